"""The host half of a generated kernel: its launches, argument packing, device tables and outputs.

A `Program` is what `Lowered.run` calls (the gfx950 counterpart of the reference's generated
`entry(*inputs)`, src/autokernel/codegen.py:456-502): it allocates the outputs with torch on the inputs'
device, uploads the kernel's constant tables once per device, runs its launches on torch's current
stream through libak, and returns the outputs.
"""

from __future__ import annotations

import struct
from dataclasses import dataclass, field
from typing import Any, Dict, List, Optional, Sequence, Tuple

import numpy as np
import torch

from .. import jaxlite, runtime
from ..errors import KernelError

__all__ = ["Arg", "Launch", "Program", "TRACE", "TRACE_FIELDS", "NOW", "CLOCK_START", "CLOCK_END"]

# A kernel generated with trace regions writes, per workgroup, TRACE_FIELDS 64-bit totals into the
# workspace buffer TRACE: input-wait ticks (pipeline fill included), fill ticks, output ticks, compute ticks
# (of the 100 MHz constant clock NOW reads), the slices (units of streamed work) it processed, then the
# shader clock's cycles (s_memtime) and the constant clock's ticks over the workgroup's whole run: their
# ratio is the clock the kernel ran at, measured on the chip rather than derived from a counter.
TRACE = "ak_trace"
TRACE_FIELDS = 7
NOW = "__builtin_amdgcn_s_memrealtime()"
CLOCK_START = ("const unsigned long long ak_cyc0 = __builtin_amdgcn_s_memtime(), "
               "ak_rt0 = __builtin_amdgcn_s_memrealtime();")
CLOCK_END = "tr[5] = __builtin_amdgcn_s_memtime() - ak_cyc0; tr[6] = __builtin_amdgcn_s_memrealtime() - ak_rt0;"


@dataclass(frozen=True)
class Arg:
    """One kernel argument: a pointer to an input, output, table or workspace buffer, or an int."""

    kind: str  # "input", "output", "table", "state", "workspace", "int"
    key: Any  # input/output position, table/workspace name, or the int's value
    ctype: str  # the C type of the struct field
    name: str


@dataclass
class Launch:
    symbol: str
    args: List[Arg]
    grid: Tuple[int, int, int]
    block: Tuple[int, int, int]
    lds: int = 0  # dynamic LDS bytes


@dataclass
class Program:
    name: str
    source: str
    launches: List[Launch]
    outputs: List[Tuple[Tuple[int, ...], jaxlite.DType]]
    inputs: List[Tuple[Tuple[int, ...], jaxlite.DType]]
    tables: Dict[str, np.ndarray] = field(default_factory=dict)
    workspace: Dict[str, int] = field(default_factory=dict)  # name -> bytes (uninitialised: launches write before reading)
    # name -> int32 count: counters kept on the device from call to call, zero when made (once per device);
    # a kernel that uses one leaves it zero again when it ends (the work queues' heads). One set per program
    # and device, shared by every call: two calls of a program with state must not overlap (on two streams
    # of one device), or each takes the other's items; nothing here checks that. No standard lowering has
    # state: the matmul family's queued tail (gemm.QUEUE_TAIL) is off, since it measured slower.
    state: Dict[str, int] = field(default_factory=dict)
    lds_bytes: int = 0
    notes: Dict[str, Any] = field(default_factory=dict)  # what the lowering chose (hardware tiles, ...)
    protocol: Any = field(default=None, repr=False, compare=False)  # the LDS ring's events (protocol.Recorder)
    parts: Tuple[Any, ...] = field(default=(), repr=False, compare=False)  # the programs a composite one joins
    _modules: Dict[int, runtime.Module] = field(default_factory=dict, repr=False)
    _tables: Dict[int, Dict[str, torch.Tensor]] = field(default_factory=dict, repr=False)

    def module(self, device: int) -> runtime.Module:
        if device not in self._modules:
            with torch.cuda.device(device):
                self._modules[device] = runtime.load(self.source, f"{self.name}.hip")
        return self._modules[device]

    def device_tables(self, device: torch.device) -> Dict[str, torch.Tensor]:
        key = device.index or 0
        if key not in self._tables:
            made = {name: torch.from_numpy(np.ascontiguousarray(t)).to(device) for name, t in self.tables.items()}
            made.update({name: torch.zeros(max(n, 1), dtype=torch.int32, device=device)
                         for name, n in self.state.items()})
            self._tables[key] = made
        return self._tables[key]

    def check_inputs(self, arrays: Sequence[torch.Tensor]) -> None:
        if len(arrays) != len(self.inputs):
            raise KernelError(f"{self.name} takes {len(self.inputs)} inputs, got {len(arrays)}")
        device = arrays[0].device
        for k, (t, (shape, dt)) in enumerate(zip(arrays, self.inputs)):
            if tuple(t.shape) != shape or t.dtype != dt.torch:
                raise KernelError(f"{self.name}: input {k} is {tuple(t.shape)} {t.dtype}, built for {shape} {dt.name}")
            if t.device != device:
                raise KernelError(f"{self.name}: inputs are on different devices")
            if not t.is_contiguous():
                raise KernelError(f"{self.name}: input {k} must be contiguous")
        if device.type != "cuda":
            raise KernelError(f"{self.name} runs on the GPU: its inputs are on {device}")

    def __call__(self, *arrays: torch.Tensor, outputs: Optional[Sequence[torch.Tensor]] = None,
                 stream: Optional[int] = None) -> Any:
        outputs, _ = self._run(arrays, outputs, stream, self.launches)
        return outputs[0] if len(outputs) == 1 else tuple(outputs)

    def run_traced(self, *arrays: torch.Tensor) -> Tuple[Any, Optional[torch.Tensor]]:
        """One call of a program generated with trace regions: its outputs, and its trace buffer (per
        workgroup: input-wait, fill, output and compute ticks of the 100 MHz clock, then steps), or None."""
        outputs, workspace = self._run(arrays, None, None, self.launches)
        trace = workspace.get(TRACE)
        result = outputs[0] if len(outputs) == 1 else tuple(outputs)
        return result, (trace.view(torch.int64) if trace is not None else None)

    def scratch_layout(self) -> Dict[str, Tuple[int, int]]:
        """Where each workspace buffer sits in the library's scratch array: name -> (offset, bytes), offsets
        256-aligned in name order. KernelError if they don't fit."""
        layout, at = {}, 0
        for name in sorted(self.workspace):
            n = max(self.workspace[name], 4)
            layout[name] = (at, n)
            at += -(-n // runtime.SCRATCH_ALIGN) * runtime.SCRATCH_ALIGN
        if at > runtime.SCRATCH_BYTES:
            raise KernelError(f"{self.name}: its workspace takes {at} bytes, more than the {runtime.SCRATCH_BYTES} "
                              "bytes of the library's scratch array: call it with a workspace allocated per call")
        return layout

    def run_no_alloc(self, *arrays: torch.Tensor, outputs: Sequence[torch.Tensor],
                     stream: Optional[int] = None) -> None:
        """One call that allocates no device memory: the caller's outputs, and every workspace buffer placed in
        the library's scratch array (ak_launch_scratch). The kernel's constant tables are uploaded on a
        device's first call (once), as for ordinary calls. Calls that overlap on one GPU share its scratch
        array and race."""
        runtime.require_gpu()
        self.check_inputs(arrays)
        device = arrays[0].device
        if len(outputs) != len(self.outputs):
            raise KernelError(f"{self.name} has {len(self.outputs)} outputs, {len(outputs)} given")
        for k, (t, (shape, dt)) in enumerate(zip(outputs, self.outputs)):
            if tuple(t.shape) != shape or t.dtype != dt.torch or t.device != device or not t.is_contiguous():
                raise KernelError(f"{self.name}: output {k} must be a contiguous {shape} {dt.name} tensor on {device}")
        layout = self.scratch_layout()
        tables = self.device_tables(device)
        module = self.module(device.index or 0)
        stream = runtime.current_stream() if stream is None else stream
        for launch in self.launches:
            placeholders = {name: _Null() for name in self.workspace}
            args = pack(launch.args, arrays, outputs, tables, placeholders)
            pointer_args = [a for a in launch.args if a.kind != "int"]
            placed = [(8 * i, *_placed(layout, a.key)) for i, a in enumerate(pointer_args) if a.kind == "workspace"]
            module.kernel(launch.symbol).launch_scratch(launch.grid, launch.block, launch.lds, args, stream, placed)

    def step_tables(self, *arrays: torch.Tensor) -> Dict[str, torch.Tensor]:
        """Run only the device step-table builder (runtime masks) and return its tables as int32 tensors:
        step_tile, step_code, count (the reference's three) and tile_steps."""
        builder = [launch for launch in self.launches if launch.symbol == self.notes.get("step_builder")]
        if not builder:
            raise KernelError(f"{self.name} has no runtime masks, so no device step tables")
        _, workspace = self._run(arrays, None, None, builder)
        return {name: t.view(torch.int32) for name, t in workspace.items()}

    def _run(self, arrays, outputs, stream, launches):
        runtime.require_gpu()
        self.check_inputs(arrays)
        device = arrays[0].device
        poison = self.notes.get("poison", False)  # a poisoned build (codegen/poison.py): outputs and workspaces NaN
        if outputs is None:
            outputs = [_poisoned(shape, dt.torch, device) if poison else torch.empty(shape, dtype=dt.torch, device=device)
                       for shape, dt in self.outputs]
        tables = self.device_tables(device)
        workspace = {name: (torch.full((max(n, 4),), 0xFF, dtype=torch.uint8, device=device) if poison
                            else torch.empty(max(n, 4), dtype=torch.uint8, device=device))
                     for name, n in self.workspace.items()}
        module = self.module(device.index or 0)
        stream = runtime.current_stream() if stream is None else stream
        for launch in launches:
            args = pack(launch.args, arrays, outputs, tables, workspace)
            module.kernel(launch.symbol).launch(launch.grid, launch.block, launch.lds, args, stream)
        return outputs, workspace


def _placed(layout: Dict[str, Tuple[int, int]], key: Any) -> Tuple[int, int]:
    """Where a workspace argument sits in the scratch array: (offset, bytes) of its buffer, or past a byte
    offset into it."""
    name, offset = key if isinstance(key, tuple) else (key, 0)
    at, n = layout[name]
    return at + offset, n - offset


def _poisoned(shape, dtype: torch.dtype, device) -> torch.Tensor:
    """An output of a poisoned build: NaN, or -1 for an integer dtype."""
    fill = float("nan") if dtype.is_floating_point else -1
    return torch.full(shape, fill, dtype=dtype, device=device)


class _Null:
    """A workspace buffer not allocated here: its pointer field is packed as 0 and filled in by the library."""

    @staticmethod
    def data_ptr() -> int:
        return 0


def pack(args: Sequence[Arg], arrays: Sequence[torch.Tensor], outputs: Sequence[torch.Tensor],
         tables: Dict[str, torch.Tensor], workspace: Dict[str, torch.Tensor]) -> bytes:
    """The kernel's argument struct: pointers first (8 bytes each), then 32-bit ints, as `c_struct` lays
    it out."""
    pointers, ints = [], []
    for a in args:
        if a.kind == "int":
            ints.append(int(a.key))
        elif a.kind == "input":
            pointers.append(arrays[a.key].data_ptr())
        elif a.kind == "output":
            pointers.append(outputs[a.key].data_ptr())
        elif a.kind in ("table", "state"):
            pointers.append(tables[a.key].data_ptr())
        elif a.kind == "workspace":  # a name, or (name, byte offset) for a pointer into the buffer
            name, offset = a.key if isinstance(a.key, tuple) else (a.key, 0)
            pointers.append(workspace[name].data_ptr() + offset if offset else workspace[name].data_ptr())
        else:
            raise KernelError(f"unknown argument kind {a.kind}")
    data = struct.pack(f"<{len(pointers)}Q", *pointers) + struct.pack(f"<{len(ints)}i", *ints)
    return data + b"\0" * (-len(data) % 8)


def c_struct(name: str, args: Sequence[Arg]) -> str:
    """The C struct a kernel takes its arguments in (pointers first, then ints)."""
    lines = [f"struct {name} {{"]
    for a in args:
        if a.kind != "int":
            lines.append(f"  {a.ctype} {a.name};")
    for a in args:
        if a.kind == "int":
            lines.append(f"  int {a.name};")
    lines.append("};")
    return "\n".join(lines)
