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

__all__ = ["Arg", "Launch", "Program", "TRACE", "TRACE_FIELDS", "NOW"]

# A kernel generated with trace regions writes, per workgroup, TRACE_FIELDS 64-bit totals into the
# workspace buffer TRACE: input-wait ticks (pipeline fill included), fill ticks, output ticks, compute ticks
# (of the 100 MHz constant clock NOW reads), then the slices (units of streamed work) it processed.
TRACE = "ak_trace"
TRACE_FIELDS = 5
NOW = "__builtin_amdgcn_s_memrealtime()"


@dataclass(frozen=True)
class Arg:
    """One kernel argument: a pointer to an input, output, table or workspace buffer, or an int."""

    kind: str  # "input", "output", "table", "workspace", "int"
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
    lds_bytes: int = 0
    notes: Dict[str, Any] = field(default_factory=dict)  # what the lowering chose (hardware tiles, ...)
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
            self._tables[key] = {name: torch.from_numpy(np.ascontiguousarray(t)).to(device)
                                 for name, t in self.tables.items()}
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
        if outputs is None:
            outputs = [torch.empty(shape, dtype=dt.torch, device=device) for shape, dt in self.outputs]
        tables = self.device_tables(device)
        workspace = {name: torch.empty(max(n, 4), dtype=torch.uint8, device=device) for name, n in self.workspace.items()}
        module = self.module(device.index or 0)
        stream = runtime.current_stream() if stream is None else stream
        for launch in launches:
            args = pack(launch.args, arrays, outputs, tables, workspace)
            module.kernel(launch.symbol).launch(launch.grid, launch.block, launch.lds, args, stream)
        return outputs, workspace


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
        elif a.kind == "table":
            pointers.append(tables[a.key].data_ptr())
        elif a.kind == "workspace":
            pointers.append(workspace[a.key].data_ptr())
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
