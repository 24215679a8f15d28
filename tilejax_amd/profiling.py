"""Where a kernel's time goes on the GPU: device time from HIP events, and the kernel's own trace regions.

The reference reads libtpu trace regions `<k>/wait`, `<k>/out_wait`, `<k>/compute` from a profiler trace
(src/autokernel/profiling.py:95-274). On gfx950 the same breakdown comes from the kernel itself: a kernel
generated with `trace=True` stamps `s_memrealtime` (the 100 MHz constant clock) around its waits for
input slices, its output stores and its compute, per workgroup, into a trace buffer; `measure` sums them.
Device time per call is measured with HIP events on the stream the kernel runs on, after a warm-up call,
as the median of `runs` calls (the reference's timing method: benchmarks/timing.py:12-22).

`KernelProfile.bottleneck` classifies as the reference does: "dma" when exposed input waits plus output
waits exceed 20 % of the device time, "overhead" when time outside every region exceeds 30 %, else
"compute"; None when no regions were recorded.
"""

from __future__ import annotations

import statistics
import time
from dataclasses import dataclass, field
from typing import Any, Dict, Optional, Sequence

from .codegen.program import TRACE_FIELDS  # per workgroup: wait, fill, out_wait, compute (ticks), steps, cycles, ticks
from .errors import KernelError

__all__ = ["DMA_BOUND_SHARE", "OVERHEAD_BOUND_SHARE", "KernelProfile", "enable_profiling", "measure", "profile",
           "summarize"]

DMA_BOUND_SHARE = 0.2
OVERHEAD_BOUND_SHARE = 0.3
CLOCK_HZ = 100e6  # s_memrealtime


@dataclass
class KernelProfile:
    """A kernel's time per call on the device (seconds), and, with trace regions, its breakdown."""

    name: str
    config: Any
    calls: int
    device_s: float
    regions: bool = False
    steps: float = 0.0
    wait_s: float = 0.0
    fill_s: float = 0.0
    out_wait_s: float = 0.0
    compute_s: float = 0.0
    scopes: Dict[str, float] = field(default_factory=dict)
    samples: Sequence[float] = ()
    clock_hz: float = 0.0  # the shader clock the traced workgroups ran at (s_memtime cycles over 100 MHz ticks)

    @property
    def exposed_wait_s(self) -> float:
        return max(0.0, self.wait_s - self.fill_s)

    @property
    def other_s(self) -> float:
        return max(0.0, self.device_s - self.wait_s - self.out_wait_s - self.compute_s)

    @property
    def bottleneck(self) -> Optional[str]:
        if not self.regions:
            return None
        if (self.exposed_wait_s + self.out_wait_s) > DMA_BOUND_SHARE * self.device_s:
            return "dma"
        if self.other_s > OVERHEAD_BOUND_SHARE * self.device_s:
            return "overhead"
        return "compute"

    def __str__(self) -> str:
        us = lambda s: f"{s * 1e6:10.1f} us"  # noqa: E731
        lines = [f"{self.name} ({self.config}): {us(self.device_s).strip()} per call over {self.calls} calls"]
        if self.regions:
            per_step = self.device_s / self.steps if self.steps else 0.0
            lines += [
                f"  steps          {self.steps:10.0f}     ({per_step * 1e6:.2f} us each)",
                f"  compute        {us(self.compute_s)}",
                f"  input waits    {us(self.exposed_wait_s)}  (+{us(self.fill_s).strip()} filling the pipeline)",
                f"  output waits   {us(self.out_wait_s)}",
                f"  other          {us(self.other_s)}  (decoding steps, starting loads, draining)",
                f"  shader clock   {self.clock_hz / 1e9:10.3f} GHz (cycles over constant-clock ticks, in the kernel)",
                f"  bottleneck: {self.bottleneck}",
            ]
        return "\n".join(lines)


def enable_profiling() -> None:
    """Kept for the reference's API (src/autokernel/profiling.py:69-79), where libtpu must be told to record
    trace regions before JAX starts. Here a kernel built with trace=True stamps its own regions, so there
    is nothing to enable."""


def summarize(stamps: Any, name: str, config: Any, calls: int, device_s: float, workgroups: int,
              slots: int = 0) -> KernelProfile:
    """A profile from a trace buffer of per-workgroup region totals (in clock ticks): rows of
    [wait, fill, out_wait, compute, steps, shader cycles, ticks], summed over `calls` calls. Time per call is
    the total over workgroups divided by the number that run side by side (`slots`, default all of them):
    with more workgroups than that, a slot runs several in turn. The shader clock is the workgroups' cycles
    over their ticks (each workgroup weighted by how long it ran)."""
    import numpy as np

    t = np.asarray(stamps, dtype=np.float64).reshape(workgroups, -1)
    per = t.sum(axis=0) / max(min(workgroups, slots or workgroups), 1) / max(calls, 1)
    ticks = 1.0 / CLOCK_HZ
    return KernelProfile(
        name=name, config=config, calls=calls, device_s=device_s, regions=True,
        wait_s=per[0] * ticks, fill_s=per[1] * ticks, out_wait_s=per[2] * ticks, compute_s=per[3] * ticks,
        steps=float(t[:, 4].sum()) / max(calls, 1),
        clock_hz=float(t[:, 5].sum() / t[:, 6].sum() * CLOCK_HZ) if t.shape[1] > 6 and t[:, 6].sum() > 0 else 0.0,
    )


def measure(lowered: Any, inputs: Sequence[Any], runs: int = 5) -> KernelProfile:
    """Time a generated kernel: one warm-up call, then `runs` calls back to back with HIP events between
    them on the current stream; the median per call (with trace regions when the kernel was generated with
    them)."""
    import torch

    from . import runtime

    runtime.require_gpu()
    stream = runtime.current_stream()
    # load the spin kernel (on its first use in the process) now: loaded between the warm-up and the timed
    # calls, it leaves the GPU idle long enough for its clock to drop, and the first kernel timed runs slow
    runtime.spin(0.0, stream)
    program = lowered.program
    workgroups = program.notes.get("trace_workgroups", 0) if lowered.trace else 0
    lowered.run(*inputs)
    torch.cuda.synchronize()
    # The calls run back to back, with an event between consecutive ones. A spin kernel queued ahead of
    # them holds the GPU for twice the host's launch time of all of them (measured on a second warm-up
    # call), so every call is queued before the GPU reaches it and host time never counts as device time.
    events = [runtime.Event() for _ in range(runs + 1)]
    traces = []
    start = time.perf_counter()
    if workgroups:
        program.run_traced(*inputs)
    else:
        lowered.run(*inputs)
    host_s = time.perf_counter() - start
    torch.cuda.synchronize()
    runtime.spin(2.0 * runs * host_s + 1e-4, stream)
    events[0].record(stream)
    for k in range(runs):
        if workgroups:
            traces.append(program.run_traced(*inputs)[1])
        else:
            lowered.run(*inputs)
        events[k + 1].record(stream)
    torch.cuda.synchronize()
    samples = [events[k].elapsed_ms(events[k + 1]) * 1e-3 for k in range(runs)]
    stamps = None
    for trace in traces:
        t = trace[: workgroups * TRACE_FIELDS].cpu()
        stamps = t if stamps is None else stamps + t
    device_s = statistics.median(samples)
    if workgroups:
        result = summarize(stamps.numpy(), lowered.plan.nest.name, lowered.config, runs, device_s, workgroups,
                           program.notes.get("trace_slots", 0))
        result.steps /= max(program.notes.get("slices_per_step", 1), 1)
        result.samples = samples
        return result
    return KernelProfile(lowered.plan.nest.name, lowered.config, runs, device_s, samples=samples)


def profile(kernel: Any, args: Sequence[Any], runs: int = 5) -> KernelProfile:
    """Where `kernel`'s time goes on the GPU for these inputs (and tunable, if given)."""
    from .api import _as_tensor as _tensor

    arrays, _ = kernel._arguments(tuple(args))
    config = kernel.lower(*args).config
    lowered = kernel.lowered(kernel.signature(*arrays), config, trace=True)
    return measure(lowered, [_tensor(a) for a in arrays], runs)
