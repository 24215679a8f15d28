"""How deeply a kernel buffers its copies: the part of a schedule that is the kernel's, not the user's.

The reference's Pipeline (src/autokernel/pipeline.py:42-147) counts VMEM slots per copy. On gfx950 the
same two numbers mean:

- `input_buffers`: LDS slots in the ring each streamed operand rotates through (1-4). A step's tiles are
  fetched `input_buffers - 1` steps ahead (across tile boundaries: the kernel is persistent), so more
  slots hide more HBM latency at the cost of LDS, which also bounds occupancy.
- `output_buffers`: with 2 or more, a tile's last step starts the next tile's first fetches before its
  output stores (the stores drain while the next tile computes); with 1, stores go first.

`default_pipeline` picks the deepest ring (3, as the reference measured best, else 2) that fits the LDS
the lowering needs per workgroup.
"""

from __future__ import annotations

from dataclasses import dataclass

from .errors import KernelError

__all__ = ["MAX_INPUT_BUFFERS", "MAX_OUTPUT_BUFFERS", "Pipeline"]

MAX_INPUT_BUFFERS = 4
MAX_OUTPUT_BUFFERS = 3


@dataclass(frozen=True, order=True)
class Pipeline:
    input_buffers: int = 3
    output_buffers: int = 2
    burst: int = 0

    def __post_init__(self) -> None:
        if self.burst:
            raise KernelError("pipelines of bursts are not lowered by the gfx950 backend")
        if not (1 <= self.input_buffers <= MAX_INPUT_BUFFERS and 1 <= self.output_buffers <= MAX_OUTPUT_BUFFERS):
            raise KernelError(
                f"a pipeline has 1 to {MAX_INPUT_BUFFERS} input buffers and 1 to {MAX_OUTPUT_BUFFERS} output "
                f"buffers, not {self.input_buffers} and {self.output_buffers}"
            )

    def __str__(self) -> str:
        return f"{self.input_buffers} input / {self.output_buffers} output buffers"
