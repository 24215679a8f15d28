"""How deeply a kernel buffers its copies: the part of a schedule that is the kernel's, not the user's.

The reference's Pipeline (src/autokernel/pipeline.py:42-147) counts VMEM slots per copy. On gfx950,
`input_buffers` is the depth of the ring each family streams its operands through (1-4):

- matmul: LDS stages of the A and B slices (at least 2, where they divide a step's slices and fit in LDS);
- attention: K and V blocks loaded `input_buffers - 1` blocks ahead through that many + 1 LDS stages;
- decode: K register sets and V LDS stages, steps fetched ahead (2-4).

`output_buffers` is accepted (1-3) for the reference's API and changes nothing here: the gfx950 kernels
store output tiles straight from registers, with no output copy to queue, so the tuner doesn't propose it.
`codegen.default_pipeline` gives each family the buffering it measured best (two stages for the matmul and
attention, three steps ahead for decode).

Bursts (the reference's one-step kernels grouping their DMA copies against HBM read/write turnaround) have
no counterpart in these kernels, which load through LDS rings and store from registers: a `burst` raises.
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
