"""Lower a planned loop nest to gfx950: HIP C++ source plus the host program that launches it.

The reference's codegen emits one Pallas kernel per loop nest (src/autokernel/codegen.py:91-1755). Here a
loop nest's traced tile code is matched against the kernel families the backend lowers, each a persistent
HIP kernel generated from the plan and schedule:

- `gemm`: `acc += a @ b` (or `@ b.T`) over a reduction loop, then a pointwise epilogue (dense, causal and
  grouped matmuls), also with two right operands whose products the epilogue combines; a feed-forward chain
  (`acc += act(x @ w1, x @ w2) @ w3` over hidden blocks, the MoE expert layer) runs as two such kernels
  (chain.py);
- `flash`: the online-softmax reduction of attention over static masks (causal flash attention);
- `decode`: the same reduction under runtime masks and runtime page windows (paged decode attention).

Every other loop nest (and one a family recognises but can't take, say a head dim it has no layout for)
lowers to `generic`: one persistent kernel evaluating the traced tile code pass by pass per tile, correct
for any nest the planner accepts and tuned for none. A nest even that can't lower raises KernelError.
"""

from __future__ import annotations

import re
from typing import Any, Dict, List, Optional, Tuple

from ..errors import KernelError
from ..pipeline import Pipeline
from ..plan import Plan
from ..schedule import Schedule
from .program import Program

__all__ = ["Program", "default_pipeline", "generate", "hardware_choices"]


def _symbol(plan: Plan) -> str:
    return "tj_" + re.sub(r"[^A-Za-z0-9_]", "_", plan.nest.name)


def _family(plan: Plan) -> Tuple[str, Any]:
    """The kernel family that takes `plan` and its match, or ("generic", error or None): the first family
    whose matcher recognises the nest; a family that recognises it but can't take it leaves its KernelError."""
    from . import chain, decode, flash, gemm

    if plan.walk:
        return "generic", None
    try:
        for name, module in (("chain", chain), ("gemm", gemm), ("flash", flash), ("decode", decode)):
            found = module.match(plan)
            if found is not None:
                return name, found
    except KernelError as e:
        return "generic", e
    return "generic", None


def default_pipeline(plan: Plan, schedule: Schedule) -> Pipeline:
    """The buffering each family measured best at the BASELINE configs: two LDS stages for the matmul (a
    256x256x64 bf16 tile fills 128 KiB with two) and for attention (two 4-wave workgroups per CU), three
    steps ahead for decode. Output buffers: the reference's default two, which change nothing here (the gfx950
    kernels store from registers, see pipeline.py)."""
    family, _ = _family(plan)
    return Pipeline(3 if family == "decode" else 2, 2)


def hardware_choices(plan: Plan, schedule: Schedule) -> List[Tuple[Tuple[str, int], ...]]:
    """The kernel shapes tuning may try for `plan` beside its buffering, as sorted (knob, value) tuples, the
    default first: the matmul's workgroup tile, attention's waves per workgroup and keys per block."""
    from . import flash, gemm

    family, found = _family(plan)
    choices: List[Dict[str, int]] = [{}]
    if family == "gemm":
        choices = gemm.hardware_choices(found)
    elif family == "flash":
        choices = flash.hardware_choices(found)
    return [()] + [tuple(sorted(c.items())) for c in choices[1:]]  # () is the default shape


def generate(plan: Plan, schedule: Schedule, pipeline: Pipeline, *, trace: bool = False,
             cursor: bool = False, hardware: Optional[Dict[str, int]] = None) -> Program:
    """The program for this plan, schedule and pipeline (and `hardware` knobs of the family's kernel shape,
    from `hardware_choices`); with `cursor`, a kernel with runtime masks finds its steps itself as it runs
    rather than from device-built step tables (the decode family). The knob `poison` builds the program's
    poisoned form (codegen/poison.py: LDS, outputs and workspaces start as NaN), for tests."""
    knobs = dict(hardware or {})
    poison = knobs.pop("poison", 0)
    program = _generate(plan, schedule, pipeline, trace=trace, cursor=cursor, hardware=knobs)
    if poison:
        from .poison import poison_program

        poison_program(program)
    return program


def _generate(plan: Plan, schedule: Schedule, pipeline: Pipeline, *, trace: bool, cursor: bool,
              hardware: Dict[str, int]) -> Program:
    from . import chain, decode, flash, gemm, generic

    name = _symbol(plan)
    if plan.walk:
        if cursor:
            raise KernelError(f"{plan.nest.name}: a plan of the tile as written finds its steps as it runs already "
                              "(no cursor mode)")
        return generic.lower_walk(plan, schedule, pipeline, name, trace=trace)
    family_error = None
    try:
        found = chain.match(plan)
        if found is not None:
            if cursor:
                raise KernelError(f"{plan.nest.name}: the matmul family reads runtime masks from device step "
                                  "tables (no cursor)")
            return chain.lower(plan, schedule, pipeline, found, name, trace=trace)
        found = gemm.match(plan)
        if found is not None:
            if cursor:
                raise KernelError(f"{plan.nest.name}: the matmul family reads runtime masks from device step "
                                  "tables (no cursor)")
            return gemm.lower(plan, schedule, pipeline, found, name, trace=trace, hardware=hardware)
        found = flash.match(plan)
        if found is not None:
            return flash.lower(plan, schedule, pipeline, found, name, trace=trace, hardware=hardware)
        found = decode.match(plan)
        if found is not None:
            return decode.lower(plan, schedule, pipeline, found, name, trace=trace, cursor=cursor, hardware=hardware)
    except KernelError as e:
        family_error = e
        if hardware:  # knobs of the family's kernel shape: that shape doesn't build, whatever else would
            raise
    if cursor:
        raise family_error or KernelError(f"{plan.nest.name}: only the decode family finds its steps with a cursor")
    try:
        return generic.lower(plan, schedule, pipeline, name, trace=trace)
    except KernelError as e:
        why = f"; {family_error}" if family_error is not None else ""
        raise KernelError(f"{plan.nest.name}: the gfx950 backend has no lowering for this loop nest: {e}{why}") from e
