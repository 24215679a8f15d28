"""The order a kernel runs its steps in, and the tables that find them.

Semantics follow the reference's schedule (src/autokernel/schedule.py:58-427) exactly, because the tables
are part of the contract (bit-exact): tiles run in the parallel loops' row-major order; a tile's steps are
its phases' steps back to back; without masks steps are arithmetic on the step index; with masks evaluated
at build time the kernel walks tables of only the tiles and steps that run:

- tile tables (a tile mask skips tiles): for every tile that runs, each inner parallel loop's block
  (`tile_<var>`), and for every skipped tile the same (`fill_<var>`), so the kernel writes its fill;
- step tables (a reduction mask skips steps): each step's tile (`step_tile`) and code (`step_code`),
  `((block * phases + phase) * iterations + iteration) << 3 | empty << 2 | first << 1 | last`, where the
  phase and iteration radices are rounded up to powers of two when the codes still fit 31 bits.

Tables cover only the loops the masks read (the innermost parallel loops from the first one any mask
reads): causal attention's masks don't read batch and head, so its tables hold one (b, h) pattern.

Masks reading index arrays (runtime masks) are evaluated on the device just before the kernel (the
generated step-table builder, codegen/steps.py): the schedule then describes every step that could run
(`capacity`), each pattern tile's inner loop values (`tile_values`) and, for phases whose masks read no
index array, which of each tile's blocks run (`static_runs`).

On gfx950 the tables live in device memory and are read through the scalar cache by the workgroup that
owns a tile: the kernel is persistent over tiles, so a workgroup decodes only its own tiles' steps.
"""

from __future__ import annotations

import ast
import itertools
import math
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np

from . import gfx950
from .plan import Plan, Range
from .syntax import used as reads

__all__ = ["CODE_SHIFT", "Schedule", "make_schedule", "STEP_TILE", "STEP_CODE", "STEP_COUNT", "TILE_TABLE",
           "FILL_TABLE"]

STEP_TILE, STEP_CODE, STEP_COUNT, TILE_TABLE, FILL_TABLE = "step_tile", "step_code", "step_count", "tile_%s", "fill_%s"
CODE_SHIFT = 3


@dataclass(frozen=True)
class Schedule:
    """Which tiles and steps a kernel runs, in order, and the tables that find them."""

    tiles: int
    total_tiles: int
    steps: int
    phase_counts: Tuple[int, ...]
    phase_steps: Tuple[int, ...]
    step_tables: bool
    outer: Tuple[Range, ...]
    inner: Tuple[Range, ...]
    pattern_tiles: int
    pattern_steps: int
    pattern_fills: int
    tile_tables: bool
    tables: Dict[str, np.ndarray] = field(default_factory=dict)
    empty: bool = False
    iterations: int = 1
    phase_radix: int = 1
    runtime: bool = False
    tile_values: Dict[str, np.ndarray] = field(default_factory=dict)
    static_runs: Dict[int, np.ndarray] = field(default_factory=dict)
    cursor: bool = False
    runtime_tiles: bool = False

    @property
    def steps_per_tile(self) -> int:
        return sum(self.phase_counts) or 1

    @property
    def repeats(self) -> int:
        return math.prod(r.count for r in self.outer)

    @property
    def fills(self) -> int:
        return self.pattern_fills * self.repeats

    def step_at(self, step: int) -> Tuple[int, int, int]:
        """(tile, phase, reduction block) of a step, as the kernel decodes it."""
        if not self.step_tables:
            tile, within = divmod(step, self.steps_per_tile)
            phase = 0
            while phase + 1 < len(self.phase_counts) and within >= self.phase_counts[phase]:
                within -= self.phase_counts[phase]
                phase += 1
            return tile, phase, within
        rep, r = divmod(step, self.pattern_steps)
        tile = rep * self.pattern_tiles + int(self.tables[STEP_TILE][r])
        phase_block = (int(self.tables[STEP_CODE][r]) >> CODE_SHIFT) // self.iterations
        return tile, phase_block % self.phase_radix, phase_block // self.phase_radix

    def first_at(self, step: int) -> bool:
        return bool(self.tables[STEP_CODE][step % self.pattern_steps] & 2)

    def empty_at(self, step: int) -> bool:
        return self.empty and bool(self.tables[STEP_CODE][step % self.pattern_steps] & 4)

    def blocks_at(self, tile: int) -> Tuple[int, ...]:
        """The parallel loops' blocks of the `tile`-th tile that runs."""
        if not self.tile_tables:
            return _mixed_radix(tile, self.outer + self.inner)
        rep, t = divmod(tile, self.pattern_tiles)
        return _mixed_radix(rep, self.outer) + tuple(int(self.tables[TILE_TABLE % r.var][t]) for r in self.inner)

    def fill_blocks_at(self, fill: int) -> Tuple[int, ...]:
        """The parallel loops' blocks of the `fill`-th skipped tile."""
        rep, t = divmod(fill, self.pattern_fills)
        return _mixed_radix(rep, self.outer) + tuple(int(self.tables[FILL_TABLE % r.var][t]) for r in self.inner)


def make_schedule(plan: Plan) -> Schedule:
    """The steps `plan`'s kernel runs; KernelError if a mask leaves nothing to run or tables don't fit."""
    nest = plan.nest
    if plan.walk:
        return _walked(plan)
    phases = [phase.range for phase in plan.phases]
    counts = tuple(r.count for r in phases)
    tile_masks = [r.mask for r in plan.parallel if r.mask is not None]
    step_masks = [r.mask for r in phases if r.mask is not None]
    if not tile_masks and not step_masks:
        return _arithmetic(plan, counts)

    instances = plan.instances
    phase_radix, iterations = _radices(plan)
    read = set().union(*(reads(m) for m in [*tile_masks, *step_masks]))
    split = next((i for i, r in enumerate(plan.parallel) if r.var in read), len(plan.parallel))
    outer, inner = plan.parallel[:split], plan.parallel[split:]

    active, skipped, steps = [], [], []
    for blocks in itertools.product(*(range(r.count) for r in inner)):
        values = _values(inner, blocks)
        if any(_holds(plan, mask, values) for mask in tile_masks):
            skipped.append(blocks)
            continue
        active.append(blocks)
        if not plan.runtime:
            steps.append([_blocks_run(plan, phases[p], values) for p, _ in instances])
    if not active:
        raise nest.error("the masks skip every output tile", nest.parallel[0].node)
    if plan.runtime:
        return _runtime(plan, counts, (phase_radix, iterations), outer, inner, active, skipped)
    step_tables = any(ks != list(range(phases[p].count)) for tile in steps for ks, (p, _) in zip(tile, instances))
    if not skipped and not step_tables:
        return _arithmetic(plan, counts)

    tables = _tile_tables(inner, active, skipped)
    empty = False
    if step_tables:
        tile_of: List[int] = []
        codes: List[int] = []
        for t, tile in enumerate(steps):
            for (p, it), ks in zip(instances, tile):
                runs = ks or [0]  # a phase none of whose blocks run takes one empty step
                empty |= not ks
                tile_of += [t] * len(runs)
                codes += [_code(kb, p, phase_radix, it, iterations, not ks, n == 0, n == len(runs) - 1)
                          for n, kb in enumerate(runs)]
        tables[STEP_TILE] = np.array(tile_of, np.int32)
        tables[STEP_CODE] = np.array(codes, np.int32)
    _check_tables(plan, tables)
    per_phase = [0] * len(phases)
    for tile in steps:
        for ks, (p, _) in zip(tile, instances):
            per_phase[p] += max(len(ks), 1)
    repeats = math.prod(r.count for r in outer)
    pattern_steps = sum(max(len(ks), 1) for tile in steps for ks in tile) or len(active)
    tiles, fills = repeats * len(active), repeats * len(skipped)
    _check_tiles(plan, tiles, fills)
    return Schedule(
        tiles=tiles, total_tiles=math.prod(r.count for r in plan.parallel), steps=repeats * pattern_steps,
        phase_counts=counts, phase_steps=tuple(repeats * per_phase[p] for p in range(len(phases))),
        step_tables=step_tables, outer=outer, inner=inner, pattern_tiles=len(active), pattern_steps=pattern_steps,
        pattern_fills=len(skipped), tile_tables=bool(skipped), tables=tables, empty=empty,
        iterations=iterations, phase_radix=phase_radix,
    )


def _radices(plan: Plan) -> Tuple[int, int]:
    phases = len(plan.phases)
    iterations = 1
    blocks = max((phase.range.count for phase in plan.phases), default=1)
    phase_radix, iteration_radix = (1 << (n - 1).bit_length() for n in (phases, iterations))
    if (blocks * phase_radix * iteration_radix) << CODE_SHIFT < 2**31:
        return phase_radix, iteration_radix
    return phases, iterations


def _runtime(plan: Plan, counts, radices, outer, inner, active, skipped) -> Schedule:
    phases = [phase.range for phase in plan.phases]
    tables = _tile_tables(inner, active, skipped)
    per_phase = [1 for _ in phases]
    capacity = len(active) * sum(count * n for count, n in zip(counts, per_phase))
    _check_tables(plan, tables, 4 * (2 * capacity + 1))
    tile_values = {r.var: np.array([r.value(blocks[i]) for blocks in active], np.int32) for i, r in enumerate(inner)}
    static_runs = {}
    for p, r in enumerate(phases):
        if r.mask is None or r.runtime:
            continue
        runs = [[not _holds(plan, r.mask, {**_values(inner, blocks), r.var: r.value(kb)}) for kb in range(r.count)]
                for blocks in active]
        static_runs[p] = np.array(runs)
    repeats = math.prod(q.count for q in outer)
    tiles = repeats * len(active)
    _check_tiles(plan, tiles, repeats * len(skipped))
    return Schedule(
        tiles=tiles, total_tiles=math.prod(r.count for r in plan.parallel), steps=repeats * capacity,
        phase_counts=counts, phase_steps=tuple(tiles * count * n for count, n in zip(counts, per_phase)),
        step_tables=True, outer=outer, inner=inner, pattern_tiles=len(active), pattern_steps=capacity,
        pattern_fills=len(skipped), tile_tables=bool(skipped), tables=tables, empty=True, runtime=True,
        tile_values=tile_values, static_runs=static_runs, iterations=radices[1], phase_radix=radices[0],
    )


def _code(block: int, phase: int, phases: int, iteration: int, iterations: int, empty: bool, first: bool, last: bool) -> int:
    return ((block * phases + phase) * iterations + iteration) << CODE_SHIFT | empty << 2 | first << 1 | last


def _values(inner: Sequence[Range], blocks: Sequence[int]) -> Dict[str, int]:
    return {r.var: r.value(b) for r, b in zip(inner, blocks)}


def _tile_tables(inner, active, skipped) -> Dict[str, np.ndarray]:
    tables: Dict[str, np.ndarray] = {}
    if skipped:
        for i, r in enumerate(inner):
            tables[TILE_TABLE % r.var] = np.array([b[i] for b in active], np.int32)
            tables[FILL_TABLE % r.var] = np.array([b[i] for b in skipped], np.int32)
    return tables


def _check_tables(plan: Plan, tables: Dict[str, np.ndarray], more: int = 0) -> None:
    size = sum(t.nbytes for t in tables.values()) + more
    size += sum(gfx950.padded_bytes(ix.shape, 4) for ix in plan.indices)
    if size > gfx950.TABLE_BUDGET:
        raise plan.nest.error(
            f"the step tables and index arrays take {size // 2**20} MiB, more than the {gfx950.TABLE_BUDGET // 2**20} "
            "MiB a kernel keeps: use bigger tiles or smaller index arrays", plan.nest.parallel[0].node)


def _check_tiles(plan: Plan, tiles: int, fills: int) -> None:
    if tiles * max(fills, 1) >= 2**31:
        raise plan.nest.error("too many output tiles for the kernel's int32 step arithmetic", plan.nest.parallel[0].node)


def _walked(plan: Plan) -> Schedule:
    """A plan of the tile as written: the kernel walks every tile of the parallel loops (evaluating tile masks
    and a runtime count of tiles itself), no tables. `steps` counts reduction-loop iterations when bounds
    and masks are static (else 0); `runtime_tiles` when the count of tiles is known only as the kernel runs."""
    from .walk import static_steps

    parallel = [plan.bounds[loop.var] for loop in plan.nest.parallel]
    runtime_tiles = not all(b.static for b in parallel)
    tiles = 0 if runtime_tiles else math.prod(b.count for b in parallel)
    steps = static_steps(plan) or 0
    return Schedule(
        tiles=tiles, total_tiles=tiles, steps=steps, phase_counts=(), phase_steps=(), step_tables=False,
        outer=plan.parallel, inner=(), pattern_tiles=tiles, pattern_steps=steps, pattern_fills=0, tile_tables=False,
        runtime_tiles=runtime_tiles,
    )


def _arithmetic(plan: Plan, counts: Tuple[int, ...]) -> Schedule:
    tiles = math.prod(r.count for r in plan.parallel)
    per_tile = sum(counts) or 1
    return Schedule(
        tiles=tiles, total_tiles=tiles, steps=tiles * per_tile, phase_counts=counts,
        phase_steps=tuple(tiles * count for count in counts), step_tables=False, outer=plan.parallel, inner=(),
        pattern_tiles=tiles, pattern_steps=tiles * per_tile, pattern_fills=0, tile_tables=False,
    )


def _blocks_run(plan: Plan, phase: Range, values: Dict[str, int]) -> List[int]:
    return [kb for kb in range(phase.count)
            if phase.mask is None or not _holds(plan, phase.mask, {**values, phase.var: phase.value(kb)})]


def _holds(plan: Plan, mask: ast.expr, values: Dict[str, int]) -> bool:
    result = plan.eval(mask, values)
    try:
        return bool(result)
    except Exception as e:
        raise plan.nest.error(
            f"masks are Python conditions on loop variables and constants, evaluated when planning; this one gave "
            f"{type(result).__name__}", mask) from e


def _mixed_radix(index: int, ranges: Sequence[Range]) -> Tuple[int, ...]:
    blocks = []
    for r in reversed(ranges):
        index, block = divmod(index, r.count)
        blocks.append(block)
    return tuple(reversed(blocks))
