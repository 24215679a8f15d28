"""The order a kernel runs its steps in, and the tables that find them.

The semantics are the reference's (src/autokernel/schedule.py:58-427), because the tables are part of the
contract and must match bit for bit: tiles run in the parallel loops' row-major order; a tile's steps are
its phases' steps back to back; without masks, steps are arithmetic on the step index; with masks
evaluated at build time the kernel walks tables of only the tiles and steps that run:

- tile tables (a tile mask skips tiles): for every tile that runs, each inner parallel loop's block
  (`tile_<var>`), and for every skipped tile the same (`fill_<var>`), so the kernel writes its fill;
- step tables (a reduction mask skips steps): each step's tile (`step_tile`) and code (`step_code`),
  `((block * phases + phase) * iterations + iteration) << 3 | empty << 2 | first << 1 | last`, where the
  phase and iteration radices are rounded up to powers of two when the codes still fit 31 bits. A phase
  none of whose blocks run in a tile still takes one step, at block 0, flagged empty.

Tables cover only the loops the masks read (the innermost parallel loops from the first one any mask
reads): causal attention's masks don't read batch and head, so its tables hold one (b, h) pattern.

How it is computed here: the masks are evaluated once per point of the covered loops into boolean
matrices, one per phase, of shape (tiles that run, the phase's blocks): `True` where the block runs. A
tile's row with no `True` gets one at block 0 (its empty step). Laying the phases' matrices side by side,
the steps of the pattern are exactly the `True` entries in row-major order, so the step tables, the
first/last flags (where the (tile, phase) group changes) and the per-phase counts are array operations
on that one matrix.

Masks reading index arrays (runtime masks) are evaluated on the device just before the kernel (the
generated step-table builder, codegen/steps.py): the schedule then describes every step that could run
(`capacity`), each pattern tile's inner loop values (`tile_values`) and, for phases whose masks read no
index array, which of each tile's blocks run (`static_runs`).

On gfx950 the tables live in device memory and are read through the scalar cache by the workgroup that
owns a tile: the kernel is persistent over tiles, so a workgroup decodes only its own tiles' steps.
"""

from __future__ import annotations

import ast
import bisect
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
EMPTY_BIT, FIRST_BIT, LAST_BIT = 4, 2, 1


@dataclass(frozen=True)
class Schedule:
    """Which tiles and steps a kernel runs, in order, and the tables that find them. A "pattern" is what
    the tables list for one combination of the outer parallel loops (those no mask reads); the run repeats
    it `repeats` times."""

    tiles: int  # tiles that run
    total_tiles: int  # every tile of the parallel loops
    steps: int  # steps over the whole run (runtime masks: the most there can be)
    phase_counts: Tuple[int, ...]  # blocks of each phase's reduction loop
    phase_steps: Tuple[int, ...]  # steps each phase takes over the whole run
    step_tables: bool  # steps found through `step_tile` / `step_code`
    outer: Tuple[Range, ...]  # parallel loops no mask reads
    inner: Tuple[Range, ...]  # parallel loops the tables cover
    pattern_tiles: int
    pattern_steps: int
    pattern_fills: int
    tile_tables: bool  # tiles found through `tile_<var>` / `fill_<var>`
    tables: Dict[str, np.ndarray] = field(default_factory=dict)
    empty: bool = False  # may a step be empty
    iterations: int = 1  # the iteration's radix in a step code
    phase_radix: int = 1  # the phase's radix in a step code
    runtime: bool = False  # step tables made on the device from runtime masks
    tile_values: Dict[str, np.ndarray] = field(default_factory=dict)
    static_runs: Dict[int, np.ndarray] = field(default_factory=dict)
    cursor: bool = False
    runtime_tiles: bool = False  # the count of tiles is known only as the kernel runs (walk plans)

    @property
    def steps_per_tile(self) -> int:
        """A tile's steps when nothing is masked: every phase's blocks, or one step without phases."""
        return max(sum(self.phase_counts), 1)

    @property
    def repeats(self) -> int:
        return int(np.prod([r.count for r in self.outer], dtype=np.int64))

    @property
    def fills(self) -> int:
        return self.repeats * self.pattern_fills

    def _code(self, step: int) -> int:
        return int(self.tables[STEP_CODE][step % self.pattern_steps])

    def step_at(self, step: int) -> Tuple[int, int, int]:
        """(tile, phase, reduction block) of a step, as the kernel decodes it."""
        if self.step_tables:
            pattern, at = divmod(step, self.pattern_steps)
            tile = pattern * self.pattern_tiles + int(self.tables[STEP_TILE][at])
            block, phase = divmod((self._code(step) >> CODE_SHIFT) // self.iterations, self.phase_radix)
            return tile, phase, block
        tile, at = divmod(step, self.steps_per_tile)
        if not self.phase_counts:
            return tile, 0, at
        ends = np.cumsum(self.phase_counts)
        phase = min(bisect.bisect_right(ends.tolist(), at), len(ends) - 1)
        return tile, phase, at - int(ends[phase] - self.phase_counts[phase])

    def first_at(self, step: int) -> bool:
        return (self._code(step) & FIRST_BIT) != 0

    def empty_at(self, step: int) -> bool:
        return self.empty and (self._code(step) & EMPTY_BIT) != 0

    def blocks_at(self, tile: int) -> Tuple[int, ...]:
        """The parallel loops' blocks of the `tile`-th tile that runs."""
        if self.tile_tables:
            pattern, at = divmod(tile, self.pattern_tiles)
            return _unravel(pattern, self.outer) + tuple(int(self.tables[TILE_TABLE % r.var][at]) for r in self.inner)
        return _unravel(tile, self.outer + self.inner)

    def fill_blocks_at(self, fill: int) -> Tuple[int, ...]:
        """The parallel loops' blocks of the `fill`-th skipped tile."""
        pattern, at = divmod(fill, self.pattern_fills)
        return _unravel(pattern, self.outer) + tuple(int(self.tables[FILL_TABLE % r.var][at]) for r in self.inner)


def _unravel(index: int, ranges: Sequence[Range]) -> Tuple[int, ...]:
    if not ranges:
        return ()
    return tuple(int(b) for b in np.unravel_index(index, [r.count for r in ranges]))


# ----------------------------------------------------------------------------------------------------------
# Building a schedule


def make_schedule(plan: Plan) -> Schedule:
    """The steps `plan`'s kernel runs; KernelError if a mask leaves nothing to run or tables don't fit."""
    if plan.walk:
        return _walked(plan)
    counts = tuple(phase.range.count for phase in plan.phases)
    masks = [r.mask for r in plan.parallel if r.mask is not None]
    masks += [phase.range.mask for phase in plan.phases if phase.range.mask is not None]
    if not masks:
        return _arithmetic(plan, counts)
    grid = _Grid.of(plan, masks)
    if plan.runtime:
        return grid.runtime_schedule(counts)
    runs = grid.static_runs(range(len(plan.phases)))
    skips_steps = any(not m.all() for m in runs)
    if not grid.skipped.size and not skips_steps:
        return _arithmetic(plan, counts)  # the masks skip nothing
    return grid.table_schedule(counts, runs, skips_steps)


@dataclass
class _Grid:
    """The points of the parallel loops the masks read (`inner`, row-major), split into the tiles that run
    (`active`) and those a tile mask skips (`skipped`), as (tiles, len(inner)) arrays of block indices."""

    plan: Plan
    outer: Tuple[Range, ...]
    inner: Tuple[Range, ...]
    active: np.ndarray
    skipped: np.ndarray

    @staticmethod
    def of(plan: Plan, masks: List[ast.expr]) -> "_Grid":
        read = set().union(*(reads(m) for m in masks))
        covered = [i for i, r in enumerate(plan.parallel) if r.var in read]
        cut = covered[0] if covered else len(plan.parallel)
        outer, inner = tuple(plan.parallel[:cut]), tuple(plan.parallel[cut:])
        shape = [r.count for r in inner]
        points = np.stack(np.unravel_index(np.arange(int(np.prod(shape, dtype=np.int64))), shape), axis=1) \
            if inner else np.zeros((1, 0), np.int64)
        tile_masks = [r.mask for r in plan.parallel if r.mask is not None]
        skip = np.array([any(_holds(plan, m, _at(inner, p)) for m in tile_masks) for p in points], dtype=bool)
        if skip.all():
            raise plan.nest.error("the masks skip every output tile", plan.nest.parallel[0].node)
        return _Grid(plan, outer, inner, points[~skip], points[skip])

    @property
    def repeats(self) -> int:
        return math.prod(r.count for r in self.outer)

    def values(self, tile: int) -> Dict[str, int]:
        return _at(self.inner, self.active[tile])

    def static_runs(self, phases) -> List[np.ndarray]:
        """Per phase: a bool matrix (active tiles, blocks), True where the phase's mask lets the block run."""
        out = []
        for p in phases:
            r = self.plan.phases[p].range
            if r.mask is None:
                out.append(np.ones((len(self.active), r.count), dtype=bool))
                continue
            out.append(np.array([[not _holds(self.plan, r.mask, {**self.values(t), r.var: r.value(kb)})
                                  for kb in range(r.count)] for t in range(len(self.active))], dtype=bool)
                       .reshape(len(self.active), r.count))
        return out

    def tile_tables(self) -> Dict[str, np.ndarray]:
        if not self.skipped.size:
            return {}
        tables: Dict[str, np.ndarray] = {}
        for axis, r in enumerate(self.inner):
            tables[TILE_TABLE % r.var] = self.active[:, axis].astype(np.int32)
            tables[FILL_TABLE % r.var] = self.skipped[:, axis].astype(np.int32)
        return tables

    def table_schedule(self, counts: Tuple[int, ...], runs: List[np.ndarray], skips_steps: bool) -> Schedule:
        plan = self.plan
        phase_radix, iterations = _code_radices(plan)
        n_active = len(self.active)
        tables = self.tile_tables()
        # one step per (tile, phase) group at least: an empty group takes block 0, flagged empty
        empty_groups = [~m.any(axis=1) for m in runs]
        slots = [np.where(e, 1, m.sum(axis=1)) for m, e in zip(runs, empty_groups)]
        per_phase = [int(s.sum()) for s in slots]
        pattern_steps = sum(per_phase) or n_active
        if skips_steps:
            tables[STEP_TILE], tables[STEP_CODE] = _step_tables(runs, empty_groups, phase_radix, iterations)
        _check_tables(plan, tables)
        tiles, fills = self.repeats * n_active, self.repeats * len(self.skipped)
        _check_tiles(plan, tiles, fills)
        return Schedule(
            tiles=tiles, total_tiles=math.prod(r.count for r in plan.parallel), steps=self.repeats * pattern_steps,
            phase_counts=counts, phase_steps=tuple(self.repeats * n for n in per_phase), step_tables=skips_steps,
            outer=self.outer, inner=self.inner, pattern_tiles=n_active, pattern_steps=pattern_steps,
            pattern_fills=len(self.skipped), tile_tables=bool(self.skipped.size), tables=tables,
            empty=skips_steps and any(e.any() for e in empty_groups), iterations=iterations, phase_radix=phase_radix,
        )

    def runtime_schedule(self, counts: Tuple[int, ...]) -> Schedule:
        """Every step that could run, for the device builder to compact; the parts it can't know itself."""
        plan = self.plan
        phase_radix, iterations = _code_radices(plan)
        n_active = len(self.active)
        capacity = n_active * sum(counts)
        tables = self.tile_tables()
        _check_tables(plan, tables, 4 * (2 * capacity + 1))
        tile_values = {r.var: (r.start + self.active[:, axis] * r.step).astype(np.int32)
                       for axis, r in enumerate(self.inner)}
        static = [p for p, ph in enumerate(plan.phases) if ph.range.mask is not None and not ph.range.runtime]
        static_runs = dict(zip(static, self.static_runs(static)))
        tiles = self.repeats * n_active
        _check_tiles(plan, tiles, self.repeats * len(self.skipped))
        return Schedule(
            tiles=tiles, total_tiles=math.prod(r.count for r in plan.parallel), steps=self.repeats * capacity,
            phase_counts=counts, phase_steps=tuple(tiles * c for c in counts), step_tables=True,
            outer=self.outer, inner=self.inner, pattern_tiles=n_active, pattern_steps=capacity,
            pattern_fills=len(self.skipped), tile_tables=bool(self.skipped.size), tables=tables, empty=True,
            runtime=True, tile_values=tile_values, static_runs=static_runs, iterations=iterations,
            phase_radix=phase_radix,
        )


def _step_tables(runs: List[np.ndarray], empty_groups: List[np.ndarray], phase_radix: int,
                 iterations: int) -> Tuple[np.ndarray, np.ndarray]:
    """The pattern's `step_tile` and `step_code`: the True entries, in row-major order, of the phases'
    run matrices laid side by side (each empty group's block 0 set)."""
    kept = [m.copy() for m in runs]
    for m, e in zip(kept, empty_groups):
        m[e, 0] = True
    side = np.concatenate(kept, axis=1)
    phase_of = np.concatenate([np.full(m.shape[1], p) for p, m in enumerate(kept)])
    block_of = np.concatenate([np.arange(m.shape[1]) for m in kept])
    tile, column = np.nonzero(side)
    phase, block = phase_of[column].astype(np.int64), block_of[column].astype(np.int64)
    group = tile.astype(np.int64) * len(kept) + phase
    first = np.ones(len(group), dtype=bool)
    first[1:] = group[1:] != group[:-1]
    last = np.ones(len(group), dtype=bool)
    last[:-1] = group[:-1] != group[1:]
    empty = np.zeros(len(group), dtype=bool)
    for p, e in enumerate(empty_groups):
        empty |= (phase == p) & e[tile]
    iteration = 0  # phases of steps run once per tile: no repeat loops
    code = ((block * phase_radix + phase) * iterations + iteration) << CODE_SHIFT
    code |= empty * EMPTY_BIT | first * FIRST_BIT | last * LAST_BIT
    return tile.astype(np.int32), code.astype(np.int32)


def _code_radices(plan: Plan) -> Tuple[int, int]:
    """The phase's and the iteration's radices in a step code: the next powers of two of their counts (so
    the kernel decodes with shifts), unless a code would then pass 31 bits; then the counts themselves."""
    n_phases, n_iterations = len(plan.phases), 1
    widest = max([phase.range.count for phase in plan.phases] or [1])
    rounded = tuple(1 << max(n - 1, 0).bit_length() for n in (n_phases, n_iterations))
    if widest * rounded[0] * rounded[1] < 1 << (31 - CODE_SHIFT):
        return rounded
    return n_phases, n_iterations


def _at(ranges: Sequence[Range], blocks) -> Dict[str, int]:
    return {r.var: r.value(int(b)) for r, b in zip(ranges, blocks)}


def _check_tables(plan: Plan, tables: Dict[str, np.ndarray], more: int = 0) -> None:
    size = more + sum(t.nbytes for t in tables.values())
    size += sum(gfx950.padded_bytes(ix.shape, 4) for ix in plan.indices)
    if size > gfx950.TABLE_BUDGET:
        raise plan.nest.error(
            f"the step tables and index arrays take {size // 2**20} MiB, more than the {gfx950.TABLE_BUDGET // 2**20} "
            "MiB a kernel keeps: use bigger tiles or smaller index arrays", plan.nest.parallel[0].node)


def _check_tiles(plan: Plan, tiles: int, fills: int) -> None:
    if tiles * max(fills, 1) >= 2**31:
        raise plan.nest.error("too many output tiles for the kernel's int32 step arithmetic", plan.nest.parallel[0].node)


def _holds(plan: Plan, mask: ast.expr, values: Dict[str, int]) -> bool:
    """Does `mask` (a build-time Python condition) skip the point `values`?"""
    result = plan.eval(mask, values)
    try:
        return bool(result)
    except Exception as e:
        raise plan.nest.error(
            f"masks are Python conditions on loop variables and constants, evaluated when planning; this one gave "
            f"{type(result).__name__}", mask) from e


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
    """No tables: tile t's blocks are t in mixed radix over the parallel loops, its steps t's share of the
    step index."""
    tiles = math.prod(r.count for r in plan.parallel)
    per_tile = max(sum(counts), 1)
    return Schedule(
        tiles=tiles, total_tiles=tiles, steps=tiles * per_tile, phase_counts=counts,
        phase_steps=tuple(tiles * c for c in counts), step_tables=False, outer=plan.parallel, inner=(),
        pattern_tiles=tiles, pattern_steps=tiles * per_tile, pattern_fills=0, tile_tables=False,
    )
