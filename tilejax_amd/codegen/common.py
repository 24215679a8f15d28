"""Pieces every gfx950 lowering shares: addressing tiles of row-major arrays, decoding tiles and steps
from the schedule, and the work lists that spread output tiles over the GPU's workgroups."""

from __future__ import annotations

import ast
import heapq
import math
from dataclasses import dataclass
from typing import Callable, Dict, List, Optional, Sequence, Tuple

import numpy as np

from .. import gfx950
from ..errors import KernelError
from ..plan import Plan, Tile, Window
from ..schedule import CODE_SHIFT, FILL_TABLE, STEP_CODE, TILE_TABLE, Schedule
from .expr import int_expr

__all__ = ["strides", "tile_base", "decode_tile", "decode_fill", "Index", "work_lists"]


def strides(shape: Sequence[int]) -> List[int]:
    out, n = [], 1
    for d in reversed(shape):
        out.append(n)
        n *= d
    return list(reversed(out))


class Index:
    """C expressions for index-array elements, `lengths[b]` -> `args.lengths[b]`, clamped into the array's
    dims where `clamp` (a runtime window index, which JAX clamps into the dim it indexes). With `constant`,
    elements are read through the constant address space (`ak_ldc`): inputs no kernel writes, so where the
    index is uniform the read is a scalar load and leaves the vector memory queue's wait counts to the data
    loads."""

    def __init__(self, plan: Plan, names: Callable[[str], Optional[str]], args: str = "args",
                 constant: bool = False) -> None:
        loops = {r.var for r in plan.loops}

        def resolve(v: str) -> Optional[str]:
            if v in loops:
                return names(v)
            value = plan.env.get(v)  # a constant of the prologue or the module (G, a block size, ...)
            if isinstance(value, bool):
                return "true" if value else "false"
            if isinstance(value, int):
                return str(value)
            return names(v)

        self.plan, self.names, self.args, self.constant = plan, resolve, args, constant

    def read(self, node: ast.Subscript) -> str:
        ix = self.plan.index(node.value.id)  # type: ignore[attr-defined]
        dims = node.slice.elts if isinstance(node.slice, ast.Tuple) else [node.slice]
        flat = "0"
        for d, (expr, stride) in enumerate(zip(dims, strides(ix.shape))):
            flat = f"({flat} + {self.expr(expr)} * {stride})"
        if self.constant:
            return f"ak_ldc({self.args}.{ix.name}, {flat})"
        return f"{self.args}.{ix.name}[{flat}]"

    def expr(self, node: ast.expr) -> str:
        return int_expr(node, self.names, self.read)


def tile_base(tile: Tile, shape: Sequence[int], index: Index, loop_value: Callable[[str], str]) -> Tuple[str, List[int]]:
    """The flat offset (C) of a tile's first element given the loop values, and the strides of its sliced
    dims. A runtime window index counts from the end when negative and is clamped into its dim, as JAX
    reads."""
    terms = []
    sliced = []
    for w, dim, stride in zip(tile.windows, shape, strides(shape)):
        if w.index is not None:
            terms.append(f"(long long)ak_index({index.read(w.index)}, {dim}) * {stride}")
        else:
            off = str(w.offset) if w.offset else ""
            if w.loop is not None:
                off = f"({loop_value(w.loop)} + {w.offset})" if w.offset else loop_value(w.loop)
            if off:
                terms.append(f"(long long)({off}) * {stride}")
        if w.size is not None:
            sliced.append(stride)
    return (" + ".join(terms) if terms else "0"), sliced


def tile_value(sch: Schedule, var: str, t: str) -> str:
    """Inner loop `var`'s value at pattern tile `t` (a runtime schedule's `tile_values`): `start + t * step`
    where that table is an arithmetic sequence (so no load waits for it), else a read of the table, which
    the kernel takes as `args.tv_<var>`."""
    vals = np.asarray(sch.tile_values[var], np.int64)
    step = int(vals[1] - vals[0]) if len(vals) > 1 else 0
    if len(vals) and np.array_equal(vals, vals[0] + step * np.arange(len(vals))):
        return f"({int(vals[0])} + ({t}) * {step})"
    return f"ak_ldc(args.tv_{var}, {t})"


def decode_tile(plan: Plan, sch: Schedule, t: str, prefix: str = "lv_", constant: bool = False) -> List[str]:
    """C statements setting `<prefix><var>` to each parallel loop's value at tile `t` (the t-th that runs);
    with `constant`, the tile tables are read through the constant address space (`ak_ldc`)."""
    lines = []
    outer, inner = sch.outer, sch.inner
    if sch.tile_tables:
        lines.append(f"const int rep_ = {t} / {sch.pattern_tiles}, tt_ = {t} % {sch.pattern_tiles};")
        rest = "rep_"
        for r in reversed(outer):
            lines.append(f"const int {prefix}{r.var} = {r.start} + ({rest} % {r.count}) * {r.step};")
            rest = f"({rest} / {r.count})"
        for r in inner:
            read = f"ak_ldc(args.{TILE_TABLE % r.var}, tt_)" if constant else f"args.{TILE_TABLE % r.var}[tt_]"
            lines.append(f"const int {prefix}{r.var} = {r.start} + {read} * {r.step};")
    else:
        rest = t
        for r in reversed(plan.parallel):
            lines.append(f"const int {prefix}{r.var} = {r.start} + (({rest}) % {r.count}) * {r.step};")
            rest = f"(({rest}) / {r.count})"
    return lines


def decode_fill(plan: Plan, sch: Schedule, f: str, prefix: str = "lv_", constant: bool = False) -> List[str]:
    """C statements setting each parallel loop's value at the f-th tile a mask skips (`constant`: as in
    `decode_tile`)."""
    lines = [f"const int frep_ = {f} / {sch.pattern_fills}, ff_ = {f} % {sch.pattern_fills};"]
    rest = "frep_"
    for r in reversed(sch.outer):
        lines.append(f"const int {prefix}{r.var} = {r.start} + ({rest} % {r.count}) * {r.step};")
        rest = f"({rest} / {r.count})"
    for r in sch.inner:
        read = f"ak_ldc(args.{FILL_TABLE % r.var}, ff_)" if constant else f"args.{FILL_TABLE % r.var}[ff_]"
        lines.append(f"const int {prefix}{r.var} = {r.start} + {read} * {r.step};")
    return lines


def static_tile_steps(sch: Schedule) -> np.ndarray:
    """For static step tables: each pattern tile's first step in the tables, and the end (one more entry)."""
    tiles = sch.tables["step_tile"]
    offsets = np.zeros(sch.pattern_tiles + 1, np.int32)
    counts = np.bincount(tiles, minlength=sch.pattern_tiles)
    offsets[1:] = np.cumsum(counts)
    return offsets


def work_lists(items: List[Tuple[int, ...]], weights: List[float], groups: List[int], grid: int) -> Tuple[np.ndarray, np.ndarray]:
    """Spread work items over `grid` persistent workgroups, longest first onto the least loaded workgroup.
    Workgroup w runs on XCD w % 8 (each XCD has its own L2). Among equally loaded workgroups the next item
    goes to the one that comes first in XCD-major order (XCD 0's workgroups, then XCD 1's, ...), and items
    of equal weight are taken in locality order (`groups`, e.g. a band of output columns, then position).
    So each round of equal items hands one XCD a run of neighbouring items, which share operand panels in
    its L2, while the balance is that of plain longest-first (a triangle of causal tiles included).
    Returns (offsets[grid + 1], items[n, width]) with each workgroup's items contiguous, in the order it
    runs them (the order they were assigned, one round after another)."""
    xcds = min(gfx950.XCDS, grid)
    slot = [(w % xcds) * ((grid + xcds - 1) // xcds) + w // xcds for w in range(grid)]
    heap = [(0.0, slot[w], w) for w in range(grid)]
    heapq.heapify(heap)
    assigned: List[List[int]] = [[] for _ in range(grid)]
    for k in sorted(range(len(items)), key=lambda k: (-weights[k], groups[k], k)):
        load, sl, w = heapq.heappop(heap)
        assigned[w].append(k)
        heapq.heappush(heap, (load + weights[k], sl, w))
    width = len(items[0]) if items else 2
    offsets = np.zeros(grid + 1, np.int32)
    flat: List[Tuple[int, ...]] = []
    for w in range(grid):
        flat.extend(items[k] for k in assigned[w])
        offsets[w + 1] = len(flat)
    return offsets, np.array(flat, np.int32).reshape(-1, width)
