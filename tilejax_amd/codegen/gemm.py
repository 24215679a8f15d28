"""Lowering of matmul-shaped loop nests: `acc += a[...] @ b[...]` (or `@ b[...].T`) over a reduction
loop, then a pointwise epilogue stored into one output tile. Dense and causal matmul
(examples/matmul.py:22-35 and examples/causal_matmul.py:23-40 of the reference) and the grouped matmul
whose right operand is a runtime window `w[group_expert[i // G], ...]` take this path.

The generated kernel is persistent: one workgroup per CU (256 threads, four waves in a 2x2 grid), each
walking its own list of work items. An item is a hardware tile of BM x BN outputs inside one spec tile
(the loop nest's tile), or a fill: a hardware tile whose value the schedule or the epilogue fixes without
computing (a tile the mask skips, or one the epilogue's `where` proves constant). For a compute item the
workgroup walks the spec tile's steps (arithmetic, or decoded from the step tables), each split into
BK-deep slices that stream through `stages` LDS stages:

- loads go straight from HBM to LDS (`buffer_load_dwordx4 ... lds`, 16 bytes a lane, one buffer resource
  per operand tile), each lane fetching the global chunk that belongs at its XOR-swizzled LDS position;
- the right operand of `a @ b` stays N-contiguous in LDS and is read transposed with
  `ds_read_b64_tr_b16`, so both MFMA operands arrive K-contiguous with no register shuffles;
- each stage is its own LDS array, which lets the compiler keep later stages' loads in flight while it
  reads this one; the barrier for a slice sits one K16 step before it, so the next slice's first fragments
  load under this slice's last MFMAs (`v_mfma_f32_32x32x16_bf16`, f32 accumulators in AGPRs), and
  `sched_group_barrier` hints interleave each MFMA with an LDS read or a global load;
- the epilogue is computed per element where the accumulator lives; for bf16 outputs a lane and lane ^ 32
  exchange halves so each stores 8 consecutive outputs (16 bytes), and a row's stores fill whole lines.
"""

from __future__ import annotations

import ast
from dataclasses import dataclass
from typing import Any, Dict, List, Optional, Tuple

import numpy as np

from .. import gfx950, jaxlite
from ..errors import KernelError
from ..jaxlite import Node
from ..pipeline import Pipeline
from ..plan import Kind, Operand, Output, Plan
from ..schedule import CODE_SHIFT, FILL_TABLE, STEP_CODE, STEP_TILE, TILE_TABLE, Schedule
from .common import Index, decode_fill, decode_tile, static_tile_steps, strides, tile_base, work_lists
from .device import PRELUDE
from .expr import ElementEmitter, Emitter, Interval, ctype, intervals, literal, nodes_between
from .program import CLOCK_END, CLOCK_START, NOW, TRACE, TRACE_FIELDS, Arg, Launch, Program, c_struct
from .protocol import ItemRecorder, Recorder

__all__ = ["GemmMatch", "match", "lower"]

THREADS = 256  # the fixup kernel's workgroup
WAVE_GRIDS = {4: (2, 2), 8: (2, 4)}  # waves of the matmul workgroup along M and N, by waves per workgroup
MFMA = 32  # 32x32x16 bf16 MFMA tiles


@dataclass
class GemmMatch:
    a: Operand
    b: Operand
    b_nt: bool  # `a @ b.T`: b's tile is (tn, tk), K-contiguous
    kvar: Optional[str]  # the reduction loop's variable (None: no reduction loop)
    tm: int
    tn: int
    tk: int
    acc: Node  # the Node standing for the accumulator in the epilogue
    init: float
    out: Output
    value: Any  # the stored value (Node, or a number)
    # A row prologue: the left operand is a pointwise function of its load and k-wise row vectors (`a_expr`,
    # None for a plain load), and other carried values are row sums of such functions (`side`: (name, summand,
    # initial value)), which the epilogue may read (the reference's examples/rmsnorm_matmul.py:33-46).
    a_expr: Optional[Node] = None
    side: Tuple[Tuple[str, Node, float], ...] = ()
    k0: int = 0  # the value of a reduction loop of one step (not among the plan's phases)
    # A first reduction loop before the matmul's (the reference's tests/test_codegen.py:580-611): carried row
    # sums of row-prologue functions of the left operand's array (`pre`: (name, summand, "tile" for a tile
    # summed elementwise and read through jnp.sum(axis=1), "row" for a (rows, 1) sum)), and the row statistics
    # the code between the loops computes from them and the matmul's prologue reads (`stats`: (name, value)).
    pre: Tuple[Tuple[str, Node, str], ...] = ()
    stats: Tuple[Tuple[str, Node], ...] = ()
    mphase: int = 0  # the matmul's reduction loop
    # A second product of the same left operand tile (`u += a[...] @ b2[...]` beside `acc += a[...] @ b[...]`,
    # b2 an array of b's shape read at b's window): the epilogue reads both accumulators (`acc2`), as a gated
    # feed-forward's gate and up projections do (the reference's examples/moe.py:180-182).
    b2: Optional[Operand] = None
    acc2: Optional[Node] = None


def _is(node: Any, op: str) -> bool:
    return isinstance(node, Node) and node.op == op


_OPERAND_TYPES = ("bfloat16", "float32")  # operand types `@` takes: bf16, or f32 as six bf16 products
# f32 operands as bf16 parts x = x1 + x2 + x3: the BK-deep slices each slice of an operand becomes, so that
# slice by slice the products are a1 b1 + a1 b2 + a2 b1 + a1 b3 + a2 b2 + a3 b1 (every pair of parts whose
# product is above about 2^-24 of a b)
F32_PARTS = {"a": (1, 1, 2, 1, 2, 3), "b": (1, 2, 1, 3, 2, 1)}
_POINTWISE = {"astype", "multiply", "add", "subtract", "divide", "negative", "maximum", "minimum", "full"}


def _row_prologue(plan: Plan, expr: Any, x: Optional[Node] = None, stats: frozenset = frozenset()) -> Optional[Node]:
    """The one 2-D load a pointwise bf16 or f32 expression is a function of, besides loads of k-wise row
    vectors ((1, n) tiles), row statistics (carried values named in `stats`) and constants; None if it is
    anything else. With `x`, that load must be `x`."""
    if not isinstance(expr, Node):
        return None
    loads = []
    for n in nodes_between(expr):
        if n.op == "load":
            loads.append(n)
        elif n.op == "carried" and n.kwargs["name"] in stats:
            continue
        elif n.op not in _POINTWISE:
            return None
    main = [n for n in loads if len(n.shape) == 2 and n.shape[0] != 1]
    if len({id(n) for n in main}) != 1 or (x is not None and main[0] is not x):
        return None
    if any(len(n.shape) != 2 or (n.shape[0] != 1 and n is not main[0]) for n in loads):
        return None
    return main[0]


def _dot_of_loads(plan: Plan, node: Node, stats: frozenset = frozenset()
                  ) -> Optional[Tuple[Operand, Operand, bool, Optional[Node], Optional[Node]]]:
    """(a's operand, b's operand, `a @ b.T`, a's expression if it isn't a plain load, a's load)."""
    if not (_is(node, "dot") or _is(node, "dot_nt")) or node.dtype.name != "float32":
        return None
    a, b = node.args[0], node.args[1]
    a_expr = None
    if not _is(a, "load"):
        x = _row_prologue(plan, a, stats=stats)
        if x is None or a.dtype.name not in _OPERAND_TYPES or a.shape != x.shape:
            return None
        a_expr, a = a, x
    if not _is(b, "load"):
        return None
    opa, opb = plan.operand(a.kwargs["operand"]), plan.operand(b.kwargs["operand"])
    if opa.tile.dtype.name not in _OPERAND_TYPES or opb.tile.dtype.name not in _OPERAND_TYPES:
        return None
    if len(opa.tile.shape) != 2 or len(opb.tile.shape) != 2:
        return None
    return opa, opb, node.op == "dot_nt", a_expr, a


def _is_f32(m: "GemmMatch") -> bool:
    """Does the product read f32 operands (`@` at HIGHEST precision, src/autokernel/mxu.py:21-43)?"""
    a_type = (m.a_expr.dtype if m.a_expr is not None else m.a.tile.dtype).name
    return "float32" in (a_type, m.b.tile.dtype.name)


_UNIFORM_OPS = _POINTWISE | {"rsqrt", "sqrt", "exp", "log", "reciprocal", "square", "tanh", "sigmoid"}


def _column_uniform(node: Node, side: set) -> bool:
    """Is `node` the same in every column: built pointwise from row sums (`side`: carried values, or the
    sums `_row_sum_name` names) and constants only?"""
    stack, seen = [node], set()
    while stack:
        n = stack.pop()
        if n.id in seen:
            continue
        seen.add(n.id)
        if n.op == "carried":
            if n.kwargs["name"] not in side:
                return False
            continue
        if n.op == "reduce_sum" and _row_sum_name(n) in side:
            continue
        if n.op not in _UNIFORM_OPS:
            return False
        stack.extend(n.inputs())
    return True


def _row_sum_name(n: Node) -> str:
    """The name a row sum in a one-step tile's epilogue goes by (a carried value's, in a loop)."""
    return f"_sum{n.id}"


def _side_sum(plan: Plan, name: str, x: Node, mp: int = 0) -> Optional[Tuple[str, Node, float]]:
    """A carried value whose update is `c + jnp.sum(h, axis=1, keepdims=True)`, h a row-prologue function of
    the left operand's load, from a constant: (name, h, initial value)."""
    body, seg0 = plan.scopes[f"body{mp}"], plan.scopes["seg0" if mp == 0 else f"end{mp - 1}"]
    new, init = body.values.get(name), seg0.values.get(name)
    leaf = body.carried_in.get(name)
    if not (isinstance(new, jaxlite.Sym) and _is(new.node, "add")) or leaf is None:
        return None
    u, v = new.node.args
    red = v if u is leaf else u if v is leaf else None
    if not (_is(red, "reduce_sum") and red.kwargs.get("axis") in (1, -1) and red.kwargs.get("keepdims")):
        return None
    h = red.args[0]
    if _row_prologue(plan, h, x) is None:
        return None
    if isinstance(init, jaxlite.Sym) and _is(init.node, "full"):
        return name, h, float(init.node.kwargs["value"])
    if isinstance(init, (int, float)):
        return name, h, float(init)
    return None


def _first_pass(plan: Plan) -> Optional[Tuple[List[Tuple[str, Node, str]], Dict[str, Node], str]]:
    """A first reduction loop of row sums, before the matmul's: (its sums, the row statistics computed from
    them between the loops and carried into the matmul's loop, the array they read); None if it is anything
    else. Each sum is `c + h` (a tile summed elementwise, read afterwards only through jnp.sum(c, axis=1,
    keepdims=True)) or `c + jnp.sum(h, axis=1, keepdims=True)`, from zero, h a row-prologue function of one
    load."""
    body, seg0, end, body1 = (plan.scopes[k] for k in ("body0", "seg0", "end0", "body1"))
    pre: List[Tuple[str, Node, str]] = []
    arrays = set()
    for name, leaf in body.carried_in.items():
        new = body.values.get(name)
        if not (isinstance(new, jaxlite.Sym) and _is(new.node, "add")):
            return None
        u, v = new.node.args
        h = v if u is leaf else u if v is leaf else None
        kind = "tile"
        if _is(h, "reduce_sum"):
            if not (h.kwargs.get("axis") in (1, -1) and h.kwargs.get("keepdims")):
                return None
            h, kind = h.args[0], "row"
        x = _row_prologue(plan, h)
        init = seg0.values.get(name)
        zero = (isinstance(init, jaxlite.Sym) and _is(init.node, "full") and float(init.node.kwargs["value"]) == 0.0) \
            or (isinstance(init, (int, float)) and float(init) == 0.0)
        if x is None or not zero or (kind == "tile" and h.shape != new.node.shape):
            return None
        arrays.add(plan.operand(x.kwargs["operand"]).tile.array)
        pre.append((name, h, kind))
    if len(arrays) != 1:
        return None
    kinds = {name: kind for name, _, kind in pre}
    stats: Dict[str, Node] = {}
    for name, leaf in body1.carried_in.items():
        got = end.values.get(name)
        if name in kinds or not isinstance(got, jaxlite.Sym) or body1.values.get(name) is None:
            continue
        if not (isinstance(body1.values[name], jaxlite.Sym) and body1.values[name].node is leaf):
            continue  # updated in the matmul's loop: not a statistic
        stack, ok = [got.node], True
        while stack and ok:
            n = stack.pop()
            if n.op == "carried":
                ok = kinds.get(n.kwargs["name"]) == "row"
            elif n.op == "reduce_sum" and _is(n.args[0], "carried") and kinds.get(n.args[0].kwargs["name"]) == "tile":
                ok = n.kwargs.get("axis") in (1, -1) and bool(n.kwargs.get("keepdims"))
            elif n.op in _UNIFORM_OPS:
                stack.extend(n.inputs())
            else:
                ok = False
        if ok:
            stats[name] = got.node
    return pre, stats, next(iter(arrays))


def match(plan: Plan) -> Optional[GemmMatch]:
    """The matmul this loop nest is, or None."""
    if len(plan.outputs) != 1 or len(plan.phases) > 2:
        return None
    mp = len(plan.phases) - 1 if plan.phases else 0
    pre: List[Tuple[str, Node, str]] = []
    stats: Dict[str, Node] = {}
    if mp == 1:
        first = _first_pass(plan)
        if first is None:
            return None
        pre, stats, pre_array = first
    out = plan.outputs[0]
    if len(out.tile.shape) != 2:
        return None
    last = plan.scopes["last"]
    value = last.stores.get(out.name)
    root = value.node if isinstance(value, jaxlite.Sym) else None
    side: List[Tuple[str, Node, float]] = []
    acc2, acc2_leaf, found2 = None, None, None  # a second product of the left operand (GemmMatch.b2)
    if plan.phases:
        body, seg0 = plan.scopes[f"body{mp}"], plan.scopes["seg0" if mp == 0 else f"end{mp - 1}"]
        products = []  # (carried value, its product's operands): the carried values matmuls accumulate into
        for name in body.carried_in:
            new = body.values.get(name)
            if not (isinstance(new, jaxlite.Sym) and _is(new.node, "add")):
                continue
            x, y = new.node.args
            leaf = body.carried_in.get(name)
            dot = y if x is leaf else x if y is leaf else None
            got = _dot_of_loads(plan, dot, frozenset(stats)) if isinstance(dot, Node) else None
            if got is not None:
                products.append((name, got))
        if not products:
            return None
        products.sort(key=lambda p_: p_[0])  # (by name: the carried values' order varies from run to run)
        acc, found = products[0]
        if len(products) == 2 and mp == 0:
            acc2, found2 = products[1]
            if not _second_product(found, found2) or \
                    tuple(plan.inputs[found[1].param].shape) != tuple(plan.inputs[found2[1].param].shape):
                return None
        elif len(products) > 1:
            return None
        if pre and plan.operand(found[4].kwargs["operand"]).tile.array != pre_array:
            return None
        init = seg0.values.get(acc)
        for name in plan.carried:  # every other carried value: a row sum of the left operand's prologue
            if name not in (acc, acc2) and name not in stats and not any(name == p_[0] for p_ in pre):
                got = _side_sum(plan, name, found[4], mp)
                if got is None:
                    return None
                side.append(got)
        if isinstance(init, jaxlite.Sym) and _is(init.node, "full"):
            init_value = float(init.node.kwargs["value"])
        elif isinstance(init, (int, float)):
            init_value = float(init)
        else:
            return None
        acc_leaf = last.carried_in.get(acc)
        if acc_leaf is None or root is None:
            return None
        if acc2 is not None:
            acc2_leaf = last.carried_in.get(acc2)
            init2 = seg0.values.get(acc2)
            same = (isinstance(init2, jaxlite.Sym) and _is(init2.node, "full")
                    and float(init2.node.kwargs["value"]) == init_value) or init2 == init_value
            if acc2_leaf is None or side or not same:
                return None
        kvar = plan.phases[mp].range.var
    else:
        if root is None:
            return None
        dots = [n for n in nodes_between(root) if n.op in ("dot", "dot_nt")]
        if len(dots) != 1:
            return None
        found = _dot_of_loads(plan, dots[0])
        if found is None:
            return None
        acc_leaf, init_value, kvar = dots[0], 0.0, None
        # a reduction of one step: the row sums a loop would carry are sums of the whole row, inline
        for n in nodes_between(root):
            if n.op == "reduce_sum":
                if not (n.kwargs.get("axis") in (1, -1) and n.kwargs.get("keepdims")
                        and _row_prologue(plan, n.args[0], found[4]) is not None):
                    return None
                side.append((_row_sum_name(n), n.args[0], 0.0))
    opa, opb, nt, a_expr, _ = found
    tm, tk = opa.tile.shape
    tn, tkb = (opb.tile.shape if nt else opb.tile.shape[::-1])
    if tkb != tk or tuple(out.tile.shape) != (tm, tn):
        return None
    # The operands' rows/columns must be the output's: same loops placing them.
    arow = [w for w in opa.tile.windows if w.size is not None]
    brow = [w for w in opb.tile.windows if w.size is not None]
    orow = [w for w in out.tile.windows if w.size is not None]
    bcol = brow[0] if nt else brow[1]
    bk = brow[1] if nt else brow[0]
    if (arow[0].loop, arow[0].offset) != (orow[0].loop, orow[0].offset):
        return None
    if (bcol.loop, bcol.offset) != (orow[1].loop, orow[1].offset):
        return None
    if kvar is not None and (arow[1].loop != kvar or bk.loop != kvar):
        return None
    k0 = 0
    if kvar is None and (arow[1].loop is not None or bk.loop is not None):
        # a reduction loop of one step joins the code around it, its variable bound to its start
        one = {r.var: r.start for r in plan.reductions if r.count == 1 and r.mask is None}
        if arow[1].loop != bk.loop or arow[1].loop not in one:
            return None
        kvar, k0 = arow[1].loop, one[arow[1].loop]
    if out.dtype.name not in ("bfloat16", "float32"):
        return None
    if pre and a_expr is None:
        a_expr = found[4]  # (the row pass writes the operand: its first loop reads the same array)
    b2 = found2[1] if found2 is not None else None
    return GemmMatch(opa, opb, nt, kvar, tm, tn, tk, acc_leaf, init_value, out, value, a_expr, tuple(side), k0,
                     tuple(pre), tuple(stats.items()), mp, b2, acc2_leaf)


def _tile_level(phase: Any) -> bool:
    """Does the reduction loop's mask (if any) leave its variable unread, so it keeps a tile's blocks all or
    none?"""
    return phase.mask is None or phase.var not in {n.id for n in ast.walk(phase.mask) if isinstance(n, ast.Name)}


def _windows(op: Operand) -> Tuple[Tuple[Any, ...], ...]:
    """Where an operand's tile sits: each dim's loop, offset and size, and its runtime index's expression."""
    return tuple((w.loop, w.offset, w.size, ast.dump(w.index) if w.index is not None else None, w.index_loops)
                 for w in op.tile.windows)


def _second_product(first: Tuple, second: Tuple) -> bool:
    """Is `second` (a `_dot_of_loads` result) a second product of `first`'s left operand tile: the same window
    of the same array, plain loads of bf16, and a right operand of another array of the same shape and dtype
    read at the same window (runtime window indices included)?"""
    opa, opb, nt, a_expr, _ = first
    opa2, opb2, nt2, a_expr2, _ = second
    if nt or nt2 or a_expr is not None or a_expr2 is not None:
        return False
    if opa.tile.array != opa2.tile.array or _windows(opa) != _windows(opa2):
        return False
    if opb.tile.array == opb2.tile.array or _windows(opb) != _windows(opb2):
        return False
    return opb.tile.shape == opb2.tile.shape and all(o.tile.dtype.name == "bfloat16" for o in (opa, opb, opb2))


@dataclass(frozen=True)
class HwTile:
    """A workgroup's share of a spec tile: BM x BN outputs, K walked in BK-deep slices through `stages` LDS
    stages (one array per stage and operand)."""

    bm: int
    bn: int
    bk: int
    stages: int
    waves: int = 4  # per workgroup: 4 (one per SIMD, 128 x 128 each of a 256 x 256 tile) or 8 (two per SIMD)
    dual: bool = False  # two right operands (GemmMatch.b2): LDS holds BN columns of each, 2 BN in all

    @property
    def grid(self) -> Tuple[int, int]:
        return WAVE_GRIDS[self.waves]

    @property
    def bn_lds(self) -> int:
        """Right-operand columns a stage holds: BN, or BN of each of two operands."""
        return 2 * self.bn if self.dual else self.bn

    @property
    def lds(self) -> int:
        return self.stages * (self.bm + self.bn_lds) * self.bk * 2


def hardware_tile(m: GemmMatch, pipeline: Pipeline, hardware: Optional[Dict[str, int]] = None) -> HwTile:
    """The workgroup tile for a spec tile (tm, tn, tk): at most 256 x 256 outputs (`hardware` may cap each
    side, "bm" and "bn"), computed by eight waves (two per SIMD, 128 x 64 each) for a 256 x 256 tile and by
    four (128 x 128 each at most) for a smaller one, unless "waves" says otherwise; K slices of 64 (32 if tk
    is an odd multiple of 64, 16 for tk = 32) so every tile's slice count is even, and the LDS stages the
    pipeline asks for where they divide a step's slices and fit in LDS."""
    hardware = hardware or {}
    dual = m.b2 is not None
    # two right operands: 128 output columns of each fill the 256 LDS columns of a plain 256 x 256 tile
    bm, bn = min(m.tm, hardware.get("bm", 256)), min(m.tn, hardware.get("bn", 128 if dual else 256))
    waves = hardware.get("waves", default_waves(bm, 2 * bn if dual else bn))
    if waves not in WAVE_GRIDS:
        raise KernelError(f"the gfx950 matmul lowering runs workgroups of 4 or 8 waves, not {waves}")
    if m.tm % bm or m.tn % bn or bm % 64 or bn % 64:
        raise KernelError(f"the gfx950 matmul lowering needs tiles that are multiples of 64 (got {m.tm} x {m.tn})")
    if m.tk % 64 and m.tk != 32:
        raise KernelError(f"the gfx950 matmul lowering needs a reduction block of 32 or a multiple of 64 (got {m.tk})")
    bk = 64 if m.tk % 128 == 0 else 32 if m.tk % 64 == 0 else 16

    def deepest(bk_: int) -> int:
        kslices = m.tk // bk_
        for s in range(max(2, pipeline.input_buffers), 1, -1):
            if kslices % s == 0 and s * (bm + (2 if dual else 1) * bn) * bk_ * 2 <= gfx950.LDS_BUDGET:
                return s
        return 2

    stages = deepest(bk)
    # More buffers than 64-deep slices can have in LDS: slices half as deep, so loads run further ahead.
    if pipeline.input_buffers > stages and bk == 64 and deepest(32) > stages:
        bk, stages = 32, deepest(32)
    wm, wn = WAVE_GRIDS[waves]
    if bm % (32 * wm) or bn % (32 * wn):
        # (with two right operands each wave takes the same whole 32-column blocks of both)
        raise KernelError(f"a {bm} x {bn} workgroup tile does not split into {waves} waves of whole 32 x 32 blocks")
    return HwTile(bm, bn, bk, stages, waves, dual)


# Small items (K-split chunks, filled and constant tiles) pulled from a shared queue once a workgroup's own
# list is done (True), or placed in the lists ahead of time like whole tiles (False). Measured on one box,
# causal 8192^3 at 512^3 tiles: 484.8-487.7 us with the queue, 479.1-483.7 us without (the queue narrows the
# workgroups' spread, but its pulls and the later stores cost more than that gains); with the last round in
# 8 chunks per tile, 480.5-483.3 against 475.9-482.8 us.
# With it on, the queue's heads are per program and device (Program.state): calls of one queued program
# must not overlap on two streams.
QUEUE_TAIL = [False]
PATCHES = [True]  # locality groups of a column band and a patch of rows (False: the column band alone)
# A locality group's column band, in workgroup tiles: an XCD's round of 32 tiles is then a patch 8 tiles wide
# and 4 high. Measured at 8192^3 (256 x 256 tiles, four rounds alternating): 8 wide 812-839 us against 817-846
# at 4 wide (dense), 456-459 against 460-465 (causal), the MoE grouped matmul level; 1, 2, 16 and 32 wide
# 1006-1026, 911-925, 856-863 and 860-866 us (dense).
BAND_TILES = [8]
# The last round's K-split: at most MAX_SPLIT chunks per tile. Its chunks run at the kernel's end, when their
# reads, f32 partials and the filled tiles' stores share HBM, and the fixup reads the partials again: causal
# 8192^3 at 512^3 tiles measured 484 us at 16 chunks of 8 slices, 475-478 at 8 of 16, 477-480 at 4 of 32.
# Running a workgroup's small items (fills, constants, its chunk) before its whole tiles, all of them or the
# fills alone, or after its first or second whole tile by workgroup, measured 5-25 us slower. The fixup inside
# this kernel (chunks first in their lists, each counted in after an agent-scope release, the fixup in parts
# last in the lists of the workgroups without a chunk, each after an agent-scope acquire) was bit-equal and
# slower: 514-523 against 461-471 us with a release per wave (each an L2 write-back), 470-474 with one per
# chunk, 465-470 with no fence at all; at 1024^3, 75, 43 and 27 against 23 us.
MAX_SPLIT = 8


def lower(plan: Plan, sch: Schedule, pipeline: Pipeline, m: GemmMatch, name: str, trace: bool = False,
          hardware: Optional[Dict[str, int]] = None) -> Program:
    hw = hardware_tile(m, pipeline, hardware)
    return _Gemm(plan, sch, pipeline, m, hw, name, trace).program()


def default_waves(bm: int, bn: int) -> int:
    """Waves per workgroup when the tuner doesn't say: eight for a 256 x 256 tile, four for a smaller one.
    Measured at 8192^3 (bf16, 512^3 spec tiles), five runs each in alternating order on one box: dense 805-824
    us with eight waves against 819-842 with four, causal 459-468 against 469-479; the grouped MoE GEMM of
    16384 x 4096 x 14336 equal (1772 against 1766 us)."""
    return 8 if (bm, bn) == (256, 256) else 4


def hardware_choices(m: GemmMatch) -> List[Dict[str, int]]:
    """The workgroup tiles tuning may try for this match, as caps on each side (256 x 256 first, the
    default; then 256 x 128, 128 x 256 and 128 x 128 where the spec tile divides into them), each also with
    the other number of waves per workgroup (four or eight) where the tile splits into them."""
    found, seen = [], set()
    dual = m.b2 is not None
    shapes = ((256, 128), (128, 128), (256, 64), (128, 64)) if dual else ((256, 256), (256, 128), (128, 256), (128, 128))
    for bm, bn in shapes:
        got = (min(m.tm, bm), min(m.tn, bn))
        if got in seen or m.tm % got[0] or m.tn % got[1]:
            continue
        seen.add(got)
        found.append({"bm": bm, "bn": bn})
    other = []
    for h in found:
        tile = (min(m.tm, h["bm"]), min(m.tn, h["bn"]))
        waves = 12 - default_waves(tile[0], tile[1] * (2 if dual else 1))  # the other of 4 and 8
        wm, wn = WAVE_GRIDS[waves]
        if tile[0] % (32 * wm) == 0 and tile[1] % (32 * wn) == 0:
            other.append({**h, "waves": waves})
    return found + other


class _Gemm:
    def __init__(self, plan: Plan, sch: Schedule, pipeline: Pipeline, m: GemmMatch, hw: HwTile, name: str,
                 trace: bool = False) -> None:
        self.plan, self.sch, self.pipeline, self.m, self.hw, self.name = plan, sch, pipeline, m, hw, name
        self.trace = trace
        self.sub_m, self.sub_n = m.tm // hw.bm, m.tn // hw.bn
        self.subs = self.sub_m * self.sub_n
        self.tables: Dict[str, np.ndarray] = {}
        self.const_value: Optional[float] = None
        self.split: Optional[Tuple[int, int, int]] = None  # (items cut, chunks per item, K slices per chunk)
        self.prologue = m.a_expr is not None or bool(m.side) or bool(m.pre)
        # f32 operands: each goes to HBM as three bf16 parts (ak_split3), and the kernel sums the six products
        # of F32_PARTS in f32 on the bf16 MFMAs, within a few 2^-24 of x y; the f32 MFMAs would run at a
        # sixteenth of the bf16 rate. The parts array has six BK-deep slices for each of the operand's.
        self.x3 = _is_f32(m)
        self.kx = len(F32_PARTS["a"]) if self.x3 else 1
        self.dual = hw.dual
        if self.dual and (self.x3 or self.prologue):
            raise KernelError("the gfx950 matmul lowering takes two right operands for bf16 loads without a prologue")
        if self.prologue:
            self._check_prologue()
        if self.x3:
            self._check_parts()

    def _check_prologue(self) -> None:
        """A row prologue runs as its own pass over the left operand's whole array: its rows are the output's
        rows and its columns the reduction, every block of which the loop visits."""
        plan, sch, m = self.plan, self.sch, self.m
        shape = plan.inputs[m.a.param].shape
        wins = [w for w in m.a.tile.windows if w.size is not None]
        if len(shape) != 2 or len(wins) != 2 or len(m.a.tile.windows) != 2:
            raise KernelError("a matmul's row prologue is lowered for a 2-D left operand only")
        rows, cols = wins
        if sch.runtime or any(ph.range.mask is not None for ph in plan.phases):
            raise KernelError("a matmul's row prologue is lowered for unmasked reduction loops only")
        if rows.offset != 0 or cols.offset != 0 or shape[1] % 8:
            raise KernelError("a matmul's row prologue needs windows from the array's start and rows of a "
                              "multiple of 8 elements")
        if plan.phases:
            r = plan.phases[m.mphase].range
            if not (r.start == 0 and r.step == m.tk and r.count * m.tk == shape[1]):
                raise KernelError("a matmul's row prologue needs a reduction loop over the whole row")
            first = plan.phases[0].range
            if m.pre and not (first.start == 0 and first.count * first.step == shape[1]):
                raise KernelError("a matmul's first reduction loop must walk the whole row")
            for _, h, _ in m.pre:  # the first loop reads the operand's rows where the matmul does
                for n in nodes_between(h):
                    if n.op != "load" or len(n.shape) != 2 or n.shape[0] == 1:
                        continue
                    w0 = [w for w in plan.operand(n.kwargs["operand"]).tile.windows if w.size is not None]
                    if len(w0) != 2 or (w0[0].loop, w0[0].offset) != (rows.loop, rows.offset) or w0[1].offset != 0 \
                            or w0[1].loop != first.var:
                        raise KernelError("a matmul's first reduction loop must read the rows the matmul reads, "
                                          "block by block along the row")
        elif m.tk != shape[1]:
            raise KernelError("a matmul's row prologue needs a reduction loop over the whole row")
        self.rows_n, self.cols_n = shape

    def _kdim(self, role: str) -> int:
        """The dim of the left ("a") or right ("b") operand's array that the reduction walks."""
        shape = self.plan.inputs[(self.m.a if role == "a" else self.m.b).param].shape
        return len(shape) - 1 if role == "a" or self.m.b_nt else len(shape) - 2

    def _shape(self, role: str) -> Tuple[int, ...]:
        """The array the kernel reads for an operand: its own, or with f32 operands its bf16 parts, whose
        reduction dim is kx times as long."""
        shape = tuple(self.plan.inputs[(self.m.a if role == "a" else self.m.b).param].shape)
        if not self.x3:
            return shape
        kd = self._kdim(role)
        return shape[:kd] + (self.kx * shape[kd],) + shape[kd + 1:]

    def _check_parts(self) -> None:
        """f32 operands: every reduction block the kernel reads starts on a BK-slice boundary of the array, so
        slice j of the operand is slices 6j..6j+5 of its parts (F32_PARTS: six bf16 slices per f32 slice)."""
        plan, m, bk = self.plan, self.m, self.hw.bk
        for role, op in (("a", m.a), ("b", m.b)):
            shape = plan.inputs[op.param].shape
            kd = self._kdim(role)
            kwin = [w for w in op.tile.windows if w.size is not None][1 if role == "a" or m.b_nt else 0]
            if shape[kd] % bk or kwin.offset % bk or shape[-1] % 8:
                raise KernelError(f"the gfx950 matmul lowering takes f32 operands whose reduction dim and windows "
                                  f"are multiples of {bk} and whose rows are multiples of 8 elements")
        if plan.phases:
            r = plan.phases[m.mphase].range  # the matmul's own loop (a row-sum loop may run before it)
            if r.start % bk or r.step % bk:
                raise KernelError(f"the gfx950 matmul lowering takes f32 operands with reduction blocks on "
                                  f"multiples of {bk}")

    def _parts_source(self, role: str) -> str:
        """The pass that writes an f32 (or bf16) operand's bf16 parts: each thread takes 8 consecutive
        elements, splits each into three bf16 parts (the second and third 0 for a bf16 operand) and stores the
        parts its slice's copies hold (F32_PARTS)."""
        op = self.m.a if role == "a" else self.m.b
        spec = self.plan.inputs[op.param]
        shape, kd, bk = tuple(spec.shape), self._kdim(role), self.hw.bk
        K, inner, numel = shape[kd], int(np.prod(shape[kd + 1:])), int(np.prod(shape))
        parts = tuple(f"p{i}" for i in F32_PARTS[role])
        kx = self.kx
        if spec.dtype.name == "float32":
            load = (f"const ak_f32x4 u0 = *(const ak_f32x4*)(args.{op.tile.array} + flat), "
                    f"u1 = *(const ak_f32x4*)(args.{op.tile.array} + flat + 4);\n"
                    "  const float v[8] = {u0[0], u0[1], u0[2], u0[3], u1[0], u1[1], u1[2], u1[3]};")
        else:
            load = (f"const ak_u32x4 u = *(const ak_u32x4*)((const ak_u16*)args.{op.tile.array} + flat);\n"
                    "  float v[8];\n"
                    "#pragma unroll\n"
                    "  for (int e = 0; e < 8; ++e) v[e] = ak_bf16_to_f32((ak_u16)(u[e >> 1] >> (16 * (e & 1))));")
        stores = "\n".join(f"  *(ak_u32x4*)(args.x3_{role} + o + {c * bk * inner}LL) = {p_};" for c, p_ in enumerate(parts))
        return f"""
// The bf16 parts of `{op.tile.array}` ({"x".join(map(str, shape))}, {spec.dtype.name}) for the f32 matmul: for each {bk}-deep
// slice of dim {kd}, the slices ({", ".join(parts)}).
extern "C" __global__ void __launch_bounds__({THREADS}) {self.name}_parts_{role}(const {self.name}_args args) {{
  const long long e8 = (long long)blockIdx.x * {THREADS} + threadIdx.x;
  if (e8 >= {numel // 8}) return;
  const long long flat = e8 * 8, kk = flat / {inner};
  const int k = (int)(kk % {K});
  const long long o = ((kk / {K}) * {kx * K} + {kx} * (k / {bk}) * {bk} + k % {bk}) * {inner} + flat % {inner};
  {load}
  unsigned q1[4], q2[4], q3[4];
#pragma unroll
  for (int e = 0; e < 8; e += 2) {{
    float a1, a2, a3, b1, b2, b3;
    ak_split3(v[e], a1, a2, a3);
    ak_split3(v[e + 1], b1, b2, b3);
    q1[e >> 1] = ak_pack_bf16x2(a1, b1); q2[e >> 1] = ak_pack_bf16x2(a2, b2); q3[e >> 1] = ak_pack_bf16x2(a3, b3);
  }}
  const ak_u32x4 p1 = {{q1[0], q1[1], q1[2], q1[3]}}, p2 = {{q2[0], q2[1], q2[2], q2[3]}}, p3 = {{q3[0], q3[1], q3[2], q3[3]}};
{stores}
}}
"""

    # ------------------------------------------------------------------ work items (host)

    def _items(self) -> Tuple[List[Tuple[int, int]], List[float], List[int]]:
        """Every (tile or fill, sub-tile | kind << 16), its weight (k slices) and locality group."""
        plan, sch, m, hw = self.plan, self.sch, self.m, self.hw
        items, weights, groups = [], [], []
        kslices = m.tk // hw.bk * self.kx
        steps_of = None
        if sch.step_tables and not sch.runtime:
            offsets = static_tile_steps(sch)
            codes = sch.tables[STEP_CODE]
            steps_of = [int(offsets[t + 1] - offsets[t]) - int(np.sum((codes[offsets[t]:offsets[t + 1]] & 4) != 0))
                        for t in range(sch.pattern_tiles)]
        per_tile = (plan.phases[m.mphase].range.count if plan.phases else 1) if not sch.step_tables else None
        out_rows, out_cols = [w for w in m.out.tile.windows if w.size is not None][:2]
        col_loop, row_loop = out_cols.loop, out_rows.loop
        # Locality groups: a band of columns (BAND_TILES workgroup tiles wide), and within it a patch of rows,
        # so that an XCD's round of equal items (32 of them, in group order) covers a patch of the output
        # whatever order the spec's loops take
        band = hw.bn * BAND_TILES[0]
        rows_per_patch = max(1, gfx950.CUS // gfx950.XCDS // max(1, band // hw.bn)) * hw.bm

        def locality(values: Dict[str, int], sm: int, sn: int) -> Tuple[int, int]:
            col = (values.get(col_loop, 0) if col_loop else 0) + sn * hw.bn
            row = (values.get(row_loop, 0) if row_loop else 0) + sm * hw.bm
            return (col // band, row // rows_per_patch) if PATCHES[0] else (col // band, 0)

        consts: set = set()
        for t in range(sch.tiles):
            blocks = sch.blocks_at(t)
            values = {r.var: r.value(b) for r, b in zip(plan.parallel, blocks)}
            if steps_of is not None:
                nsteps = steps_of[t % sch.pattern_tiles]
            elif sch.runtime:
                nsteps = sch.phase_counts[0] if sch.phase_counts else 1
            else:
                nsteps = per_tile if plan.phases else 1
            for s in range(self.subs):
                sm, sn = divmod(s, self.sub_n)
                kind, weight = 0, max(nsteps, 1) * kslices + 1
                if not sch.runtime:
                    const = self._constant(values, sm, sn)
                    if const is not None:
                        consts.add(const)
                        kind, weight = 2, 0.25
                items.append((t, s | (kind << 16)))
                weights.append(weight)
                groups.append(locality(values, sm, sn))
        for f in range(sch.fills):
            blocks = sch.fill_blocks_at(f)
            values = {r.var: r.value(b) for r, b in zip(plan.parallel, blocks)}
            for s in range(self.subs):
                sm, sn = divmod(s, self.sub_n)
                items.append((f, s | (1 << 16)))
                weights.append(0.25)
                groups.append(locality(values, sm, sn))
        if len(consts) > 1:  # one constant per kernel: compute the others
            keep = sorted(consts)[0]
            items = [(t, s & 0xFFFF) if (s >> 16) == 2 and self._constant_of(t, s) != keep else (t, s)
                     for t, s in items]
            consts = {keep}
        self.const_value = next(iter(consts)) if consts else None
        items3 = [(t, s, 0) for t, s in items]
        if not sch.runtime:
            items3, weights, groups = self._split_remainder(items3, weights, groups)
        return items3, weights, groups

    def _split_remainder(self, items, weights, groups):
        """Balance the last round. With n equal compute items on G workgroups, n = q G + r and r <= G / 2,
        the last round would leave most workgroups idle: r of the items are cut along the reduction into
        `split` chunks each (r * split <= G, split <= MAX_SPLIT). A chunk writes its f32 partial sums to a
        workspace slot, and a fixup kernel adds a tile's partials in chunk order and applies the epilogue."""
        hw, G = self.hw, gfx950.CUS
        compute = [k for k, (_, c, _) in enumerate(items) if (c >> 16) == 0]
        if not compute or len({weights[k] for k in compute}) != 1:
            return items, weights, groups
        r = len(compute) % G
        T = int(round(weights[compute[0]])) - 1  # K slices per item
        if r == 0 or 2 * r > G or self.dual:  # (two accumulators: no partial-sum fixup for them)
            return items, weights, groups
        split = 1
        while (2 * split * r <= G and 2 * split <= MAX_SPLIT and T % (2 * split) == 0 and (T // (2 * split)) % hw.stages == 0
               and T // (2 * split) >= max(4, 2 * hw.stages)):
            split *= 2
        if split == 1:
            return items, weights, groups
        chosen = compute[-r:]
        self.split = (r, split, T // split)
        self.tables["split_items"] = np.array([items[k][:2] for k in chosen], np.int32).reshape(-1)
        out, w_out, g_out = [], [], []
        chosen_set = set(chosen)
        for k, item in enumerate(items):
            if k not in chosen_set:
                out.append(item)
                w_out.append(weights[k])
                g_out.append(groups[k])
        for p, k in enumerate(chosen):
            t, c, _ = items[k]
            for ch in range(split):
                out.append((t, (c & 0xFFFF) | (3 << 16), p * split + ch))
                w_out.append(T / split + 1)
                # chunks are ordered by K range and equally loaded workgroups are taken an XCD at a time, so an
                # XCD takes every remainder tile's chunks over the same K ranges (two of eight at 16 tiles): the
                # tiles' A and B panels over those ranges are read into its L2 once
                g_out.append((ch * gfx950.XCDS // split, 0))
        return out, w_out, g_out

    def _constant_of(self, t: int, s: int) -> Optional[float]:
        blocks = self.sch.blocks_at(t)
        values = {r.var: r.value(b) for r, b in zip(self.plan.parallel, blocks)}
        sm, sn = divmod(s & 0xFFFF, self.sub_n)
        return self._constant(values, sm, sn)

    def _constant(self, values: Dict[str, int], sm: int, sn: int) -> Optional[float]:
        """The epilogue's value over a whole hardware sub-tile if it can't depend on the accumulator."""
        m, hw = self.m, self.hw
        root = m.value.node if isinstance(m.value, jaxlite.Sym) else None
        if root is None:
            return None
        rows = (sm * hw.bm, sm * hw.bm + hw.bm - 1)
        cols = (sn * hw.bn, sn * hw.bn + hw.bn - 1)

        def leaf(n: Node) -> Optional[Interval]:
            if n is m.acc or n.op in ("carried", "load", "dot", "dot_nt"):
                return Interval(data=True)
            if n.op == "iota":
                dim = n.kwargs["dimension"]
                lo, hi = rows if dim == len(n.shape) - 2 else cols if dim == len(n.shape) - 1 else (None, None)
                return Interval(lo, hi) if lo is not None else Interval()
            if n.op == "loop":
                v = values.get(n.kwargs["var"])
                return Interval(v, v) if v is not None else Interval()
            if n.op == "full":
                v = n.kwargs["value"]
                return Interval(v, v, const=v)
            if n.op == "index":
                return Interval()
            return None

        got = intervals(root, leaf)
        if not got.data and got.const is not None:
            return float(got.const)
        return None

    # ------------------------------------------------------------------ source

    def program(self) -> Program:
        plan, sch, m, hw = self.plan, self.sch, self.m, self.hw
        items, weights, groups = self._items()
        grid = max(1, min(len(items), gfx950.CUS))
        # Whole tiles go to workgroups ahead of time (longest first, XCD-aware: work_lists). The small items
        # (K-split chunks, filled and constant tiles) form one queue that workgroups pull from when their
        # own list is done, so the workgroups that finish early (a faster XCD, a lighter list) take more of
        # them. The queue's head and a count of finished workgroups are kept on the device; the last
        # workgroup to finish sets both back to zero for the next call.
        whole = [k for k, it in enumerate(items) if (it[1] >> 16) == 0]
        small = [k for k, it in enumerate(items) if (it[1] >> 16) != 0]
        if not whole or not QUEUE_TAIL[0]:
            whole, small = list(range(len(items))), []
        offsets, flat = work_lists([items[k] for k in whole], [weights[k] for k in whole],
                                   [groups[k] for k in whole], grid)
        self.tables["wg_items"] = offsets
        self.tables["items"] = flat.reshape(-1) if flat.size else np.zeros(3, np.int32)
        small.sort(key=lambda k: (-weights[k], groups[k], k))
        self.n_small = len(small)
        if small:
            self.tables["small_items"] = np.array([items[k] for k in small], np.int32).reshape(-1)
            self.state = {"queue": 2}
        else:
            self.state = {}
        for name, t in sch.tables.items():
            if name in (STEP_TILE,):
                continue
            self.tables[name] = t
        if sch.step_tables and not sch.runtime:
            self.tables["tile_steps"] = static_tile_steps(sch)
        args = self._args()
        source = self._source(args)
        launches = [Launch(self.name, args, (grid, 1, 1), (64 * hw.waves, 1, 1), 0)]
        workspace = {}
        if self.x3:
            for role in ("b",) if self.prologue else ("a", "b"):
                source += self._parts_source(role)
                workspace[f"x3_{role}"] = 2 * int(np.prod(self._shape(role)))
                groups8 = int(np.prod(self.plan.inputs[(m.a if role == "a" else m.b).param].shape)) // 8
                launches.insert(0, Launch(f"{self.name}_parts_{role}", args, (-(-groups8 // THREADS), 1, 1),
                                          (THREADS, 1, 1), 0))
        if self.prologue:
            source += self._rows_source()
            workspace["rn_a"] = self.rows_n * self.cols_n * 2 * self.kx
            for name, _, _ in m.side:
                workspace[f"rn_{name}"] = self.rows_n * 4
            launches.insert(0, Launch(f"{self.name}_rows", args, (-(-self.rows_n // 4), 1, 1), (THREADS, 1, 1), 0))
        if self.trace:
            workspace[TRACE] = grid * TRACE_FIELDS * 8
        if self.split:
            r, split, _ = self.split
            workspace["gm_part"] = r * split * hw.bm * hw.bn * 4
            launches.append(Launch(f"{self.name}_fixup", args, (r * hw.bm * hw.bn // (4 * THREADS), 1, 1),
                                   (THREADS, 1, 1), 0))
        inputs = [(spec.shape, spec.dtype) for spec in plan.inputs]
        prog = Program(
            name=self.name, source=source, launches=launches, outputs=[(m.out.shape, m.out.dtype)], inputs=inputs,
            tables=dict(self.tables), workspace=workspace, state=dict(self.state), lds_bytes=hw.lds,
            protocol=self.protocol,
            notes={"family": "gemm", "hw_tile": (hw.bm, hw.bn, hw.bk), "stages": hw.stages, "waves": hw.waves, "grid": grid,
                   "items": len(items), "constant_items": sum(1 for _, s, _ in items if (s >> 16) == 2),
                   "queued_items": self.n_small,
                   "split": self.split, "dual": self.dual, "trace_workgroups": grid if self.trace else 0,
                   "slices_per_step": m.tk // hw.bk * self.kx * self.subs, "f32_operands": self.x3},
        )
        if sch.runtime:
            from .steps import attach_step_builder

            attach_step_builder(prog, plan, sch, self.name)
        return prog

    def _args(self) -> List[Arg]:
        plan, m = self.plan, self.m
        args = []
        for k, name in enumerate(plan.nest.params):
            spec = plan.inputs[k]
            if any(ix.name == name for ix in plan.indices):
                args.append(Arg("input", k, "const int* __restrict__", name))
            else:
                args.append(Arg("input", k, f"const {_cstore(spec.dtype)}* __restrict__", name))
        args.append(Arg("output", 0, f"{_cstore(m.out.dtype)}* __restrict__", m.out.name + "_out"))
        for name in self.tables:
            args.append(Arg("table", name, "const int* __restrict__", name))
        for name in self.state:
            args.append(Arg("state", name, "int* __restrict__", name))
        args.append(Arg("int", 2 * self._pitch("a"), "int", "ak_pitch_a"))
        args.append(Arg("int", 2 * self._pitch("b"), "int", "ak_pitch_b"))
        if self.split:
            args.append(Arg("workspace", "gm_part", "float* __restrict__", "gm_part"))
        if self.trace:
            args.append(Arg("workspace", TRACE, "unsigned long long* __restrict__", TRACE))
        if self.x3:
            for role in ("b",) if self.prologue else ("a", "b"):
                args.append(Arg("workspace", f"x3_{role}", "ak_u16* __restrict__", f"x3_{role}"))
        if self.prologue:
            args.append(Arg("workspace", "rn_a", "ak_u16* __restrict__", "rn_a"))
            for name, _, _ in m.side:
                args.append(Arg("workspace", f"rn_{name}", "float* __restrict__", f"rn_{name}"))
        if self.sch.runtime:
            args.append(Arg("workspace", "step_code", "const int* __restrict__", "rt_step_code"))
            args.append(Arg("workspace", "tile_steps", "const int* __restrict__", "rt_tile_steps"))
        return args

    def _rows_source(self) -> str:
        """The row prologue's pass: one wave per row of the left operand, eight columns a lane at a time. It
        writes the operand the matmul reads (the prologue's bf16 value per element) and each row sum, a
        lane's partial sums added across the wave. With a first reduction loop, the wave first sums that
        loop's row sums over the whole row and computes the row statistics the operand reads."""
        plan, m = self.plan, self.m
        zero = Index(plan, lambda v: "0")
        pre_k = {name: k for k, (name, _, _) in enumerate(m.pre)}
        stat_k = {name: k for k, (name, _) in enumerate(m.stats)}

        def leaves(n: Node, idx: Tuple[str, ...]) -> Optional[str]:
            if n.op == "carried" and n.kwargs["name"] in stat_k:
                return f"st_{stat_k[n.kwargs['name']]}"
            if n.op == "carried" and n.kwargs["name"] in pre_k:  # a (rows, 1) sum
                return f"ps_{pre_k[n.kwargs['name']]}"
            if n.op == "reduce_sum" and _is(n.args[0], "carried") and n.args[0].kwargs["name"] in pre_k:
                return f"ps_{pre_k[n.args[0].kwargs['name']]}"  # a tile summed elementwise, then along its rows
            if n.op == "load":
                op = plan.operand(n.kwargs["operand"])
                shape = plan.inputs[op.param].shape
                base, st = tile_base(op.tile, shape, zero, lambda v: "0")
                flat = " + ".join(f"(long long)({i}) * {s_}" for i, s_ in zip(idx, st)) or "0"
                if op.tile.dtype.name == "float32":
                    return f"args.{op.tile.array}[({base}) + {flat}]"
                if op.tile.dtype.name != "bfloat16":
                    raise KernelError("a matmul's row prologue reads bf16 or f32 operands")
                return f"ak_bf16_to_f32(((const ak_u16*)args.{op.tile.array})[({base}) + {flat}])"
            return None

        em = ElementEmitter(leaves)
        a_node = m.a_expr
        if a_node is None:  # (only row sums: the operand is copied as it is)
            a_node = next(n for n in nodes_between(m.side[0][1]) if n.op == "load")
        D = self.cols_n
        sums = "".join(f" float rs_{k} = 0.f;" for k in range(len(m.side)))
        adds = "\n".join(f"        rs_{k} += (float)({em.at(h, ('r', 'c'))}) + (float)({em.at(h, ('r', 'c + 1'))});"
                          for k, (_, h, _) in enumerate(m.side))
        outs = "\n".join(f"  rs_{k} = ak_wave_sum(rs_{k}); if (lane == 0) args.rn_{name}[r] = rs_{k};"
                          for k, (name, _, _) in enumerate(m.side))
        first = ""
        if m.pre:
            first = ("  // the first reduction loop's sums over the whole row, then the row statistics\n"
                     + "".join(f"  float ps_{k} = 0.f;\n" for k in range(len(m.pre)))
                     + f"  for (int c0 = lane * 8; c0 < {self.cols_n}; c0 += 512) {{\n#pragma unroll\n"
                     + "    for (int e = 0; e < 8; ++e) {\n      const int c = c0 + e;\n"
                     + "".join(f"      ps_{k} += (float)({em.at(h, ('r', 'c'))});\n" for k, (_, h, _) in enumerate(m.pre))
                     + "    }\n  }\n"
                     + "".join(f"  ps_{k} = ak_wave_sum(ps_{k});\n" for k in range(len(m.pre)))
                     + "".join(f"  const float st_{k} = (float)({em.at(v, ('r', '0'))});\n"
                               for k, (_, v) in enumerate(m.stats)))
        if self.x3:  # the operand's bf16 parts: for each of its BK-deep slices, the slices F32_PARTS names
            bk, kx = self.hw.bk, self.kx
            value = (f"const float v0 = {em.at(a_node, ('r', 'c'))}, v1 = {em.at(a_node, ('r', 'c + 1'))};\n"
                     "      float a1, a2, a3, b1, b2, b3;\n"
                     "      ak_split3(v0, a1, a2, a3);\n"
                     "      ak_split3(v1, b1, b2, b3);\n"
                     "      q1[e >> 1] = ak_pack_bf16x2(a1, b1); q2[e >> 1] = ak_pack_bf16x2(a2, b2); "
                     "q3[e >> 1] = ak_pack_bf16x2(a3, b3);")
            store = (f"ak_u16* dst = args.rn_a + (long long)r * {kx * D} + {kx} * (c0 / {bk}) * {bk} + c0 % {bk};\n"
                     + "\n".join(f"    *(ak_u32x4*)(dst + {c * bk}) = ak_u32x4{{q{i}[0], q{i}[1], q{i}[2], q{i}[3]}};"
                                  for c, i in enumerate(F32_PARTS["a"])))
        else:
            value = (f"q1[e >> 1] = ak_pack_bf16x2((float)({em.at(a_node, ('r', 'c'))}), "
                     f"(float)({em.at(a_node, ('r', 'c + 1'))}));")
            store = f"*(ak_u32x4*)(args.rn_a + (long long)r * {D} + c0) = ak_u32x4{{q1[0], q1[1], q1[2], q1[3]}};"
        return f"""
// The row prologue of `{plan.nest.name}`: rows {self.rows_n} x {D}, one wave per row.
extern "C" __global__ void __launch_bounds__({THREADS}) {self.name}_rows(const {self.name}_args args) {{
  const int r = blockIdx.x * {THREADS // 64} + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (r >= {self.rows_n}) return;
{first} {sums}
  for (int c0 = lane * 8; c0 < {D}; c0 += 512) {{
    unsigned q1[4], q2[4], q3[4];
#pragma unroll
    for (int e = 0; e < 8; e += 2) {{
      const int c = c0 + e;
      {value}
{adds}
    }}
    (void)q2; (void)q3;
    {store}
  }}
{outs}
}}
"""

    def _pitch(self, role: str) -> int:
        """Elements between consecutive rows of an operand tile (its first sliced dim's stride) in the array
        the kernel reads."""
        op = self.m.a if role == "a" else self.m.b
        return [s for w, s in zip(op.tile.windows, strides(self._shape(role))) if w.size is not None][0]

    def _source(self, args: List[Arg]) -> str:
        plan, sch, m, hw = self.plan, self.sch, self.m, self.hw
        bm, bn, bk, S = hw.bm, hw.bn, hw.bk, hw.stages
        WM, WN = hw.grid
        T = 64 * WM * WN  # threads of the workgroup
        dual, bnl = hw.dual, hw.bn_lds
        wtm, wtn = bm // WM, bnl // WN
        mi, ni = wtm // MFMA, wtn // MFMA
        # Output columns per wave and 32-column blocks of them: with two right operands a wave's fragments j and
        # j + nio read the same columns of b and b2 (LDS holds b's BN columns, then b2's), and its outputs are
        # the epilogue of each pair.
        nio, wto = (ni // 2, wtn // 2) if dual else (ni, wtn)
        k16s = bk // 16
        kslices = m.tk // bk * self.kx  # K slices per step (with f32 operands, of the parts arrays)
        split, split_slices = (self.split[1], self.split[2]) if self.split else (1, 0)
        kvar = m.kvar
        # tables and index inputs are read through the constant address space: scalar loads, which leave the
        # vector memory queue's in-order wait counts to the LDS loads in flight (a vector load of a table at an
        # item's start would wait for the next item's prefetched slices too)
        index = Index(plan, lambda v: f"lv_{v}", constant=True)
        a_shape, b_shape = self._shape("a"), self._shape("b")
        no_k = lambda v: "0" if v == kvar else f"lv_{v}"  # the reduction loop's offset goes per slice
        a_base, a_str = tile_base(m.a.tile, a_shape, index, no_k)
        b_base, b_str = tile_base(m.b.tile, b_shape, index, no_k)
        b2_base = tile_base(m.b2.tile, b_shape, index, no_k)[0] if dual else None
        o_base, o_str = tile_base(m.out.tile, m.out.shape, index, lambda v: f"lv_{v}")
        if a_str[1] != 1 or b_str[1] != 1 or o_str[1] != 1:
            raise KernelError("the gfx950 matmul lowering reads and writes tiles whose last dim is the array's last")
        for name, shape in ((m.a.tile.array, a_shape), (m.b.tile.array, b_shape)):
            if 2 * int(np.prod(shape)) >= 2**31:
                raise KernelError(f"`{name}` is 2 GiB or more: the gfx950 matmul lowering addresses operands with "
                                  "32-bit buffer offsets")
        lda, ldb, ldo = a_str[0], b_str[0], o_str[0]
        nt = m.b_nt
        kca = bk // 8  # 16-byte chunks per K-contiguous row
        nc = bn // 8  # 16-byte chunks per N-contiguous row (B of `a @ b`)
        a_ld = bm * bk // 8 // T
        b_ld = bnl * bk // 8 // T  # (with two right operands, half for each)
        if a_ld < 1 or b_ld < 1 or (not nt and 64 % nc):
            raise KernelError(f"matmul hardware tile {bm} x {bn} x {bk} is too small for a {T}-thread workgroup")

        def swa(row: str) -> str:  # K-contiguous rows: chunk XOR, conflict-free ds_read_b128 (64 banks)
            return {8: f"((({row}) >> 1) & 7)", 4: f"((({row}) >> 2) & 3)", 2: f"((({row}) >> 3) & 1)"}[kca]

        def swb(k: str) -> str:  # N-contiguous rows: chunk XOR, conflict-free ds_read_b64_tr_b16
            return f"(((({k}) & 3) << 2) & {nc - 1})"

        # How a tile's steps are found: `nsteps` and the reduction loop's value at step `st_`.
        phase = plan.phases[m.mphase].range if plan.phases else None
        if phase is None:
            steps_setup = ["const int nsteps = 1;"]
            kval = str(m.k0)
        elif not sch.step_tables:
            steps_setup = [f"const int nsteps = {phase.count};"]
            kval = f"({phase.start} + st_ * {phase.step})"
        else:
            codes, offs = (f"args.{STEP_CODE}", "args.tile_steps") if not sch.runtime else ("args.rt_step_code",
                                                                                            "args.rt_tile_steps")
            steps_setup = [
                f"const int tt_s = t % {sch.pattern_tiles};",
                f"const int sbeg = __builtin_amdgcn_readfirstlane(ak_ldc({offs}, tt_s)), send = ak_ldc({offs}, tt_s + 1);",
                f"const int nsteps = ((ak_ldc({codes}, sbeg) >> 2) & 1) ? 0 : send - sbeg;",
            ]
            if _tile_level(phase) and len(plan.phases) == 1:
                # A mask that doesn't read the reduction loop's variable keeps all of a tile's blocks or none:
                # a kept tile's steps are the loop's blocks in order, so the K offset is arithmetic. (Read from
                # the step code, it is a global load and a wait for it before every slice's loads are issued.)
                kval = f"({phase.start} + st_ * {phase.step})"
            else:
                kval = (f"({phase.start} + ((ak_ldc({codes}, sbeg + st_) >> {CODE_SHIFT}) / {sch.iterations} / "
                        f"{sch.phase_radix}) * {phase.step})")
        if self.x3:  # the parts arrays hold kx slices for each of the operand's
            kval = f"({self.kx} * {kval})"

        # The epilogue, per accumulator element.
        def leaf(n: Node) -> Optional[str]:
            if n is m.acc:
                return "acc_v"
            if dual and n is m.acc2:
                return "acc2_v"
            if n.op == "iota":
                dim = n.kwargs["dimension"]
                if dim == len(n.shape) - 2:
                    return "er"
                if dim == len(n.shape) - 1:
                    return "ec"
                return "0"
            if n.op == "loop":
                var = n.kwargs["var"]
                if var not in {r.var for r in plan.parallel}:
                    raise KernelError(f"the epilogue reads `{var}`, which isn't defined there")
                return f"lv_{var}"
            if n.op == "full":
                return literal(n.kwargs["value"], n.dtype)
            if n.op == "index":
                ix = plan.index(n.kwargs["array"])
                flat = " + ".join(f"({em.value(i)}) * {s}" for i, s in zip(n.args, strides(ix.shape))) or "0"
                return f"args.{ix.name}[{flat}]"
            if n.op == "tile" and isinstance(n.args[0], Node) and _column_uniform(n.args[0], {x[0] for x in m.side}):
                return em.emit(n.args[0])  # tiling a row statistic along the columns repeats each row's value
            sided = n.kwargs["name"] if n.op == "carried" else _row_sum_name(n) if n.op == "reduce_sum" else None
            if sided is not None and any(sided == name for name, _, _ in m.side):
                # a row sum: the same for every column; the tile's rows are the left operand's
                name, _, init = next(x for x in m.side if x[0] == sided)
                rows = [w for w in m.a.tile.windows if w.size is not None][0]
                row = f"(lv_{rows.loop}) + er" if rows.loop else "er"
                return f"({literal(init, n.dtype)} + args.rn_{name}[{row}])"
            if n.op in ("carried", "load"):
                raise KernelError("the matmul epilogue reads only the accumulator, positions and loop values")
            return None

        em = Emitter(leaf, m.out.tile.shape, prefix="e")
        result = em.emit(m.value.node) if isinstance(m.value, jaxlite.Sym) else literal(m.value)
        epi = "\n              ".join(em.lines)
        out_bf16 = m.out.dtype.name == "bfloat16"
        struct = c_struct(f"{self.name}_args", args)
        # with a row prologue the left operand is its pass's output, laid out as the operand's array
        A = "args.rn_a" if self.prologue else "args.x3_a" if self.x3 else f"args.{m.a.tile.array}"
        B = "args.x3_b" if self.x3 else f"args.{m.b.tile.array}"
        B2 = f"args.{m.b2.tile.array}" if dual else None
        O = f"args.{m.out.name}_out"
        a_numel, b_numel = int(np.prod(a_shape)), int(np.prod(b_shape))
        fill_value = literal(m.out.fill if m.out.fill is not None else 0, m.out.dtype)
        const_value = literal(self.const_value if self.const_value is not None else 0.0, m.out.dtype)
        tile_decode = "\n    ".join(decode_tile(plan, sch, "t", constant=True))
        fill_block = ""
        # a traced kernel counts the stores of filled and constant tiles as output time
        tr_s0 = f"const unsigned long long tr_s0 = {NOW}; " if self.trace else ""
        tr_s1 = f" tr_out += {NOW} - tr_s0;" if self.trace else ""
        if sch.fills:
            fill_decode = "\n      ".join(decode_fill(plan, sch, "t", constant=True))
            fill_block = (f"if (kind == 1) {{\n      {fill_decode}\n      const long long obase = {o_base};\n      "
                          f"{tr_s0}{_store_constant(bm, bn, out_bf16, O, 'obase', ldo, fill_value, T)}{tr_s1}\n"
                          f"      continue;\n    }}")
        setup = "\n    ".join(steps_setup)

        L: List[str] = []
        w = L.append
        w(f"""// Generated by tilejax_amd for `{plan.nest.name}`: a persistent gfx950 matmul kernel.
// spec tile {m.tm} x {m.tn} x {m.tk}; workgroup tile {bm} x {bn}, K slices of {bk} through {S} LDS stages;
// {sch.tiles} tiles of {sch.total_tiles} ({sch.fills} filled), {sch.steps} steps.
{PRELUDE}
{struct}""")
        for s in range(S):  # one array per stage and operand: the compiler then keeps prefetches in flight
            w(f"__shared__ __attribute__((aligned(1024))) ak_u16 ak_sa{s}[{bm * bk}];")
            w(f"__shared__ __attribute__((aligned(1024))) ak_u16 ak_sb{s}[{bnl * bk}];")
        w(f"""
extern "C" __global__ void __launch_bounds__({T}) {self.name}(const {self.name}_args args) {{
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: LDS addresses stay in SGPRs
  const int wm = wave / {WN}, wn = wave % {WN};
  // Each wave's buffer_load ... lds fills 1 KiB of a stage, lane l's 16 bytes at 16 l: the lane loads the
  // global chunk that belongs at that (swizzled) position.
  const int a_row = wave * {64 // kca} + lane / {kca};
  // Row pitches (bytes) come in as kernel arguments: as literals the compiler precomputes every load's
  // offset into registers and spills them inside the K loop.
  const unsigned pa = (unsigned)args.ak_pitch_a, pb = (unsigned)args.ak_pitch_b;
  const unsigned a_voff = a_row * pa + (unsigned)((((lane % {kca}) ^ {swa('a_row')}) * 16));""")
        if nt:
            w(f"""  const unsigned b_voff = a_row * pb + (unsigned)((((lane % {kca}) ^ {swa('a_row')}) * 16));""")
        else:
            w(f"""  const int b_k = wave * {64 // nc} + lane / {nc};
  const unsigned b_voff = b_k * pb + (unsigned)((((lane % {nc}) ^ {swb('b_k')}) * 16));""")
        w(f"  int a_roff[{k16s}], b_roff[{k16s if nt else ni}];")
        for k16 in range(k16s):
            w(f"  {{ const int row = wm * {wtm} + (lane & 31); a_roff[{k16}] = row * {bk * 2} + "
              f"((({2 * k16} + (lane >> 5)) ^ {swa('row')}) * 16); }}")
            if nt:
                w(f"  {{ const int row = wn * {wtn} + (lane & 31); b_roff[{k16}] = row * {bk * 2} + "
                  f"((({2 * k16} + (lane >> 5)) ^ {swa('row')}) * 16); }}")
        if not nt:
            w("  { const int G = lane >> 4, s = lane & 15, k = 8 * (G >> 1) + (s >> 2);")
            for j in range(ni):
                half, jj = divmod(j, nio)  # (which right operand: 0 but with two)
                at = f"{half * bk * bn * 2} + " if dual else ""
                w(f"    {{ const int n = wn * {wto} + {jj * 32} + 16 * (G & 1) + 4 * (s & 3);"
                  f" b_roff[{j}] = {at}k * {bn * 2} + (((n >> 3) ^ {swb('k')}) << 4) + (n & 7) * 2; }}")
            w("  }")
        trace_write = (f"if (tid == 0) {{ unsigned long long* tr = args.{TRACE} + blockIdx.x * {TRACE_FIELDS}; "
                       f"tr[0] = tr_fill + tr_wait; tr[1] = tr_fill; tr[2] = tr_out; tr[3] = tr_comp - tr_wait; "
                       f"tr[4] = tr_slices; {CLOCK_END} }}" if self.trace else "")
        trace_decl = (f"{CLOCK_START} unsigned long long tr_wait = 0, tr_fill = 0, tr_out = 0, tr_comp = 0, "
                      "tr_slices = 0;" if self.trace else "")
        now = NOW
        if self.n_small:
            pull = f"""    int t, code, slot;
    if (q < q_end) {{
      t = ak_ldc(args.items, 3 * q); code = ak_ldc(args.items, 3 * q + 1); slot = ak_ldc(args.items, 3 * q + 2); ++q;
    }} else {{  // this workgroup's own list is done: the next item of the shared queue, if any is left
      if (tid == 0) ak_pulled = atomicAdd(&args.queue[0], 1);
      __syncthreads();
      const int k = __builtin_amdgcn_readfirstlane(ak_pulled);
      __syncthreads();
      if (k >= {self.n_small}) break;
      t = args.small_items[3 * k]; code = args.small_items[3 * k + 1]; slot = args.small_items[3 * k + 2];
    }}"""
            loop_head = "  for (int q = q_begin;;) {"
            tail = """  if (tid == 0) {  // the last workgroup to finish leaves the queue at zero for the next call
    if (atomicAdd(&args.queue[1], 1) == (int)gridDim.x - 1) {
      __hip_atomic_store(&args.queue[0], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&args.queue[1], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
"""
        else:
            pull = ("    const int t = ak_ldc(args.items, 3 * q), code = ak_ldc(args.items, 3 * q + 1), "
                    "slot = ak_ldc(args.items, 3 * q + 2);")
            loop_head = "  for (int q = q_begin; q < q_end; ++q) {"
            tail = ""
        self._queue_tail = tail
        # Without the shared queue a workgroup knows its whole list: the next item that loads gets its first S
        # slices issued in place of this item's last S slices' refills, so its fill overlaps this item's last
        # slices and epilogue (`cross`). With the queue, each item fills its stages itself.
        cross = self.cross = not self.n_small
        sb_cur = "sbeg" if sch.step_tables else "0"
        a_off_expr = f"({a_base}) + (long long)(sm * {bm}) * {lda}"
        b_off_expr = f"({b_base}) + (long long)(sn * {bn}) * {ldb}" if nt else f"({b_base}) + sn * {bn}"
        b2_off_expr = f"({b2_base}) + sn * {bn}" if dual else None
        probe = ""
        if cross:
            probe = f"""
  // Slice g of an item whose K slices start at g0 (T of them; past the last, the last again), its K offset.
  auto k_at = [&](int g0, int T, int sbeg, int g) -> int {{
    const int gg = g0 + (g < T ? g : (T > 0 ? T - 1 : 0));
    const int st_ = gg / {kslices};
    return {kval} + (gg % {kslices}) * {bk};
  }};
  // Item q2's loads: its slices and operand offsets; false if it loads nothing (a filled or constant tile,
  // or one without steps).
  auto probe = [&](int q2, int& T_, int& g0_, int& sb_, long long& aoff_, long long& boff_{", long long& boff2_" if dual else ""}) -> bool {{
    const int t = ak_ldc(args.items, 3 * q2), code = ak_ldc(args.items, 3 * q2 + 1), slot = ak_ldc(args.items, 3 * q2 + 2);
    const int sub = code & 0xffff, kind = code >> 16;
    (void)slot;
    if (kind == 1 || kind == 2) return false;
    const int sm = sub / {self.sub_n}, sn = sub % {self.sub_n};
    {tile_decode}
    {setup}
    int T = nsteps * {kslices}, g0 = 0;
    if (kind == 3) {{ g0 = (slot % {split}) * {split_slices}; T = {split_slices}; }}
    T_ = T; g0_ = g0; sb_ = {sb_cur};
    aoff_ = {a_off_expr};
    boff_ = {b_off_expr};{f"{chr(10)}    boff2_ = {b2_off_expr};" if dual else ""}
    return T > 0;
  }};
  int pf_q = -1;  // the item whose first {S} slices are in flight"""
        w(f"""  const int q_begin = ak_ldc(args.wg_items, blockIdx.x), q_end = ak_ldc(args.wg_items, blockIdx.x + 1);
  {"__shared__ int ak_pulled;" if self.n_small else ""}
  {trace_decl}{probe}
{loop_head}
{pull}
    const int sub = code & 0xffff, kind = code >> 16;
    const int sm = sub / {self.sub_n}, sn = sub % {self.sub_n};
    {fill_block}
    {tile_decode}
    const long long obase = {o_base};
    if (kind == 2) {{
      {tr_s0}{_store_constant(bm, bn, out_bf16, O, "obase", ldo, const_value, T)}{tr_s1}
      continue;
    }}
    {setup}
    int T = __builtin_amdgcn_readfirstlane(nsteps * {kslices});  // K slices (even; one value per wave)
    int g0 = 0;  // the first K slice (a chunk of a tile cut along the reduction starts later)
    if (kind == 3) {{ g0 = (slot % {split}) * {split_slices}; T = {split_slices}; }}
    asm volatile("" : "+s"(T));  // an opaque trip count: a known one makes the compiler spill in the loop
    const long long a_off = {a_off_expr};
    const long long b_off = {b_off_expr};
    const __amdgpu_buffer_rsrc_t rsa = __builtin_amdgcn_make_buffer_rsrc((void*)({A} + a_off), (short)0,
        (int)({a_numel}LL * 2 - a_off * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t rsb = __builtin_amdgcn_make_buffer_rsrc((void*)({B} + b_off), (short)0,
        (int)({b_numel}LL * 2 - b_off * 2), 0x00020000);""")
        if dual:
            w(f"""    const long long b2_off = {b2_off_expr};
    const __amdgpu_buffer_rsrc_t rsb2 = __builtin_amdgcn_make_buffer_rsrc((void*)({B2} + b2_off), (short)0,
        (int)({b_numel}LL * 2 - b2_off * 2), 0x00020000);""")
        if cross:
            w(f"""    // the next item in this workgroup's list that loads (its first slices are issued during this item's last)
    int nx_q = q_end, nx_T = 0, nx_g0 = 0, nx_sb = 0;
    long long nx_aoff = 0, nx_boff = 0{", nx_boff2 = 0" if dual else ""};
    for (int q2 = q + 1; q2 < q_end; ++q2)
      if (probe(q2, nx_T, nx_g0, nx_sb, nx_aoff, nx_boff{", nx_boff2" if dual else ""})) {{ nx_q = q2; break; }}
    const __amdgpu_buffer_rsrc_t nx_rsa = __builtin_amdgcn_make_buffer_rsrc((void*)({A} + nx_aoff), (short)0,
        (int)({a_numel}LL * 2 - nx_aoff * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t nx_rsb = __builtin_amdgcn_make_buffer_rsrc((void*)({B} + nx_boff), (short)0,
        (int)({b_numel}LL * 2 - nx_boff * 2), 0x00020000);
    const int sb = {sb_cur};""")
            if dual:
                w(f"""    const __amdgpu_buffer_rsrc_t nx_rsb2 = __builtin_amdgcn_make_buffer_rsrc((void*)({B2} + nx_boff2), (short)0,
        (int)({b_numel}LL * 2 - nx_boff2 * 2), 0x00020000);""")
        w(f"""
    // A tile's chunks are summed by the fixup kernel: only the first starts from the initial value.
    const float acc_init = (kind == 3 && g0 != 0) ? 0.0f : {literal(m.init)};
    ak_f32x16 acc[{mi}][{ni}];
#pragma unroll
    for (int i_ = 0; i_ < {mi}; ++i_)
#pragma unroll
      for (int j_ = 0; j_ < {ni}; ++j_)
#pragma unroll
        for (int r_ = 0; r_ < 16; ++r_) acc[i_][j_][r_] = acc_init;
    ak_bf16x8 fa[2][{mi}], fb[2][{ni}];""")
        if not cross:
            w(f"""    // Slice g's loads into stage s: the slice's step and K offset (slices past the tile's last reload it).
    auto k_of = [&](int g) -> int {{
      const int gg = g0 + (g < T ? g : (T > 0 ? T - 1 : 0));
      const int st_ = gg / {kslices};
      return {kval} + (gg % {kslices}) * {bk};
    }};""")

        def issue(g: str, s: int, ind: str, refill: bool = False) -> List[str]:
            if cross and refill:  # past this item's last slice, the next loading item's first ones
                # the inputs are selected, then one k_at: no branch splits the MFMA stream here
                out = [f"{ind}{{ const int gi = {g}; const bool nxt = gi >= T && nx_q < q_end;",
                       f"{ind}  const int k0 = k_at(nxt ? nx_g0 : g0, nxt ? nx_T : T, nxt ? nx_sb : sb, nxt ? gi - T : gi);",
                       f"{ind}  const __amdgpu_buffer_rsrc_t ra = nxt ? nx_rsa : rsa, rb = nxt ? nx_rsb : rsb;"]
                if dual:
                    out.append(f"{ind}  const __amdgpu_buffer_rsrc_t rb2 = nxt ? nx_rsb2 : rsb2;")
            elif cross:
                out = [f"{ind}{{ const int k0 = k_at(g0, T, sb, {g}); const __amdgpu_buffer_rsrc_t ra = rsa, rb = rsb;"]
                if dual:
                    out.append(f"{ind}  const __amdgpu_buffer_rsrc_t rb2 = rsb2;")
            else:
                out = [f"{ind}{{ const int k0 = k_of({g}); const __amdgpu_buffer_rsrc_t ra = rsa, rb = rsb;"]
                if dual:
                    out.append(f"{ind}  const __amdgpu_buffer_rsrc_t rb2 = rsb2;")
            rows_a = T // kca
            for c in range(a_ld):
                out.append(f"{ind}  __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, AK_LDS(&ak_sa{s}[({c * T} + wave * 64) * 8]), "
                           f"16, a_voff, {c * rows_a}u * pa + (unsigned)k0 * 2u, 0, 0);")
            halves = (("rb", 0), ("rb2", bk * bn)) if dual else (("rb", 0),)
            for rsrc, base in halves:  # with two right operands, b's BK x BN slice, then b2's after it
                for c in range(b_ld // len(halves)):
                    if nt:
                        soff = f"{c * rows_a}u * pb + (unsigned)k0 * 2u"
                    else:
                        soff = f"(unsigned)(k0 + {c * (T // nc)}) * pb"
                    at = f"{base} + " if base else ""
                    out.append(f"{ind}  __builtin_amdgcn_raw_ptr_buffer_load_lds({rsrc}, AK_LDS(&ak_sb{s}[{at}({c * T} + wave * 64) * 8]), "
                               f"16, b_voff, {soff}, 0, 0);")
            out.append(f"{ind}}}")
            return out

        def reads(s: int, k16: int, b: int, ind: str) -> List[str]:
            out = [f"{ind}fa[{b}][{i}] = *(const ak_bf16x8*)((const char*)ak_sa{s} + a_roff[{k16}] + {i * 32 * bk * 2});"
                   for i in range(mi)]
            for j in range(ni):
                if nt:
                    out.append(f"{ind}fb[{b}][{j}] = *(const ak_bf16x8*)((const char*)ak_sb{s} + b_roff[{k16}] + {j * 32 * bk * 2});")
                else:
                    o = k16 * 16 * bn * 2
                    out.append(f"{ind}{{ ak_i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(AK_LDS4((const char*)ak_sb{s} + b_roff[{j}] + {o}));"
                               f" ak_i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(AK_LDS4((const char*)ak_sb{s} + b_roff[{j}] + {o + 4 * bn * 2}));"
                               f" fb[{b}][{j}] = __builtin_bit_cast(ak_bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7)); }}")
            return out

        def mfmas(b: int, ind: str) -> List[str]:
            return [f"{ind}acc[{i}][{j}] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[{b}][{j}], fa[{b}][{i}], acc[{i}][{j}], 0, 0, 0);"
                    for i in range(mi) for j in range(ni)]

        n_reads = mi + (ni if nt else 2 * ni)
        per_slice = a_ld + b_ld

        def hints(ind: str, issue_too: bool) -> List[str]:
            # Interleave: each MFMA followed by one LDS read (and one global load where the slice issues).
            out, r, v = [], n_reads, per_slice if issue_too else 0
            for _ in range(mi * ni):
                out.append(f"{ind}__builtin_amdgcn_sched_group_barrier(0x008, 1, 0);")
                if r:
                    out.append(f"{ind}__builtin_amdgcn_sched_group_barrier(0x100, 1, 0);")
                    r -= 1
                if v:
                    out.append(f"{ind}__builtin_amdgcn_sched_group_barrier(0x020, 1, 0);")
                    v -= 1
            return out

        # The LDS events of an item's slices, as emitted: `protocol.check` replays items back to back. In the
        # cross-item form (ItemRecorder) block ids are global: gid(k) is the item's k-th slice, then the next
        # loading item's, or the item's last slice reloaded where none follows.
        if cross:
            rec = self.protocol = ItemRecorder()
            ind = "      "
            w(f"    if (T > 0) {{  // (an item without steps loads nothing: it stores the initial value)")
            if self.trace:
                w(f"{ind}const unsigned long long tr_i0 = {now}; tr_slices += T;")
            w(f"{ind}if (pf_q != q) {{  // not loaded during the previous item: fill the stages now")
            for s in range(S):
                L.extend(issue(str(s), s, ind + "  "))
                rec.add(lambda b, n, nxt, gid, s=s: ("load", s, gid(s), per_slice), lambda n, nxt, pre: n > 0 and not pre)
            w(f"{ind}}}")
            rec.add(lambda b, n, nxt, gid: ("wait_vm", per_slice * (S - 1)), lambda n, nxt, pre: n > 0)
            rec.add(lambda b, n, nxt, gid: ("barrier",), lambda n, nxt, pre: n > 0)
            rec.add(lambda b, n, nxt, gid: ("read", 0, gid(0)), lambda n, nxt, pre: n > 0)
        else:
            rec = self.protocol = Recorder()
            ind = "    "
            if self.trace:
                w(f"{ind}const unsigned long long tr_i0 = {now}; tr_slices += T;")
            for s in range(S):
                L.extend(issue(str(s), s, ind))
                rec.add(("load", s, s, per_slice))
            rec.add(("wait_vm", per_slice * (S - 1)))
            rec.add(("barrier",))
            rec.add(("read", 0, 0))
        # Slice 0 has landed here (at most S - 1 slices' loads are younger; the epilogue's stores, issued after
        # them, are waited for too where they are still in flight) and, after the barrier, every wave's.
        w(f"{ind}AK_WAIT_VM({per_slice * (S - 1)});")
        w(f'{ind}asm volatile("s_barrier" ::: "memory");')
        if self.trace:
            w(f"{ind}const unsigned long long tr_c0 = {now}; tr_fill += tr_c0 - tr_i0;")
        L.extend(reads(0, 0, 0, ind))
        rec.loop(S)
        w(f"{ind}for (int g = 0; g < T; g += {S}) {{")
        ind2 = ind + "  "
        for s in range(S):
            for k16 in range(k16s):
                cur = (s * k16s + k16) & 1
                w(f"{ind2}{{")
                if k16 < k16s - 1:
                    L.extend(reads(s, k16 + 1, cur ^ 1, ind2 + "  "))
                    if cross:
                        rec.at(s, lambda b, n, nxt, gid, st=s: ("read", st, gid(b)))
                    else:
                        rec.at(s, lambda b, n, st=s: ("read", st, b))
                    L.extend(mfmas(cur, ind2 + "  "))
                    L.extend(hints(ind2 + "  ", False))
                else:
                    # Last K16 of slice g + s: our reads of its stage are done, and (after the barrier) every
                    # wave's; slice g + s + 1 has landed. Refill this stage with slice g + s + S and read the
                    # next slice's first fragments while this slice's last MFMAs run.
                    if self.trace:
                        w(f"{ind2}  const unsigned long long tr_w0 = {now};")
                    w(f"{ind2}  AK_WAIT_LGKM0();")
                    w(f"{ind2}  AK_WAIT_VM({per_slice * (S - 2)});")
                    w(f'{ind2}  asm volatile("s_barrier" ::: "memory");')
                    if self.trace:
                        w(f"{ind2}  tr_wait += {now} - tr_w0;")
                    L.extend(issue(f"g + {s + S}", s, ind2 + "  ", refill=True))
                    L.extend(reads((s + 1) % S, 0, cur ^ 1, ind2 + "  "))
                    if cross:
                        rec.at(s, lambda b, n, nxt, gid: ("wait_lgkm",))
                        rec.at(s, lambda b, n, nxt, gid: ("wait_vm", per_slice * (S - 2)))
                        rec.at(s, lambda b, n, nxt, gid: ("barrier",))
                        rec.at(s, lambda b, n, nxt, gid, st=s: ("load", st, gid(b + S), per_slice))
                        rec.at(s, lambda b, n, nxt, gid, st=(s + 1) % S: ("read", st, gid(b + 1)))
                    else:
                        rec.at(s, lambda b, n: ("wait_lgkm",))
                        rec.at(s, lambda b, n: ("wait_vm", per_slice * (S - 2)))
                        rec.at(s, lambda b, n: ("barrier",))
                        rec.at(s, lambda b, n, st=s: ("load", st, b + S, per_slice))
                        rec.at(s, lambda b, n, st=(s + 1) % S: ("read", st, b + 1))
                    L.extend(mfmas(cur, ind2 + "  "))
                    L.extend(hints(ind2 + "  ", True))
                w(f"{ind2}}}")
        w(f"{ind}}}")
        rec.end_loop()
        if cross:
            # The next loading item's first slices are in flight in the stages: no drain here. The last loads
            # are waited for once, before the workgroup ends.
            w(f"{ind}pf_q = nx_q < q_end ? nx_q : -1;")
            if self.trace:
                w(f"{ind}tr_comp += {now} - tr_c0;")
            w("    }")
            rec.end.append(("wait_vm", 0))
            self._queue_tail = "  AK_WAIT_VM(0);  // no load into LDS in flight when the workgroup ends\n"
            if self.trace:
                w(f"    const unsigned long long tr_o0 = {now};")
        else:
            # every load and LDS read of the item done, in every wave, before the next item's loads reuse the stages
            w(f"{ind}AK_WAIT_VM(0); AK_WAIT_LGKM0();")
            w(f'{ind}asm volatile("s_barrier" ::: "memory");')
            rec.add(("wait_vm", 0))
            rec.add(("wait_lgkm",))
            rec.add(("barrier",))
            if self.trace:
                w(f"{ind}const unsigned long long tr_o0 = {now}; tr_comp += tr_o0 - tr_c0;")
        if self.split:
            w(f"""    if (kind == 3) {{  // a chunk: its f32 partial sums go to workspace slot `slot`, lane-contiguous
      // The lane index goes through an empty asm, as in the epilogue: the stores' addresses are then computed
      // here, not hoisted above the K loop where they would take the registers it needs.
      int lane_p = lane;
      asm volatile("" : "+v"(lane_p));
      float* part = args.gm_part + (long long)slot * {bm * bn} + (wave * {mi * ni * 4 * 64} + lane_p) * 4;
      // One accumulator tile at a time through VGPRs (the empty asm orders the copies).
#pragma unroll
      for (int i_ = 0; i_ < {mi}; ++i_)
#pragma unroll
        for (int j_ = 0; j_ < {ni}; ++j_) {{
          ak_f32x16 t_ = acc[i_][j_];
          asm volatile("" : "+v"(t_));
#pragma unroll
          for (int g4 = 0; g4 < 4; ++g4)
            *(ak_f32x4*)(part + ((i_ * {ni} + j_) * 4 + g4) * 256) = ak_f32x4{{t_[g4 * 4], t_[g4 * 4 + 1], t_[g4 * 4 + 2], t_[g4 * 4 + 3]}};
        }}
      {"tr_out += " + now + " - tr_o0;" if self.trace else ""}
      continue;
    }}""")
        # the second accumulator of each pair (two right operands), at the same output position
        acc2_line = " const float acc2_v = acc[i_][j_ + " + str(nio) + "][g4 * 4 + e4];" if dual else ""
        old_loop = f"""#pragma unroll
      for (int j_ = 0; j_ < {nio}; ++j_) {{
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {{
          const int ec0 = sn * {bn} + wn * {wto} + j_ * 32 + g4 * 8 + (lane_e >> 5) * 4;
          float res[4];
#pragma unroll
          for (int e4 = 0; e4 < 4; ++e4) {{
            const int ec = ec0 + e4;
            const float acc_v = acc[i_][j_][g4 * 4 + e4];{acc2_line}
            (void)ec; (void)er;
            {epi}
            res[e4] = (float)({result});
          }}
          {_store4(O, "obase", ldo, out_bf16)}
        }}
      }}
    }}"""
        paired_loop = f"""#pragma unroll
      for (int j_ = 0; j_ < {nio}; ++j_) {{
#pragma unroll
        for (int p2 = 0; p2 < 2; ++p2) {{
          // groups 2 p2 and 2 p2 + 1, then one exchange with lane ^ 32: each lane stores 8 consecutive
          // outputs (16 bytes), the lower half-wave columns 16 p2 .. + 7, the upper 16 p2 + 8 .. + 15
          unsigned pk[2][2];
#pragma unroll
          for (int h2 = 0; h2 < 2; ++h2) {{
            const int g4 = 2 * p2 + h2;
            const int ec0 = sn * {bn} + wn * {wto} + j_ * 32 + g4 * 8 + (lane_e >> 5) * 4;
            float res[4];
#pragma unroll
            for (int e4 = 0; e4 < 4; ++e4) {{
              const int ec = ec0 + e4;
              const float acc_v = acc[i_][j_][g4 * 4 + e4];{acc2_line}
              (void)ec; (void)er;
              {epi}
              res[e4] = (float)({result});
            }}
            pk[h2][0] = ak_pack_bf16x2(res[0], res[1]);
            pk[h2][1] = ak_pack_bf16x2(res[2], res[3]);
          }}
          const bool up = lane_e >= 32;
          // lane and lane ^ 32 swap halves: the low lanes keep pk[0] and take their partner's pk[0], the high
          // lanes take their partner's pk[1] and keep pk[1] (v_permlane32_swap, no LDS crossbar)
          const auto s0 = __builtin_amdgcn_permlane32_swap(pk[0][0], pk[1][0], false, false);
          const auto s1 = __builtin_amdgcn_permlane32_swap(pk[0][1], pk[1][1], false, false);
          const ak_u32x4 v = ak_u32x4{{s0[0], s1[0], s0[1], s1[1]}};
          const int ec8 = sn * {bn} + wn * {wto} + j_ * 32 + 16 * p2 + (up ? 8 : 0);
          *(ak_u32x4*)((ak_u16*){O} + obase + (long long)er * {ldo} + ec8) = v;
        }}
      }}
    }}"""
        if out_bf16 and ldo % 8:
            raise KernelError("the gfx950 matmul lowering stores bf16 outputs 16 bytes at a time: rows of a multiple "
                              f"of 8 elements, not {ldo}")
        EPILOGUE_LOOP = paired_loop if out_bf16 else old_loop
        w(f"""    // Epilogue: the accumulator holds C transposed (lane: one row, four consecutive columns per group).
    // The lane index goes through an empty asm so the stores' addresses are computed here, not hoisted
    // above the K loop where they would take registers the loop needs.
    int lane_e = lane;
    asm volatile("" : "+v"(lane_e));
#pragma unroll
    for (int i_ = 0; i_ < {mi}; ++i_) {{
      const int er = sm * {bm} + wm * {wtm} + i_ * 32 + (lane_e & 31);
{EPILOGUE_LOOP}
    {"tr_out += " + now + " - tr_o0;" if self.trace else ""}
  }}
{self._queue_tail}  {trace_write}
}}""")
        if self.split:
            r, split, _ = self.split
            per_item = bm * bn // (4 * THREADS)
            w(f"""
// The fixup of tiles cut along the reduction: each thread adds one float4 of the {split} chunks' partial sums
// (in chunk order), then applies the epilogue to those four outputs.
extern "C" __global__ void __launch_bounds__({THREADS}) {self.name}_fixup(const {self.name}_args args) {{
  const int p = blockIdx.x / {per_item};
  const int e = (blockIdx.x % {per_item}) * {THREADS} + threadIdx.x;
  const int lane_e = e & 63, g4 = (e >> 6) & 3, j_ = (e >> 8) % {ni}, i_ = (e >> 8) / {ni} % {mi};
  const int wave = (e >> 8) / {ni * mi}, wm = wave / {WN}, wn = wave % {WN};
  const float* part = args.gm_part + (long long)p * {split * bm * bn} + e * 4;
  ak_f32x4 sum = *(const ak_f32x4*)part;
#pragma unroll
  for (int c = 1; c < {split}; ++c) {{
    const ak_f32x4 v = *(const ak_f32x4*)(part + (long long)c * {bm * bn});
    sum[0] += v[0]; sum[1] += v[1]; sum[2] += v[2]; sum[3] += v[3];
  }}
  const int t = args.split_items[2 * p], sub = args.split_items[2 * p + 1] & 0xffff;
  const int sm = sub / {self.sub_n}, sn = sub % {self.sub_n};
  {tile_decode}
  const long long obase = {o_base};
  const int er = sm * {bm} + wm * {wtm} + i_ * 32 + (lane_e & 31);
  const int ec0 = sn * {bn} + wn * {wtn} + j_ * 32 + g4 * 8 + (lane_e >> 5) * 4;
  float res[4];
#pragma unroll
  for (int e4 = 0; e4 < 4; ++e4) {{
    const int ec = ec0 + e4;
    const float acc_v = sum[e4];
    (void)ec; (void)er;
    {epi}
    res[e4] = (float)({result});
  }}
  {_store4(O, "obase", ldo, out_bf16)}
}}""")
        return "\n".join(L)


def _cstore(dt: jaxlite.DType) -> str:
    return {"bfloat16": "__bf16", "float32": "float", "int32": "int", "float16": "_Float16"}.get(dt.name, "void")


def _store4(O: str, obase: str, ldo: int, bf16: bool) -> str:
    if bf16:
        return (f"*(ak_u32x2*)((ak_u16*){O} + {obase} + (long long)er * {ldo} + ec0) = "
                "ak_u32x2{ak_pack_bf16x2(res[0], res[1]), ak_pack_bf16x2(res[2], res[3])};")
    return f"*(ak_f32x4*)({O} + {obase} + (long long)er * {ldo} + ec0) = ak_f32x4{{res[0], res[1], res[2], res[3]}};"


def _store_constant(bm: int, bn: int, bf16: bool, O: str, obase: str, ldo: int, value: str, threads: int) -> str:
    """Source storing one value over the workgroup's hardware sub-tile (sm, sn)."""
    if bf16:
        return (
            f"{{ const unsigned w_ = ak_bf16_bits((float)({value})) * 0x10001u; const ak_u32x4 v_ = {{w_, w_, w_, w_}};\n"
            f"        for (int c_ = tid; c_ < {bm * bn // 8}; c_ += {threads}) {{\n"
            f"          const int r_ = c_ / {bn // 8}, k_ = c_ % {bn // 8};\n"
            f"          *(ak_u32x4*)((ak_u16*){O} + {obase} + (long long)(sm * {bm} + r_) * {ldo} + sn * {bn} + k_ * 8) = v_;\n"
            "        } }"
        )
    return (
        f"{{ const float f_ = (float)({value}); const ak_f32x4 v_ = {{f_, f_, f_, f_}};\n"
        f"        for (int c_ = tid; c_ < {bm * bn // 4}; c_ += {threads}) {{\n"
        f"          const int r_ = c_ / {bn // 4}, k_ = c_ % {bn // 4};\n"
        f"          *(ak_f32x4*)({O} + {obase} + (long long)(sm * {bm} + r_) * {ldo} + sn * {bn} + k_ * 4) = v_;\n"
        "        } }"
    )
