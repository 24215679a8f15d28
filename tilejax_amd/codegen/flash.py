"""Lowering of online-softmax attention loop nests to one gfx950 flash-attention kernel.

The family is the reference's causal attention spec (examples/causal_attention.py:37-63): per output tile
of query rows, a reduction loop over key/value blocks whose body is

    s  = score(q_tile @ k_block.T)                      # pointwise in s, positions, loop values
    m' = maximum(m, max(s, axis=1))                     # m, l: row statistics (row-uniform)
    p  = exp(s - m')
    l' = exp(m - m') * l + sum(p, axis=1)
    acc' = exp(m - m') * acc + p.astype(v.dtype) @ v_block
    m  = m'

and whose output is a pointwise function of acc and l. `match` recognises that structure in the traced
tile code (whatever the spelling: widened statistics, `jnp.tile`, operand order) and extracts the two
pointwise pieces, `score` and the epilogue, which are emitted per element.

The kernel (one workgroup per block of BQ query rows, BQ = 32 x waves, or 64 x waves with the knob `rows`;
blocks largest-first so the GPU balances them):

- each wave owns 32 query rows (or two halves of 32 that share every K and V fragment it reads) and
  computes S^T = K Q^T with `v_mfma_f32_32x32x16_bf16`, so a lane holds one query row's scores: the row
  max and sum are an in-lane reduction plus one exchange with lane ^ 32;
- P^T (bf16) feeds O^T = V^T P^T straight from the S^T accumulators, V read transposed from LDS with
  `ds_read_b64_tr_b16` in the order the accumulator layout gives the key positions;
- K and V blocks of BKV rows stream HBM -> LDS (`buffer_load_dwordx4 ... lds`) through two stages, the next
  block's loads in flight under this block's MFMAs;
- the key blocks a work item visits are the spec's (its step tables), split into BKV-row blocks; per wave,
  the host's interval analysis of `score` over each block's rectangle marks blocks where the mask keeps
  every score (computed without it) and, after a block that gives every row a real score, blocks where it
  keeps none (skipped: their probabilities are exactly zero).
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Any, Dict, List, Optional, Sequence, Tuple

import numpy as np

from .. import gfx950, jaxlite
from ..errors import KernelError
from ..jaxlite import Node
from ..pipeline import Pipeline
from ..plan import Kind, Operand, Output, Plan
from ..schedule import CODE_SHIFT, STEP_CODE, Schedule
from .common import Index, decode_tile, static_tile_steps, strides, tile_base
from .device import PRELUDE
from .expr import Emitter, Interval, intervals, literal, nodes_between
from .program import CLOCK_END, CLOCK_START, NOW, TRACE, TRACE_FIELDS, Arg, Launch, Program, c_struct
from .protocol import Recorder

__all__ = ["FlashMatch", "match", "lower"]

LOG2E = 1.4426950408889634
RESCALE_SLACK = 8.0  # natural-log units: p stays below e^8 between rescales
MASKED_BELOW = -1e20  # a constant score this low contributes exp(c - m) == 0 once a row has a real score
# Workgroups of 4 waves (128 query rows) with two LDS stages (64 KiB): two workgroups share a CU, and as
# they keep no step with each other, one's MFMA work runs beside the other's softmax. Measured against one
# workgroup of 8 waves (256 rows) and four stages: equal at (4, 16, 2048, 128), 5 % faster at
# (1, 16, 4096, 128).
# K and V blocks are loaded `ahead` blocks ahead of use (the pipeline's input buffers less one, at most
# MAX_AHEAD) through ahead + 1 LDS stages, one barrier per block; block-table entries of blocks b .. b + ahead
# + 1 are kept in a ring of ahead + 2 scalars, at b modulo the ring.
MAX_AHEAD = 3
WAVES = 4  # waves per workgroup (None: 8 for tiles of a multiple of 256 query rows, else 4)
ROWS = 32  # query rows per wave (the knob `rows`: 32, or 64 as two halves sharing the K and V fragments)
BKV = 64  # keys per block (a multiple of 32)
K_AHEAD = 8  # K fragments in flight ahead of the S MFMAs
# With K in registers (knob `kreg`): register sets of K fragments. With two, the next block's set is loaded
# while this block's is read; with one, it is loaded over this block's once the S product has read it.
KREG_SETS = 1
V_AHEAD = 4  # V fragments in flight ahead of the O MFMAs
# Split-KV: a work item's cost is its key blocks plus ITEM_COST (its Q load, pipeline fill and stores); a
# workgroup's share is the total over the resident workgroups (two per CU). Items above SPLIT_ABOVE shares
# are cut into chunks of about a share, and of at least MIN_CHUNK blocks (a chunk's partial (m, l, acc) and
# its merge cost about that much). Measured at 512 x 512 spec blocks: (1, 16, 4096, 128) 90.5 -> 87.5 us,
# (1, 8, 8192, 128) 170 -> 155 us, (2, 4, 1024, 128) 25.3 -> 22.0 us; 1.25 shares split too much, and
# (4, 16, 2048, 128) has no item above 1.5. Static per-workgroup work lists balanced by the same cost (LPT)
# measured no faster than the dispatcher's own order: of two workgroups on a CU the older one issues more,
# so equal work does not finish together.
ITEM_COST = 2
SPLIT_ABOVE = 1.5
MIN_CHUNK = 3


@dataclass
class FlashMatch:
    q: Operand  # TILE: (R, D) query rows
    k: Operand  # STREAM: (bk, D)
    v: Operand  # STREAM: (bk, Dv)
    jvar: str  # the reduction loop over key blocks
    scores: Node  # dot_nt(q, k): S
    score: Node  # score(S): what the max and exp read
    m_init: float
    out: Output
    value: Any  # the stored value (Node)
    acc_leaf: Node  # acc in the end scope
    sum_leaf: Node  # l in the end scope
    rows: int
    bk: int
    d: int
    dv: int


def _is(n: Any, op: str) -> bool:
    return isinstance(n, Node) and n.op == op


def _strip(n: Any) -> Any:
    """A value without the row broadcasts the spec spells (jnp.tile / broadcast_to, or a slice of its
    leading columns): they don't change a row-uniform value."""
    while isinstance(n, Node):
        if n.op in ("tile", "broadcast_to"):
            n = n.args[0]
        elif n.op == "getitem" and isinstance(n.args[1], tuple) and len(n.args[1]) == 2 and \
                n.args[1][0] == slice(None) and isinstance(n.args[1][1], slice):
            n = n.args[0]
        else:
            break
    return n


def _pair(n: Node, op: str) -> Optional[Tuple[Any, Any]]:
    if _is(n, op):
        return n.args[0], n.args[1]
    return None


def _either(pair: Optional[Tuple[Any, Any]], test) -> Optional[Tuple[Any, Any]]:
    """(x, other) where x passes `test`, trying both orders of a commutative pair."""
    if pair is None:
        return None
    a, b = pair
    if test(a):
        return a, b
    if test(b):
        return b, a
    return None


def _full_value(v: Any) -> Optional[float]:
    if isinstance(v, jaxlite.Sym) and _is(v.node, "full"):
        return float(v.node.kwargs["value"])
    if isinstance(v, (int, float)):
        return float(v)
    return None


@dataclass
class Softmax:
    """The online-softmax reduction of a loop nest's body, as `softmax_structure` finds it."""

    qk: Node  # dot_nt(queries, keys)
    pv: Node  # dot(p.astype, values)
    score: Node
    m_name: str
    l_name: str
    acc_name: str
    m_init: float
    consts: Tuple[str, ...]  # carried values the body never changes: per-tile values of the setup code


def softmax_structure(plan: Plan) -> Optional[Softmax]:
    """The online softmax of the body (the module docstring's form), or None. Besides the three statistics,
    carried values may only be per-tile constants (assigned before the loop, read in it or after it)."""
    if len(plan.outputs) != 1 or len(plan.phases) != 1:
        return None
    body, seg0 = plan.scopes["body0"], plan.scopes["seg0"]
    dots = [n for n in body.nodes if n.op in ("dot", "dot_nt")]
    if len(dots) != 2:
        return None
    qk = next((n for n in dots if n.op == "dot_nt"), None)
    pv = next((n for n in dots if n.op == "dot"), None)
    if qk is None or pv is None or not (_is(qk.args[1], "load") and _is(pv.args[1], "load")):
        return None
    new = {c: body.values.get(c) for c in plan.carried}
    leaf = body.carried_in
    consts = tuple(c for c, val in new.items() if isinstance(val, jaxlite.Sym) and val.node is leaf.get(c))
    consts += tuple(c for c in plan.carried if c not in new or new[c] is None)
    acc = next((c for c, val in new.items() if isinstance(val, jaxlite.Sym) and _pair(val.node, "add")
                and pv in val.node.args), None)
    if acc is None:
        return None
    rest = [c for c in plan.carried if c != acc and c not in consts]
    if len(rest) != 2:
        return None
    m_name = next((c for c in rest if isinstance(new[c], jaxlite.Sym) and _is(_strip(new[c].node), "maximum")), None)
    if m_name is None:
        return None
    l_name = next(c for c in rest if c != m_name)
    m_in, l_in, acc_in = leaf.get(m_name), leaf.get(l_name), leaf.get(acc)
    if m_in is None or l_in is None or acc_in is None:
        return None
    # m' = maximum(m, max(score, axis=1))
    m_new = _strip(new[m_name].node)
    got = _either(_pair(m_new, "maximum"), lambda x: _strip(x) is m_in)
    if got is None or not _is(got[1], "reduce_max") or got[1].kwargs.get("axis") not in (1, -1):
        return None
    score = got[1].args[0]
    # p = exp(score - m'); alpha = exp(m - m')
    exps = [n for n in body.nodes if n.op == "exp"]
    p = next((n for n in exps if _is(n.args[0], "subtract") and n.args[0].args[0] is score
              and _strip(n.args[0].args[1]) is m_new), None)
    alpha = next((n for n in exps if _is(n.args[0], "subtract") and _strip(n.args[0].args[0]) is m_in
                  and _strip(n.args[0].args[1]) is m_new), None)
    if p is None or alpha is None:
        return None
    # l' = alpha * l + sum(p, axis=1)
    l_new = new[l_name].node if isinstance(new[l_name], jaxlite.Sym) else None
    got = _either(_pair(l_new, "add"), lambda x: _is(x, "reduce_sum") and x.args[0] is p)
    if got is None or _either(_pair(got[1], "multiply"), lambda x: _strip(x) is alpha) is None:
        return None
    if _strip(_either(_pair(got[1], "multiply"), lambda x: _strip(x) is alpha)[1]) is not l_in:
        return None
    # acc' = alpha * acc + p.astype(v.dtype) @ v
    scaled = _either(_pair(new[acc].node, "add"), lambda x: x is pv)[1]
    got = _either(_pair(scaled, "multiply"), lambda x: _strip(x) is alpha)
    if got is None or got[1] is not acc_in:
        return None
    p16 = pv.args[0]  # p.astype(v.dtype): bf16 (or p itself, f32, where the cast changes nothing)
    if not ((_is(p16, "astype") and p16.args[0] is p and p16.dtype.name in ("bfloat16", "float32"))
            or (p16 is p and p.dtype.name == "float32")):
        return None
    # The score is pointwise in S: everything between S and it is elementwise on positions and loop values.
    stack, seen = [score], set()
    while stack:
        n = stack.pop()
        if n.id in seen or n is qk:
            continue
        seen.add(n.id)
        if n.op in ("dot", "dot_nt", "load", "reduce_max", "reduce_sum", "reshape", "concatenate"):
            return None
        if n.op == "carried" and n.kwargs["name"] not in consts:
            return None
        stack.extend(n.inputs())
    # Initial values: m a constant, l and acc zero.
    m_init = _full_value(seg0.values.get(m_name))
    if m_init is None or _full_value(seg0.values.get(l_name)) != 0.0 or _full_value(seg0.values.get(acc)) != 0.0:
        return None
    return Softmax(qk, pv, score, m_name, l_name, acc, m_init, consts)


def match(plan: Plan) -> Optional[FlashMatch]:
    """The attention this loop nest is (queries a TILE read, keys and values streamed, static masks), or
    None."""
    sm = softmax_structure(plan)
    if sm is None or sm.consts or plan.runtime:
        return None
    qk, pv, score, m_init = sm.qk, sm.pv, sm.score, sm.m_init
    if not _is(qk.args[0], "load"):
        return None
    q, k, v = (plan.operand(n.kwargs["operand"]) for n in (qk.args[0], qk.args[1], pv.args[1]))
    if q.kind is not Kind.TILE or k.kind is not Kind.STREAM or v.kind is not Kind.STREAM:
        return None
    if len({op.tile.dtype.name for op in (q, k, v)}) != 1 or q.tile.dtype.name not in ("bfloat16", "float32"):
        return None
    if (q.tile.dtype.name == "float32") != (pv.args[0].dtype.name == "float32"):
        return None
    phase = plan.phases[0].range
    last = plan.scopes["last"]
    acc, l_name = sm.acc_name, sm.l_name
    out = plan.outputs[0]
    value = last.stores.get(out.name)
    if not isinstance(value, jaxlite.Sym):
        return None
    acc_leaf, sum_leaf = last.carried_in.get(acc), last.carried_in.get(l_name)
    if acc_leaf is None or sum_leaf is None:
        return None
    rows, d = q.tile.shape
    bk, dk = k.tile.shape
    bv, dv = v.tile.shape
    if dk != d or bv != bk or tuple(out.tile.shape[-2:]) != (rows, dv) or qk.shape != (rows, bk):
        return None
    return FlashMatch(q, k, v, phase.var, qk, score, m_init, out, value, acc_leaf, sum_leaf, rows, bk, d, dv)


# ---------------------------------------------------------------------------------------------- host side


def _loop_window(op: Operand, var: str) -> Tuple[int, Any]:
    """(dim, window) of the tile dim the loop `var` places."""
    for dim, w in enumerate(op.tile.windows):
        if w.loop == var:
            return dim, w
    raise KernelError(f"`{op.tile.text}` is not placed by loop `{var}`")


class _Flash:
    def __init__(self, plan: Plan, sch: Schedule, pipeline: Pipeline, m: FlashMatch, name: str,
                 trace: bool = False, hardware: Optional[Dict[str, int]] = None) -> None:
        self.plan, self.sch, self.pipeline, self.m, self.name = plan, sch, pipeline, m, name
        self.trace = trace
        hardware = hardware or {}
        # K and V blocks loaded `ahead` blocks ahead through ahead + 1 LDS stages: the pipeline's input buffers
        self.ahead = max(1, min(pipeline.input_buffers - 1, MAX_AHEAD))
        self.stages, self.ring = self.ahead + 1, self.ahead + 2
        if m.d % 32 or m.dv % 32 or m.d > 128 or m.dv > 128:
            raise KernelError(f"the gfx950 attention lowering takes head dims that are multiples of 32 up to 128 "
                              f"(got {m.d} and {m.dv})")
        self.nw = hardware.get("waves", WAVES) or (8 if m.rows % 256 == 0 else 4 if m.rows % 128 == 0 else 0)
        # query rows per wave: 32, or 64 as two 32-row halves that share every K and V fragment it reads
        self.wr = hardware.get("rows", ROWS)
        if self.wr not in (32, 64):
            raise KernelError(f"the attention knob rows is 32 or 64 query rows a wave (got {self.wr})")
        if not self.nw or m.rows % (self.wr * self.nw):
            raise KernelError(f"the gfx950 attention lowering needs query tiles of a multiple of "
                              f"{self.wr * (self.nw or 4)} rows (got {m.rows})")
        self.bq = self.wr * self.nw
        self.bkv = hardware.get("bkv", BKV)
        # K fragments loaded from memory straight into registers (a register set per block, the next block's
        # loaded after this block's S product) rather than through LDS, which then holds V only
        self.kreg = bool(hardware.get("kreg", 0))
        if self.kreg and self.ahead != 1:
            raise KernelError("K fragments in registers are loaded one block ahead: two LDS stages for V")
        # split-KV above this many shares, in tenths (0: never split)
        self.split_tenths = hardware.get("split", round(10 * SPLIT_ABOVE))
        if self.split_tenths < 0:
            raise KernelError(f"the split share is a number of tenths of a share, 0 or more (got {self.split_tenths})")
        if m.bk % self.bkv:
            raise KernelError(f"the gfx950 attention lowering needs key blocks of a multiple of {self.bkv} (got {m.bk})")
        lds = self.stages * self.bkv * ((0 if getattr(self, 'kreg', False) else m.d) + m.dv) * 2
        if lds > gfx950.LDS_BUDGET:
            raise KernelError(f"{self.stages} LDS stages of {self.bkv} keys (head dims {m.d}, {m.dv}) take {lds} bytes of "
                              f"LDS per workgroup; gfx950 has {gfx950.LDS_BUDGET}")
        if plan.runtime or sch.runtime:
            raise KernelError("attention with runtime masks is lowered by the decode path, not this one")
        self.jr = plan.phases[0].range
        self.kdim, self.kwin = _loop_window(m.k, m.jvar)
        self.vdim, self.vwin = _loop_window(m.v, m.jvar)

    # The blocks each work item visits, and the per-wave mask classes.
    def _classify(self, values: Dict[str, int], r0: int, r1: int, c0: int, c1: int) -> str:
        """'full' if score == S over rows [r0, r1] x cols [c0, c1] of the tile (spec-local positions) at these
        loop values; 'none' if it is a constant below MASKED_BELOW there; else 'partial'."""
        m = self.m
        marker = Interval(data=True)

        def leaf(n: Node) -> Optional[Interval]:
            if n is m.scores:
                return marker
            if n.op == "iota":
                dim = n.kwargs["dimension"]
                if dim == len(n.shape) - 2:
                    return Interval(r0, r1)
                if dim == len(n.shape) - 1:
                    return Interval(c0, c1)
                return Interval()
            if n.op == "loop":
                val = values.get(n.kwargs["var"])
                return Interval(val, val) if val is not None else Interval()
            if n.op == "full":
                return Interval(n.kwargs["value"], n.kwargs["value"], const=n.kwargs["value"])
            if n.op in ("load", "carried", "index"):
                return Interval(data=True)
            return None

        got = intervals(m.score, leaf)
        if got is marker:
            return "full"
        if not got.data and got.const is not None and float(got.const) <= MASKED_BELOW:
            return "none"
        return "partial"

    def _items(self):
        plan, sch, m = self.plan, self.sch, self.m
        jr, bq = self.jr, self.bq
        subs = m.rows // bq
        offsets = static_tile_steps(sch) if sch.step_tables else None
        codes = sch.tables.get(STEP_CODE)
        patterns: Dict[Tuple, Tuple[List[Tuple[int, int]], List[Tuple[int, int]]]] = {}
        items, weights, blocks = [], [], []
        for t in range(sch.tiles):
            blocks_t = sch.blocks_at(t)
            values = {r.var: r.value(b) for r, b in zip(plan.parallel, blocks_t)}
            if offsets is not None:
                pt = t % sch.pattern_tiles
                steps = range(int(offsets[pt]), int(offsets[pt + 1]))
                kbs = [((int(codes[s]) >> CODE_SHIFT) // sch.iterations // sch.phase_radix) for s in steps
                       if not (int(codes[s]) & 4)]
            else:
                kbs = list(range(jr.count))
            inner = tuple(values[r.var] for r in sch.inner) if sch.tile_tables or sch.step_tables else ()
            key = (inner, tuple(kbs)) if (sch.tile_tables or sch.step_tables) else ("all",)
            for sub in range(subs):
                pkey = key + (sub,)
                if pkey not in patterns:
                    patterns[pkey] = self._pattern(values, kbs, sub)
                blist, waves = patterns[pkey]
                items.append((t, sub, len(blocks), len(blist), waves))
                weights.append(sum(n for _, n in waves))
                blocks.extend(blist)
        return items, weights, blocks

    def _pattern(self, values: Dict[str, int], kbs: Sequence[int], sub: int):
        """For one work item: its hardware key blocks [(j value, offset in the spec block)], and per wave
        (blocks computed without the mask, blocks to compute)."""
        m, bkv, bq = self.m, self.bkv, self.bq
        per_spec = m.bk // bkv
        cand = [(self.jr.value(kb), o * bkv) for kb in kbs for o in range(per_spec)]
        classes = []
        for jv, off in cand:
            vals = {**values, m.jvar: jv}
            row = []
            for wv in range(self.nw):
                r0 = sub * bq + wv * self.wr
                row.append(self._classify(vals, r0, r0 + self.wr - 1, off, off + bkv - 1))
            classes.append(row)
        # Blocks after which each wave's rows all have a real score: a block whose first column keeps every
        # one of the wave's scores.
        keep_until = [len(cand)] * self.nw
        for wv in range(self.nw):
            established = False
            last = 0
            for b, (jv, off) in enumerate(cand):
                if classes[b][wv] != "none" or not established:
                    last = b + 1
                if not established:
                    r0 = sub * bq + wv * self.wr
                    first = self._classify({**values, m.jvar: jv}, r0, r0 + self.wr - 1, off, off)
                    established = first == "full"
            keep_until[wv] = last
        n_blocks = max(keep_until) if keep_until else 0
        blist = cand[:n_blocks]
        waves = []
        for wv in range(self.nw):
            full = 0
            while full < keep_until[wv] and classes[full][wv] == "full":
                full += 1
            waves.append((full, keep_until[wv]))
        return blist, waves

    # ------------------------------------------------------------------------------------------ program

    def _split(self, items, weights, lanes: int):
        """Split-KV for balance: items with more than `split_tenths` / 10 times one workgroup's share of all
        the work (`lanes` workgroups at a time) are cut into chunks of consecutive blocks. A chunk runs the same
        online softmax over its blocks and writes its (m, l, acc) to a workspace slot; the merge kernel
        combines a tile's chunks. Returns the items (t, sub, block offset, blocks, per-wave counts, slot or
        -1), their weights and the merge table rows (t, sub, first slot, chunks)."""
        total = sum(it[3] + ITEM_COST for it in items)
        share = max(MIN_CHUNK, -(-total // lanes))
        out, w_out, merges = [], [], []
        slot = 0
        for it, wt in zip(items, weights):
            t, sub, off, cnt, waves = it
            parts = -(-cnt // share) if self.split_tenths and 10 * cnt > share * self.split_tenths else 1
            if parts == 1:
                out.append((t, sub, off, cnt, waves, -1))
                w_out.append(wt)
                continue
            bounds = [cnt * c // parts for c in range(parts + 1)]
            merges.append((t, sub, slot, parts))
            for c in range(parts):
                b0, b1 = bounds[c], bounds[c + 1]
                cw = [(min(max(f - b0, 0), b1 - b0), min(max(u - b0, 0), b1 - b0)) for f, u in waves]
                out.append((t, sub, off + b0, b1 - b0, cw, slot))
                w_out.append(sum(u for _, u in cw))
                slot += 1
        return out, w_out, merges

    def program(self) -> Program:
        plan, sch, m = self.plan, self.sch, self.m
        items, weights, blocks = self._items()
        lds = self.stages * self.bkv * ((0 if getattr(self, 'kreg', False) else m.d) + m.dv) * 2
        # workgroups at a time: two a CU where their LDS fits, one with 64-row waves (their registers)
        lanes = gfx950.CUS * (1 if self.wr == 64 else max(1, min(2, gfx950.LDS_BYTES // lds)))
        items, weights, merges = self._split(items, weights, lanes)
        self.slots = sum(c for _, _, _, c in merges)
        order = sorted(range(len(items)), key=lambda i: (-weights[i], i))
        grid = max(len(items), 1)
        nw = self.nw
        stride = 5 + 2 * nw
        table = np.zeros((max(len(items), 1), stride), np.int32)
        for row, i in enumerate(order):
            t, sub, off, cnt, waves, slot = items[i]
            table[row, :5] = (t, sub, off, cnt, slot)
            for wv, (full, upto) in enumerate(waves):
                table[row, 5 + 2 * wv] = full
                table[row, 6 + 2 * wv] = upto
        # one padding entry at the end: an item without blocks (its offset the table's length) still reads an
        # entry in bounds where the kernel loads its first entries unconditionally
        kvtab = np.array(list(blocks) + [(0, 0)], np.int32).reshape(-1)
        tables = {"fa_items": table.reshape(-1), "fa_blocks": kvtab}
        if merges:
            tables["fa_merge"] = np.array(merges, np.int32).reshape(-1)
        for name, t in sch.tables.items():
            if name.startswith("tile_") or name.startswith("fill_"):
                tables[name] = t
        self.tables = tables
        args = self._args()
        source = self._source(args, stride)
        launches = [Launch(self.name, args, (grid, 1, 1), (64 * nw, 1, 1), 0)]
        workspace = {}
        if self.trace:
            workspace[TRACE] = max(len(items), 1) * TRACE_FIELDS * 8
        if merges:
            workspace["fa_part"] = self.slots * self.bq * (m.dv + 2) * 4
            per_item = self.bq * m.dv // 4 // 256
            launches.append(Launch(f"{self.name}_merge", args, (len(merges) * per_item, 1, 1), (256, 1, 1), 0))
        flop = 2.0 * sum(w for w in weights) * self.wr * self.bkv * (m.d + m.dv)
        return Program(
            name=self.name, source=source, launches=launches, outputs=[(m.out.shape, m.out.dtype)],
            inputs=[(s.shape, s.dtype) for s in plan.inputs], tables=tables, workspace=workspace,
            lds_bytes=lds, protocol=getattr(self, "protocol", None),
            notes={"family": "flash", "block_q": self.bq, "block_kv": self.bkv, "waves": nw, "items": len(items),
                   "executed_flop": flop, "split_items": len(merges), "chunks": self.slots,
                   # the reference's step is (query tile, key block) of the spec; a workgroup's slice here is
                   # one block of bkv keys for its bq rows
                   "trace_workgroups": grid if self.trace else 0,
                   "trace_slots": min(grid, lanes),
                   "slices_per_step": (m.rows // self.bq) * (m.bk // self.bkv)},
        )

    def _args(self) -> List[Arg]:
        plan, m = self.plan, self.m
        args = []
        for k, name in enumerate(plan.nest.params):
            if any(ix.name == name for ix in plan.indices):
                args.append(Arg("input", k, "const int* __restrict__", name))
            else:
                args.append(Arg("input", k, "const ak_u16* __restrict__", name))
        args.append(Arg("output", 0, "ak_u16* __restrict__", m.out.name + "_out"))
        for name in self.tables:
            args.append(Arg("table", name, "const int* __restrict__", name))
        if "fa_merge" in self.tables:
            args.append(Arg("workspace", "fa_part", "float* __restrict__", "fa_part"))
        if self.trace:
            args.append(Arg("workspace", TRACE, "unsigned long long* __restrict__", TRACE))
        return args

    def _setup(self, args: List[Arg]) -> Dict[str, Any]:
        """What every form of the kernel's source shares: the shapes of its fragments and loads, the operands'
        bases and pitches, and the score and epilogue as C expressions per element."""
        plan, sch, m = self.plan, self.sch, self.m
        nw, bq, bkv = self.nw, self.bq, self.bkv
        D, DV = m.d, m.dv
        T = 64 * nw
        kt, ds, ks, dt_n = bkv // 32, D // 16, bkv // 16, DV // 32
        chk, chv = D // 8, DV // 8
        ldk_n = bkv * D // 8 // T
        ldv_n = bkv * DV // 8 // T
        vo_n = max(1, 16 // (T // chk)) if chk >= 16 else 1
        if ldk_n < 1 or ldv_n < 1 or 64 % chk or 64 % chv:
            raise KernelError("attention block too small for the workgroup")
        index = Index(plan, lambda v: f"lv_{v}")
        jvar = m.jvar
        no_j = lambda v: "0" if v == jvar else f"lv_{v}"
        q_shape = plan.inputs[m.q.param].shape
        k_shape = plan.inputs[m.k.param].shape
        v_shape = plan.inputs[m.v.param].shape
        q_base, q_str = tile_base(m.q.tile, q_shape, index, lambda v: f"lv_{v}")
        k_base, k_str = tile_base(m.k.tile, k_shape, index, no_j)
        v_base, v_str = tile_base(m.v.tile, v_shape, index, no_j)
        o_base, o_str = tile_base(m.out.tile, m.out.shape, index, lambda v: f"lv_{v}")
        if q_str[-1] != 1 or k_str[-1] != 1 or v_str[-1] != 1 or o_str[-1] != 1:
            raise KernelError("the gfx950 attention lowering reads rows whose last dim is contiguous")
        ldq, ldk, ldv, ldo = q_str[0], k_str[0], v_str[0], o_str[0]
        kstride_j = strides(k_shape)[self.kdim]
        vstride_j = strides(v_shape)[self.vdim]
        for arr, shape in ((m.k.tile.array, k_shape), (m.v.tile.array, v_shape)):
            if 2 * math.prod(shape) >= 2**31:
                raise KernelError(f"`{arr}` is 2 GiB or more: the attention lowering uses 32-bit buffer offsets")
        k_numel, v_numel = math.prod(k_shape), math.prod(v_shape)

        # score(S) per element: S is `sv`; rows/cols spec-local; the key loop's value is `lv_j`.
        def sleaf(n: Node) -> Optional[str]:
            if n is m.scores:
                return "sv"
            if n.op == "iota":
                dim = n.kwargs["dimension"]
                return "er" if dim == len(n.shape) - 2 else "ec" if dim == len(n.shape) - 1 else "0"
            if n.op == "loop":
                return f"lv_{n.kwargs['var']}"
            if n.op == "full":
                return literal(n.kwargs["value"], n.dtype)
            if n.op == "index":
                ix = plan.index(n.kwargs["array"])
                flat = " + ".join(f"({sem.value(i)}) * {s}" for i, s in zip(n.args, strides(ix.shape))) or "0"
                return f"args.{ix.name}[{flat}]"
            return None

        sem = Emitter(sleaf, (m.rows, m.bk), prefix="sc")
        score_expr = sem.emit(m.score)
        score_lines = " ".join(sem.lines)

        # The stored value per element: acc (this element), l (the row's sum).
        def eleaf(n: Node) -> Optional[str]:
            if n is m.acc_leaf:
                return "acc_v"
            if _strip(n) is m.sum_leaf:
                return "l_run"
            if n.op == "iota":
                dim = n.kwargs["dimension"]
                return "er" if dim == len(n.shape) - 2 else "ed" if dim == len(n.shape) - 1 else "0"
            if n.op == "loop":
                return f"lv_{n.kwargs['var']}"
            if n.op == "full":
                return literal(n.kwargs["value"], n.dtype)
            if n.op in ("carried", "load"):
                raise KernelError("the attention epilogue reads only the accumulator and the row sum")
            return None

        eem = Emitter(eleaf, m.out.tile.shape, prefix="e")
        out_expr = eem.emit(m.value.node)
        epi_lines = "\n        ".join(eem.lines)
        struct = c_struct(f"{self.name}_args", args)
        tile_decode = "\n  ".join(decode_tile(plan, sch, "t"))
        Q, K, V, O = (f"args.{m.q.tile.array}", f"args.{m.k.tile.array}", f"args.{m.v.tile.array}",
                      f"args.{m.out.name}_out")
        return locals()

    def _source(self, args: List[Arg], stride: int) -> str:
        c = self._setup(args)
        plan, m = self.plan, self.m
        nw, bq, bkv = self.nw, self.bq, self.bkv
        (D, DV, T, kt, ds, ks, dt_n, chk, chv, ldk_n, ldv_n, vo_n, jvar, q_base, k_base, v_base, o_base, ldq, ldk,
         ldv, ldo, kstride_j, vstride_j, k_numel, v_numel, score_lines, score_expr, epi_lines, out_expr, struct,
         tile_decode, Q, K, V, O) = (c[n] for n in (
            "D", "DV", "T", "kt", "ds", "ks", "dt_n", "chk", "chv", "ldk_n", "ldv_n", "vo_n", "jvar", "q_base",
            "k_base", "v_base", "o_base", "ldq", "ldk", "ldv", "ldo", "kstride_j", "vstride_j", "k_numel",
            "v_numel", "score_lines", "score_expr", "epi_lines", "out_expr", "struct", "tile_decode", "Q", "K", "V",
            "O"))
        L: List[str] = []
        w = L.append
        w(f"""// Generated by tilejax_amd for `{plan.nest.name}`: a gfx950 flash-attention kernel.
// spec tile {m.rows} x {m.bk} (head dims {D}, {DV}); workgroup {bq} query rows in {nw} waves, key blocks of {bkv}.
{PRELUDE}
{struct}""")
        kreg = self.kreg
        two = self.wr == 64  # a wave's rows in two halves: rows er (state as named) and er_b (the same, `_b`)
        if two and kreg:
            raise KernelError("64 query rows a wave read K from LDS (the knob kreg is for 32)")
        if kreg and ldk != kstride_j:
            raise KernelError("K fragments in registers need key rows one row pitch apart")
        for s in range(self.stages):
            if not kreg:
                w(f"__shared__ __attribute__((aligned(1024))) ak_u16 ak_sk{s}[{bkv * D}];")
            w(f"__shared__ __attribute__((aligned(1024))) ak_u16 ak_sv{s}[{bkv * DV}];")
        w(f"""
extern "C" __global__ void __launch_bounds__({T}, {1 if two else 2}) {self.name}(const {self.name}_args args) {{
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int* item = args.fa_items + blockIdx.x * {stride};
  const int t = ak_ldc(item, 0), sub = ak_ldc(item, 1), boff = ak_ldc(item, 2), nblk = ak_ldc(item, 3);
  const int slot = ak_ldc(item, 4);  // a chunk of a tile split along the keys: its workspace slot (else -1)
  const int f_w = ak_ldc(item, 5 + 2 * wave), n_w = ak_ldc(item, 6 + 2 * wave);
  (void)slot;
  {tile_decode}
  {f"const int er = sub * {bq} + wave * 64 + (lane & 31), er_b = er + 32;  // this lane's query rows in the spec tile (two halves)" if two else
   f"const int er = sub * {bq} + wave * 32 + (lane & 31);   // this lane's query row in the spec tile"}
  // Q^T fragments (srcB of S^T = K Q^T): row er, head dims 16 s + 8 (lane / 32) .. + 8
  ak_bf16x8 qf[{ds}];{f" ak_bf16x8 qf_b[{ds}];" if two else ""}
  {{
    const ak_u16* qp = {Q} + ({q_base}) + (long long)er * {ldq} + 8 * (lane >> 5);
#pragma unroll
    for (int s = 0; s < {ds}; ++s) qf[s] = *(const ak_bf16x8*)(qp + 16 * s);{f'''
#pragma unroll
    for (int s = 0; s < {ds}; ++s) qf_b[s] = *(const ak_bf16x8*)(qp + 32LL * {ldq} + 16 * s);''' if two else ""}
  }}
  const long long k_off = {k_base};
  const long long v_off = {v_base};
  const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc((void*)({K} + k_off), (short)0,
      (int)({k_numel}LL * 2 - k_off * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc((void*)({V} + v_off), (short)0,
      (int)({v_numel}LL * 2 - v_off * 2), 0x00020000);
  // K rows XOR-swizzled for ds_read_b128 (chunk ^ row & 15), V rows for ds_read_b64_tr_b16 (chunk ^ (row & 3) << 2)
  const int k_row = (wave * 64 + lane) / {chk}, v_row = (wave * 64 + lane) / {chv};
  // A load step covers {T // chk} K rows; with fewer than 16 the swizzle (row & 15) differs between steps, so
  // the lanes keep one offset per step position modulo 16 rows.
  unsigned k_voff[{vo_n}];
#pragma unroll
  for (int p = 0; p < {vo_n}; ++p)
    k_voff[p] = (unsigned)(k_row * {ldk * 2} + (((lane % {chk}) ^ ((p * {T // chk} + k_row) & {min(15, chk - 1)})) * 16));
  const unsigned v_voff = (unsigned)(v_row * {ldv * 2} + (((lane % {chv}) ^ (((v_row & 3) << 2) & {chv - 1})) * 16));
  int k_roff[{ds}];
#pragma unroll
  for (int s = 0; s < {ds}; ++s) {{
    const int row = lane & 31;
    k_roff[s] = row * {D * 2} + (((2 * s + (lane >> 5)) ^ (row & {min(15, chk - 1)})) * 16);
  }}
  int v_roff[{dt_n}];
  {{
    const int G = lane >> 4, s = lane & 15, kv = 4 * (G >> 1) + (s >> 2);
#pragma unroll
    for (int dt = 0; dt < {dt_n}; ++dt) {{
      const int d = 32 * dt + 16 * (G & 1) + 4 * (s & 3);
      v_roff[dt] = kv * {DV * 2} + ((((d >> 3) ^ (((kv & 3) << 2) & {chv - 1}))) << 4) + (d & 7) * 2;
    }}
  }}
  ak_f32x16 acc[{dt_n}];{f" ak_f32x16 acc_b[{dt_n}];" if two else ""}
#pragma unroll
  for (int i = 0; i < {dt_n}; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;{f'''
#pragma unroll
  for (int i = 0; i < {dt_n}; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc_b[i][r] = 0.f;''' if two else ""}
  float m_run = {literal(m.m_init)}, l_run = 0.f;{f" float m_run_b = {literal(m.m_init)}, l_run_b = 0.f;" if two else ""}""")
        if kreg:
            w(f"""  // K fragments straight from memory (srcA of S^T = K Q^T): key row 32 t + lane % 32 of the block, head dims
  // 16 s + 8 (lane / 32) .. + 8; one register set per block, alternating
  const unsigned kr_voff = (unsigned)((lane & 31) * {ldk * 2} + 16 * (lane >> 5));
  {" ".join(f"ak_bf16x8 kr{k}[{kt * ds}];" for k in range(KREG_SETS))}""")
        tr = self.trace
        if tr:
            # trace regions: the wait for block 0 is the pipeline fill; later blocks' waits (their loads and the
            # barrier) are input waits; the rest of the loop is compute; the stores are output
            w(f"  unsigned long long tr_fill = 0, tr_wait = 0;")
            w(f"  {CLOCK_START} const unsigned long long tr_i0 = {NOW};")
        # the last wave writes: its rows see every key block the tile visits, so its waits are for data
        # (and the barrier), never for want of work
        trace_write = (f"if (tid == {T - 64}) {{ const unsigned long long tr_e = {NOW}; "
                       f"unsigned long long* tr = args.{TRACE} + blockIdx.x * {TRACE_FIELDS}; "
                       f"tr[0] = tr_fill + tr_wait; tr[1] = tr_fill; tr[2] = tr_e - tr_c1; "
                       f"tr[3] = tr_c1 - tr_i0 - tr_fill - tr_wait; tr[4] = (unsigned long long)nblk; {CLOCK_END} }}") if tr else ""

        # A block's table entry (key block start, column offset) is loaded into a ring of scalars one block
        # before it is first needed, so no scalar load's latency follows a barrier.
        def entry_load(x: str, r: int, ind: str) -> str:
            return (f"{ind}{{ const int* bp = args.fa_blocks + 2 * (boff + ak_imax(ak_imin({x}, nblk - 1), 0)); "
                    f"bj[{r}] = ak_ldc(bp, 0); bc[{r}] = ak_ldc(bp, 1); }}")

        def issue(r: int, s: int, ind: str) -> List[str]:
            out = [f"{ind}{{ const int kpos = bj[{r}] + {self.kwin.offset} + bc[{r}], vpos = bj[{r}] + {self.vwin.offset} + bc[{r}];"]
            if kreg:
                out[0] += " (void)kpos;"
            rows_k, rows_v = T // chk, T // chv
            for c in range(0 if kreg else ldk_n):
                out.append(f"{ind}  __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, AK_LDS(&ak_sk{s}[({c * T} + wave * 64) * 8]), 16, k_voff[{c % vo_n}], "
                           f"(unsigned)((kpos + {c * rows_k}) * {kstride_j * 2}), 0, 0);")
            for c in range(ldv_n):
                out.append(f"{ind}  __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, AK_LDS(&ak_sv{s}[({c * T} + wave * 64) * 8]), 16, v_voff, "
                           f"(unsigned)((vpos + {c * rows_v}) * {vstride_j * 2}), 0, 0);")
            out.append(f"{ind}}}")
            return out

        v_order = [(kk, dt) for kk in range(ks) for dt in range(dt_n)]
        v_ahead = min(V_AHEAD, len(v_order))
        k_order = [(t, sl) for sl in range(ds) for t in range(kt)]

        def k_issue(r: int, kset: int, ind: str) -> List[str]:
            """The K fragments of the block at ring slot r into register set `kset` (with `kreg`)."""
            out = [f"{ind}{{ const unsigned ko_ = (unsigned)((bj[{r}] + {self.kwin.offset} + bc[{r}]) * {ldk * 2});"]
            for i, (t, sl) in enumerate(k_order):
                out.append(f"{ind}  kr{kset}[{i}] = __builtin_bit_cast(ak_bf16x8, __builtin_amdgcn_raw_buffer_load_b128(rk, "
                           f"kr_voff + {t * 32 * ldk * 2 + sl * 32}u, ko_, 0));")
            out.append(f"{ind}}}")
            return out

        def v_read(i: int, ind: str) -> str:
            kk, dt = v_order[i]
            o1 = kk * 16 * DV * 2
            return (f"{ind}  {{ const ak_i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(AK_LDS4(vs + v_roff[{dt}] + {o1}));"
                    f" const ak_i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(AK_LDS4(vs + v_roff[{dt}] + {o1 + 8 * DV * 2}));"
                    f" vf[{i}] = __builtin_bit_cast(ak_bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7)); }}")

        def pv(ind: str) -> List[str]:
            """O^T += V^T P^T from the V stage `vs` and `pf`: the first V_AHEAD fragments are in `vf`
            already, the rest are read V_AHEAD MFMAs ahead of use."""
            o: List[str] = []
            a = o.append
            for i, (kk, dt) in enumerate(v_order):
                a(f"{ind}  acc[{dt}] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf[{i}], pf[{kk}], acc[{dt}], 0, 0, 0);")
                if two:  # the same V fragment for the second half's rows
                    a(f"{ind}  acc_b[{dt}] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf[{i}], pf_b[{kk}], acc_b[{dt}], 0, 0, 0);")
                if i + v_ahead < len(v_order):
                    a(v_read(i + v_ahead, ind))
            for i in range(len(v_order)):
                a(f"{ind}  __builtin_amdgcn_sched_group_barrier(0x008, {2 if two else 1}, 0);")
                if i + v_ahead < len(v_order):
                    a(f"{ind}  __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);")
            return o

        def softmax(ind: str, x: str) -> List[str]:
            """The mask's scores in place and the online softmax of the half with state suffix `x` ('' or
            '_b'), into pf{x}."""
            o: List[str] = []
            a = o.append
            st, er_x = f"st{x}", f"er{x}"
            # the mask's scores in place (blocks the mask keeps whole skip it); then one max for both
            a(f"{ind}  if (b_ >= f_w) {{")
            if x:
                a(f"{ind}    const int er = {er_x}; (void)er;")
            for t in range(kt):
                a(f"{ind}    #pragma unroll")
                a(f"{ind}    for (int r = 0; r < 16; ++r) {{")
                a(f"{ind}      const int ec = ec0 + {32 * t} + (r >> 2) * 8 + (r & 3); (void)ec;")
                a(f"{ind}      const float sv = {st}[{t}][r];")
                a(f"{ind}      {score_lines}")
                a(f"{ind}      {st}[{t}][r] = (float)({score_expr});")
                a(f"{ind}    }}")
            a(f"{ind}  }}")
            a(f"{ind}  {{")
            a(f"{ind}  float mx = -__builtin_inff();")
            for t in range(kt):
                a(f"{ind}  #pragma unroll")
                a(f"{ind}  for (int r = 0; r < 16; ++r) mx = fmaxf(mx, {st}[{t}][r]);")
            a(f"{ind}  mx = ak_xor32_max(mx);")
            a(f"{ind}  const float m_new = ak_maximum(m_run{x}, mx);")
            # Lazy rescaling: the running max moves (and acc, l are rescaled) only when some row's new max
            # exceeds it by more than RESCALE_SLACK; otherwise p = exp(s - m_run) stays below e^slack and
            # acc, l keep one common scale, so acc / l is unchanged.
            a(f"{ind}  if (__ballot(!(m_new <= m_run{x} + {RESCALE_SLACK}f))) {{")
            a(f"{ind}    const float alpha = ak_exp(m_run{x} - m_new);")
            a(f"{ind}    l_run{x} *= alpha;")
            a(f"{ind}    m_run{x} = m_new;")
            a(f"{ind}    #pragma unroll")
            a(f"{ind}    for (int i = 0; i < {dt_n}; ++i) acc{x}[i] *= alpha;")
            a(f"{ind}  }}")
            # p = exp(s - m) as one fma and v_exp_f32 (2^x)
            a(f"{ind}  const float mb = -m_run{x} * {LOG2E!r}f;")
            a(f"{ind}  float ps = 0.f;")
            for t in range(kt):
                for half in range(2):
                    a(f"{ind}  {{ unsigned pk[4];")
                    a(f"{ind}    #pragma unroll")
                    a(f"{ind}    for (int r = 0; r < 8; r += 2) {{")
                    a(f"{ind}      const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf({st}[{t}][{8 * half} + r], {LOG2E!r}f, mb));")
                    a(f"{ind}      const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf({st}[{t}][{8 * half} + r + 1], {LOG2E!r}f, mb));")
                    a(f"{ind}      ps += p0 + p1; pk[r >> 1] = ak_pack_bf16x2(p0, p1); }}")
                    a(f"{ind}    pf{x}[{2 * t + half}] = __builtin_bit_cast(ak_bf16x8, (ak_u32x4){{pk[0], pk[1], pk[2], pk[3]}}); }}")
            a(f"{ind}  ps = ak_xor32_sum(ps);")
            a(f"{ind}  l_run{x} += ps;")
            a(f"{ind}  }}")
            return o

        def compute(s: int, ind: str, r: Optional[int] = None, kset: int = 0) -> List[str]:
            """Block b_ from stage s: S^T, the mask, the online softmax into `pf`, and O^T += V^T P^T (with
            `kreg`, K from register set `kset`, and the next block's K loaded into the other after S)."""
            o: List[str] = []
            a = o.append
            a(f"{ind}if (b_ < n_w) {{")
            if kreg:
                a(f"{ind}  const char* vs = (const char*)ak_sv{s};")
            else:
                a(f"{ind}  const char* ks = (const char*)ak_sk{s}; const char* vs = (const char*)ak_sv{s}; (void)vs;")
            r = s if r is None else r
            a(f"{ind}  const int lv_{jvar} = bj[{r}], ec0 = bc[{r}] + (lane >> 5) * 4;")
            a(f"{ind}  ak_f32x16 st[{kt}];")
            for t in range(kt):
                a(f"{ind}  #pragma unroll")
                a(f"{ind}  for (int r = 0; r < 16; ++r) st[{t}][r] = 0.f;")
            if two:
                a(f"{ind}  ak_f32x16 st_b[{kt}];")
                for t in range(kt):
                    a(f"{ind}  #pragma unroll")
                    a(f"{ind}  for (int r = 0; r < 16; ++r) st_b[{t}][r] = 0.f;")
            # S^T = K Q^T: the key tiles' MFMA chains alternate (a chain's next MFMA waits for its last), and
            # the K fragments are read K_AHEAD MFMAs ahead of use, so LDS latency stays hidden.
            order = k_order
            ahead = 0 if kreg else min(K_AHEAD, len(order))
            if kreg:
                for i, (t, sl) in enumerate(order):
                    a(f"{ind}  st[{t}] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kr{kset}[{i}], qf[{sl}], st[{t}], 0, 0, 0);")
                # the next block's K into the other set, beside the softmax and O^T of this one
                a(f"{ind}  if (b_ + 1 < n_w) {{")
                o.extend(k_issue((r + 1) % self.ring, KREG_SETS - 1 - kset, ind + "    "))
                a(f"{ind}  }}")
            else:
                a(f"{ind}  ak_bf16x8 kf[{len(order)}];")
                for i, (t, sl) in enumerate(order[:ahead]):
                    a(f"{ind}  kf[{i}] = *(const ak_bf16x8*)(ks + k_roff[{sl}] + {t * 32 * D * 2});")
                for i, (t, sl) in enumerate(order):
                    a(f"{ind}  st[{t}] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[{i}], qf[{sl}], st[{t}], 0, 0, 0);")
                    if two:  # the same K fragment for the second half's rows
                        a(f"{ind}  st_b[{t}] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[{i}], qf_b[{sl}], st_b[{t}], 0, 0, 0);")
                    if i + ahead < len(order):
                        t2, sl2 = order[i + ahead]
                        a(f"{ind}  kf[{i + ahead}] = *(const ak_bf16x8*)(ks + k_roff[{sl2}] + {t2 * 32 * D * 2});")
            # O^T += V^T P^T: its first V_AHEAD fragments (two transposed reads each) go out now, beside the
            # S MFMAs and the softmax.
            a(f"{ind}  ak_bf16x8 vf[{len(v_order)}];")
            for i in range(v_ahead):
                a(v_read(i, ind))
            if ahead:
                a(f"{ind}  __builtin_amdgcn_sched_group_barrier(0x100, {ahead}, 0);")
            for i in range(len(order)):
                a(f"{ind}  __builtin_amdgcn_sched_group_barrier(0x008, {2 if two else 1}, 0);")
                if ahead and i + ahead < len(order):
                    a(f"{ind}  __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);")
            a(f"{ind}  __builtin_amdgcn_sched_group_barrier(0x100, {2 * v_ahead}, 0);")
            if two:
                o.extend(softmax(ind, ""))
                o.extend(softmax(ind, "_b"))
                o.extend(pv(ind))
                a(f"{ind}}}")
                return o
            # the mask's scores in place (blocks the mask keeps whole skip it); then one max for both
            a(f"{ind}  if (b_ >= f_w) {{")
            for t in range(kt):
                a(f"{ind}    #pragma unroll")
                a(f"{ind}    for (int r = 0; r < 16; ++r) {{")
                a(f"{ind}      const int ec = ec0 + {32 * t} + (r >> 2) * 8 + (r & 3); (void)ec;")
                a(f"{ind}      const float sv = st[{t}][r];")
                a(f"{ind}      {score_lines}")
                a(f"{ind}      st[{t}][r] = (float)({score_expr});")
                a(f"{ind}    }}")
            a(f"{ind}  }}")
            a(f"{ind}  float mx = -__builtin_inff();")
            for t in range(kt):
                a(f"{ind}  #pragma unroll")
                a(f"{ind}  for (int r = 0; r < 16; ++r) mx = fmaxf(mx, st[{t}][r]);")
            a(f"{ind}  mx = ak_xor32_max(mx);")
            a(f"{ind}  const float m_new = ak_maximum(m_run, mx);")
            # Lazy rescaling: the running max moves (and acc, l are rescaled) only when some row's new max
            # exceeds it by more than RESCALE_SLACK; otherwise p = exp(s - m_run) stays below e^slack and
            # acc, l keep one common scale, so acc / l is unchanged.
            a(f"{ind}  if (__ballot(!(m_new <= m_run + {RESCALE_SLACK}f))) {{")
            a(f"{ind}    const float alpha = ak_exp(m_run - m_new);")
            a(f"{ind}    l_run *= alpha;")
            a(f"{ind}    m_run = m_new;")
            a(f"{ind}    #pragma unroll")
            a(f"{ind}    for (int i = 0; i < {dt_n}; ++i) acc[i] *= alpha;")
            a(f"{ind}  }}")
            # p = exp(s - m) as one fma and v_exp_f32 (2^x)
            a(f"{ind}  const float mb = -m_run * {LOG2E!r}f;")
            a(f"{ind}  float ps = 0.f;")
            for t in range(kt):
                for half in range(2):
                    a(f"{ind}  {{ unsigned pk[4];")
                    a(f"{ind}    #pragma unroll")
                    a(f"{ind}    for (int r = 0; r < 8; r += 2) {{")
                    a(f"{ind}      const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(st[{t}][{8 * half} + r], {LOG2E!r}f, mb));")
                    a(f"{ind}      const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(st[{t}][{8 * half} + r + 1], {LOG2E!r}f, mb));")
                    a(f"{ind}      ps += p0 + p1; pk[r >> 1] = ak_pack_bf16x2(p0, p1); }}")
                    a(f"{ind}    pf[{2 * t + half}] = __builtin_bit_cast(ak_bf16x8, (ak_u32x4){{pk[0], pk[1], pk[2], pk[3]}}); }}")
            a(f"{ind}  ps = ak_xor32_sum(ps);")
            a(f"{ind}  l_run += ps;")
            o.extend(pv(ind))
            a(f"{ind}}}")
            return o

        # K and V blocks stream through `stages` LDS stages, loaded `ahead` blocks ahead. At the barrier that opens
        # block b every wave has finished reading the stage block b + ahead goes into (that of block
        # b + ahead - stages, stages = ahead + 1), so that load is issued right after it.
        per_block = ldk_n + ldv_n

        unroll = self.stages * self.ring // math.gcd(self.stages, self.ring)  # positions: stage p % stages, slot p % ring
        rec = self.protocol = Recorder()  # the loop's LDS events (a stage holds a block's K and V), as emitted
        w(f"  int bj[{self.ring}], bc[{self.ring}];  // table entries of blocks b .. b + {self.ring - 1}, at b mod {self.ring}")
        for x in range(self.ahead + 1):
            w(entry_load(str(x), x, "  "))
        if kreg:
            per_block = ldv_n  # (the LDS ring holds V only)
        for s in range(self.ahead):
            w(f"  if ({s} < nblk) {{")
            L.extend(issue(s, s, "    "))
            rec.add(("load", s, s, per_block), lambda n, s=s: s < n)
            w("  }")
        if kreg:
            w("  if (0 < n_w) {")
            L.extend(k_issue(0, 0, "    "))
            w("  }")
        rec.loop(unroll)
        w("  ak_bf16x8 pf[" + str(ks) + "];  // P^T of the block (srcB of O^T = V^T P^T)")
        if two:
            w(f"  ak_bf16x8 pf_b[{ks}];  // (the second half's)")
        w(f"  for (int b = 0; b < nblk; b += {unroll}) {{")
        for p_ in range(unroll):
            s, r_ = p_ % self.stages, p_ % self.ring
            w(f"    {{ const int b_ = b + {p_};")
            w("      if (b_ < nblk) {")
            if tr:
                w(f"        const unsigned long long tr_w0 = {NOW};")
            # Block b_ has landed; the (at most self.ahead - 1) later blocks issued may still be in flight.
            for ahead in range(self.ahead - 1, 0, -1):
                w(f"        {'if' if ahead == self.ahead - 1 else 'else if'} (b_ + {ahead} < nblk) {{ AK_WAIT_VM({ahead * per_block}); }}")
            w("        " + ("else " if self.ahead > 1 else "") + "{ AK_WAIT_VM(0); }")
            rec.at(p_, lambda b, n, A=self.ahead: ("wait_vm", next((a * per_block for a in range(A - 1, 0, -1)
                                                                     if b + a < n), 0)))
            w("        AK_WAIT_LGKM0();")
            w('        asm volatile("s_barrier" ::: "memory");')
            rec.at(p_, lambda b, n: ("wait_lgkm",))
            rec.at(p_, lambda b, n: ("barrier",))
            if tr:
                w(f"        {{ const unsigned long long tr_w1 = {NOW}; if (b_ == 0) tr_fill = tr_w1 - tr_i0; else tr_wait += tr_w1 - tr_w0; }}")
            w(f"        if (b_ + {self.ahead} < nblk) {{")
            L.extend(issue((r_ + self.ahead) % self.ring, (s + self.ahead) % self.stages, "          "))
            rec.at(p_, lambda b, n, st=(s + self.ahead) % self.stages, A=self.ahead: ("load", st, b + A, per_block),
                   lambda b, n, A=self.ahead: b + A < n)
            w("        }")
            w(entry_load(f"b_ + {self.ahead + 1}", (r_ + self.ahead + 1) % self.ring, "        "))
            L.extend(compute(s, "        ", r_, p_ % KREG_SETS))
            rec.at(p_, lambda b, n, st=s: ("read", st, b))
            w("      }")
            w("    }")
        w("  }")
        if tr:
            w(f"  const unsigned long long tr_c1 = {NOW};")
        if self.slots:
            def part_store(x: str, lr: str) -> str:
                return f"""  {{
    const int lr = {lr};
#pragma unroll
    for (int dt = 0; dt < {dt_n}; ++dt)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4)
        *(ak_f32x4*)(part + lr * {DV} + 32 * dt + g4 * 8 + (lane >> 5) * 4) =
            ak_f32x4{{acc{x}[dt][4 * g4], acc{x}[dt][4 * g4 + 1], acc{x}[dt][4 * g4 + 2], acc{x}[dt][4 * g4 + 3]}};
    if (lane < 32) {{ part[{bq * DV} + lr] = m_run{x}; part[{bq * DV + bq} + lr] = l_run{x}; }}
    }}"""
            if two:
                stores = part_store("", "wave * 64 + (lane & 31)") + "\n" + part_store("_b", "wave * 64 + 32 + (lane & 31)")
            else:
                stores = f"""    const int lr = wave * 32 + (lane & 31);
#pragma unroll
    for (int dt = 0; dt < {dt_n}; ++dt)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4)
        *(ak_f32x4*)(part + lr * {DV} + 32 * dt + g4 * 8 + (lane >> 5) * 4) =
            ak_f32x4{{acc[dt][4 * g4], acc[dt][4 * g4 + 1], acc[dt][4 * g4 + 2], acc[dt][4 * g4 + 3]}};
    if (lane < 32) {{ part[{bq * DV} + lr] = m_run; part[{bq * DV + bq} + lr] = l_run; }}"""
            w(f"""  if (slot >= 0) {{  // a chunk: (m, l, acc) of its rows to the workspace, for the merge kernel
    float* part = args.fa_part + (long long)slot * {bq * (DV + 2)};
{stores}
    {trace_write}
    return;
  }}""")
        w(f"""  // Output: lane = query row er, acc[dt][r] = head dim 32 dt + (r / 4) * 8 + (lane / 32) * 4 + r % 4.
  ak_u16* op = (ak_u16*){O} + ({o_base}) + (long long)er * {ldo};
#pragma unroll
  for (int dt = 0; dt < {dt_n}; ++dt)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {{
      float res[4];
#pragma unroll
      for (int e4 = 0; e4 < 4; ++e4) {{
        const int ed = 32 * dt + g4 * 8 + (lane >> 5) * 4 + e4; (void)ed;
        const float acc_v = acc[dt][4 * g4 + e4];
        {epi_lines}
        res[e4] = (float)({out_expr});
      }}
      *(ak_u32x2*)(op + 32 * dt + g4 * 8 + (lane >> 5) * 4) = ak_u32x2{{ak_pack_bf16x2(res[0], res[1]), ak_pack_bf16x2(res[2], res[3])}};
    }}{f'''
  {{  // the second half's rows: the epilogue sees its row and row sum under the same names
    const int er = er_b; const float l_run = l_run_b; (void)l_run;
    ak_u16* op_b = (ak_u16*){O} + ({o_base}) + (long long)er * {ldo};
#pragma unroll
    for (int dt = 0; dt < {dt_n}; ++dt)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {{
        float res[4];
#pragma unroll
        for (int e4 = 0; e4 < 4; ++e4) {{
          const int ed = 32 * dt + g4 * 8 + (lane >> 5) * 4 + e4; (void)ed;
          const float acc_v = acc_b[dt][4 * g4 + e4];
          {epi_lines}
          res[e4] = (float)({out_expr});
        }}
        *(ak_u32x2*)(op_b + 32 * dt + g4 * 8 + (lane >> 5) * 4) = ak_u32x2{{ak_pack_bf16x2(res[0], res[1]), ak_pack_bf16x2(res[2], res[3])}};
      }}
  }}''' if two else ""}
  {trace_write}
}}""")
        if self.slots:
            w(self._merge_kernel(c))
        return "\n".join(L)

    def _merge_kernel(self, c: Dict[str, Any]) -> str:
        """The merge of tiles split along the keys: each thread combines four output elements of one row over
        the tile's chunks with the online softmax's own rule (weights exp(m_c - M)), then applies the
        epilogue."""
        bq, DV = self.bq, self.m.dv
        per_item = bq * DV // 4 // 256
        tile_decode, O, o_base, ldo = c["tile_decode"], c["O"], c["o_base"], c["ldo"]
        epi_lines, out_expr = c["epi_lines"], c["out_expr"]
        return f"""
// The merge of tiles split along the keys: each thread combines four output elements of one row over the
// tile's chunks with the online softmax's own rule (weights exp(m_c - M)), then applies the epilogue.
extern "C" __global__ void __launch_bounds__(256) {self.name}_merge(const {self.name}_args args) {{
  const int p = blockIdx.x / {per_item};
  const int e = (blockIdx.x % {per_item}) * 256 + threadIdx.x;
  const int lr = e / {DV // 4}, d0 = (e % {DV // 4}) * 4;
  const int t = ak_ldc(args.fa_merge, 4 * p), sub = ak_ldc(args.fa_merge, 4 * p + 1);
  const int first = ak_ldc(args.fa_merge, 4 * p + 2), chunks = ak_ldc(args.fa_merge, 4 * p + 3);
  {tile_decode}
  float mx = -__builtin_inff();
  for (int c = 0; c < chunks; ++c) mx = fmaxf(mx, args.fa_part[(long long)(first + c) * {bq * (DV + 2)} + {bq * DV} + lr]);
  float l_run = 0.f;
  ak_f32x4 a = {{0.f, 0.f, 0.f, 0.f}};
  for (int c = 0; c < chunks; ++c) {{
    const float* part = args.fa_part + (long long)(first + c) * {bq * (DV + 2)};
    const float w = ak_exp(part[{bq * DV} + lr] - mx);
    l_run += w * part[{bq * DV + bq} + lr];
    const ak_f32x4 v = *(const ak_f32x4*)(part + lr * {DV} + d0);
    a[0] += w * v[0]; a[1] += w * v[1]; a[2] += w * v[2]; a[3] += w * v[3];
  }}
  const int er = sub * {bq} + lr; (void)er;
  ak_u16* op = (ak_u16*){O} + ({o_base}) + (long long)er * {ldo} + d0;
  float res[4];
#pragma unroll
  for (int e4 = 0; e4 < 4; ++e4) {{
    const int ed = d0 + e4; (void)ed;
    const float acc_v = a[e4];
    {epi_lines}
    res[e4] = (float)({out_expr});
  }}
  *(ak_u32x2*)op = ak_u32x2{{ak_pack_bf16x2(res[0], res[1]), ak_pack_bf16x2(res[2], res[3])}};
}}"""


class _FlashF32(_Flash):
    """f32 q, k and v (`@` at full precision): a plain f32 kernel on the vector ALUs, for the parity of the
    spec's f32 form rather than speed. One thread per query row (128 per workgroup), the key blocks of the
    bf16 kernel's work items staged through LDS (K, V and the block's scores), per 64-key block the row max,
    then exp and the sums, in f32 throughout."""

    THREADS = 128

    def __init__(self, plan: Plan, sch: Schedule, pipeline: Pipeline, m: FlashMatch, name: str,
                 trace: bool = False) -> None:
        self.plan, self.sch, self.pipeline, self.m, self.name = plan, sch, pipeline, m, name
        self.trace = trace
        if m.d % 4 or m.dv % 4 or m.d > 128 or m.dv > 128:
            raise KernelError(f"the gfx950 f32 attention lowering takes head dims that are multiples of 4 up to 128 "
                              f"(got {m.d} and {m.dv})")
        self.nw = 4  # rows in groups of 32 for the block lists' mask classes: 128 rows per work item
        self.wr = 32
        self.bq = 128
        self.bkv = BKV
        if m.rows % self.bq or m.bk % self.bkv:
            raise KernelError(f"the gfx950 attention lowering needs query tiles of a multiple of {self.bq} rows "
                              f"and key blocks of a multiple of {self.bkv} (got {m.rows} and {m.bk})")
        if plan.runtime or sch.runtime:
            raise KernelError("attention with runtime masks is lowered by the decode path, not this one")
        self.jr = plan.phases[0].range
        self.kdim, self.kwin = _loop_window(m.k, m.jvar)
        self.vdim, self.vwin = _loop_window(m.v, m.jvar)

    def program(self) -> Program:
        plan, m = self.plan, self.m
        items, weights, blocks = self._items()
        order = sorted(range(len(items)), key=lambda i: (-weights[i], i))
        table = np.zeros((max(len(items), 1), 4), np.int32)
        for row, i in enumerate(order):
            t, sub, off, cnt, _ = items[i]
            table[row] = (t, sub, off, cnt)
        kvtab = np.array(blocks, np.int32).reshape(-1) if blocks else np.zeros(2, np.int32)
        self.tables = {"fa_items": table.reshape(-1), "fa_blocks": kvtab}
        for name, t in self.sch.tables.items():
            if name.startswith("tile_") or name.startswith("fill_"):
                self.tables[name] = t
        args = self._args()
        grid = max(len(items), 1)
        workspace = {TRACE: grid * TRACE_FIELDS * 8} if self.trace else {}
        lds = 4 * self.bkv * (m.d + m.dv + self.THREADS)
        return Program(
            name=self.name, source=self._source32(args), launches=[Launch(self.name, args, (grid, 1, 1),
                                                                          (self.THREADS, 1, 1), 0)],
            outputs=[(m.out.shape, m.out.dtype)], inputs=[(s_.shape, s_.dtype) for s_ in plan.inputs],
            tables=self.tables, workspace=workspace, lds_bytes=lds,
            notes={"family": "flash", "f32_operands": True, "block_q": self.bq, "block_kv": self.bkv,
                   "items": len(items), "trace_workgroups": grid if self.trace else 0,
                   "trace_slots": min(grid, gfx950.CUS * max(1, gfx950.LDS_BYTES // lds)),
                   "slices_per_step": (m.rows // self.bq) * (m.bk // self.bkv)})

    def _args(self) -> List[Arg]:
        plan, m = self.plan, self.m
        args = []
        for k, name in enumerate(plan.nest.params):
            if any(ix.name == name for ix in plan.indices):
                args.append(Arg("input", k, "const int* __restrict__", name))
            else:
                args.append(Arg("input", k, "const float* __restrict__", name))
        out_t = "float" if m.out.dtype.name == "float32" else "ak_u16"
        args.append(Arg("output", 0, f"{out_t}* __restrict__", m.out.name + "_out"))
        for name in self.tables:
            args.append(Arg("table", name, "const int* __restrict__", name))
        if self.trace:
            args.append(Arg("workspace", TRACE, "unsigned long long* __restrict__", TRACE))
        return args

    def _source32(self, args: List[Arg]) -> str:
        plan, sch, m = self.plan, self.sch, self.m
        D, DV, bkv, T = m.d, m.dv, self.bkv, self.THREADS
        index = Index(plan, lambda v: f"lv_{v}")
        jvar = m.jvar
        no_j = lambda v: "0" if v == jvar else f"lv_{v}"
        q_shape, k_shape, v_shape = (plan.inputs[op.param].shape for op in (m.q, m.k, m.v))
        q_base, q_str = tile_base(m.q.tile, q_shape, index, lambda v: f"lv_{v}")
        k_base, k_str = tile_base(m.k.tile, k_shape, index, no_j)
        v_base, v_str = tile_base(m.v.tile, v_shape, index, no_j)
        o_base, o_str = tile_base(m.out.tile, m.out.shape, index, lambda v: f"lv_{v}")
        if q_str[-1] != 1 or k_str[-1] != 1 or v_str[-1] != 1 or o_str[-1] != 1:
            raise KernelError("the gfx950 attention lowering reads rows whose last dim is contiguous")
        ldq, ldo = q_str[0], o_str[0]
        kstride_j, vstride_j = strides(k_shape)[self.kdim], strides(v_shape)[self.vdim]

        def sleaf(n: Node) -> Optional[str]:
            if n is m.scores:
                return "sv"
            if n.op == "iota":
                dim = n.kwargs["dimension"]
                return "er" if dim == len(n.shape) - 2 else "ec" if dim == len(n.shape) - 1 else "0"
            if n.op == "loop":
                return f"lv_{n.kwargs['var']}"
            if n.op == "full":
                return literal(n.kwargs["value"], n.dtype)
            if n.op == "index":
                ix = plan.index(n.kwargs["array"])
                flat = " + ".join(f"({sem.value(i)}) * {s_}" for i, s_ in zip(n.args, strides(ix.shape))) or "0"
                return f"args.{ix.name}[{flat}]"
            return None

        sem = Emitter(sleaf, (m.rows, m.bk), prefix="sc")
        score_expr = sem.emit(m.score)
        score_lines = " ".join(sem.lines)

        def eleaf(n: Node) -> Optional[str]:
            if n is m.acc_leaf:
                return "acc_v"
            if _strip(n) is m.sum_leaf:
                return "l_run"
            if n.op == "iota":
                dim = n.kwargs["dimension"]
                return "er" if dim == len(n.shape) - 2 else "ed" if dim == len(n.shape) - 1 else "0"
            if n.op == "loop":
                return f"lv_{n.kwargs['var']}"
            if n.op == "full":
                return literal(n.kwargs["value"], n.dtype)
            if n.op in ("carried", "load"):
                raise KernelError("the attention epilogue reads only the accumulator and the row sum")
            return None

        eem = Emitter(eleaf, m.out.tile.shape, prefix="e")
        out_expr = eem.emit(m.value.node)
        epi_lines = "\n      ".join(eem.lines)
        store = ("op[ed] = res;" if m.out.dtype.name == "float32"
                 else "op[ed] = (ak_u16)ak_bf16_bits(res);")
        tile_decode = "\n  ".join(decode_tile(plan, sch, "t"))
        Q, K, V, O = (f"args.{m.q.tile.array}", f"args.{m.k.tile.array}", f"args.{m.v.tile.array}",
                      f"args.{m.out.name}_out")
        tr0 = f"{CLOCK_START} const unsigned long long tr_0 = {NOW};" if self.trace else ""
        tr1 = (f"if (tid == 0) {{ unsigned long long* tr = args.{TRACE} + blockIdx.x * {TRACE_FIELDS}; tr[0] = 0; "
               f"tr[1] = 0; tr[2] = 0; tr[3] = {NOW} - tr_0; tr[4] = nblk; {CLOCK_END} }}" if self.trace else "")
        return f"""// Generated by tilejax_amd for `{plan.nest.name}`: f32 attention on the vector ALUs.
// spec tile {m.rows} x {m.bk} (head dims {D}, {DV}); {T} query rows per workgroup, key blocks of {bkv}.
{PRELUDE}
{c_struct(f"{self.name}_args", args)}
extern "C" __global__ void __launch_bounds__({T}) {self.name}(const {self.name}_args args) {{
  __shared__ float ks[{bkv * D}], vs[{bkv * DV}], ss[{bkv * T}];
  const int tid = threadIdx.x;
  {tr0}
  const int* item = args.fa_items + blockIdx.x * 4;
  const int t = item[0], sub = item[1], boff = item[2], nblk = item[3];
  {tile_decode}
  const int er = sub * {T} + tid;  // this thread's query row in the spec tile
  float q[{D}], acc[{DV}];
  const float* qp = {Q} + ({q_base}) + (long long)er * {ldq};
#pragma unroll
  for (int d = 0; d < {D}; ++d) q[d] = qp[d];
#pragma unroll
  for (int d = 0; d < {DV}; ++d) acc[d] = 0.f;
  float m_run = {literal(m.m_init)}, l_run = 0.f;
  const long long k_off = {k_base}, v_off = {v_base};
  for (int b = 0; b < nblk; ++b) {{
    const int lv_{jvar} = args.fa_blocks[2 * (boff + b)], bc = args.fa_blocks[2 * (boff + b) + 1];
    const int kpos = lv_{jvar} + {self.kwin.offset} + bc, vpos = lv_{jvar} + {self.vwin.offset} + bc;
    __syncthreads();  // the previous block's reads are done
    for (int e = tid; e < {bkv * D // 4}; e += {T}) {{
      const int r = e / {D // 4}, c = e % {D // 4};
      *(ak_f32x4*)(ks + 4 * e) = *(const ak_f32x4*)({K} + k_off + (long long)(kpos + r) * {kstride_j} + 4 * c);
    }}
    for (int e = tid; e < {bkv * DV // 4}; e += {T}) {{
      const int r = e / {DV // 4}, c = e % {DV // 4};
      *(ak_f32x4*)(vs + 4 * e) = *(const ak_f32x4*)({V} + v_off + (long long)(vpos + r) * {vstride_j} + 4 * c);
    }}
    __syncthreads();
    float mx = m_run;
    for (int key = 0; key < {bkv}; ++key) {{
      float sv = 0.f;
#pragma unroll
      for (int d = 0; d < {D}; ++d) sv = __builtin_fmaf(q[d], ks[key * {D} + d], sv);
      const int ec = bc + key;
      {score_lines}
      const float sc = {score_expr};
      ss[key * {T} + tid] = sc;
      mx = ak_maximum(mx, sc);
    }}
    const float alpha = ak_exp(m_run - mx);
    float lsum = 0.f;
#pragma unroll
    for (int d = 0; d < {DV}; ++d) acc[d] *= alpha;
    for (int key = 0; key < {bkv}; ++key) {{
      const float p = ak_exp(ss[key * {T} + tid] - mx);
      lsum += p;
#pragma unroll
      for (int d = 0; d < {DV}; ++d) acc[d] = __builtin_fmaf(p, vs[key * {DV} + d], acc[d]);
    }}
    l_run = alpha * l_run + lsum;
    m_run = mx;
  }}
  auto* op = {O} + ({o_base}) + (long long)er * {ldo};
#pragma unroll
  for (int ed = 0; ed < {DV}; ++ed) {{
    const float acc_v = acc[ed];
    {epi_lines}
    const float res = (float)({out_expr});
    {store}
  }}
  {tr1}
}}
"""


def lower(plan: Plan, sch: Schedule, pipeline: Pipeline, m: FlashMatch, name: str, trace: bool = False,
          hardware: Optional[Dict[str, int]] = None) -> Program:
    if m.q.tile.dtype.name == "float32":
        if m.out.dtype.name not in ("float32", "bfloat16"):
            raise KernelError("the gfx950 attention lowering stores f32 or bf16 outputs")
        return _FlashF32(plan, sch, pipeline, m, name, trace).program()
    if m.out.dtype.name != "bfloat16":
        raise KernelError("the gfx950 attention lowering stores bf16 outputs")
    return _Flash(plan, sch, pipeline, m, name, trace, hardware).program()


def hardware_choices(m: FlashMatch) -> List[Dict[str, int]]:
    """The kernel shapes tuning may try for this match: waves per workgroup (32 query rows each), keys per
    block, and, for the first of those, where split-KV starts (never, or above one share instead of 1.5).
    The first is the default."""
    if m.q.tile.dtype.name == "float32":
        return [{}]
    found = []
    for waves in (WAVES, 8 if WAVES == 4 else 4):
        for bkv in (BKV, 32 if BKV == 64 else 64):
            if m.rows % (32 * waves) == 0 and m.bk % bkv == 0:
                found.append({"waves": waves, "bkv": bkv})
    if found:
        found += [{**found[0], "split": 0}, {**found[0], "split": 10}]
    return found or [{}]
