"""Lowering of runtime-masked online-softmax loop nests (decode attention over a KV cache) to gfx950.

The family is the reference's `paged_gqa_decode` (examples/decode.py:199-223) and `gqa_decode` over a
contiguous cache (:175-196): per output tile (one sequence) some setup code computes the query rows once
(`block_diagonal(query_rows(q[b]))`), then a reduction loop over the cache's pages or blocks, under a
runtime mask (`p * P >= lengths[b]`, `j >= lengths[b]`) and reading each through a window (a runtime
one, `k_pages[block_tables[b, p], :, :]`, or `k_cache[b, j : j + bk, :]`), runs the online softmax that
`flash.softmax_structure` recognises, and the output is some epilogue of the accumulator and the row sum
(`finish(own_blocks(acc))`). It computes exactly that, as two or three launches on one stream:

1. with step tables, the device step-table builder (codegen/steps.py) evaluates the runtime mask: every
   sequence's pages in order, compacted; more workgroups of the same launch materialise each tile's query
   rows (the setup code's value, per element) in a workspace. With a cursor there is no builder: the
   attention kernel evaluates the mask itself, and computes its query rows itself (`qrows`) or, where the
   waves own no rows, a setup launch materialises them;
2. the attention kernel works in kernel steps of SUB = 16 positions (a table step of P positions is P / 16
   of them, in order) and splits the compacted list of them evenly over one workgroup per CU (a sequence's
   pages may span several workgroups, a workgroup several short sequences). It decodes its range's steps
   (tile, code, page offsets) into LDS first, then streams pages with three in flight under each step's
   compute: K fragments HBM -> registers (`buffer_load_dwordx4`, three register sets), V rows HBM -> LDS
   (`buffer_load_dwordx4 ... lds`, three stages); only a tile change drains the queue. Its eight waves each
   take an eighth of the query rows' width. Where the spec's block-diagonal query rows put every row's
   values in one wave's columns (`row_owners`), each wave scores its own rows against its own columns and
   loads its own columns of V, with a workgroup barrier only every few steps; otherwise S = Q K^T is eight
   partial products (`v_mfma_f32_16x16x32_bf16`, in four chains) summed through LDS behind an LDS-only
   barrier. The softmax rescales only when a row's max grows by more than e^8, and `p @ V` runs on
   `v_mfma_f32_32x32x16_bf16` with V read transposed (`ds_read_b64_tr_b16`). When a workgroup leaves a
   sequence it writes its partial (row max, row sum, accumulator) to a workspace slot;
3. a merge kernel per sequence rescales and sums its partials (the online softmax's own merge rule:
   exact reassociation of the same sums) and evaluates the epilogue per output element.
"""

from __future__ import annotations

import ast
import math
from dataclasses import dataclass
from typing import Any, Dict, List, Optional, Tuple

import numpy as np

from .. import gfx950, jaxlite
from ..errors import KernelError
from ..jaxlite import Node
from ..pipeline import Pipeline
from ..plan import Kind, Operand, Output, Plan
from ..schedule import CODE_SHIFT, Schedule
from ..syntax import element_reads
from .common import Index, strides, tile_base, tile_value
from .device import PRELUDE
from .expr import ElementEmitter, literal
from .flash import RESCALE_SLACK, Softmax, _is, _strip, softmax_structure
from .protocol import Recorder
from .program import CLOCK_END, CLOCK_START, NOW, TRACE, TRACE_FIELDS, Arg, Launch, Program, c_struct
from .steps import attach_step_builder

__all__ = ["DecodeMatch", "match", "lower"]

WAVES = 8
THREADS = 64 * WAVES
RP = 32  # query rows the kernels work on: a spec's R <= 32 rows, the rest zero
SUB = 16  # key positions per kernel step: a spec step of P positions (a page, a cache block) is P / SUB of them
SP = SUB + 4  # floats per row of a wave's partial S in LDS (padded: rows 80 bytes apart)
DEPTH = 3  # K register sets and V LDS stages (steps fetched ahead of the one computed): the default
MAX_DEPTH = 4
# The merge in the attention kernel (`_Decode._fold_merge`, the hardware knob "fold") rather than a launch of
# its own: correct (tests/test_gpu_decode.py), but slower. At BASELINE config 5 the call took 312 us with a
# release fence in every wave and 249 us with one per workgroup, against 214 us with the merge launch: each
# agent-scope release writes the XCD's L2 back, each acquire invalidates it, and the merges then read the
# partials from memory. With own rows (partials of 16 KB, not 128) it still took 231 against 201 us, and
# with the partials stored and loaded at agent scope (sc1) and no fence at all, 245 us: the cost is the last
# workgroup of each sequence merging it alone at the kernel's end, where the merge launch spreads it over
# 512 workgroups. So it is off unless asked for.
FOLD_DEFAULT = False
# Waves that own their query rows (`row_owners`), where the spec's structure shows it (the hardware knob "own",
# on unless set to 0): each wave scores its own rows against its own columns, loads its own columns of V into
# a region of the stage only it reads, and the step has no workgroup barrier. Every other wave's columns
# contributed exact zeros to those rows' scores, so the output is bit-equal to the shared-score kernel's; at
# BASELINE config 5 the call went from 222 to 202 us with step tables and from 226 to 208 us with a cursor.
OWN_DEFAULT = True
# With own rows nothing else synchronises a workgroup's waves, and they drift apart: at config 5 the first
# wave ended 38-43 us before the workgroup's last (3.6 us with shared scores), the early waves winning the
# memory queues. A bare s_barrier (the loads stay in flight) every SYNC_DEFAULT steps, the hardware knob
# "sync" (0: none), keeps them together: 199.9-201.9 us per call without, 195.9-197.5 with one every 6 or
# 8 steps (tables; 206 against 202-203 us with a cursor), every count bit-equal.
SYNC_DEFAULT = 8
# The query rows computed by the attention kernel itself (the hardware knob "qrows"): each wave evaluates the
# spec's setup code for its own fragments' elements when it starts a tile, so no workgroup materialises them
# in a workspace first (with a cursor that is a launch of its own, with step tables more workgroups of the
# builder's launch). The same per-element code and rounding: the same bits. Only a wave's own rows are nonzero
# in its columns, so it needs owned rows. A tile start then costs about 3 us more (the tile's loop values,
# then the query loads, where the workspace took one load); with a cursor it saves a launch of 6 us, with
# tables only the builder launch's extra workgroups. At config 5: tables 190.9 us without, 194.0 with; a
# cursor 196.4 without, 193.0 with. None: with a cursor only.
QROWS_DEFAULT = None


@dataclass
class DecodeMatch:
    sm: Softmax
    k: Operand
    v: Operand
    q_node: Node  # the query rows' value: a setup-code value (carried) or a tile read
    rows: int  # R: query rows
    page: int  # P: key rows per step
    width: int  # W: query/key width (= value width)
    out: Output
    value: Any
    acc_leaf: Node
    sum_leaf: Node


def row_owners(plan: Plan, m: DecodeMatch, span: int) -> Optional[List[int]]:
    """For each query row, the one span of `span` columns its query values can be nonzero in, if every row
    has one and the epilogue reads each row's accumulator only there; else None. The spec's own setup and
    epilogue code is run eagerly on concrete inputs (four draws: normal, normal times 1e4, uniform in
    [0.5, 1.5), and its negation): a value zero in all of them is taken to be zero by construction (the
    block-diagonal query rows of GQA decode: a query head's values sit in its kv head's columns). Setup or
    epilogue code that reads an integer input (an index array, whose values the probe cannot know) makes it
    decline. For the epilogue, the accumulator is NaN outside each row's span, and the output must come out
    finite. Rows with no nonzero value (none, for real queries) are given span 0."""
    import torch

    nest = plan.nest
    seg0, last = plan.segments[0], plan.segments[-1]
    qn = m.sm.qk.args[0]
    if not (_is(qn, "carried") and qn.kwargs["name"] in m.sm.consts):
        return None
    q_name = qn.kwargs["name"]
    rows, width = m.rows, m.width
    if width % span:
        return None
    integers = {name for name, spec in zip(nest.params, plan.inputs) if spec.dtype.name in ("int32", "int64")}
    read = {n.id for stmt in (*seg0, *last) for n in ast.walk(stmt) if isinstance(n, ast.Name)}
    if integers & read:
        return None

    def run(stmts, env):
        exec(compile(ast.Module(body=list(stmts), type_ignores=[]), f"<{nest.name}: row owners>", "exec"), env)

    def draw(kind, shape, g):
        if kind < 2:
            return torch.randn(shape, generator=g) * (1e4 if kind else 1.0)
        u = torch.rand(shape, generator=g) + 0.5
        return u if kind == 2 else -u

    nonzero = None
    envs = []
    for kind in range(4):
        g = torch.Generator().manual_seed(kind + 1)
        env = dict(plan.env)
        for name, spec in zip(nest.params, plan.inputs):
            if name in read:
                t = draw(kind, spec.shape, g).to(spec.dtype.torch)
            else:  # an input the setup and epilogue don't read (the cache): zeros of its shape, no memory
                t = torch.zeros((), dtype=spec.dtype.torch).expand(spec.shape)
            env[name] = jaxlite.asarray(t)
        for r in plan.parallel:
            env[r.var] = r.start + (r.count - 1) * r.step * (kind % 2)  # the first tile, then the last
        try:
            run(seg0, env)
        except Exception:
            return None
        qt = env.get(q_name)
        t = getattr(qt, "t", None) if qt is not None else None
        if t is None or tuple(t.shape) != (rows, width):
            return None
        nz = t.float() != 0
        nonzero = nz if nonzero is None else nonzero | nz
        envs.append(env)
    owners = []
    for r in range(rows):
        spans = sorted({int(c) // span for c in torch.nonzero(nonzero[r]).flatten().tolist()})
        if len(spans) > 1:
            return None
        owners.append(spans[0] if spans else 0)
    # the epilogue reads each row's accumulator only in its span
    env = envs[0]
    acc = torch.full((rows, width), float("nan"))
    for r, o in enumerate(owners):
        acc[r, o * span:(o + 1) * span] = torch.rand(span) + 0.5
    env[m.sm.acc_name] = jaxlite.asarray(acc)
    for name in (m.sm.l_name, m.sm.m_name):
        cur = env.get(name)
        shape = tuple(cur.t.shape) if getattr(cur, "t", None) is not None else (rows, 128)
        env[name] = jaxlite.asarray(torch.rand(shape) + 0.5)
    out = m.out
    env[out.name] = jaxlite.zeros(out.shape, out.dtype)
    try:
        run(last, env)
    except Exception:
        return None
    result = getattr(env.get(out.name), "t", None)
    if result is None or not torch.isfinite(result.float()).all():
        return None
    return owners


def match(plan: Plan) -> Optional[DecodeMatch]:
    """Decode attention (runtime-masked online softmax), or None."""
    if not plan.runtime:
        return None
    sm = softmax_structure(plan)
    if sm is None:
        return None
    k = plan.operand(sm.qk.args[1].kwargs["operand"])
    v = plan.operand(sm.pv.args[1].kwargs["operand"])
    # K and V stream with the loop, or (a loop of one block) stay per tile; either way the kernel reads each
    # step's window at the address its indices give
    if k.kind not in (Kind.STREAM, Kind.TILE) or v.kind not in (Kind.STREAM, Kind.TILE) \
            or k.tile.dtype.name != "bfloat16" or v.tile.dtype.name != "bfloat16":
        return None
    qn = sm.qk.args[0]
    seg0 = plan.scopes["seg0"]
    if _is(qn, "carried") and qn.kwargs["name"] in sm.consts:
        val = seg0.values.get(qn.kwargs["name"])
        if not isinstance(val, jaxlite.Sym):
            return None
        q_node = val.node
    elif _is(qn, "load"):
        q_node = qn
    else:
        return None
    if q_node.dtype.name != "bfloat16":
        return None
    rows, width = qn.shape
    page, kw = k.tile.shape
    vp, vw = v.tile.shape
    if kw != width or vp != page or vw != width:
        return None
    last = plan.scopes["last"]
    out = plan.outputs[0]
    value = last.stores.get(out.name)
    acc_leaf, sum_leaf = last.carried_in.get(sm.acc_name), last.carried_in.get(sm.l_name)
    if not isinstance(value, jaxlite.Sym) or acc_leaf is None or sum_leaf is None:
        return None
    return DecodeMatch(sm, k, v, q_node, rows, page, width, out, value, acc_leaf, sum_leaf)


class _Decode:
    def __init__(self, plan: Plan, sch: Schedule, m: DecodeMatch, name: str, trace: bool = False,
                 cursor: bool = False, depth: int = DEPTH, fold: bool = FOLD_DEFAULT, own: bool = OWN_DEFAULT,
                 sync: int = SYNC_DEFAULT, qrows: bool = False) -> None:
        self.plan, self.sch, self.m, self.name = plan, sch, m, name
        self.trace, self.cursor, self.depth, self.sync, self.qrows = trace, cursor, depth, sync, qrows
        # eight waves where the width splits into them (an eighth each, a multiple of 32), else four
        self.waves = WAVES if m.width % (32 * WAVES) == 0 else 4
        self.threads = 64 * self.waves
        if m.rows > RP or m.page % SUB or m.width % (32 * self.waves):
            raise KernelError(f"the gfx950 decode lowering takes up to {RP} query rows, pages (or cache blocks) of a multiple "
                              f"of {SUB} positions and widths that are multiples of {32 * self.waves} "
                              f"(got {m.rows}, {m.page}, {m.width})")
        self.sub = m.page // SUB  # kernel steps per spec step
        # Each query row's one wave (`row_owners`): with them, a wave computes its own rows' scores alone and
        # loads its own columns of V, and the step needs no workgroup barrier
        self.owners = row_owners(plan, m, m.width // self.waves) if own else None
        # Query rows in the kernel need owned rows: a wave's fragments are zero outside its own rows, whose
        # block (rows x its columns, bf16) it stages in its partial-S area of LDS
        if self.owners is None:
            self.qrows = False
        else:
            most = max(self.owners.count(w_) for w_ in range(self.waves))
            if most * (m.width // self.waves) * 2 > RP * SP * 4:
                self.qrows = False
        if sch.repeats != 1:
            raise KernelError("decode with parallel loops the runtime mask doesn't read is not lowered yet")
        self.grid = gfx950.CUS
        self.slots = self.grid + sch.pattern_tiles
        self.max_per = -(-sch.pattern_steps * self.sub // self.grid)  # most kernel steps one workgroup takes
        self.lds = self.depth * SUB * m.width * 2 + self.waves * RP * SP * 4 + 20 * self.max_per
        # with a cursor the attention kernel evaluates the mask itself: a 64-block word per tile and word
        self.words = sch.pattern_tiles * -(-plan.phases[0].range.count // 64)
        if cursor:
            self.lds += 8 * self.words + 4 * (sch.pattern_tiles + 1) + 4 * self.threads
        if self.lds > gfx950.LDS_BYTES:
            raise KernelError(f"decode over {sch.pattern_steps} pattern steps of {m.page} x {m.width} needs "
                              f"{self.lds} bytes of LDS per workgroup (gfx950 has {gfx950.LDS_BYTES})")
        self.phase = plan.phases[0].range
        # partials per tile: at most its kernel steps or the grid (+1 for the division's edges)
        self.maxs = min(self.grid, self.phase.count * self.sub) + 1
        if 2 * self.maxs * RP * 4 > 96 * 1024:  # the merge kernel's weights and row sums per partial and row
            raise KernelError("too many pages per sequence for the merge kernel's LDS")
        # With `fold` the merge runs in the attention kernel (the last workgroup to finish a tile merges it), its
        # LDS (the partials' weights and row sums) beside the kernel's own; else it is a launch of its own.
        merge_lds = self.maxs * m.rows * 4 + m.rows * 4 + 16
        if fold and self.lds + merge_lds > gfx950.LDS_BYTES:
            raise KernelError(f"the decode merge in the attention kernel needs {self.lds + merge_lds} bytes of LDS "
                              f"per workgroup (gfx950 has {gfx950.LDS_BYTES})")
        self.fold = fold
        if self.fold:
            self.lds += merge_lds
        self.index = Index(plan, lambda v: f"lv_{v}")
        self.seg0 = plan.scopes["seg0"]
        # The setup and merge kernels split each tile's elements over `chunks` workgroups (grid y), enough for
        # about four workgroups per CU over all tiles, each thread keeping at least one element.
        want = -(-4 * gfx950.CUS // sch.pattern_tiles)
        self.setup_chunks = max(1, min(RP * m.width // self.threads, want))
        self.merge_chunks = max(1, min(math.prod(m.out.tile.shape) // self.threads, want))

    # -------------------------------------------------------------------------------- element emitters

    def _emitter(self, extra) -> ElementEmitter:
        """Per-element code of the tile code with the common leaves; `extra(node, idx)` adds the caller's."""
        plan, m = self.plan, self.m
        consts = set(m.sm.consts)
        em: Optional[ElementEmitter] = None

        def leaves(n: Node, idx: Tuple[str, ...]) -> Optional[str]:
            got = extra(n, idx)
            if got is not None:
                return got
            if n.op == "loop":
                return f"lv_{n.kwargs['var']}"
            if n.op == "index":
                ix = plan.index(n.kwargs["array"])
                flat = " + ".join(f"({em.at(i, ()) if isinstance(i, Node) else literal(i)}) * {s}"
                                  for i, s in zip(n.args, strides(ix.shape))) or "0"
                return f"ak_ldc(args.{ix.name}, {flat})"
            if n.op == "carried" and n.kwargs["name"] in consts:
                return em.at(self.seg0.values[n.kwargs["name"]].node, idx)
            if n.op == "load":
                op = plan.operand(n.kwargs["operand"])
                if op.kind is Kind.STREAM:
                    raise KernelError("setup and epilogue code may read only per-tile tiles")
                shape = plan.inputs[op.param].shape
                base, st = tile_base(op.tile, shape, self.index, lambda v: f"lv_{v}")
                flat = " + ".join(f"(long long)({i}) * {s}" for i, s in zip(idx, st)) or "0"
                return f"ak_bf16_to_f32(args.{op.tile.array}[({base}) + {flat}])"
            return None

        em = ElementEmitter(leaves)
        return em

    # ------------------------------------------------------------------------------------------ program

    def program(self) -> Program:
        plan, sch, m = self.plan, self.sch, self.m
        R, W = m.rows, m.width
        args: List[Arg] = []
        for k, name in enumerate(plan.nest.params):
            ctype = "const int* __restrict__" if any(ix.name == name for ix in plan.indices) else \
                "const ak_u16* __restrict__"
            args.append(Arg("input", k, ctype, name))
        args.append(Arg("output", 0, "ak_u16* __restrict__", m.out.name + "_out"))
        tables: Dict[str, np.ndarray] = {}
        for r in sch.inner:
            tables[f"tv_{r.var}"] = np.asarray(sch.tile_values[r.var], np.int32)
            args.append(Arg("table", f"tv_{r.var}", "const int* __restrict__", f"tv_{r.var}"))
        workspace = {"dc_m": 4 * self.slots * RP, "dc_l": 4 * self.slots * RP, "dc_acc": 4 * self.slots * RP * W}
        if not self.qrows:
            workspace["dc_q"] = 2 * sch.pattern_tiles * RP * W
        # the step tables (device-built) or, with a cursor, only what the merge reads: the count and each
        # tile's first step, which the attention kernel's workgroup 0 writes
        for ws in (("count", "tile_steps") if self.cursor else ("step_tile", "step_code", "count", "tile_steps")):
            args.append(Arg("workspace", ws, "int* __restrict__", f"rt_{ws}"))
        if self.cursor:
            workspace["count"] = 4
            workspace["tile_steps"] = 4 * (sch.pattern_tiles + 1)
        if not self.qrows:
            args.append(Arg("workspace", "dc_q", "ak_u16* __restrict__", "dc_q"))
        for ws in ("dc_m", "dc_l", "dc_acc"):
            args.append(Arg("workspace", ws, "float* __restrict__", ws))
        if self.trace:
            workspace[TRACE] = self.grid * TRACE_FIELDS * 8
            args.append(Arg("workspace", TRACE, "unsigned long long* __restrict__", TRACE))
        # with the merge in the attention kernel: per tile, the workgroups done with it (zero between calls)
        state = {"dc_arrive": sch.pattern_tiles} if self.fold else {}
        if self.fold:
            args.append(Arg("state", "dc_arrive", "int* __restrict__", "dc_arrive"))
        struct = c_struct(f"{self.name}_args", args)
        # Unless the attention kernel computes them itself (`qrows`), the query rows are set up by extra workgroups
        # of the table builder's launch (they need no table), or with a cursor by a launch of their own.
        setup = self.cursor and not self.qrows
        source = "\n".join([f"// Generated by tilejax_amd for `{plan.nest.name}`: gfx950 split-KV decode attention.",
                            PRELUDE, struct, self._setup_source() if setup else "", self._attention_source(),
                            "" if self.fold else self._merge_source()])
        launches = [Launch(self.name, args, (self.grid, 1, 1), (self.threads, 1, 1), 0)]
        if not self.fold:
            launches.append(Launch(f"{self.name}_merge", args, (sch.pattern_tiles, self.merge_chunks, 1),
                                   (self.threads, 1, 1), 0))
        if setup:
            launches.insert(0, Launch(f"{self.name}_setup", args, (sch.pattern_tiles, self.setup_chunks, 1),
                                      (self.threads, 1, 1), 0))
        prog = Program(
            name=self.name, source=source,
            launches=launches,
            outputs=[(m.out.shape, m.out.dtype)], inputs=[(s.shape, s.dtype) for s in plan.inputs],
            tables=tables, workspace=workspace, state=state, lds_bytes=self.lds, protocol=self.protocol,
            notes={"family": "decode", "grid": self.grid, "slots": self.slots, "rows": R, "width": W, "page": m.page,
                   "cursor": self.cursor, "merge_folded": self.fold, "own_rows": self.owners is not None,
                   "query_rows_in_kernel": self.qrows,
                   # trace regions cover the attention kernel; a slice is one kernel step, SUB positions
                   "trace_workgroups": self.grid if self.trace else 0, "slices_per_step": self.sub},
        )
        if not self.cursor and self.qrows:
            attach_step_builder(prog, plan, sch, self.name)
        elif not self.cursor:
            setup_args = [a for a in args if a.kind in ("input", "table") or a.key == "dc_q"]
            attach_step_builder(prog, plan, sch, self.name,
                                extra=self._setup_body(f"xb_ / {self.setup_chunks}", f"xb_ % {self.setup_chunks}"),
                                extra_args=setup_args, extra_groups=sch.pattern_tiles * self.setup_chunks)
        return prog

    def _decode_tile(self, t: str) -> str:
        return " ".join(f"const int lv_{r.var} = {tile_value(self.sch, r.var, t)};" for r in self.sch.inner)

    def _tile_values(self, t: str) -> str:
        """The attention kernel's loop values of tile `t` after the cursor's scan: from its copy in LDS (with
        step tables, from the table)."""
        if not self.cursor:
            return self._decode_tile(t)
        return " ".join(f"const int lv_{r.var} = cs_lv_{r.var}[{t}];" for r in self.sch.inner)

    def _setup_body(self, t: str, y: str) -> str:
        """Chunk `y` of tile `t`'s query rows (the setup code's value, per element), by the workgroup's
        threads."""
        m = self.m
        R, W = m.rows, m.width
        em = self._emitter(lambda n, idx: None)
        expr = em.at(m.q_node, ("qr", "qc"))
        per = -(-RP * W // self.setup_chunks)
        return f"""  {{ const int t = {t}, y_ = {y};
    {self._decode_tile("t")}
    ak_u16* dst = args.dc_q + (long long)t * {RP * W};
    const int e1 = ak_imin((y_ + 1) * {per}, {RP * W});
    for (int e = y_ * {per} + (int)threadIdx.x; e < e1; e += (int)blockDim.x) {{
      const int qr = e / {W}, qc = e % {W};
      dst[e] = qr < {R} ? (ak_u16)ak_bf16_bits((float)({expr})) : (ak_u16)0;  // rows past R are zero
    }}
  }}"""

    def _setup_source(self) -> str:
        return f"""
// The tile's query rows, materialised once per tile; workgroup (t, y) writes chunk y of tile t's elements.
extern "C" __global__ void __launch_bounds__({self.threads}) {self.name}_setup(const {self.name}_args args) {{
{self._setup_body("(int)blockIdx.x", "(int)blockIdx.y")}
}}
"""

    def _attention_source(self) -> str:
        plan, sch, m = self.plan, self.sch, self.m
        P, W = SUB, m.width
        U = self.sub
        WQ = W // self.waves  # a wave's share of the width
        slabs = WQ // 32  # K = 32 slabs of S^T = K Q^T per wave
        dtiles = WQ // 32  # 32-wide tiles of acc^T per wave
        loads = P * W // 8 // self.threads  # 16-byte V loads per thread per step
        D = self.depth
        phase, index = self.phase, self.index
        radix = sch.phase_radix * sch.iterations
        jvar = phase.var
        k_shape, v_shape = plan.inputs[m.k.param].shape, plan.inputs[m.v.param].shape
        k_base, k_str = tile_base(m.k.tile, k_shape, index, lambda v: f"lv_{v}")
        v_base, v_str = tile_base(m.v.tile, v_shape, index, lambda v: f"lv_{v}")
        if k_str[-1] != 1 or v_str[-1] != 1:
            raise KernelError("the decode lowering reads pages whose last dim is contiguous")
        ldk, ldv = k_str[0], v_str[0]
        for arr, shape in ((m.k.tile.array, k_shape), (m.v.tile.array, v_shape)):
            if 2 * math.prod(shape) >= 2**31:
                raise KernelError(f"`{arr}` is 2 GiB or more: the decode lowering uses 32-bit buffer offsets")

        # score(S) per element: S is `sv`, rows `er`, positions `ep` (in the step's block).
        def sleaf(n: Node, idx: Tuple[str, ...]) -> Optional[str]:
            if n is m.sm.qk:
                return "sv"
            return None

        score = self._emitter(sleaf).at(m.sm.score, ("er", "ep"))
        chunks = W // 8
        own = self.owners is not None
        cw = WQ // 8  # 16-byte chunks of a wave's columns per row
        vrow = WQ if own else W  # elements per V row in a stage (a wave's region, or the whole width)
        acc_store = (f"""float* ap = args.dc_acc + (long long)slot * {RP * W} + row * {W} + cb + (lane >> 5) * 4;
#pragma unroll
    for (int dt = 0; dt < {dtiles}; ++dt)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4)
        *(ak_f32x4*)(ap + 32 * dt + 8 * g4) = ak_f32x4{{acc[dt][4 * g4], acc[dt][4 * g4 + 1], acc[dt][4 * g4 + 2], acc[dt][4 * g4 + 3]}};""")
        if own:
            # each row's statistics and accumulator come from the wave that owns it (rows past R: none)
            flush_body = (f"""if (dc_owner[row] == wave) {{  // this wave's rows: their statistics and columns
      if (lane < 32) {{
        args.dc_m[slot * {RP} + row] = m_run;
        args.dc_l[slot * {RP} + row] = l_run;
      }}
      {acc_store}
    }}""")
        else:
            flush_body = (f"""if (wave == 0 && lane < 32) {{
      args.dc_m[slot * {RP} + row] = m_run;
      args.dc_l[slot * {RP} + row] = l_run;
    }}
    {acc_store}""")
        if own:
            # each wave loads its own columns of V into its own region of the stage (rows of WQ elements)
            v_load_setup = f"""// V loads: each wave its own {WQ} columns, into its own region of the stage: chunk position
  // p = c * 64 + lane, row p / {cw}, chunk p % {cw}, rows swizzled for ds_read_b64_tr_b16 (chunk ^ (row & 3) << 2).
  unsigned v_voff[{loads}];
#pragma unroll
  for (int c = 0; c < {loads}; ++c) {{
    const int p = c * 64 + lane, row = p / {cw}, ch = p % {cw};
    v_voff[c] = (unsigned)(row * {ldv * 2} + cb * 2 + ((ch ^ (((row & 3) << 2) & {cw - 1})) * 16));
  }}"""
            v_roff_line = (f"const int c = 32 * dt + 16 * (G & 1) + 4 * (s & 3); v_roff[dt] = wave * {P * WQ * 2} + "
                           f"pos * {WQ * 2} + ((((c >> 3) ^ (((pos & 3) << 2) & {cw - 1}))) << 4) + (c & 7) * 2;")
        else:
            v_load_setup = f"""// V loads: LDS chunk position p = c * {self.threads} + tid: row p / {chunks}, chunk p % {chunks}, rows swizzled
  // for ds_read_b64_tr_b16 (chunk ^ (row & 3) << 2).
  unsigned v_voff[{loads}];
#pragma unroll
  for (int c = 0; c < {loads}; ++c) {{
    const int p = c * {self.threads} + tid, row = p / {chunks}, ch = p % {chunks};
    v_voff[c] = (unsigned)(row * {ldv * 2} + ((ch ^ ((row & 3) << 2)) * 16));
  }}"""
            v_roff_line = ("const int c = cb + 32 * dt + 16 * (G & 1) + 4 * (s & 3);\n"
                           f"      v_roff[dt] = pos * {W * 2} + ((((c >> 3) ^ ((pos & 3) << 2))) << 4) + (c & 7) * 2;")
        # the Q^T fragments of tile t (srcB of S^T, 16x16x32): query rows lane % 16 and 16 + lane % 16, columns
        # cb + 32 s + 8 (lane / 16) .. + 8
        table_lines: List[str] = []  # file-scope constant tables they read
        if self.qrows:
            # Evaluated here from the setup code, per element, as the setup kernel would write them. Only this
            # wave's own rows are nonzero in its columns: the lanes evaluate that block (its elements spread over
            # the wave, their loads all in flight at once) into the wave's partial-S area of LDS, and each
            # fragment is read back from there, or is zero for a row of another wave's. (LDS operations of one
            # wave run in order: no barrier.)
            owned = [[r for r, o in enumerate(self.owners) if o == w_] for w_ in range(self.waves)]
            most = max(len(rows) for rows in owned)
            per_lane = -(-most * WQ // 64)
            slot_of = [[rows.index(r) if r in rows else -1 for r in range(RP)] for rows in owned]
            table_lines.append(f"// per wave: its own query rows, in order (-1 past them), and each row's place among them")
            table_lines.append(f"__constant__ int dc_rows[{self.waves}][{max(most, 1)}] = {{"
                               + ", ".join("{" + ", ".join(map(str, rows + [-1] * (max(most, 1) - len(rows)))) + "}"
                                           for rows in owned) + "};")
            table_lines.append(f"__constant__ int dc_slot[{self.waves}][{RP}] = {{"
                               + ", ".join("{" + ", ".join(map(str, sl)) + "}" for sl in slot_of) + "};")
            q_expr = self._emitter(lambda n, idx: None).at(m.q_node, ("qr", "qc"))
            q_load = f"""{self._tile_values("t")}
    ak_u16* stg = (ak_u16*)&dc_sp[wave][0][0];  // this wave's own rows x its {WQ} columns
#pragma unroll
    for (int i = 0; i < {per_lane}; ++i) {{
      const int e = lane + 64 * i, k = e / {WQ}, col = e % {WQ};
      const int qr = k < {most} ? dc_rows[wave][k] : -1, qc = cb + col;
      if (qr >= 0) stg[e] = (ak_u16)ak_bf16_bits((float)({q_expr}));
    }}
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {{
      const int k = dc_slot[wave][(lane & 15) + 16 * tt];
#pragma unroll
      for (int s = 0; s < {slabs}; ++s)
        qf[tt][s] = k >= 0 ? *(const ak_bf16x8*)&stg[k * {WQ} + 32 * s + 8 * (lane >> 4)] : ak_bf16x8{{}};
    }}"""
        else:
            q_load = f"""const ak_u16* qp = args.dc_q + (long long)t * {RP * W} + cb + 8 * (lane >> 4);
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int s = 0; s < {slabs}; ++s)
        qf[tt][s] = *(const ak_bf16x8*)(qp + (long long)((lane & 15) + 16 * tt) * {W} + 32 * s);"""
        L: List[str] = []
        w = L.append
        for s in range(D):  # one array per stage: the compiler then keeps the other stages' loads in flight
            w(f"__shared__ __attribute__((aligned(1024))) ak_u16 dc_sv{s}[{P * W}];")
        # each wave's partial S, row-major: a row's positions are contiguous (one 16-byte write per MFMA result
        # and two 16-byte reads per lane), rows padded to SP floats so 16 lanes' rows fall in distinct banks
        w(f"__shared__ __attribute__((aligned(16))) float dc_sp[{self.waves}][{RP}][{SP}];")
        w(f"__shared__ __attribute__((aligned(16))) int dc_st[{self.max_per}][5];")
        if own:
            owner = list(self.owners) + [-1] * (RP - len(self.owners))
            w(f"// each query row's wave (its values lie in that wave's columns only); rows past R: none")
            w(f"__constant__ int dc_owner[{RP}] = {{{', '.join(map(str, owner))}}};")
        L.extend(table_lines)
        w(f"""
extern "C" __global__ void __launch_bounds__({self.threads}) {self.name}(const {self.name}_args args) {{
  {f"__shared__ float dc_w[{self.maxs}][{m.rows}], dc_lsum[{m.rows}]; __shared__ int dc_last;" if self.fold else ""}
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  {self._trace_start()}
  {self._cursor_scan() if self.cursor else ""}
  const int count = {"cs_start[" + str(sch.pattern_tiles) + "]" if self.cursor else "args.rt_count[0]"} * {U};  // kernel steps: {U} of {P} positions per table step
  const int per = (count + {self.grid - 1}) / {self.grid};
  const int g0 = blockIdx.x * per, n = ak_imin(g0 + per, count) - g0;
  if (n <= 0) {{ {self._trace_write("0")} return; }}
  // The range's steps, decoded once into LDS: tile, code, K and V page byte offsets. The loop then reads
  // them from LDS, so no global load other than the pages themselves sits in the vector memory queue.
  for (int j = tid; j < n; j += {self.threads}) {{
    const int x = g0 + j, js = x / {U}, su = x - js * {U};  // the table's step, and the part of its block
    {self._cursor_step() if self.cursor else "const int t = args.rt_step_tile[js], code = args.rt_step_code[js];"}
    {self._tile_values("t")}
    const int lv_{jvar} = {phase.start} + ((code >> {CODE_SHIFT}) / {radix}) * {phase.step};
    dc_st[j][0] = t;
    dc_st[j][1] = code;
    dc_st[j][2] = (int)(({k_base} + (long long)su * {P * ldk}) * 2);
    dc_st[j][3] = (int)(({v_base} + (long long)su * {P * ldv}) * 2);
    dc_st[j][4] = su;
  }}
  __syncthreads();
  const int cb = wave * {WQ};  // this wave's columns of the width
  const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc((void*)args.{m.k.tile.array}, (short)0,
      (int)({math.prod(k_shape)}LL * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc((void*)args.{m.v.tile.array}, (short)0,
      (int)({math.prod(v_shape)}LL * 2), 0x00020000);
  {v_load_setup}
  // K fragments (srcA of S^T, 16x16x32) straight from HBM into registers: position lane % 16, columns
  // cb + 32 s + 8 (lane / 16)
  const unsigned k_voff = (unsigned)((lane & 15) * {ldk * 2} + (cb + 8 * (lane >> 4)) * 2);
  // V^T fragment (srcA of acc^T, 32x32x16), tr16 reads: group G = lane / 16, s = lane % 16
  int v_roff[{dtiles}];
  {{
    const int G = lane >> 4, s = lane & 15, pos = 8 * (G >> 1) + (s >> 2);
#pragma unroll
    for (int dt = 0; dt < {dtiles}; ++dt) {{
      {v_roff_line}
    }}
  }}
  ak_bf16x8 qf[2][{slabs}];
  {" ".join(f"ak_bf16x8 kb{s}[{slabs}];" for s in range(D))}
  ak_f32x16 acc[{dtiles}];
  float m_run = {literal(m.sm.m_init)}, l_run = 0.f;
  int cur_t = -1;
  auto flush = [&](int t) {{
    {f"const unsigned long long tr_f0 = {NOW};" if self.trace else ""}
    const int slot = t + blockIdx.x;
    const int row = lane & 31;
    {flush_body}
    {f"tr_out += {NOW} - tr_f0;" if self.trace else ""}
  }};
  auto start_tile = [&](int t) {{
    {q_load}
#pragma unroll
    for (int i = 0; i < {dtiles}; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;
    m_run = {literal(m.sm.m_init)};
    l_run = 0.f;
  }};""")
        # Issue order, one group per arrow: ... -> V(j + D - 1) -> K(j + D) -> ... (step j issues the V page
        # D - 1 steps ahead after its first barrier and the K fragments D steps ahead once its S product has
        # read kb). Steps past the range issue the same loads out of the buffers' bounds (offset + 2^31: no
        # memory access, zeros), so every step adds the same count and one wait count fits every step: K(j)
        # and V(j) are done once the groups after V(j) (K(j+1) .. K(j+D-1)) alone are outstanding.
        wait_n = (D - 1) * slabs + (D - 2) * loads

        def issue_k(x: str, ks: int, ind: str) -> List[str]:
            return [
                f"{ind}{{ const int x_ = {x}; const unsigned ob_ = x_ < n ? 0u : 0x80000000u;",
                f"{ind}  const int ko_ = __builtin_amdgcn_readfirstlane(dc_st[ak_imin(x_, n - 1)][2]);",
                *(f"{ind}  kb{ks}[{q}] = __builtin_bit_cast(ak_bf16x8, __builtin_amdgcn_raw_buffer_load_b128(rk, k_voff + ob_ + {64 * q}, ko_, 0));"
                  for q in range(slabs)),
                f"{ind}}}",
            ]

        def v_dest(c: int) -> str:
            """The stage element instruction c of this thread's V loads starts at (1 KiB per wave)."""
            return f"wave * {P * WQ} + {c * 64 * 8}" if own else f"({c * self.threads} + wave * 64) * 8"

        def issue_v(x: str, vs: int, ind: str) -> List[str]:
            return [
                f"{ind}{{ const int x_ = {x}; const unsigned ob_ = x_ < n ? 0u : 0x80000000u;",
                f"{ind}  const int vo_ = __builtin_amdgcn_readfirstlane(dc_st[ak_imin(x_, n - 1)][3]);",
                *(f"{ind}  __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, AK_LDS(&dc_sv{vs}[{v_dest(c)}]), 16, "
                  f"v_voff[{c}] + ob_, vo_, 0, 0);" for c in range(loads)),
                f"{ind}}}",
            ]

        rec = self.protocol = Recorder()  # V pages through LDS stages, K fragments through register sets

        def step(j: str, u: int, ind: str) -> List[str]:
            """Step j (= u modulo D): its K fragments in kb{u}, its V page in dc_sv{u}."""
            o: List[str] = []
            a = o.append
            record = not rec.body.get(u)  # each position's events once (the loop and the tail emit the same)
            a(f"{ind}{{ const int j_ = {j};")
            a(f"{ind}  const int t = __builtin_amdgcn_readfirstlane(dc_st[j_][0]), code = __builtin_amdgcn_readfirstlane(dc_st[j_][1]);")
            if self.trace:
                a(f"{ind}  const unsigned long long tr_w0 = {NOW}, tr_o0 = tr_out;")
            a(f"{ind}  if (t != cur_t) {{ if (cur_t >= 0) flush(cur_t); start_tile(t); cur_t = t; AK_WAIT_VM(0); }}")
            a(f"{ind}  AK_WAIT_VM({wait_n});")
            if own:  # V(j) is in this wave's own region: its own wait suffices
                if record:
                    rec.at(u, lambda b, n: ("wait_vm", wait_n))
                if self.sync:
                    # nothing else holds a workgroup's waves together: without a barrier now and then they
                    # drift apart (the first waves win the memory queues), and the last ones finish alone
                    a(f'{ind}  if (j_ % {self.sync} == 0) asm volatile("s_barrier" ::: "memory");')
                    if record:
                        rec.at(u, lambda b, n: ("barrier",), lambda b, n, k=self.sync: b % k == 0)
            else:
                # every wave is past step j - 1, so its V stage is free; every thread's part of V(j) has landed
                a(f'{ind}  asm volatile("s_barrier" ::: "memory");')
                if record:
                    rec.at(u, lambda b, n: ("wait_vm", wait_n))
                    rec.at(u, lambda b, n: ("barrier",))
            if self.trace:
                # the first step's wait is the pipeline fill; a flush inside the wait is output time
                a(f"{ind}  {{ const unsigned long long d_ = {NOW} - tr_w0 - (tr_out - tr_o0);"
                  f" if (j_ == 0) tr_fill = d_; else tr_wait += d_; }}")
            o.extend(issue_v(f"j_ + {D - 1}", (u + D - 1) % D, ind + "  "))
            if record:
                rec.at(u, lambda b, n, st=(u + D - 1) % D: ("load", st, b + D - 1, loads))
                # V(j) is visible (its wait, then the barrier): its V^T fragments are read now, so the P V
                # MFMAs after the softmax don't wait for LDS
                rec.at(u, lambda b, n, st=u: ("read_mine" if own else "read", st, b))
                rec.at(u, lambda b, n, ku=u: ("read_own", ("k", ku), b))  # the S product reads kb{u}
            a(f"{ind}  const bool run = !(code & 4);")
            a(f"{ind}  ak_bf16x8 vf[{dtiles}];")
            # partial S^T over this wave's columns, in four MFMA chains (even and odd slabs apart)
            a(f"{ind}  if (run) {{")
            a(f"{ind}    const char* vs = (const char*)dc_sv{u};")
            a(f"{ind}    #pragma unroll")
            a(f"{ind}    for (int dt = 0; dt < {dtiles}; ++dt) {{")
            a(f"{ind}      const ak_i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(AK_LDS4(vs + v_roff[dt]));")
            a(f"{ind}      const ak_i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(AK_LDS4(vs + v_roff[dt] + {4 * vrow * 2}));")
            a(f"{ind}      vf[dt] = __builtin_bit_cast(ak_bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));")
            a(f"{ind}    }}")
            a(f"{ind}    ak_f32x4 st[4] = {{ak_f32x4{{0.f, 0.f, 0.f, 0.f}}, ak_f32x4{{0.f, 0.f, 0.f, 0.f}}, ak_f32x4{{0.f, 0.f, 0.f, 0.f}}, ak_f32x4{{0.f, 0.f, 0.f, 0.f}}}};")
            a(f"{ind}    #pragma unroll")
            a(f"{ind}    for (int q = 0; q < {slabs}; ++q) {{")
            a(f"{ind}      st[2 * (q & 1)] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kb{u}[q], qf[0][q], st[2 * (q & 1)], 0, 0, 0);")
            a(f"{ind}      st[2 * (q & 1) + 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kb{u}[q], qf[1][q], st[2 * (q & 1) + 1], 0, 0, 0);")
            a(f"{ind}    }}")
            a(f"{ind}    st[0] += st[2];")
            a(f"{ind}    st[1] += st[3];")
            # st[h][r] is S^T at position 4 (lane / 16) + r, query row 16 h + lane % 16
            a(f"{ind}    *(ak_f32x4*)&dc_sp[wave][lane & 15][4 * (lane >> 4)] = st[0];")
            a(f"{ind}    *(ak_f32x4*)&dc_sp[wave][16 + (lane & 15)][4 * (lane >> 4)] = st[1];")
            a(f"{ind}  }}")
            # kb{u} has been read: refill it D steps ahead
            o.extend(issue_k(f"j_ + {D}", u, ind + "  "))
            if record:
                rec.at(u, lambda b, n, ku=u: ("load", ("k", ku), b + D, slabs))
            a(f"{ind}  if (run) {{")
            a(f"{ind}    {self._decode_tile('t')}")
            a(f"{ind}    const int lv_{jvar} = {phase.start} + ((code >> {CODE_SHIFT}) / {radix}) * {phase.step}; (void)lv_{jvar};")
            a(f"{ind}    const int su = __builtin_amdgcn_readfirstlane(dc_st[j_][4]); (void)su;")
            # an LDS-only barrier: the pages in flight stay in flight (with rows of its own, a wave reads back
            # only its own partial S: its own wait suffices)
            a(f"{ind}    AK_WAIT_LGKM0();")
            if not own:
                a(f'{ind}    asm volatile("s_barrier" ::: "memory");')
            if record:
                rec.at(u, lambda b, n: ("wait_lgkm",))
                if not own:
                    rec.at(u, lambda b, n: ("barrier",))
            # softmax: lane = query row er, positions 8 (lane / 32) + e
            # the lane's row; the mask sees rows past R (zero queries, never stored) as row R - 1
            a(f"{ind}    const int lr = lane & 31, er = {'lr' if m.rows == RP else f'ak_imin(lr, {m.rows - 1})'};")
            a(f"{ind}    float sc[8];")
            if own:
                # the rows this wave owns have their whole S here (the other waves' are zeros for them); its
                # other rows are computed but never stored
                a(f"{ind}    const ak_f32x4 s_lo = *(const ak_f32x4*)&dc_sp[wave][lr][8 * (lane >> 5)], s_hi = *(const ak_f32x4*)&dc_sp[wave][lr][8 * (lane >> 5) + 4];")
            else:
                a(f"{ind}    ak_f32x4 s_lo = *(const ak_f32x4*)&dc_sp[0][lr][8 * (lane >> 5)], s_hi = *(const ak_f32x4*)&dc_sp[0][lr][8 * (lane >> 5) + 4];")
                a(f"{ind}    #pragma unroll")
                a(f"{ind}    for (int w_ = 1; w_ < {self.waves}; ++w_) {{")
                a(f"{ind}      s_lo += *(const ak_f32x4*)&dc_sp[w_][lr][8 * (lane >> 5)];")
                a(f"{ind}      s_hi += *(const ak_f32x4*)&dc_sp[w_][lr][8 * (lane >> 5) + 4];")
                a(f"{ind}    }}")
            a(f"{ind}    float mx = -__builtin_inff();")
            a(f"{ind}    #pragma unroll")
            a(f"{ind}    for (int e = 0; e < 8; ++e) {{")
            a(f"{ind}      const int el = 8 * (lane >> 5) + e;  // the position in this kernel step")
            a(f"{ind}      const int ep = {P} * su + el;  // the position in the table step's block")
            a(f"{ind}      const float sv = e < 4 ? s_lo[e] : s_hi[e - 4];")
            a(f"{ind}      sc[e] = (float)({score});")
            a(f"{ind}      mx = fmaxf(mx, sc[e]);")
            a(f"{ind}    }}")
            a(f"{ind}    mx = fmaxf(mx, __shfl_xor(mx, 32));")
            a(f"{ind}    const float m_new = ak_maximum(m_run, mx);")
            # Lazy rescaling: the running max moves (and acc, l are rescaled) only when some row's new max
            # exceeds it by more than RESCALE_SLACK; otherwise p = exp(s - m_run) stays below e^slack and
            # acc, l keep one common scale, so acc / l is unchanged.
            a(f"{ind}    if (__ballot(!(m_new <= m_run + {RESCALE_SLACK}f))) {{")
            a(f"{ind}      const float alpha = ak_exp(m_run - m_new);")
            a(f"{ind}      l_run *= alpha;")
            a(f"{ind}      m_run = m_new;")
            a(f"{ind}      #pragma unroll")
            a(f"{ind}      for (int dt = 0; dt < {dtiles}; ++dt) acc[dt] *= alpha;")
            a(f"{ind}    }}")
            a(f"{ind}    float ps = 0.f;")
            a(f"{ind}    unsigned pk[4];")
            a(f"{ind}    #pragma unroll")
            a(f"{ind}    for (int e = 0; e < 8; e += 2) {{")
            a(f"{ind}      const float p0 = ak_exp(sc[e] - m_run), p1 = ak_exp(sc[e + 1] - m_run);")
            a(f"{ind}      ps += p0 + p1; pk[e >> 1] = ak_pack_bf16x2(p0, p1);")
            a(f"{ind}    }}")
            a(f"{ind}    ps += __shfl_xor(ps, 32);")
            a(f"{ind}    l_run += ps;")
            a(f"{ind}    const ak_bf16x8 pf = __builtin_bit_cast(ak_bf16x8, ak_u32x4{{pk[0], pk[1], pk[2], pk[3]}});")
            a(f"{ind}    #pragma unroll")
            a(f"{ind}    for (int dt = 0; dt < {dtiles}; ++dt)")
            a(f"{ind}      acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf[dt], pf, acc[dt], 0, 0, 0);")
            a(f"{ind}  }}")
            a(f"{ind}}}")
            return o

        # prologue: what steps -D .. -1 would have issued: K(0), then V(x) and K(x + 1) for x < D - 1
        L.extend(issue_k("0", 0, "  "))
        rec.add(("load", ("k", 0), 0, slabs))
        for x in range(D - 1):
            L.extend(issue_v(str(x), x, "  "))
            L.extend(issue_k(str(x + 1), x + 1, "  "))
            rec.add(("load", x, x, loads))
            rec.add(("load", ("k", x + 1), x + 1, slabs))
        rec.loop(D)
        # whole rounds of D steps with no condition between them (the compiler's wait counts stay exact),
        # then the last steps; no wait drains the queue except at a tile change
        w("  int j = 0;")
        w(f"  for (; j + {D} <= n; j += {D}) {{")
        for u in range(D):
            L.extend(step(f"j + {u}", u, "    "))
        w("  }")
        ind = "  "
        for u in range(D - 1):
            w(f"{ind}if (j + {u} < n) {{")
            L.extend(step(f"j + {u}", u, ind + "  "))
            ind += "  "
        for u in range(D - 1):
            ind = ind[:-2]
            w(f"{ind}}}")
        w("  flush(cur_t);")
        if self.fold:
            if self.trace:
                w(f"  const unsigned long long tr_m0 = {NOW};")
            w(self._fold_merge("cs_start[{}]" if self.cursor else "args.rt_tile_steps[{}]"))
            if self.trace:
                w(f"  tr_out += {NOW} - tr_m0;  // the merges count as output time")
        if self.trace:
            w(f"  {self._trace_write('n')}")
        w("}")
        return "\n".join(L)

    def _cursor_scan(self) -> str:
        """With a cursor: the runtime mask of every (tile, block), a ballot per 64 blocks into LDS words (each
        wave takes every `waves`-th tile, decoding its loop values once); each tile's kept count (a tile with
        no block running keeps one empty step, as the step tables do) and their exclusive scan, cs_start.
        Workgroup 0 writes the count and the tiles' first steps for the merge kernel."""
        plan, sch = self.plan, self.sch
        phase = plan.phases[0].range
        pt, count, nb = sch.pattern_tiles, phase.count, -(-phase.count // 64)
        mask = Index(plan, lambda v: f"lv_{v}").expr(phase.mask)
        per_t = -(-pt // self.threads)
        rounds = -(-pt // self.waves)  # tiles per wave
        kb_run = (f"const int kb = wi * 64 + lane;\n        bool run = false;\n"
                  f"        if (kb < {count}) {{ const int lv_{phase.var} = {phase.start} + kb * {phase.step}; run = !({mask}); }}")
        inner = self.sch.inner
        # whether the mask's index-array reads are the tile's alone (`lengths[b]`), not the block's
        reads = element_reads(phase.mask, {ix.name for ix in plan.indices})
        tile_reads = all(phase.var not in {n.id for n in ast.walk(r.slice) if isinstance(n, ast.Name)} for r in reads)
        if rounds * nb <= 64 and tile_reads:
            # A lane per (tile, word): its tile's loop values (one vector load), then the mask's index reads
            # (the same for the word's 64 blocks, so loaded once), then the word's bits in a loop.
            ballots = f"""{{
    const int i_ = lane / {nb}, wi = lane % {nb}, t = wave + {self.waves} * i_;
    if (lane < {rounds * nb} && t < {pt}) {{
      {" ".join(f"const int lv_{r.var} = {tile_value(sch, r.var, 't')};" for r in inner)}
      unsigned long long word_ = 0;
      for (int b_ = 0; b_ < 64; ++b_) {{
        const int kb = wi * 64 + b_;
        bool run = false;
        if (kb < {count}) {{ const int lv_{phase.var} = {phase.start} + kb * {phase.step}; run = !({mask}); }}
        word_ |= (unsigned long long)run << b_;
      }}
      cs_run[t * {nb} + wi] = word_;
    }}
  }}"""
        elif rounds * nb <= 64:
            # Straight-line code: all the wave's tiles' loop values are loaded at once, then their masks' index
            # reads, so the latencies overlap; each ballot word is kept by one lane (a select, no branch) and
            # the lanes store them together.
            ballots = f"""{{
    {" ".join(f"int lvA_{r.var}[{rounds}];" for r in inner)}
#pragma unroll
    for (int i = 0; i < {rounds}; ++i) {{
      const int t_ = ak_imin(wave + {self.waves} * i, {pt - 1});
      {" ".join(f"lvA_{r.var}[i] = {tile_value(sch, r.var, 't_')};" for r in inner)}
    }}
    unsigned long long word_ = 0;
#pragma unroll
    for (int i = 0; i < {rounds}; ++i) {{
      {" ".join(f"const int lv_{r.var} = lvA_{r.var}[i];" for r in inner)}
#pragma unroll
      for (int wi = 0; wi < {nb}; ++wi) {{
        {kb_run}
        const unsigned long long m_ = __ballot(run);
        word_ = lane == i * {nb} + wi ? m_ : word_;
      }}
    }}
    const int t_ = wave + {self.waves} * (lane / {nb});
    if (lane < {rounds * nb} && t_ < {pt}) cs_run[t_ * {nb} + lane % {nb}] = word_;
  }}"""
        else:
            ballots = f"""// (unrolled so that several tiles' loop values and index reads are in flight at once)
#pragma unroll 8
  for (int t = wave; t < {pt}; t += {self.waves}) {{
    {self._decode_tile("t")}
    for (int wi = 0; wi < {nb}; ++wi) {{
      {kb_run}
      const unsigned long long m_ = __ballot(run);
      if (lane == 0) cs_run[t * {nb} + wi] = m_;
    }}
  }}"""
        # every tile's loop values, for the steps' decode and the tiles' starts (one load a thread, beside
        # the ballots)
        lv_copy = "\n  ".join(f"__shared__ int cs_lv_{r.var}[{pt}];\n  for (int t_ = tid; t_ < {pt}; t_ += {self.threads}) "
                              f"cs_lv_{r.var}[t_] = {tile_value(sch, r.var, 't_')};" for r in inner)
        return f"""__shared__ unsigned long long cs_run[{self.words}];
  __shared__ int cs_start[{pt + 1}], cs_part[{self.threads}];
  {lv_copy}
  {ballots}
  __syncthreads();
  {{  // kept steps per tile, summed over runs of {per_t} tiles per thread; a scan within each wave (shuffles),
    // then over the waves' totals
    const int t0 = tid * {per_t}, t1 = ak_imin(t0 + {per_t}, {pt});
    int mine = 0;
    for (int t = t0; t < t1; ++t) {{
      int k = 0;
      for (int wi = 0; wi < {nb}; ++wi) k += __popcll(cs_run[t * {nb} + wi]);
      cs_start[t] = k ? k : 1;
      mine += k ? k : 1;
    }}
    int inc = mine;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {{
      const int y_ = __shfl_up(inc, d);
      if (lane >= d) inc += y_;
    }}
    if (lane == 63) cs_part[wave] = inc;
    __syncthreads();
    int before = 0;
    for (int w_ = 0; w_ < wave; ++w_) before += cs_part[w_];
    int at = before + inc - mine;
    for (int t = t0; t < t1; ++t) {{ const int k = cs_start[t]; cs_start[t] = at; at += k; }}
    if (tid == {self.threads - 1}) cs_start[{pt}] = before + inc;
    __syncthreads();
    if (blockIdx.x == 0) {{
      for (int t = tid; t <= {pt}; t += {self.threads}) args.rt_tile_steps[t] = cs_start[t];
      if (tid == 0) args.rt_count[0] = cs_start[{pt}];
    }}
  }}"""

    def _cursor_step(self) -> str:
        """With a cursor: table step js's tile (the last tile starting at or before it) and block (the
        tile's (js - start)-th running block, or block 0 of a tile with none: an empty step), as the code
        the step tables would hold (the kernel reads its block and its empty flag)."""
        sch = self.sch
        pt, nb = sch.pattern_tiles, -(-self.plan.phases[0].range.count // 64)
        radix = sch.phase_radix * sch.iterations
        return f"""int t = 0;
    {{ int hi = {pt - 1};
      while (t < hi) {{ const int mid = (t + hi + 1) >> 1; if (cs_start[mid] <= js) t = mid; else hi = mid - 1; }} }}
    int code = 4;  // an empty step at block 0, unless a running block is found
    {{ int r = js - cs_start[t];
      for (int wi = 0; wi < {nb}; ++wi) {{
        unsigned long long w_ = cs_run[t * {nb} + wi];
        const int c = __popcll(w_);
        if (r < c) {{  // the word's r-th set bit, by halving: is it among the low `h` bits of what is left?
          int pos = 0;
#pragma unroll
          for (int h = 32; h >= 1; h >>= 1) {{
            const int lo = __popcll(w_ & ((1ull << h) - 1));
            if (r >= lo) {{ r -= lo; w_ >>= h; pos += h; }}
          }}
          code = ((wi * 64 + pos) * {radix}) << {CODE_SHIFT};
          break;
        }}
        r -= c;
      }} }}"""

    def _trace_start(self) -> str:
        if not self.trace:
            return ""
        return (f"{CLOCK_START} unsigned long long tr_fill = 0, tr_wait = 0, tr_out = 0; "
                f"const unsigned long long tr_i0 = {NOW};")

    def _trace_write(self, steps: str) -> str:
        """Wave 0 writes the workgroup's region totals: waits (fill included), fill, output, compute, steps."""
        if not self.trace:
            return ""
        return (f"if (threadIdx.x == 0) {{ const unsigned long long tr_e = {NOW}; "
                f"unsigned long long* tr = args.{TRACE} + blockIdx.x * {TRACE_FIELDS}; "
                f"tr[0] = tr_fill + tr_wait; tr[1] = tr_fill; tr[2] = tr_out; "
                f"tr[3] = tr_e - tr_i0 - tr_fill - tr_wait - tr_out; tr[4] = (unsigned long long)({steps}); {CLOCK_END} }}")

    def _merge_body(self, e_begin: str, e_end: str) -> str:
        """Merge tile `t`'s `n` partials (slots t + w0 onwards: row max m, row sum l, accumulator) and write
        its output elements [e_begin, e_end), per element, by the workgroup's threads; `dc_w`, `dc_lsum` and
        (without `fold`) `dc_lw` are LDS arrays of the caller's."""
        m = self.m
        R, W = m.rows, m.width
        out_shape = m.out.tile.shape
        o_base, o_str = tile_base(m.out.tile, m.out.shape, self.index, lambda v: f"lv_{v}")

        def mleaf(n: Node, idx: Tuple[str, ...]) -> Optional[str]:
            if n is m.acc_leaf:
                return f"dc_acc_at(({idx[0]}), ({idx[1]}))"
            if _strip(n) is m.sum_leaf or n is m.sum_leaf:
                return f"dc_lsum[{idx[0]}]"
            if n.op == "carried" and n.kwargs["name"] not in m.sm.consts:
                raise KernelError("the decode epilogue reads only the accumulator and the row sum")
            return None

        expr = self._emitter(mleaf).at(m.value.node, tuple(f"o{k}" for k in range(len(out_shape))))
        unravel = []
        rest = "e"
        for k, st in enumerate(strides(out_shape)):
            unravel.append(f"const int o{k} = ({rest}) / {st};")
            rest = f"({rest}) % {st}"
        flat_out = " + ".join(f"(long long)o{k} * {s}" for k, s in enumerate(o_str))
        # the row sums: loaded with the maxima into LDS `dc_lw` (one round of loads; the merge launch), or read
        # in the second pass (the fold, whose LDS holds the attention kernel's too)
        together = not self.fold
        lw = (lambda k: f"dc_lw[{k}][r]") if together else (lambda k: f"lp[({k}) * {RP}]")
        keep_l = (f"\n      dc_lw[k][r] = lp[k * {RP}]; dc_lw[k + 1][r] = lp[(k + 1) * {RP}]; "
                  f"dc_lw[k + 2][r] = lp[(k + 2) * {RP}]; dc_lw[k + 3][r] = lp[(k + 3) * {RP}];") if together else ""
        return f"""  {self._decode_tile("t")}
  // The partials' loads go out four at a time (they are independent){", the row maxima and row sums together" if together else ""};
  // the sums run in partial order.
  for (int r = threadIdx.x; r < {R}; r += {self.threads}) {{
    const float* mp = args.dc_m + (t + w0) * {RP} + r;
    const float* lp = args.dc_l + (t + w0) * {RP} + r;
    float mm = -__builtin_inff();
    int k = 0;
    for (; k + 4 <= n; k += 4) {{
      const float a0 = mp[k * {RP}], a1 = mp[(k + 1) * {RP}], a2 = mp[(k + 2) * {RP}], a3 = mp[(k + 3) * {RP}];{keep_l}
      dc_w[k][r] = a0; dc_w[k + 1][r] = a1; dc_w[k + 2][r] = a2; dc_w[k + 3][r] = a3;
      mm = fmaxf(fmaxf(fmaxf(fmaxf(mm, a0), a1), a2), a3);
    }}
    for (; k < n; ++k) {{ const float a = mp[k * {RP}]; {f"dc_lw[k][r] = lp[k * {RP}]; " if together else ""}dc_w[k][r] = a; mm = fmaxf(mm, a); }}
    float ls = 0.f;
    for (k = 0; k + 4 <= n; k += 4) {{
      const float l0 = {lw("k")}, l1 = {lw("k + 1")}, l2 = {lw("k + 2")}, l3 = {lw("k + 3")};
      const float e0 = ak_exp(dc_w[k][r] - mm), e1 = ak_exp(dc_w[k + 1][r] - mm);
      const float e2 = ak_exp(dc_w[k + 2][r] - mm), e3 = ak_exp(dc_w[k + 3][r] - mm);
      dc_w[k][r] = e0; dc_w[k + 1][r] = e1; dc_w[k + 2][r] = e2; dc_w[k + 3][r] = e3;
      ls += e0 * l0; ls += e1 * l1; ls += e2 * l2; ls += e3 * l3;
    }}
    for (; k < n; ++k) {{ const float e = ak_exp(dc_w[k][r] - mm); dc_w[k][r] = e; ls += e * {lw("k")}; }}
    dc_lsum[r] = ls;
  }}
  __syncthreads();
  auto dc_acc_at = [&](int r, int c) -> float {{
    const float* ap = args.dc_acc + (long long)(t + w0) * {RP * W} + r * {W} + c;
    float v = 0.f;
    int k = 0;
    for (; k + 4 <= n; k += 4) {{
      const float a0 = ap[(long long)k * {RP * W}], a1 = ap[(long long)(k + 1) * {RP * W}];
      const float a2 = ap[(long long)(k + 2) * {RP * W}], a3 = ap[(long long)(k + 3) * {RP * W}];
      v += dc_w[k][r] * a0; v += dc_w[k + 1][r] * a1; v += dc_w[k + 2][r] * a2; v += dc_w[k + 3][r] * a3;
    }}
    for (; k < n; ++k) v += dc_w[k][r] * ap[(long long)k * {RP * W}];
    return v;
  }};
  ak_u16* op = args.{m.out.name}_out + ({o_base});
#pragma unroll 4
  for (int e = {e_begin} + (int)threadIdx.x; e < {e_end}; e += {self.threads}) {{
    {" ".join(unravel)}
    op[{flat_out}] = (ak_u16)ak_bf16_bits((float)({expr}));
  }}"""

    def _merge_source(self) -> str:
        """The merge kernel, where the attention kernel doesn't merge (`fold` off): workgroup (t, y) merges
        tile t's partials and writes chunk y of its elements, each computing the tile's partial weights."""
        R = self.m.rows
        total = math.prod(self.m.out.tile.shape)
        chunk = -(-total // self.merge_chunks)
        return f"""
// Merge a tile's partials (row max m, row sum l, accumulator) and write its output, per element; workgroup
// (t, y) writes chunk y of tile t's elements, each computing the tile's partial weights.
extern "C" __global__ void __launch_bounds__({self.threads}) {self.name}_merge(const {self.name}_args args) {{
  __shared__ float dc_w[{self.maxs}][{R}], dc_lw[{self.maxs}][{R}];
  __shared__ float dc_lsum[{R}];
  const int t = blockIdx.x;
  const int count = args.rt_count[0] * {self.sub};  // kernel steps, as the attention kernel divides them
  const int per = (count + {self.grid - 1}) / {self.grid};
  const int ts = args.rt_tile_steps[t] * {self.sub}, te = args.rt_tile_steps[t + 1] * {self.sub};
  const int w0 = ts / per, w1 = (te - 1) / per;
  const int n = w1 - w0 + 1;
{self._merge_body(f"(int)blockIdx.y * {chunk}", f"ak_imin((int)(blockIdx.y + 1) * {chunk}, {total})")}
}}
"""

    def _fold_merge(self, tile_start: str) -> str:
        """The attention kernel's exit: the merge, by the last workgroup to finish each tile. One release
        fence makes this workgroup's partials visible device-wide; then, for each tile its steps covered
        (`tile_start(t)`: the tile's first table step), a count of the workgroups done with it (device
        state, left at zero for the next call by the one that merges). A tile wholly inside this workgroup
        is merged at once; the workgroup that brings a shared tile's count to its number of workgroups
        takes an acquire fence and merges it."""
        U = self.sub
        total = math.prod(self.m.out.tile.shape)
        return f"""  // every thread's partial stores have reached the L2; then one wave's release fence writes the XCD's L2
  // back for the whole workgroup (a fence in every wave would write it back once per wave)
  AK_WAIT_VM(0);
  __syncthreads();
  if (wave == 0) __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  {{
    const int t_lo = dc_st[0][0], t_hi = dc_st[n - 1][0];
    for (int t = t_lo; t <= t_hi; ++t) {{
      const int ts = ({tile_start.format("t")}) * {U}, te = ({tile_start.format("t + 1")}) * {U};
      const int w0 = ts / per, w1 = (te - 1) / per;
      if (w1 > w0) {{
        if (tid == 0) dc_last = atomicAdd(&args.dc_arrive[t], 1) == w1 - w0;
        __syncthreads();
        const bool last = dc_last;
        __syncthreads();
        if (!last) continue;
        if (tid == 0) __hip_atomic_store(&args.dc_arrive[t], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // the other workgroups' partials: one wave invalidates the CU's L1 and the XCD's L2 for all
        if (wave == 0) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        __syncthreads();
      }}
      {{
        const int n = w1 - w0 + 1;
{self._merge_body("0", str(total))}
      }}
      __syncthreads();  // (dc_w and dc_lsum are the next tile's)
    }}
  }}
"""


def lower(plan: Plan, sch: Schedule, pipeline: Pipeline, m: DecodeMatch, name: str, trace: bool = False,
          cursor: bool = False, hardware: Optional[Dict[str, int]] = None) -> Program:
    """The decode program; its depth (K register sets and V LDS stages: steps fetched ahead) is the
    pipeline's input buffers, 2 to MAX_DEPTH. The `hardware` knob "fold" (0 or 1) puts the merge in the
    attention kernel."""
    if m.out.dtype.name != "bfloat16":
        raise KernelError("the gfx950 decode lowering stores bf16 outputs")
    knobs = dict(hardware or {})
    fold = bool(knobs.pop("fold", FOLD_DEFAULT))
    own = bool(knobs.pop("own", OWN_DEFAULT))
    sync = int(knobs.pop("sync", SYNC_DEFAULT))
    qrows = bool(knobs.pop("qrows", QROWS_DEFAULT if QROWS_DEFAULT is not None else cursor))
    if knobs:
        raise KernelError(f"the decode lowering has no hardware knobs {sorted(knobs)}")
    if sync < 0:
        raise KernelError(f"the decode knob sync is a count of steps (0: no barrier), not {sync}")
    depth = max(2, min(pipeline.input_buffers, MAX_DEPTH))
    return _Decode(plan, sch, m, name, trace, cursor, depth, fold, own, sync, qrows).program()
