"""Lowering of matmul-shaped loop nests: `acc += a[...] @ b[...]` (or `@ b[...].T`) over a reduction
loop, then a pointwise epilogue stored into one output tile. Dense and causal matmul
(examples/matmul.py:22-35 and examples/causal_matmul.py:23-40 of the reference) and the grouped matmul
whose right operand is a runtime window `w[group_expert[i // G], ...]` take this path.

The generated kernel is persistent: one workgroup per CU (256 threads, four waves in a 2x2 grid), each
walking its own list of work items. An item is a hardware tile of BM x BN outputs inside one spec tile
(the loop nest's tile), or a fill: a hardware tile whose value the schedule or the epilogue fixes without
computing (a tile the mask skips, or one the epilogue's `where` proves constant). For a compute item the
workgroup walks the spec tile's steps (arithmetic, or decoded from the step tables), each split into
BK-deep slices: operand slices go global -> registers -> LDS (a ring of `input_buffers` slots, swizzled
16-byte chunks; the right operand of `a @ b` transposed in registers on the way, so both MFMA operands
read K-contiguous), the next slices' loads in flight while the MFMAs of this one run
(`v_mfma_f32_32x32x16_bf16`, f32 accumulators in registers), and the epilogue computed per element where
the accumulator lives and stored as packed bf16.
"""

from __future__ import annotations

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
from .expr import Emitter, Interval, ctype, intervals, literal, nodes_between
from .program import Arg, Launch, Program, c_struct

__all__ = ["GemmMatch", "match", "lower"]

THREADS = 256
MFMA = 32  # 32x32x16 bf16 MFMA tiles


@dataclass
class GemmMatch:
    a: Operand
    b: Operand
    b_nt: bool  # `a @ b.T`: b's tile is (tn, tk), K-contiguous
    kvar: Optional[str]  # the reduction loop's variable (None: one step per tile)
    tm: int
    tn: int
    tk: int
    acc: Node  # the Node standing for the accumulator in the epilogue
    init: float
    out: Output
    value: Any  # the stored value (Node, or a number)


def _is(node: Any, op: str) -> bool:
    return isinstance(node, Node) and node.op == op


def _dot_of_loads(plan: Plan, node: Node) -> Optional[Tuple[Operand, Operand, bool]]:
    if not (_is(node, "dot") or _is(node, "dot_nt")) or node.dtype.name != "float32":
        return None
    a, b = node.args[0], node.args[1]
    if not (_is(a, "load") and _is(b, "load")):
        return None
    opa, opb = plan.operand(a.kwargs["operand"]), plan.operand(b.kwargs["operand"])
    if opa.tile.dtype.name != "bfloat16" or opb.tile.dtype.name != "bfloat16":
        return None
    if len(opa.tile.shape) != 2 or len(opb.tile.shape) != 2:
        return None
    return opa, opb, node.op == "dot_nt"


def match(plan: Plan) -> Optional[GemmMatch]:
    """The matmul this loop nest is, or None."""
    if len(plan.outputs) != 1 or len(plan.phases) > 1:
        return None
    out = plan.outputs[0]
    if len(out.tile.shape) != 2:
        return None
    last = plan.scopes["last"]
    value = last.stores.get(out.name)
    root = value.node if isinstance(value, jaxlite.Sym) else None
    if plan.phases:
        if set(plan.carried) != {name for name in plan.carried} or len(plan.carried) != 1:
            return None
        (acc,) = plan.carried
        body, seg0 = plan.scopes["body0"], plan.scopes["seg0"]
        new = body.values.get(acc)
        init = seg0.values.get(acc)
        if not (isinstance(new, jaxlite.Sym) and _is(new.node, "add")):
            return None
        x, y = new.node.args
        leaf = body.carried_in.get(acc)
        dot = y if x is leaf else x if y is leaf else None
        if dot is None:
            return None
        found = _dot_of_loads(plan, dot)
        if found is None:
            return None
        if isinstance(init, jaxlite.Sym) and _is(init.node, "full"):
            init_value = float(init.node.kwargs["value"])
        elif isinstance(init, (int, float)):
            init_value = float(init)
        else:
            return None
        acc_leaf = last.carried_in.get(acc)
        if acc_leaf is None or root is None:
            return None
        kvar = plan.phases[0].range.var
        if plan.phases[0].range.mask is not None and plan.phases[0].range.runtime is False and False:
            return None
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
    opa, opb, nt = found
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
    if kvar is None and (arow[1].loop is not None or bk.loop is not None):
        return None
    if out.dtype.name not in ("bfloat16", "float32"):
        return None
    return GemmMatch(opa, opb, nt, kvar, tm, tn, tk, acc_leaf, init_value, out, value)


@dataclass(frozen=True)
class HwTile:
    bm: int
    bn: int
    bk: int
    stages: int

    @property
    def lds(self) -> int:
        return self.stages * (self.bm + self.bn) * self.bk * 2


def hardware_tile(m: GemmMatch, pipeline: Pipeline) -> HwTile:
    """The workgroup's tile for a spec tile (tm, tn, tk) and the LDS ring depth the pipeline asks for."""
    bm, bn = min(m.tm, 256), min(m.tn, 256)
    if m.tm % bm or m.tn % bn or bm % 64 or bn % 64:
        raise KernelError(f"the gfx950 matmul lowering needs tiles that are multiples of 64 (got {m.tm} x {m.tn})")
    stages = max(2, pipeline.input_buffers)
    bk = 64
    while m.tk % bk and bk > 16:
        bk //= 2
    if m.tk % bk:
        raise KernelError(f"the gfx950 matmul lowering needs a reduction block that is a multiple of 16 (got {m.tk})")
    while stages * (bm + bn) * bk * 2 > gfx950.LDS_BUDGET:
        if bk > 32 and m.tk % (bk // 2) == 0:
            bk //= 2
        else:
            stages -= 1
    if stages < 2:
        raise KernelError("the matmul's tiles don't fit in LDS double-buffered")
    return HwTile(bm, bn, bk, stages)


def lower(plan: Plan, sch: Schedule, pipeline: Pipeline, m: GemmMatch, name: str) -> Program:
    hw = hardware_tile(m, pipeline)
    return _Gemm(plan, sch, pipeline, m, hw, name).program()


class _Gemm:
    def __init__(self, plan: Plan, sch: Schedule, pipeline: Pipeline, m: GemmMatch, hw: HwTile, name: str) -> None:
        self.plan, self.sch, self.pipeline, self.m, self.hw, self.name = plan, sch, pipeline, m, hw, name
        self.sub_m, self.sub_n = m.tm // hw.bm, m.tn // hw.bn
        self.subs = self.sub_m * self.sub_n
        self.tables: Dict[str, np.ndarray] = {}
        self.const_value: Optional[float] = None

    # ------------------------------------------------------------------ work items (host)

    def _items(self) -> Tuple[List[Tuple[int, int]], List[float], List[int]]:
        """Every (tile or fill, sub-tile | kind << 16), its weight (k slices) and locality group."""
        plan, sch, m, hw = self.plan, self.sch, self.m, self.hw
        items, weights, groups = [], [], []
        kslices = m.tk // hw.bk
        steps_of = None
        if sch.step_tables and not sch.runtime:
            offsets = static_tile_steps(sch)
            codes = sch.tables[STEP_CODE]
            steps_of = [int(offsets[t + 1] - offsets[t]) - int(np.sum((codes[offsets[t]:offsets[t + 1]] & 4) != 0))
                        for t in range(sch.pattern_tiles)]
        per_tile = sch.steps_per_tile if not sch.step_tables else None
        out_cols = [w for w in m.out.tile.windows if w.size is not None][1]
        col_loop = out_cols.loop
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
                col = (values.get(col_loop, 0) if col_loop else 0) + sn * hw.bn
                items.append((t, s | (kind << 16)))
                weights.append(weight)
                groups.append(col // max(hw.bn * 4, 1024))
        for f in range(sch.fills):
            blocks = sch.fill_blocks_at(f)
            values = {r.var: r.value(b) for r, b in zip(plan.parallel, blocks)}
            for s in range(self.subs):
                sn = s % self.sub_n
                col = (values.get(col_loop, 0) if col_loop else 0) + sn * hw.bn
                items.append((f, s | (1 << 16)))
                weights.append(0.25)
                groups.append(col // max(hw.bn * 4, 1024))
        if len(consts) > 1:  # one constant per kernel: compute the others
            keep = sorted(consts)[0]
            items = [(t, s & 0xFFFF) if (s >> 16) == 2 and self._constant_of(t, s) != keep else (t, s)
                     for t, s in items]
            consts = {keep}
        self.const_value = next(iter(consts)) if consts else None
        return items, weights, groups

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
        offsets, flat = work_lists(items, weights, groups, grid)
        self.tables["wg_items"] = offsets
        self.tables["items"] = flat.reshape(-1) if flat.size else np.zeros(2, np.int32)
        for name, t in sch.tables.items():
            if name in (STEP_TILE,):
                continue
            self.tables[name] = t
        if sch.step_tables and not sch.runtime:
            self.tables["tile_steps"] = static_tile_steps(sch)
        args = self._args()
        source = self._source(args)
        launch = Launch(self.name, args, (grid, 1, 1), (THREADS, 1, 1), 0)
        inputs = [(spec.shape, spec.dtype) for spec in plan.inputs]
        prog = Program(
            name=self.name, source=source, launches=[launch], outputs=[(m.out.shape, m.out.dtype)], inputs=inputs,
            tables=dict(self.tables), lds_bytes=hw.lds,
            notes={"family": "gemm", "hw_tile": (hw.bm, hw.bn, hw.bk), "stages": hw.stages, "grid": grid,
                   "items": len(items), "constant_items": sum(1 for _, s in items if (s >> 16) == 2)},
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
        if self.sch.runtime:
            args.append(Arg("workspace", "step_code", "const int* __restrict__", "rt_step_code"))
            args.append(Arg("workspace", "tile_steps", "const int* __restrict__", "rt_tile_steps"))
        return args

    def _source(self, args: List[Arg]) -> str:
        plan, sch, m, hw = self.plan, self.sch, self.m, self.hw
        bm, bn, bk, stages = hw.bm, hw.bn, hw.bk, hw.stages
        wtm, wtn = bm // 2, bn // 2
        mi, ni = wtm // MFMA, wtn // MFMA
        index = Index(plan, lambda v: f"lv_{v}")
        a_shape = plan.inputs[m.a.param].shape
        b_shape = plan.inputs[m.b.param].shape
        a_base, a_str = tile_base(m.a.tile, a_shape, index, lambda v: f"lv_{v}")
        b_base, b_str = tile_base(m.b.tile, b_shape, index, lambda v: f"lv_{v}")
        o_base, o_str = tile_base(m.out.tile, m.out.shape, index, lambda v: f"lv_{v}")
        if a_str[1] != 1 or b_str[-1] != 1 or o_str[1] != 1:
            raise KernelError("the gfx950 matmul lowering reads and writes tiles whose last dim is the array's last")
        lda, ldb, ldo = a_str[0], b_str[0], o_str[0]
        ca = bm * bk // 8 // THREADS  # 16-byte chunks of A per thread per slice
        if ca < 1:
            raise KernelError("matmul tile too small for a 256-thread workgroup")
        kvar = m.kvar
        phase = plan.phases[0].range if plan.phases else None
        kslices = m.tk // bk

        # How a tile's steps are found.
        if phase is None:
            steps_setup = ["const int nsteps = 1;"]
            step_k = "0"
        elif not sch.step_tables:
            steps_setup = [f"const int nsteps = {phase.count};"]
            step_k = f"({phase.start} + (s_) * {phase.step})"
        elif not sch.runtime:
            steps_setup = [
                f"const int tt_s = t % {sch.pattern_tiles};",
                "const int sbeg = args.tile_steps[tt_s], send = args.tile_steps[tt_s + 1];",
                f"const int nsteps = ((args.{STEP_CODE}[sbeg] >> 2) & 1) ? 0 : send - sbeg;",
            ]
            step_k = (f"({phase.start} + ((args.{STEP_CODE}[sbeg + (s_)] >> {CODE_SHIFT}) / {sch.iterations} / "
                      f"{sch.phase_radix}) * {phase.step})")
        else:
            steps_setup = [
                f"const int tt_s = t % {sch.pattern_tiles};",
                "const int sbeg = args.rt_tile_steps[tt_s], send = args.rt_tile_steps[tt_s + 1];",
                "const int nsteps = ((args.rt_step_code[sbeg] >> 2) & 1) ? 0 : send - sbeg;",
            ]
            step_k = (f"({phase.start} + ((args.rt_step_code[sbeg + (s_)] >> {CODE_SHIFT}) / {sch.iterations} / "
                      f"{sch.phase_radix}) * {phase.step})")

        # The epilogue, per accumulator element.
        def leaf(n: Node) -> Optional[str]:
            if n is m.acc:
                return "acc_v"
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
            if n.op in ("carried", "load"):
                raise KernelError("the matmul epilogue reads only the accumulator, positions and loop values")
            return None

        em = Emitter(leaf, m.out.tile.shape, prefix="e")
        if isinstance(m.value, jaxlite.Sym):
            result = em.emit(m.value.node)
        else:
            result = literal(m.value)
        epi_lines = em.lines
        out_bf16 = m.out.dtype.name == "bfloat16"

        struct = c_struct(f"{self.name}_args", args)
        A = f"args.{m.a.tile.array}"
        B = f"args.{m.b.tile.array}"
        O = f"args.{m.out.name}_out"
        fill_value = literal(m.out.fill if m.out.fill is not None else 0, m.out.dtype)
        const_value = literal(self.const_value if self.const_value is not None else 0.0, m.out.dtype)
        tile_decode = "\n        ".join(decode_tile(plan, sch, "t"))
        fill_decode = "\n        ".join(decode_fill(plan, sch, "t")) if sch.fills else ""
        fill_block = ""
        if sch.fills:
            fill_block = (f"if (kind == 1) {{\n      {{\n        {fill_decode}\n        const long long obase = {o_base};\n"
                          f"        {_store_constant(bm, bn, out_bf16, O, 'obase', ldo, fill_value)}\n      }}\n      continue;\n    }}")
        epi = "\n              ".join(epi_lines)
        setup = "\n        ".join(steps_setup)
        b_loader = self._b_loader(bn, bk, ldb, m.b_nt)

        return f"""// Generated by tilejax_amd for `{plan.nest.name}`: a persistent gfx950 matmul kernel.
// spec tile {m.tm} x {m.tn} x {m.tk}; hardware tile {bm} x {bn}, K slices of {bk}, {stages} LDS slots;
// {sch.tiles} tiles of {sch.total_tiles} ({sch.fills} filled), {sch.steps} steps.
{PRELUDE}
{struct}

extern "C" __global__ void __launch_bounds__({THREADS}) {self.name}(const {self.name}_args args) {{
  // LDS rings: A slices [BM][BK] and B slices transposed [BN][BK], 16-byte chunks XOR-swizzled by row.
  __shared__ __attribute__((aligned(16))) ak_u16 lds_a[{stages}][{bm * bk}];
  __shared__ __attribute__((aligned(16))) ak_u16 lds_b[{stages}][{bn * bk}];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int q_begin = args.wg_items[blockIdx.x], q_end = args.wg_items[blockIdx.x + 1];
  for (int q = q_begin; q < q_end; ++q) {{
    const int t = args.items[2 * q], code = args.items[2 * q + 1];
    const int sub = code & 0xffff, kind = code >> 16;
    const int sm = sub / {self.sub_n}, sn = sub % {self.sub_n};
    {fill_block}
    {tile_decode}
    const long long obase = {o_base};
    if (kind == 2) {{
      {_store_constant(bm, bn, out_bf16, O, "obase", ldo, const_value)}
      continue;
    }}
    {setup}
    const int total = nsteps * {kslices};
    ak_f32x16 acc[{mi}][{ni}];
#pragma unroll
    for (int i_ = 0; i_ < {mi}; ++i_)
#pragma unroll
      for (int j_ = 0; j_ < {ni}; ++j_)
#pragma unroll
        for (int r_ = 0; r_ < 16; ++r_) acc[i_][j_][r_] = {literal(m.init)};

    ak_u32x4 ra[{ca}];
    {b_loader["decl"]}
    // Fetch slice g (step g / {kslices}, K offset within it) into registers.
    auto fetch = [&](int g) {{
      const int s_ = g / {kslices}, kk = (g % {kslices}) * {bk};
      {"const int lv_" + kvar + " = " + step_k + ";" if kvar else ""}
      const __bf16* ap = {A} + ({a_base}) + (long long)(sm * {bm}) * {lda} + kk;
      const __bf16* bp = {B} + ({b_base}) + {("(long long)(sn * " + str(bn) + ") * " + str(ldb) + " + kk") if m.b_nt else ("(long long)kk * " + str(ldb) + " + sn * " + str(bn))};
#pragma unroll
      for (int c = 0; c < {ca}; ++c) {{
        const int chunk = tid + c * {THREADS};
        const int row = chunk / {bk // 8}, kc = chunk % {bk // 8};
        ra[c] = *(const ak_u32x4*)(ap + (long long)row * {lda} + kc * 8);
      }}
      {b_loader["fetch"]}
    }};
    auto stash = [&](int stage) {{
#pragma unroll
      for (int c = 0; c < {ca}; ++c) {{
        const int chunk = tid + c * {THREADS};
        const int row = chunk / {bk // 8}, kc = chunk % {bk // 8};
        *(ak_u32x4*)(&lds_a[stage][row * {bk} + ((kc ^ (row & 7)) * 8)]) = ra[c];
      }}
      {b_loader["stash"]}
    }};
    if (total > 0) {{
      fetch(0);
      stash(0);
      for (int p = 1; p < {stages - 1} && p < total; ++p) {{
        fetch(p);
        stash(p);
      }}
      if ({stages - 1} < total) fetch({stages - 1});
      __syncthreads();
      for (int g = 0; g < total; ++g) {{
        const int stage = g % {stages};
        const ak_u16* sa = lds_a[stage];
        const ak_u16* sb = lds_b[stage];
#pragma unroll
        for (int k16 = 0; k16 < {bk // 16}; ++k16) {{
          ak_bf16x8 af[{mi}], bf[{ni}];
          const int chunk = k16 * 2 + (lane >> 5);
#pragma unroll
          for (int i_ = 0; i_ < {mi}; ++i_) {{
            const int row = wm * {wtm} + i_ * 32 + (lane & 31);
            af[i_] = *(const ak_bf16x8*)(&sa[row * {bk} + ((chunk ^ (row & 7)) * 8)]);
          }}
#pragma unroll
          for (int j_ = 0; j_ < {ni}; ++j_) {{
            const int row = wn * {wtn} + j_ * 32 + (lane & 31);
            bf[j_] = *(const ak_bf16x8*)(&sb[row * {bk} + ((chunk ^ (row & 7)) * 8)]);
          }}
#pragma unroll
          for (int i_ = 0; i_ < {mi}; ++i_)
#pragma unroll
            for (int j_ = 0; j_ < {ni}; ++j_)
              acc[i_][j_] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bf[j_], af[i_], acc[i_][j_], 0, 0, 0);
        }}
        if (g + {stages - 1} < total) stash((g + {stages - 1}) % {stages});
        if (g + {stages} < total) fetch(g + {stages});
        __syncthreads();
      }}
    }}
    // Epilogue: the accumulator holds C transposed (lane: one row, four consecutive columns per group).
#pragma unroll
    for (int i_ = 0; i_ < {mi}; ++i_) {{
      const int er = sm * {bm} + wm * {wtm} + i_ * 32 + (lane & 31);
#pragma unroll
      for (int j_ = 0; j_ < {ni}; ++j_) {{
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {{
          const int ec0 = sn * {bn} + wn * {wtn} + j_ * 32 + g4 * 8 + (lane >> 5) * 4;
          float res[4];
#pragma unroll
          for (int e4 = 0; e4 < 4; ++e4) {{
            const int ec = ec0 + e4;
            const float acc_v = acc[i_][j_][g4 * 4 + e4];
            (void)ec; (void)er;
            {epi}
            res[e4] = (float)({result});
          }}
          {_store4(O, "obase", ldo, out_bf16)}
        }}
      }}
    }}
  }}
}}
"""

    def _b_loader(self, bn: int, bk: int, ldb: int, nt: bool) -> Dict[str, str]:
        if nt:  # b tile (tn, tk), K-contiguous: loaded like A
            cb = bn * bk // 8 // THREADS
            return {
                "decl": f"ak_u32x4 rb[{cb}];",
                "fetch": f"""#pragma unroll
      for (int c = 0; c < {cb}; ++c) {{
        const int chunk = tid + c * {THREADS};
        const int row = chunk / {bk // 8}, kc = chunk % {bk // 8};
        rb[c] = *(const ak_u32x4*)(bp + (long long)row * {ldb} + kc * 8);
      }}""",
                "stash": f"""#pragma unroll
      for (int c = 0; c < {cb}; ++c) {{
        const int chunk = tid + c * {THREADS};
        const int row = chunk / {bk // 8}, kc = chunk % {bk // 8};
        *(ak_u32x4*)(&lds_b[stage][row * {bk} + ((kc ^ (row & 7)) * 8)]) = rb[c];
      }}""",
            }
        # b tile (tk, tn), N-contiguous: 8x8 blocks loaded row by row, transposed in registers.
        blocks = (bk // 8) * (bn // 8)
        per = (blocks + THREADS - 1) // THREADS
        return {
            "decl": f"ak_u32x4 rb[{per}][8];",
            "fetch": f"""#pragma unroll
      for (int c = 0; c < {per}; ++c) {{
        const int blk = tid + c * {THREADS};
        if (blk < {blocks}) {{
          const int kb8 = blk / {bn // 8}, nb8 = blk % {bn // 8};
#pragma unroll
          for (int r = 0; r < 8; ++r) rb[c][r] = *(const ak_u32x4*)(bp + (long long)(kb8 * 8 + r) * {ldb} + nb8 * 8);
        }}
      }}""",
            "stash": f"""#pragma unroll
      for (int c = 0; c < {per}; ++c) {{
        const int blk = tid + c * {THREADS};
        if (blk < {blocks}) {{
          const int kb8 = blk / {bn // 8}, nb8 = blk % {bn // 8};
          ak_u32x4 col[8];
          ak_transpose8x8_b16(rb[c], col);
#pragma unroll
          for (int cc = 0; cc < 8; ++cc) {{
            const int row = nb8 * 8 + cc;
            *(ak_u32x4*)(&lds_b[stage][row * {bk} + ((kb8 ^ (row & 7)) * 8)]) = col[cc];
          }}
        }}
      }}""",
        }


def _cstore(dt: jaxlite.DType) -> str:
    return {"bfloat16": "__bf16", "float32": "float", "int32": "int", "float16": "_Float16"}.get(dt.name, "void")


def _store4(O: str, obase: str, ldo: int, bf16: bool) -> str:
    if bf16:
        return (f"*(ak_u32x2*)((ak_u16*){O} + {obase} + (long long)er * {ldo} + ec0) = "
                "ak_u32x2{ak_pack_bf16x2(res[0], res[1]), ak_pack_bf16x2(res[2], res[3])};")
    return f"*(ak_f32x4*)({O} + {obase} + (long long)er * {ldo} + ec0) = ak_f32x4{{res[0], res[1], res[2], res[3]}};"


def _store_constant(bm: int, bn: int, bf16: bool, O: str, obase: str, ldo: int, value: str) -> str:
    """Source storing one value over the workgroup's hardware sub-tile (sm, sn)."""
    if bf16:
        return (
            f"{{ const unsigned w_ = ak_bf16_bits((float)({value})) * 0x10001u; const ak_u32x4 v_ = {{w_, w_, w_, w_}};\n"
            f"        for (int c_ = tid; c_ < {bm * bn // 8}; c_ += {THREADS}) {{\n"
            f"          const int r_ = c_ / {bn // 8}, k_ = c_ % {bn // 8};\n"
            f"          *(ak_u32x4*)((ak_u16*){O} + {obase} + (long long)(sm * {bm} + r_) * {ldo} + sn * {bn} + k_ * 8) = v_;\n"
            "        } }"
        )
    return (
        f"{{ const float f_ = (float)({value}); const ak_f32x4 v_ = {{f_, f_, f_, f_}};\n"
        f"        for (int c_ = tid; c_ < {bm * bn // 4}; c_ += {THREADS}) {{\n"
        f"          const int r_ = c_ / {bn // 4}, k_ = c_ % {bn // 4};\n"
        f"          *(ak_f32x4*)({O} + {obase} + (long long)(sm * {bm} + r_) * {ldo} + sn * {bn} + k_ * 4) = v_;\n"
        "        } }"
    )
