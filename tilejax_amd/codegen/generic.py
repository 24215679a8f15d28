"""Lowering of any planned loop nest to one persistent gfx950 kernel that evaluates the traced tile code.

The matmul, flash and decode families lower the loop nests they recognise to hand-scheduled kernels. Every
other nest the planner accepts (several phases with values carried between them, per-head lists of
products, whole attention blocks, nests whose shapes a family doesn't take) lowers here, as the reference
lowers any nest to one kernel (src/autokernel/codegen.py:91-1755): correct for every nest, not tuned for any.

The kernel walks the same schedule the other families do: output tiles from per-workgroup work lists
(XCD-aware, longest first), masked tiles filled, each tile's steps from the static or device-built step
tables or arithmetically, phase after phase. Within a tile it runs the traced IR (plan.scopes) as passes
over elements by the workgroup's 256 threads:

- values every element of a consumer needs whole (products, reductions) and values that outlive their
  scope (carried values, the stored outputs) are materialized: a pass computes each element into the
  workgroup's tile memory (global memory, L2-resident), then a barrier;
- everything else (pointwise arithmetic, casts, `where`, iota, slices, reshapes, concatenation, stacking,
  broadcasts, tile reads through their windows, index-array elements) is fused into the pass that reads
  it, element by element (ElementEmitter), so it is never stored;
- a product accumulates in f32 (i64 for integers) with fused multiply-adds, a reduction in f32 for 16-bit
  inputs, as the reference semantics (jaxlite) compute them; results round to their dtypes.

A carried value's new value goes to a staging buffer first and is copied over the old one after every
update of the scope is computed, so updates that read other carried values see the old ones.
"""

from __future__ import annotations

import ast
import copy
import inspect
import math
from typing import Any, Callable, Dict, List, Optional, Sequence, Set, Tuple, Union

import numpy as np

from .. import gfx950, jaxlite
from ..errors import KernelError
from ..jaxlite import DType, Node
from ..pipeline import Pipeline
from ..plan import Plan
from ..schedule import CODE_SHIFT, STEP_CODE, Schedule
from ..syntax import bound, used
from .common import Index, decode_fill, decode_tile, static_tile_steps, strides, work_lists
from .device import PRELUDE
from .expr import ElementEmitter, _broadcast_index, _rounded, ctype, int_expr, literal
from .program import CLOCK_END, CLOCK_START, NOW, TRACE, TRACE_FIELDS, Arg, Launch, Program, c_struct

__all__ = ["lower", "lower_walk"]

THREADS = 256
MEM_BUDGET = 2 << 30  # bytes of tile memory over the whole grid
MAX_GRID = 1024
ALIGN = 256
MFMA_PRODUCTS = [True]  # bf16 products of 32-multiple shapes on the matrix cores (else scalar f32 FMAs)

# Ops a pass must compute whole before anything reads an element of them.
_WHOLE = {"reduce_max", "reduce_min", "reduce_sum", "reduce_mean", "reduce_any", "argmax", "dot", "dot_nt"}

_FUNCS = {
    "reduce_max": jaxlite.max, "reduce_min": jaxlite.min, "reduce_sum": jaxlite.sum, "reduce_mean": jaxlite.mean,
    "reduce_any": jaxlite.any_, "argmax": jaxlite.argmax, "dot": jaxlite.matmul, "dot_nt": jaxlite.matmul_nt,
    "stack": jaxlite.stack, "clip": jaxlite.clip, "pad": jaxlite.pad, "repeat": jaxlite.repeat,
    "concatenate": jaxlite.concatenate,
}


def _bound_args(n: Node) -> Dict[str, Any]:
    """A Node's arguments by parameter name, defaults filled in (positional or keyword as traced)."""
    fn = _FUNCS[n.op]
    fn = getattr(fn, "__wrapped__", fn)
    got = inspect.signature(fn).bind(*n.args, **n.kwargs)
    got.apply_defaults()
    return dict(got.arguments)


def _stype(dt: DType) -> str:
    """The C type a materialized value is kept in (16-bit floats as float: already rounded)."""
    if dt.kind == "f":
        return "double" if dt.itemsize == 8 else "float"
    if dt.kind == "b":
        return "int"
    if dt.kind == "u":
        return "unsigned long long" if dt.itemsize == 8 else "unsigned"
    return "long long" if dt.itemsize == 8 else "int"


def _unflatten(shape: Sequence[int], e: str, names: Sequence[str]) -> List[str]:
    lines = []
    for d, (n, s) in enumerate(zip(shape, strides(shape))):
        lines.append(f"const int {names[d]} = ({e} / {s}) % {n};" if n != 1 else f"const int {names[d]} = 0;")
    return lines


def _flat(shape: Sequence[int], idx: Sequence[str]) -> str:
    terms = [f"({i}) * {s}" for i, s, n in zip(idx, strides(shape), shape) if n != 1]
    return " + ".join(terms) if terms else "0"


class _Elements(ElementEmitter):
    """ElementEmitter plus the elementwise and data-movement ops of tile code the families don't meet."""

    def _at(self, n: Node, idx: Tuple[str, ...]) -> str:
        leaf = self.leaves(n, idx)
        if leaf is not None:
            return leaf
        op, a, dt, shape = n.op, n.args, n.dtype, tuple(n.shape)
        ct = ctype(dt)
        if op in ("exp", "exp2", "log", "sqrt", "rsqrt", "tanh", "reciprocal", "square", "sigmoid", "sign", "abs",
                  "gelu_exact"):
            x = self._val(a[0], idx, shape, dt)
            if dt.kind != "f":
                if op == "abs":
                    return f"(({x}) < 0 ? -({x}) : ({x}))"
                if op == "square":
                    return f"(({x}) * ({x}))"
                if op == "sign":
                    return f"((({x}) > 0) - (({x}) < 0))"
                raise KernelError(f"`{op}` of integers is not lowered")
            fn = {"exp": "ak_exp", "exp2": "ak_exp2", "log": "__logf", "sqrt": "sqrtf", "rsqrt": "ak_rsqrt",
                  "tanh": "tanhf", "reciprocal": "ak_rcp", "square": "ak_square", "sigmoid": "ak_sigmoid",
                  "sign": "ak_sign", "abs": "fabsf", "gelu_exact": "ak_gelu_exact"}[op]
            if dt.itemsize == 8:
                return f"(double){fn}((float)({x}))"
            return _rounded(f"{fn}((float)({x}))", dt)
        if op == "power":
            x, y = self._val(a[0], idx, shape, dt), self._val(a[1], idx, shape, dt)
            if dt.kind == "f":
                return _rounded(f"powf((float)({x}), (float)({y}))", dt)
            return f"ak_ipow({x}, {y})"
        if op in ("floor_divide", "remainder"):
            x, y = self._val(a[0], idx, shape, dt), self._val(a[1], idx, shape, dt)
            if dt.kind in "iu":
                return f"{'ak_floordiv' if op == 'floor_divide' else 'ak_floormod'}({x}, {y})"
            if op == "floor_divide":
                return _rounded(f"floorf((float)({x}) / (float)({y}))", dt)
            return _rounded(f"ak_fmod_floor((float)({x}), (float)({y}))", dt)
        if op == "bitwise_xor" or op == "left_shift" or op == "right_shift":
            return super()._at(n, idx)
        if op == "clip":
            b = _bound_args(n)
            v = self._val(b["x"], idx, shape, dt)
            lo, hi = b.get("lo"), b.get("hi")
            if dt.kind == "f":
                if lo is not None:
                    v = f"ak_maximum(({ct})({v}), ({ct})({self._val(lo, idx, shape, dt)}))"
                if hi is not None:
                    v = f"ak_minimum(({ct})({v}), ({ct})({self._val(hi, idx, shape, dt)}))"
                return _rounded(v, dt)
            if lo is not None:
                lv = self._val(lo, idx, shape, dt)
                v = f"((({v}) < ({lv})) ? ({lv}) : ({v}))"
            if hi is not None:
                hv = self._val(hi, idx, shape, dt)
                v = f"((({v}) > ({hv})) ? ({hv}) : ({v}))"
            return v
        if op == "stack":
            b = _bound_args(n)
            pieces, axis = list(b["xs"]), b["axis"] % len(shape)
            rest = tuple(i for k, i in enumerate(idx) if k != axis)
            texts = [self._at(p, rest) if isinstance(p, Node) else literal(p, dt) for p in pieces]
            expr = f"({ct})({texts[-1]})"
            for k in range(len(pieces) - 2, -1, -1):
                expr = f"((({idx[axis]}) == {k}) ? ({ct})({texts[k]}) : {expr})"
            return expr
        if op == "concatenate":
            b = _bound_args(n)
            pieces, axis = list(b["xs"]), b["axis"] % len(shape)
            expr, start, branches = None, 0, []
            for p in pieces:
                size = p.shape[axis]
                sub = tuple(f"(({i}) - {start})" if k == axis and start else i for k, i in enumerate(idx))
                branches.append((start + size, self._at(p, sub)))
                start += size
            expr = f"({ct})({branches[-1][1]})"
            for hi, text in reversed(branches[:-1]):
                expr = f"((({idx[axis]}) < {hi}) ? ({ct})({text}) : {expr})"
            return expr
        if op == "pad":
            b = _bound_args(n)
            src, widths = b["x"], b["pad_width"]
            widths = [tuple(w) for w in (widths if isinstance(widths[0], (tuple, list)) else [widths] * len(shape))]
            inside, inner = [], []
            for k, ((lo, _), d) in enumerate(zip(widths, src.shape)):
                inner.append(f"(({idx[k]}) - {lo})")
                inside.append(f"(({idx[k]}) >= {lo} && ({idx[k]}) < {lo + d})")
            cond = " && ".join(inside) or "true"
            return f"(({cond}) ? ({ct})({self._at(src, tuple(inner))}) : ({ct})0)"
        if op == "bitcast_convert_type":  # the same width: f32 <-> 32-bit integers, 16-bit <-> 16-bit
            src = a[0]
            v = self._at(src, idx)
            sdt = src.dtype
            if sdt.itemsize == 4 and dt.itemsize == 4:
                return f"__builtin_bit_cast({ct}, ({ctype(sdt)})({v}))" if sdt.kind != dt.kind else f"({ct})({v})"
            if sdt.itemsize == 2 and dt.itemsize == 2:
                return _from_bits16(_bits16(v, sdt), dt)
            raise KernelError(f"bitcast_convert_type from {sdt.name} to {dt.name} is not lowered")
        if op == "pairs":  # (..., 2, d) 16-bit -> (..., d) words: row 0 in the low half
            src = a[0]
            lo = _bits16(self._at(src, (*idx[:-1], "0", idx[-1])), src.dtype)
            hi = _bits16(self._at(src, (*idx[:-1], "1", idx[-1])), src.dtype)
            return f"((unsigned)({lo}) | ((unsigned)({hi}) << 16))"
        if op == "unpairs":  # (..., d) words -> (..., 2, d) 16-bit: row r from the word's half r
            w = self._at(a[0], (*idx[:-2], idx[-1]))
            return _from_bits16(f"((((unsigned)({w})) >> (16 * ({idx[-2]}))) & 0xFFFFu)", dt)
        if op == "getitem" and any(isinstance(k, Node) for k in (a[1] if isinstance(a[1], tuple) else (a[1],))):
            # an element chosen by a traced integer (`weights[c // D]`): clamped into its dim, as JAX clamps
            src, key = a[0], (a[1] if isinstance(a[1], tuple) else (a[1],))
            inner, k_out = [], 0
            for k, d in enumerate(src.shape):
                sel = key[k] if k < len(key) else slice(None)
                if isinstance(sel, Node):
                    inner.append(f"ak_index((int)({self._at(sel, ())}), {d})")
                elif isinstance(sel, slice):
                    start, _, step = sel.indices(d)
                    inner.append(f"({start} + ({idx[k_out]}) * {step})")
                    k_out += 1
                elif isinstance(sel, int):
                    inner.append(str(sel % d))
                else:
                    raise KernelError("tile values are indexed per element by integers, slices and traced integers")
            return self._at(src, tuple(inner))
        if op == "repeat":
            b = _bound_args(n)
            src, reps, axis = b["x"], b["repeats"], b["axis"]
            if axis is None:
                raise KernelError("jnp.repeat without an axis is not lowered")
            axis %= len(shape)
            inner = tuple(f"(({i}) / {reps})" if k == axis else i for k, i in enumerate(idx))
            return self._at(src, inner)
        return super()._at(n, idx)


class _Buffers:
    """The workgroup's tile memory: named buffers at fixed offsets."""

    def __init__(self) -> None:
        self.offsets: Dict[str, int] = {}
        self.types: Dict[str, str] = {}
        self.size = 0

    def add(self, name: str, count: int, stype: str) -> str:
        if name not in self.offsets:
            width = 8 if stype in ("double", "long long", "unsigned long long") else 4
            self.offsets[name] = self.size
            self.types[name] = stype
            self.size += -(-max(count, 1) * width // ALIGN) * ALIGN
        return name

    def ref(self, name: str) -> str:
        return f"(({self.types[name]}*)(ak_mem + {self.offsets[name]}))"


class _Generic:
    def __init__(self, plan: Plan, sch: Schedule, name: str, trace: bool) -> None:
        self.plan, self.sch, self.name, self.trace = plan, sch, name, trace
        if plan.repeats:
            raise KernelError(f"{plan.nest.name}: repeat loops are not lowered by the gfx950 backend yet")
        self.buf = _Buffers()
        self.index = Index(plan, lambda v: f"lv_{v}")
        self.tables: Dict[str, np.ndarray] = {}
        self.lines: List[str] = []
        phase_vars = {ph.range.var for ph in plan.phases}
        # reduction loops of one iteration and no mask run inline: their variable is their one value
        self.inline = {r.var: r.start for r in plan.reductions if r.var not in phase_vars}
        self.types: Dict[str, Any] = plan.carried  # the values a tile keeps in its memory between scopes
        for c, car in plan.carried.items():
            self.buf.add(f"c_{c}", math.prod(car.shape), _stype(car.dtype))

    # ------------------------------------------------------------------------------------------ elements

    def _load(self, n: Node, idx: Tuple[str, ...]) -> str:
        op = self.plan.operand(n.kwargs["operand"])
        shape = self.plan.inputs[op.param].shape
        terms, k = [], 0
        for w, dim, stride in zip(op.tile.windows, shape, strides(shape)):
            if w.index is not None:
                base = f"ak_index({self.index.read(w.index)}, {dim})"
            else:
                base = f"(lv_{w.loop} + {w.offset})" if w.loop else str(w.offset)
            if w.size is not None:
                coord = f"({base} + ({idx[k]}))"
                k += 1
            else:
                coord = base
            terms.append(f"(long long)({coord}) * {stride}")
        addr = " + ".join(terms) or "0"
        src = f"args.{op.tile.array}[{addr}]"
        dt = op.tile.dtype
        if dt.name == "bfloat16":
            return f"ak_bf16_to_f32({src})"
        if dt.name == "float16":
            return f"(float)__builtin_bit_cast(_Float16, {src})"
        return f"({ctype(dt)})({src})"

    def _elements(self, materialized: Dict[int, str]) -> _Elements:
        plan = self.plan

        def leaves(n: Node, idx: Tuple[str, ...]) -> Optional[str]:
            if n.id in materialized:
                name = materialized[n.id]
                return f"{self.buf.ref(name)}[{_flat(n.shape, idx)}]"
            if n.op == "load":
                return self._load(n, idx)
            if n.op == "carried":
                name = f"c_{n.kwargs['name']}"
                if name not in self.buf.offsets:
                    raise KernelError(f"carried value `{n.kwargs['name']}` has no type the plan settled")
                return f"{self.buf.ref(name)}[{_flat(n.shape, idx)}]"
            if n.op == "loop":
                return f"lv_{n.kwargs['var']}"
            if n.op == "index":  # an index-array element, clamped into the array as JAX clamps
                ix = plan.index(n.kwargs["array"])
                parts = [em.at(i, ()) if isinstance(i, Node) else literal(i) for i in n.args]
                flat = " + ".join(f"ak_index((int)({p}), {d}) * {s}"
                                  for p, s, d in zip(parts, strides(ix.shape), ix.shape)) or "0"
                return f"args.{ix.name}[{flat}]"
            if n.op in _WHOLE:
                raise KernelError(f"`{n.op}` read before it is computed")
            return None

        em = _Elements(leaves)
        return em

    # ------------------------------------------------------------------------------------------ passes

    def _pass(self, shape: Sequence[int], body: Callable[[Tuple[str, ...]], List[str]], ind: str) -> List[str]:
        """A loop of the workgroup's threads over every element of `shape`, then a barrier."""
        size = math.prod(shape)
        names = tuple(f"i{d}" for d in range(len(shape)))
        out = [f"{ind}for (int e_ = tid; e_ < {size}; e_ += {THREADS}) {{"]
        out += [f"{ind}  {line}" for line in _unflatten(shape, "e_", names)]
        out += [f"{ind}  {line}" for line in body(names)]
        out += [f"{ind}}}", f"{ind}__syncthreads();"]
        return out

    def _store_into(self, name: str, dt: DType, expr: str) -> str:
        return f"{self.buf.ref(name)}[e_] = ({self.buf.types[name]})({expr});"

    def _materialize(self, n: Node, materialized: Dict[int, str], ind: str) -> List[str]:
        """A pass computing every element of `n` into a buffer of its own."""
        name = self.buf.add(f"m{n.id}", math.prod(n.shape), _stype(n.dtype))
        if n.op in ("dot", "dot_nt"):
            code = self._dot(n, name, materialized, ind)
        elif n.op in _WHOLE:
            code = self._reduce(n, name, materialized, ind)
        else:
            em = self._elements(materialized)
            code = self._pass(n.shape, lambda idx: [self._store_into(name, n.dtype, em.at(n, idx))], ind)
        materialized[n.id] = name
        return code

    def _dot(self, n: Node, name: str, materialized: Dict[int, str], ind: str) -> List[str]:
        b = _bound_args(n)
        x, y = b["a"], b["b"]
        if not (isinstance(x, Node) and isinstance(y, Node)) or len(x.shape) != 2 or len(y.shape) != 2:
            raise KernelError("the generic gfx950 lowering takes products of two matrices")
        M, K = x.shape
        N = y.shape[0] if n.op == "dot_nt" else y.shape[1]
        em = self._elements(materialized)
        dt = n.dtype
        if (MFMA_PRODUCTS[0] and x.dtype.name == y.dtype.name == "bfloat16" and dt.name in ("float32", "bfloat16")
                and M % 32 == 0 and N % 32 == 0 and K % 16 == 0):
            return self._dot_mfma(n, name, x, y, M, N, K, em, ind)
        integer = dt.kind in "iub"
        acc_t = "long long" if integer else ("double" if dt.itemsize == 8 else "float")

        def body(idx: Tuple[str, ...]) -> List[str]:
            i, j = idx
            xv = em.at(x, (i, "kk_"))
            yv = em.at(y, (j, "kk_")) if n.op == "dot_nt" else em.at(y, ("kk_", j))
            if integer:
                step = f"acc_ += (long long)({xv}) * (long long)({yv});"
            elif acc_t == "double":
                step = f"acc_ = __builtin_fma((double)({xv}), (double)({yv}), acc_);"
            else:
                step = f"acc_ = __builtin_fmaf((float)({xv}), (float)({yv}), acc_);"
            res = "acc_" if integer or dt.kind != "f" else _rounded("acc_", dt)
            return [f"{acc_t} acc_ = 0;", f"for (int kk_ = 0; kk_ < {K}; ++kk_) {{ {step} }}",
                    self._store_into(name, dt, res)]

        return self._pass((M, N), body, ind)

    def _dot_mfma(self, n: Node, name: str, x: Node, y: Node, M: int, N: int, K: int, em: "_Elements",
                  ind: str) -> List[str]:
        """A product of bf16 matrices on the matrix cores: each wave takes 32 x 32 blocks of the output in
        turn and accumulates them in f32 over K in steps of 16 (v_mfma_f32_32x32x16_bf16); a lane computes
        the 8 operand elements its fragments hold (whatever fuses into the operands) and packs them. C's
        element (i, j) of a block is lane j % 32's register 8 (r / 4) + 4 (lane / 32) + r % 4 == i."""
        nt = n.op == "dot_nt"
        blocks_n = N // 32
        xa = em.at(x, ("(ib_ + (lane_ & 31))", "(k0_ + 8 * (lane_ >> 5) + e_)"))
        yb = (em.at(y, ("(jb_ + (lane_ & 31))", "(k0_ + 8 * (lane_ >> 5) + e_)")) if nt
              else em.at(y, ("(k0_ + 8 * (lane_ >> 5) + e_)", "(jb_ + (lane_ & 31))")))
        out = self.buf.ref(name)
        res = "acc_[r_]" if n.dtype.name == "float32" else _rounded("acc_[r_]", n.dtype)
        return [
            f"{ind}{{ const int lane_ = tid & 63, wave_ = tid >> 6;",
            f"{ind}  for (int blk_ = wave_; blk_ < {(M // 32) * blocks_n}; blk_ += {THREADS // 64}) {{",
            f"{ind}    const int ib_ = (blk_ / {blocks_n}) * 32, jb_ = (blk_ % {blocks_n}) * 32;",
            f"{ind}    ak_f32x16 acc_ = {{}};",
            f"{ind}    for (int k0_ = 0; k0_ < {K}; k0_ += 16) {{",
            f"{ind}      unsigned pa_[4], pb_[4];",
            f"{ind}      #pragma unroll",
            f"{ind}      for (int e2_ = 0; e2_ < 4; ++e2_) {{",
            f"{ind}        float va_[2], vb_[2];",
            f"{ind}        #pragma unroll",
            f"{ind}        for (int h_ = 0; h_ < 2; ++h_) {{",
            f"{ind}          const int e_ = 2 * e2_ + h_;",
            f"{ind}          va_[h_] = (float)({xa});",
            f"{ind}          vb_[h_] = (float)({yb});",
            f"{ind}        }}",
            f"{ind}        pa_[e2_] = ak_pack_bf16x2(va_[0], va_[1]);",
            f"{ind}        pb_[e2_] = ak_pack_bf16x2(vb_[0], vb_[1]);",
            f"{ind}      }}",
            f"{ind}      acc_ = __builtin_amdgcn_mfma_f32_32x32x16_bf16(",
            f"{ind}          __builtin_bit_cast(ak_bf16x8, ak_u32x4{{pa_[0], pa_[1], pa_[2], pa_[3]}}),",
            f"{ind}          __builtin_bit_cast(ak_bf16x8, ak_u32x4{{pb_[0], pb_[1], pb_[2], pb_[3]}}), acc_, 0, 0, 0);",
            f"{ind}    }}",
            f"{ind}    #pragma unroll",
            f"{ind}    for (int r_ = 0; r_ < 16; ++r_)",
            f"{ind}      {out}[(ib_ + 8 * (r_ >> 2) + 4 * (lane_ >> 5) + (r_ & 3)) * {N} + jb_ + (lane_ & 31)] = "
            f"({self.buf.types[name]})({res});",
            f"{ind}  }}",
            f"{ind}}}",
            f"{ind}__syncthreads();",
        ]

    def _reduce(self, n: Node, name: str, materialized: Dict[int, str], ind: str) -> List[str]:
        b = _bound_args(n)
        src = b["x"]
        if not isinstance(src, Node):
            raise KernelError(f"`{n.op}` of a constant is not lowered")
        nd = len(src.shape)
        axes = b.get("axis")
        axes = tuple(range(nd)) if axes is None else ((axes,) if isinstance(axes, int) else tuple(axes))
        axes = tuple(sorted(a % nd for a in axes))
        keep = bool(b.get("keepdims", False))
        em = self._elements(materialized)
        red_shape = [src.shape[a] for a in axes]
        count = math.prod(red_shape)
        dt, sdt = n.dtype, src.dtype
        op = n.op
        wide = sdt.kind == "f" and sdt.itemsize == 8

        def body(idx: Tuple[str, ...]) -> List[str]:
            # the source index: output dims where kept, reduced dims from the inner counter
            out_dims = [d for d in range(nd) if d not in axes]
            inner = [None] * nd
            if keep:
                for d in out_dims:
                    inner[d] = idx[d]
            else:
                for k, d in enumerate(out_dims):
                    inner[d] = idx[k]
            lines = []
            for k, (a, s) in enumerate(zip(axes, strides(red_shape))):
                inner[a] = f"r{k}_"
            unflat = [f"const int r{k}_ = (rr_ / {s}) % {red_shape[k]};" for k, s in enumerate(strides(red_shape))]
            v = em.at(src, tuple(inner))
            if op == "reduce_sum" or op == "reduce_mean":
                if sdt.kind == "f":
                    acc_t, init, step = ("double" if wide else "float"), "0", f"acc_ += ({'double' if wide else 'float'})({v});"
                elif sdt.kind == "b":
                    acc_t, init, step = "long long", "0", f"acc_ += ({v}) ? 1 : 0;"
                else:
                    acc_t, init, step = "long long", "0", f"acc_ += (long long)({v});"
                if op == "reduce_mean":
                    res = f"(({'double' if wide else 'float'})acc_ / {count})"
                    res = _rounded(res, dt) if dt.kind == "f" else res
                else:
                    res = _rounded("acc_", dt) if dt.kind == "f" else "acc_"
            elif op in ("reduce_max", "reduce_min"):
                fn = "ak_maximum" if op == "reduce_max" else "ak_minimum"
                if sdt.kind == "f":
                    acc_t = "double" if wide else "float"
                    init = "(-__builtin_inff())" if op == "reduce_max" else "__builtin_inff()"
                    step = f"acc_ = {fn}(acc_, ({acc_t})({v}));"
                else:
                    acc_t = "long long"
                    init = "(-(1LL << 62))" if op == "reduce_max" else "(1LL << 62)"
                    cmp = ">" if op == "reduce_max" else "<"
                    step = f"{{ const long long v_ = (long long)({v}); if (v_ {cmp} acc_) acc_ = v_; }}"
                res = "acc_"
            elif op == "reduce_any":
                acc_t, init, step, res = "bool", "false", f"acc_ = acc_ || (({v}) != 0);", "acc_"
            elif op == "argmax":
                if len(axes) != 1:
                    raise KernelError("argmax over several axes is not lowered")
                acc_t, init = "float", "(-__builtin_inff())"
                step = f"{{ const float v_ = (float)({v}); if (v_ > acc_ || (v_ != v_ && acc_ == acc_)) {{ acc_ = v_; at_ = rr_; }} }}"
                res = "at_"
            else:
                raise KernelError(f"`{op}` is not lowered")
            lines += [f"{acc_t} acc_ = {init};", "int at_ = 0; (void)at_;",
                      f"for (int rr_ = 0; rr_ < {count}; ++rr_) {{ {' '.join(unflat)} {step} }}",
                      self._store_into(name, dt, res)]
            return lines

        return self._pass(n.shape, body, ind)

    # ------------------------------------------------------------------------------------------ scopes

    def _needed(self, roots: Sequence[Node]) -> List[Node]:
        """Every Node the roots read, each after its inputs."""
        order: List[Node] = []
        seen: Set[int] = set()
        stack: List[Tuple[Node, bool]] = [(r, False) for r in reversed(list(roots))]
        while stack:
            node, done = stack.pop()
            if done:
                order.append(node)
                continue
            if node.id in seen:
                continue
            seen.add(node.id)
            stack.append((node, True))
            for i in reversed(node.inputs()):
                if i.id not in seen:
                    stack.append((i, False))
        return order

    def _scope(self, key: str, ind: str, store: bool = False) -> List[str]:
        """The code of one traced scope: its passes, then its carried values' updates (and, for the last
        scope, the output stores)."""
        plan = self.plan
        scope = plan.scopes[key]
        updates = self._updates(scope, [c for c in plan.carried if c in scope.values])
        stores = [(o, scope.stores[o.name]) for o in plan.outputs] if store else []
        return self._emit(updates, stores, ind)

    @staticmethod
    def _updates(scope: Any, names: Sequence[str]) -> List[Tuple[str, Any]]:
        """The kept values a scope assigns anew (not those it leaves as they came in)."""
        out = []
        for c in names:
            v = scope.values[c]
            leaf = scope.carried_in.get(c)
            if isinstance(v, jaxlite.Sym) and leaf is not None and v.node is leaf:
                continue  # unchanged
            out.append((c, v))
        return out

    def _emit(self, updates: List[Tuple[str, Any]], stores: List[Tuple[Any, Any]], ind: str) -> List[str]:
        """Passes computing what the updates and stores read, the updates (staged), the stores, then the
        staged values copied over the kept ones."""
        roots = [v.node for _, v in updates if isinstance(v, jaxlite.Sym)]
        roots += [val.node for _, val in stores if isinstance(val, jaxlite.Sym)]
        out: List[str] = []
        materialized: Dict[int, str] = {}
        order = self._needed(roots)
        # every whole-value op, and the operands of products that aren't cheap to read, get a pass
        force: Set[int] = set()
        for n in order:
            if n.op in ("dot", "dot_nt"):
                for operand in n.args[:2]:
                    if isinstance(operand, Node) and operand.op not in ("load", "carried", "full", "iota"):
                        force.add(operand.id)
        for n in order:
            if n.op in _WHOLE or n.id in force:
                out += self._materialize(n, materialized, ind)
        # carried updates: staged, then copied over the old values
        em = self._elements(materialized)
        staged = []
        for c, v in updates:
            car = self.types[c]
            stage = self.buf.add(f"u_{c}", math.prod(car.shape), _stype(car.dtype))
            staged.append((c, stage))
            if isinstance(v, jaxlite.Sym):
                src = v.node
                expr = lambda idx, src=src, car=car: em.at(src, _broadcast_index(src.shape, car.shape, idx))
            else:
                expr = lambda idx, v=v, car=car: literal(v, car.dtype)
            out += self._pass(car.shape, lambda idx, stage=stage, car=car, expr=expr:
                              [self._store_into(stage, car.dtype, _cast(expr(idx), car.dtype))], ind)
        # the stores read the scope's values, which read the carried values as they were at its start:
        # they go before the staged values are copied over those
        for o, val in stores:
            out += self._output_store(o, val, em, ind)
        if staged:
            lines = []
            for c, stage in staged:
                car = self.types[c]
                size = math.prod(car.shape)
                lines.append(f"{ind}for (int e_ = tid; e_ < {size}; e_ += {THREADS}) "
                             f"{self.buf.ref('c_' + c)}[e_] = {self.buf.ref(stage)}[e_];")
            out += lines + [f"{ind}__syncthreads();"]
        return out

    def _output_store(self, o: Any, val: Any, em: _Elements, ind: str) -> List[str]:
        tile = o.tile
        kept = tile.shape
        shape = o.shape

        def body(idx: Tuple[str, ...]) -> List[str]:
            terms, k = [], 0
            for w, dim, stride in zip(tile.windows, shape, strides(shape)):
                base = f"(lv_{w.loop} + {w.offset})" if w.loop else str(w.offset)
                if w.size is not None:
                    coord = f"({base} + ({idx[k]}))"
                    k += 1
                else:
                    coord = base
                terms.append(f"(long long)({coord}) * {stride}")
            addr = " + ".join(terms) or "0"
            if isinstance(val, jaxlite.Sym):
                v = em.at(val.node, _broadcast_index(val.node.shape, kept, idx))
            else:
                v = literal(val, o.dtype)
            return [_write(f"args.{o.name}_out", addr, o.dtype, v)]

        return self._pass(kept, body, ind)

    def _fill(self, ind: str) -> List[str]:
        out = []
        for o in self.plan.outputs:
            fill = o.fill if o.fill is not None else 0

            def body(idx: Tuple[str, ...], o=o, fill=fill) -> List[str]:
                terms, k = [], 0
                for w, dim, stride in zip(o.tile.windows, o.shape, strides(o.shape)):
                    base = f"(lv_{w.loop} + {w.offset})" if w.loop else str(w.offset)
                    coord = f"({base} + ({idx[k]}))" if w.size is not None else base
                    k += w.size is not None
                    terms.append(f"(long long)({coord}) * {stride}")
                return [_write(f"args.{o.name}_out", " + ".join(terms) or "0", o.dtype, literal(fill, o.dtype))]

            out += self._pass(o.tile.shape, body, ind)
        return out

    # ------------------------------------------------------------------------------------------ program

    def _steps(self, ind: str) -> List[str]:
        """The tile's steps, phase by phase: each step's body (unless empty), each phase's code after its
        last step."""
        plan, sch = self.plan, self.sch
        out: List[str] = []
        if not plan.phases:
            return out
        if not sch.step_tables and not sch.runtime:
            for p, ph in enumerate(plan.phases):
                r = ph.range
                out.append(f"{ind}for (int kb_ = 0; kb_ < {r.count}; ++kb_) {{")
                out.append(f"{ind}  const int lv_{r.var} = {r.start} + kb_ * {r.step}; (void)lv_{r.var};")
                out += self._scope(f"body{p}", ind + "  ")
                out.append(f"{ind}}}")
                out += self._scope(f"end{p}", ind, store=(p == len(plan.phases) - 1))
            return out
        codes, offs = ((f"args.{STEP_CODE}", "args.tile_steps") if not sch.runtime
                       else ("args.rt_step_code", "args.rt_tile_steps"))
        out += [f"{ind}const int tt_s = t % {sch.pattern_tiles};",
                f"{ind}const int sbeg = {offs}[tt_s], send = {offs}[tt_s + 1];",
                f"{ind}for (int st_ = sbeg; st_ < send; ++st_) {{",
                f"{ind}  const int code_ = {codes}[st_];",
                f"{ind}  const int pb_ = (code_ >> {CODE_SHIFT}) / {sch.iterations};",
                f"{ind}  const int ph_ = pb_ % {sch.phase_radix}, kb_ = pb_ / {sch.phase_radix};"]
        last = len(plan.phases) - 1
        for p, ph in enumerate(plan.phases):
            r = ph.range
            out.append(f"{ind}  if (ph_ == {p}) {{")
            out.append(f"{ind}    const int lv_{r.var} = {r.start} + kb_ * {r.step}; (void)lv_{r.var};")
            out.append(f"{ind}    if (!(code_ & 4)) {{")
            out += self._scope(f"body{p}", ind + "      ")
            out.append(f"{ind}    }}")
            out.append(f"{ind}    if (code_ & 1) {{")
            out += self._scope(f"end{p}", ind + "      ", store=(p == last))
            out.append(f"{ind}    }}")
            out.append(f"{ind}  }}")
        out.append(f"{ind}}}")
        return out

    def program(self) -> Program:
        plan, sch = self.plan, self.sch
        # one work item per tile that runs (kind 0) or a mask skips (kind 1)
        items, weights, groups = [], [], []
        per_tile = sch.steps_per_tile
        for t in range(sch.tiles):
            items.append((t, 0))
            weights.append(float(per_tile) + 1.0)
            groups.append(t)
        for f in range(sch.fills):
            items.append((f, 1))
            weights.append(0.25)
            groups.append(f)
        tile_code = self._scope("seg0", "    ", store=not plan.phases) + self._steps("    ")
        fill_code = self._fill("      ") if sch.fills else []
        per_wg = max(self.buf.size, ALIGN)
        grid = max(1, min(len(items), MAX_GRID, MEM_BUDGET // per_wg))
        if per_wg > MEM_BUDGET:
            raise KernelError(f"{plan.nest.name}: a tile needs {per_wg} bytes of tile memory, more than the generic "
                              f"lowering's {MEM_BUDGET}")
        offsets, flat = work_lists(items, weights, groups, grid)
        self.tables["wg_items"] = offsets
        self.tables["items"] = flat.reshape(-1) if flat.size else np.zeros(2, np.int32)
        for name, tab in sch.tables.items():
            if name.startswith("tile_") or name.startswith("fill_") or name == STEP_CODE:
                self.tables[name] = tab
        if sch.step_tables and not sch.runtime:
            self.tables["tile_steps"] = static_tile_steps(sch)
        args = self._args()
        src = self._source(args, tile_code, fill_code)
        workspace = {"gx_mem": per_wg * grid}
        if self.trace:
            workspace[TRACE] = grid * TRACE_FIELDS * 8
        prog = Program(
            name=self.name, source=src, launches=[Launch(self.name, args, (grid, 1, 1), (THREADS, 1, 1), 0)],
            outputs=[(o.shape, o.dtype) for o in plan.outputs], inputs=[(s.shape, s.dtype) for s in plan.inputs],
            tables=dict(self.tables), workspace=workspace, lds_bytes=0,
            notes={"family": "generic", "grid": grid, "items": len(items), "tile_memory": per_wg,
                   "trace_workgroups": grid if self.trace else 0, "trace_slots": grid,
                   "slices_per_step": 1})
        if sch.runtime:
            from .steps import attach_step_builder

            attach_step_builder(prog, plan, sch, self.name)
        return prog

    def _args(self) -> List[Arg]:
        plan = self.plan
        args = []
        for k, name in enumerate(plan.nest.params):
            dt = plan.inputs[k].dtype
            args.append(Arg("input", k, f"const {_ctype_in(dt)}* __restrict__", name))
        for o in plan.outputs:
            args.append(Arg("output", plan.outputs.index(o), f"{_ctype_in(o.dtype)}* __restrict__", f"{o.name}_out"))
        for name in self.tables:
            args.append(Arg("table", name, "const int* __restrict__", name))
        args.append(Arg("workspace", "gx_mem", "char* __restrict__", "gx_mem"))
        if self.trace:
            args.append(Arg("workspace", TRACE, "unsigned long long* __restrict__", TRACE))
        if self.sch.runtime:
            args.append(Arg("workspace", "step_code", "const int* __restrict__", "rt_step_code"))
            args.append(Arg("workspace", "tile_steps", "const int* __restrict__", "rt_tile_steps"))
        return args

    def _source(self, args: List[Arg], tile_code: List[str], fill_code: List[str]) -> str:
        plan, sch = self.plan, self.sch
        inline = "\n  ".join(f"const int lv_{v} = {val}; (void)lv_{v};" for v, val in self.inline.items())
        decode = "\n    ".join(decode_tile(plan, sch, "t"))
        fdecode = "\n      ".join(decode_fill(plan, sch, "t")) if sch.fills else ""
        fills = ""
        if fill_code:
            fills = f"""    if (kind == 1) {{
      {fdecode}
{chr(10).join(fill_code)}
      continue;
    }}"""
        t0 = f"{CLOCK_START} const unsigned long long tr_0 = {NOW};" if self.trace else ""
        t1 = (f"if (tid == 0) {{ unsigned long long* tr = args.{TRACE} + blockIdx.x * {TRACE_FIELDS}; tr[0] = 0; "
              f"tr[1] = 0; tr[2] = 0; tr[3] = {NOW} - tr_0; tr[4] = q_end - q_begin; {CLOCK_END} }}" if self.trace else "")
        return f"""// Generated by tilejax_amd for `{plan.nest.name}`: the generic gfx950 lowering (tile code evaluated
// pass by pass in each workgroup's tile memory of {self.buf.size} bytes).
{PRELUDE}
AK_INLINE float ak_gelu_exact(float x) {{ return 0.5f * x * (1.0f + erff(x * 0.70710678118654752f)); }}
AK_INLINE int ak_ipow(int b, int e) {{ int r = 1; for (int k = 0; k < e; ++k) r *= b; return e < 0 ? 0 : r; }}
AK_INLINE float ak_fmod_floor(float a, float b) {{ const float r = fmodf(a, b); return (r != 0.0f && ((r < 0.0f) != (b < 0.0f))) ? r + b : r; }}
{c_struct(f"{self.name}_args", args)}
extern "C" __global__ void __launch_bounds__({THREADS}) {self.name}(const {self.name}_args args) {{
  const int tid = threadIdx.x;
  char* ak_mem = args.gx_mem + (long long)blockIdx.x * {max(self.buf.size, ALIGN)};
  (void)ak_mem;
  {inline}
  {t0}
  const int q_begin = args.wg_items[blockIdx.x], q_end = args.wg_items[blockIdx.x + 1];
  for (int q = q_begin; q < q_end; ++q) {{
    const int t = args.items[2 * q], kind = args.items[2 * q + 1];
    (void)kind;
{fills}
    {decode}
{chr(10).join(tile_code)}
    __syncthreads();
  }}
  {t1}
}}
"""


class _Walk(_Generic):
    """The generic kernel for a plan of the tile as written (tilejax_amd/walk.py): each tile walks the
    plan's tree of blocks, straight-line code as passes, reduction and repeat loops as loops whose bounds and
    masks it evaluates as it runs (from loop variables, constants, index-array elements and elements of
    index arrays the tile code computed), reading windows whose starts it evaluates the same way (clamped
    into their dims, as JAX clamps) and storing outputs where the stores' windows say. Before it, a launch
    fills every output: with its allocation's value, or, for an input updated in place, with that input.
    A runtime count of tiles is counted on the device; the kernel is persistent over tiles either way."""

    def __init__(self, plan: Plan, sch: Schedule, name: str, trace: bool) -> None:
        self.plan, self.sch, self.name, self.trace = plan, sch, name, trace
        self.buf = _Buffers()
        self.index = Index(plan, lambda v: f"lv_{v}")
        self.tables = {}
        self.lines = []
        self.inline = {}
        self.types = plan.kept
        for c, car in plan.kept.items():
            self.buf.add(f"c_{c}", math.prod(car.shape), _stype(car.dtype))
        nest = plan.nest
        self.loop_vars = {loop.var for loop in nest.loops}
        self.runtime = self.loop_vars | {ix.name for ix in plan.indices} | bound(nest.tile)

    # ------------------------------------------------------------------------------------------ integers

    def _fold(self, node: ast.expr) -> ast.expr:
        """`node` with every subexpression that reads nothing the kernel learns as it runs evaluated now."""
        plan, runtime = self.plan, self.runtime

        class Fold(ast.NodeTransformer):
            def visit(self, n: ast.AST) -> ast.AST:
                if isinstance(n, ast.expr) and not isinstance(n, ast.Constant) and not used(n) & runtime:
                    value = plan.eval(n)
                    if isinstance(value, (bool, np.bool_)):
                        return ast.copy_location(ast.Constant(bool(value)), n)
                    if isinstance(value, (int, np.integer)):
                        return ast.copy_location(ast.Constant(int(value)), n)
                return self.generic_visit(n)

        return Fold().visit(copy.deepcopy(node))  # type: ignore[return-value]

    def _name(self, v: str) -> Optional[str]:
        if v in self.loop_vars:
            return f"lv_{v}"
        value = self.plan.env.get(v)
        if isinstance(value, (bool, np.bool_)):
            return "true" if value else "false"
        if isinstance(value, (int, np.integer)):
            return str(int(value))
        return None

    def _element(self, sub: ast.Subscript) -> str:
        """An element of an index array (an input) or of an int32 array the tile keeps, clamped into it."""
        if not isinstance(sub.value, ast.Name):
            raise KernelError(f"`{ast.unparse(sub)}` isn't an element of an index array")
        name = sub.value.id
        if name in {ix.name for ix in self.plan.indices}:
            shape, ref = self.plan.index(name).shape, f"args.{name}"
        elif name in self.plan.kept and self.plan.kept[name].dtype.kind in "iu":
            shape, ref = self.plan.kept[name].shape, self.buf.ref(f"c_{name}")
        else:
            what = (f"{self.plan.kept[name].dtype.name} values" if name in self.plan.kept else "a value no later part keeps")
            raise KernelError(f"`{ast.unparse(sub)}`: an element placing a window comes from an index array or an int32 "
                              f"array the tile code computed and keeps; `{name}` is {what}")
        dims = list(sub.slice.elts) if isinstance(sub.slice, ast.Tuple) else [sub.slice]
        if len(dims) != len(shape) or any(isinstance(d, ast.Slice) for d in dims):
            raise KernelError(f"`{ast.unparse(sub)}`: index every dim of `{name}` with an integer")
        flat = " + ".join(f"ak_index({self._int(d)}, {n}) * {st}"
                          for d, n, st in zip(dims, shape, strides(shape))) or "0"
        return f"{ref}[{flat}]"

    def _int(self, node: Union[int, ast.expr]) -> str:
        if isinstance(node, int):
            return str(node)
        return f"(int)({int_expr(self._fold(node), self._name, self._element)})"

    # ------------------------------------------------------------------------------------------ windows

    def _gather(self, sub: ast.Subscript, e: str, dim: int) -> str:
        """Element e of `ids[..., a : a + n]`, an index into a dim of `dim` (clamped into both)."""
        name = sub.value.id  # type: ignore[attr-defined]
        dims = list(sub.slice.elts) if isinstance(sub.slice, ast.Tuple) else [sub.slice]
        if name in {ix.name for ix in self.plan.indices}:
            shape, ref = self.plan.index(name).shape, f"args.{name}"
        else:
            shape, ref = self.plan.kept[name].shape, self.buf.ref(f"c_{name}")
        terms = []
        for d, n, st in zip(dims, shape, strides(shape)):
            at = f"({self._int(d.lower)} + ({e}))" if isinstance(d, ast.Slice) else self._int(d)  # type: ignore[arg-type]
            terms.append(f"ak_index({at}, {n}) * {st}")
        return f"{ref}[{' + '.join(terms)}]"

    def _coords(self, acc: Any, shape: Sequence[int], idx: Tuple[str, ...], store: bool
                ) -> Tuple[str, List[str]]:
        """The flat element address of `acc` at tile index `idx`, and the conditions a store writes under
        (rows before `stop`; gathered elements and element indices inside the dim once a negative one counts
        from the end: JAX drops updates out of the array). Reads clamp into the dim instead."""
        terms, conds, k = [], [], 0
        for d, dim, stride in zip(acc.dims, shape, strides(shape)):
            if d.gather is not None:
                g = self._gather(d.gather, idx[k], dim)
                k += 1
                if store:
                    coord = f"ak_wrap({g}, {dim})"
                    conds.append(f"(unsigned)({coord}) < {dim}u")
                else:
                    coord = f"ak_index({g}, {dim})"
            elif d.size is None:
                if isinstance(d.start, int):
                    coord = self._int(d.start)
                elif store:  # an update at an index out of the dim is dropped
                    coord = f"ak_wrap({self._int(d.start)}, {dim})"
                    conds.append(f"(unsigned)({coord}) < {dim}u")
                else:
                    coord = f"ak_index({self._int(d.start)}, {dim})"
            elif d.stop is not None:
                at = f"({self._int(d.start)} + ({idx[k]}))"
                k += 1
                if store:
                    conds.append(f"{at} < {self._int(d.stop)} && (unsigned){at} < {dim}u")
                    coord = at
                else:
                    coord = f"ak_clamp({at}, 0, {dim - 1})"
            else:
                base = (self._int(d.start) if isinstance(d.start, int)
                        else f"ak_clamp({self._int(d.start)}, 0, {dim - d.size})")
                coord = f"({base} + ({idx[k]}))"
                k += 1
            terms.append(f"(long long)({coord}) * {stride}")
        return " + ".join(terms) or "0", conds

    def _load(self, n: Node, idx: Tuple[str, ...]) -> str:
        acc = self.plan.accesses[n.kwargs["operand"]]
        addr, _ = self._coords(acc, self.plan.inputs[acc.param].shape, idx, store=False)
        src = f"args.{acc.array}[{addr}]"
        dt = acc.dtype
        if dt.name == "bfloat16":
            return f"ak_bf16_to_f32({src})"
        if dt.name == "float16":
            return f"(float)__builtin_bit_cast(_Float16, {src})"
        return f"({ctype(dt)})({src})"

    def _output_store(self, o: Any, val: Any, em: _Elements, ind: str) -> List[str]:
        acc = self.plan.placed[o.name]
        kept = acc.shape

        def body(idx: Tuple[str, ...]) -> List[str]:
            addr, conds = self._coords(acc, o.shape, idx, store=True)
            if isinstance(val, jaxlite.Sym):
                v = em.at(val.node, _broadcast_index(val.node.shape, kept, idx))
            else:
                v = literal(val, o.dtype)
            line = _write(f"args.{o.name}_out", addr, o.dtype, v)
            return [f"if ({' && '.join(conds)}) {line}"] if conds else [line]

        return self._pass(kept, body, ind)

    # ------------------------------------------------------------------------------------------ the tree

    def _block(self, b: Any, ind: str) -> List[str]:
        scope = b.scope
        updates = self._updates(scope, [c for c in b.binds if c in self.plan.kept and c in scope.values])
        outputs = {o.name: o for o in self.plan.outputs}
        stores = [(outputs[name], value) for name, value in scope.stores.items()]
        return self._emit(updates, stores, ind)

    def _tree(self, blocks: Sequence[Any], ind: str) -> List[str]:
        out: List[str] = []
        for b in blocks:
            if b.kind == "code":
                out += self._block(b, ind)
                continue
            bd = self.plan.bounds[b.loop]
            v = bd.var
            out.append(f"{ind}{{ const int b0_{v} = {self._int(bd.start)}, b1_{v} = {self._int(bd.stop)};")
            out.append(f"{ind}for (int lv_{v} = b0_{v}; lv_{v} < b1_{v}; lv_{v} += {bd.step}) {{")
            if bd.mask is not None:
                out.append(f"{ind}  if ({self._int(bd.mask)}) continue;")
            out += self._block(b, ind + "  ") if b.kind == "loop" else self._tree(b.children, ind + "  ")
            out.append(f"{ind}}} }}")
        return out

    def _tiles(self) -> Tuple[List[str], str]:
        """Setting each parallel loop's value from the tile index t (the outermost slowest), and the count
        of tiles (an expression the kernel evaluates when the outermost loop's bounds are read as it runs)."""
        plan = self.plan
        parallel = [plan.bounds[loop.var] for loop in plan.nest.parallel]
        inner = parallel[1:]
        inner_count = math.prod(b.count for b in inner)
        first = parallel[0]
        if first.static:
            total = str(first.count * inner_count)
            setup = ""
        else:
            setup = (f"const int p0_ = {self._int(first.start)}, p1_ = {self._int(first.stop)}; "
                     f"const long long total_ = p1_ > p0_ ? (long long)((p1_ - p0_ + {first.step - 1}) / {first.step}) * "
                     f"{inner_count} : 0;")
            total = "total_"
        lines = ["long long r_ = t;"]
        for b in reversed(inner):
            lines.append(f"const int lv_{b.var} = {b.start} + (int)(r_ % {b.count}) * {b.step}; r_ /= {b.count};")
        start0 = str(first.start) if first.static else "p0_"
        lines.append(f"const int lv_{first.var} = {start0} + (int)r_ * {first.step};")
        masks = [self._int(b.mask) for b in parallel if b.mask is not None]
        if masks:
            lines.append(f"if ({' || '.join(masks)}) continue;")
        return [setup] + lines, total

    def _init(self) -> str:
        """The launch before the kernel: every output filled, with its allocation's value or its input."""
        lines = []
        for o in self.plan.outputs:
            n = math.prod(o.shape)
            if o.name in self.plan.aliases:
                src = self.plan.nest.params[self.plan.aliases[o.name]]
                body = f"args.{o.name}_out[e] = args.{src}[e];"
            else:
                body = _write(f"args.{o.name}_out", "e", o.dtype, literal(o.fill if o.fill is not None else 0, o.dtype))
            lines.append(f"  for (long long e = (long long)blockIdx.x * {THREADS} + threadIdx.x; e < {n}LL; "
                         f"e += (long long)gridDim.x * {THREADS}) {body}")
        return "\n".join(lines)

    def program(self) -> Program:
        plan, sch = self.plan, self.sch
        decode, total = self._tiles()
        tile_code = self._tree(plan.tree, "    ")
        per_wg = max(self.buf.size, ALIGN)
        if per_wg > MEM_BUDGET:
            raise KernelError(f"{plan.nest.name}: a tile needs {per_wg} bytes of tile memory, more than the generic "
                              f"lowering's {MEM_BUDGET}")
        most = MAX_GRID if sch.runtime_tiles else max(1, min(sch.tiles, MAX_GRID))
        grid = max(1, min(most, MEM_BUDGET // per_wg))
        args = self._args()
        src = self._walk_source(args, decode, total, tile_code)
        elements = max(math.prod(o.shape) for o in plan.outputs)
        init_grid = max(1, min(-(-elements // THREADS), 2048))
        workspace = {"gx_mem": per_wg * grid}
        if self.trace:
            workspace[TRACE] = grid * TRACE_FIELDS * 8
        launches = [Launch(f"{self.name}_init", args, (init_grid, 1, 1), (THREADS, 1, 1), 0),
                    Launch(self.name, args, (grid, 1, 1), (THREADS, 1, 1), 0)]
        return Program(
            name=self.name, source=src, launches=launches,
            outputs=[(o.shape, o.dtype) for o in plan.outputs], inputs=[(s.shape, s.dtype) for s in plan.inputs],
            tables={}, workspace=workspace, lds_bytes=0,
            notes={"family": "generic", "walk": True, "grid": grid, "items": sch.tiles, "tile_memory": per_wg,
                   "trace_workgroups": grid if self.trace else 0, "trace_slots": grid, "slices_per_step": 1})

    def _walk_source(self, args: List[Arg], decode: List[str], total: str, tile_code: List[str]) -> str:
        plan = self.plan
        t0 = f"{CLOCK_START} const unsigned long long tr_0 = {NOW};" if self.trace else ""
        t1 = (f"if (tid == 0) {{ unsigned long long* tr = args.{TRACE} + blockIdx.x * {TRACE_FIELDS}; tr[0] = 0; "
              f"tr[1] = 0; tr[2] = 0; tr[3] = {NOW} - tr_0; tr[4] = tiles_; {CLOCK_END} }}" if self.trace else "")
        body = "\n    ".join(decode[1:])
        return f"""// Generated by tilejax_amd for `{plan.nest.name}`: the generic gfx950 lowering of the tile as written
// (blocks walked per tile in each workgroup's tile memory of {self.buf.size} bytes).
{PRELUDE}
AK_INLINE float ak_gelu_exact(float x) {{ return 0.5f * x * (1.0f + erff(x * 0.70710678118654752f)); }}
AK_INLINE int ak_ipow(int b, int e) {{ int r = 1; for (int k = 0; k < e; ++k) r *= b; return e < 0 ? 0 : r; }}
AK_INLINE float ak_fmod_floor(float a, float b) {{ const float r = fmodf(a, b); return (r != 0.0f && ((r < 0.0f) != (b < 0.0f))) ? r + b : r; }}
{c_struct(f"{self.name}_args", args)}
extern "C" __global__ void __launch_bounds__({THREADS}) {self.name}_init(const {self.name}_args args) {{
{self._init()}
}}
extern "C" __global__ void __launch_bounds__({THREADS}) {self.name}(const {self.name}_args args) {{
  const int tid = threadIdx.x;
  char* ak_mem = args.gx_mem + (long long)blockIdx.x * {max(self.buf.size, ALIGN)};
  (void)ak_mem;
  {t0}
  long long tiles_ = 0; (void)tiles_;
  {decode[0]}
  for (long long t = blockIdx.x; t < {total}; t += gridDim.x) {{
    {body}
    ++tiles_;
{chr(10).join(tile_code)}
    __syncthreads();
  }}
  {t1}
}}
"""


def _bits16(value: str, dt: DType) -> str:
    """The 16 bits of a 16-bit float value (carried as a float, exactly) or integer."""
    if dt.name == "bfloat16":
        return f"(ak_bf16_bits((float)({value})) & 0xFFFFu)"
    if dt.name == "float16":
        return f"(unsigned)__builtin_bit_cast(unsigned short, (_Float16)(float)({value}))"
    return f"((unsigned)({value}) & 0xFFFFu)"


def _from_bits16(bits: str, dt: DType) -> str:
    """A 16-bit value of `dt` from its bits, as the emitter carries it (16-bit floats as float)."""
    if dt.name == "bfloat16":
        return f"__builtin_bit_cast(float, (unsigned)({bits}) << 16)"
    if dt.name == "float16":
        return f"(float)__builtin_bit_cast(_Float16, (unsigned short)({bits}))"
    if dt.kind == "i":
        return f"(int)(short)(unsigned short)({bits})"
    return f"(unsigned)({bits})"


def _ctype_in(dt: DType) -> str:
    return {"bfloat16": "ak_u16", "float16": "ak_u16", "float32": "float", "float64": "double", "int32": "int",
            "int64": "long long", "int16": "short", "int8": "signed char", "uint8": "unsigned char",
            "uint32": "unsigned", "bool": "bool"}[dt.name]


def _cast(expr: str, dt: DType) -> str:
    if dt.kind == "f":
        return _rounded(f"({ctype(dt)})({expr})", dt) if dt.itemsize < 4 else f"({ctype(dt)})({expr})"
    if dt.kind == "b":
        return f"(({expr}) != 0)"
    return f"({ctype(dt)})({expr})"


def _write(ptr: str, addr: str, dt: DType, value: str) -> str:
    if dt.name == "bfloat16":
        return f"{ptr}[{addr}] = (ak_u16)ak_bf16_bits((float)({value}));"
    if dt.name == "float16":
        return f"{ptr}[{addr}] = __builtin_bit_cast(ak_u16, (_Float16)(float)({value}));"
    if dt.kind == "b":
        return f"{ptr}[{addr}] = (({value}) != 0);"
    return f"{ptr}[{addr}] = ({_ctype_in(dt)})({value});"


def lower(plan: Plan, sch: Schedule, pipeline: Pipeline, name: str, trace: bool = False) -> Program:
    return _Generic(plan, sch, name, trace).program()


def lower_walk(plan: Plan, sch: Schedule, pipeline: Pipeline, name: str, trace: bool = False) -> Program:
    return _Walk(plan, sch, name, trace).program()
