"""Lowering of a feed-forward chain to two matmul-family kernels.

The nest this takes (the reference's examples/moe.py:167-187 `expert_ffn`, and any nest of its form):

    for i ...:                                         # parallel loops (masks allowed)
        acc = jnp.zeros((G, D), jnp.float32)
        for f in range(0, F, bf):                      # one reduction loop over hidden blocks (mask allowed)
            if <mask>: continue
            xt = x[<rows>, :]                          # (optional aliases of input windows)
            g = xt @ w1[<idx>, :, f : f + bf]          # one or two products of the same full-depth left
            u = xt @ w2[<idx>, :, f : f + bf]          #   window with hidden-block windows of the weights
            acc += <act(g, u)> @ w3[<idx>, f : f + bf, :]
        out = out.at[<rows>, ...].set(<of acc>)

Each step computes `act` of products that contract the whole feature dim, so in the nest as written every
step re-reads the full-depth left window. Here the chain runs as two programs of the `gemm` family, built
from two nests this module writes out and lowers like any other:

- the gate kernel: `h[<rows>, f : f + bf] = act(g, u)` for every (tile, hidden block), g and u accumulated
  over the feature dim in f32 slices by one kernel that holds both weights' slices in LDS and reads the
  left slice once for both (GemmMatch.b2), `act` computed on the accumulators in registers and stored in
  h's dtype (the dtype the spec gives it before the down product);
- the down kernel: the original nest with its reduction body replaced by `acc += h[<rows>, f : f + bf] @
  w3[...]`, a grouped matmul with the original mask, runtime windows and epilogue.

h is a workspace buffer (rows x F elements). The arithmetic is the spec's: g and u are f32 sums over the
whole feature dim, `act` is applied to them in f32 and rounded to h's dtype, and the down products are
summed in f32 over the hidden blocks; only the f32 summation order differs.
"""

from __future__ import annotations

import ast
import copy
import itertools
import linecache
import math
import re
from dataclasses import dataclass
from typing import Any, Dict, List, Optional, Tuple

from .. import jaxlite
from ..errors import KernelError
from ..parse import Code, Reduction, parse
from ..pipeline import Pipeline
from ..plan import Plan, Spec, make_plan
from ..schedule import Schedule, make_schedule
from .device import PRELUDE
from .program import TRACE, TRACE_FIELDS, Arg, Launch, Program

__all__ = ["ChainMatch", "match", "lower"]

H = "ak_h"  # the hidden activations' workspace, and the down kernel's parameter naming it
_names = itertools.count()


@dataclass
class ChainMatch:
    gate_source: str  # the gate kernel's nest (a function of the original's inputs and tunable)
    down_source: str  # the down kernel's nest (a function of h, then the original's inputs and tunable)
    gate_name: str
    down_name: str
    h_shape: Tuple[int, ...]
    h_dtype: jaxlite.DType
    products: int  # 1 or 2


def _subscript_of(node: ast.expr, params: Tuple[str, ...]) -> Optional[ast.Subscript]:
    return node if isinstance(node, ast.Subscript) and isinstance(node.value, ast.Name) \
        and node.value.id in params else None


def _dims(sub: ast.Subscript) -> List[ast.expr]:
    s = sub.slice
    return list(s.elts) if isinstance(s, ast.Tuple) else [s]


def _full(e: ast.expr) -> bool:
    return isinstance(e, ast.Slice) and e.lower is None and e.upper is None and e.step is None


def _text(e: ast.expr) -> str:
    return ast.unparse(e)


def _window(array: str, dims: List[str]) -> str:
    return f"{array}[{', '.join(dims)}]"


def _products(expr: ast.expr, aliases: Dict[str, ast.Subscript], named: Dict[str, Tuple[ast.Subscript, ast.Subscript]],
              params: Tuple[str, ...]) -> Optional[Tuple[ast.expr, List[Tuple[ast.Subscript, ast.Subscript]]]]:
    """`expr` with each product (named, or written inline as `x[...] @ w[...]`) replaced by a name
    `ak_p<n>`, and the products in that order; None if a product isn't of two input windows."""
    found: List[Tuple[ast.Subscript, ast.Subscript]] = []
    bad = []

    class Swap(ast.NodeTransformer):
        def visit_Name(self, node: ast.Name) -> ast.expr:
            if node.id in named:
                found.append(named[node.id])
                return ast.Name(f"ak_p{len(found) - 1}", ast.Load())
            if node.id in aliases:
                bad.append(node.id)  # an input window read pointwise: not a chain this lowering takes
            return node

        def visit_Subscript(self, node: ast.Subscript) -> ast.expr:
            if _subscript_of(node, params) is not None:
                bad.append(node.value.id)  # an input window read outside a product
            return self.generic_visit(node)

        def visit_BinOp(self, node: ast.BinOp) -> ast.expr:
            if isinstance(node.op, ast.MatMult):
                left = aliases.get(node.left.id) if isinstance(node.left, ast.Name) else _subscript_of(node.left, params)
                right = _subscript_of(node.right, params)
                if left is None or right is None:
                    bad.append("@")
                    return node
                found.append((left, right))
                return ast.Name(f"ak_p{len(found) - 1}", ast.Load())
            return self.generic_visit(node)

    out = Swap().visit(copy.deepcopy(expr))
    if bad or not found:
        return None
    # a product used twice is computed once
    unique: List[Tuple[ast.Subscript, ast.Subscript]] = []
    renames: Dict[str, str] = {}
    for k, (l, r) in enumerate(found):
        key = (ast.dump(l), ast.dump(r))
        at = next((j for j, (l2, r2) in enumerate(unique) if (ast.dump(l2), ast.dump(r2)) == key), None)
        if at is None:
            unique.append((l, r))
            at = len(unique) - 1
        renames[f"ak_p{k}"] = f"ak_p{at}"

    class Rename(ast.NodeTransformer):
        def visit_Name(self, node: ast.Name) -> ast.expr:
            return ast.Name(renames.get(node.id, node.id), node.ctx)

    return Rename().visit(out), unique


def _inline(expr: ast.expr, exprs: Dict[str, ast.expr]) -> ast.expr:
    """`expr` with the names of earlier values of the body replaced by their expressions."""

    class Inline(ast.NodeTransformer):
        def visit_Name(self, node: ast.Name) -> ast.expr:
            return copy.deepcopy(exprs[node.id]) if node.id in exprs else node

    return Inline().visit(copy.deepcopy(expr))


def match(plan: Plan) -> Optional[ChainMatch]:
    """The two nests this plan's chain lowers to, or None if it isn't a chain of this form."""
    nest = plan.nest
    if plan.walk or plan.repeats or len(plan.outputs) != 1 or len(plan.phases) != 1:
        return None
    parts = nest.parts
    if len(parts) != 3 or not isinstance(parts[0], Code) or not isinstance(parts[1], Reduction) \
            or not isinstance(parts[2], Code):
        return None
    red = parts[1]
    body = list(red.body)
    last = body[-1] if body else None
    if not (isinstance(last, ast.AugAssign) and isinstance(last.op, ast.Add) and isinstance(last.target, ast.Name)
            and isinstance(last.value, ast.BinOp) and isinstance(last.value.op, ast.MatMult)):
        return None
    acc = last.target.id
    params = nest.params
    aliases: Dict[str, ast.Subscript] = {}
    named: Dict[str, Tuple[ast.Subscript, ast.Subscript]] = {}
    exprs: Dict[str, ast.expr] = {}  # other values the body computes: inlined into the activation
    for st in body[:-1]:
        if not (isinstance(st, ast.Assign) and len(st.targets) == 1 and isinstance(st.targets[0], ast.Name)):
            return None
        name, value = st.targets[0].id, st.value
        sub = _subscript_of(value, params)
        if sub is not None:
            aliases[name] = sub
            continue
        if isinstance(value, ast.BinOp) and isinstance(value.op, ast.MatMult):
            left = aliases.get(value.left.id) if isinstance(value.left, ast.Name) else _subscript_of(value.left, params)
            right = _subscript_of(value.right, params)
            if left is None or right is None:
                return None
            named[name] = (left, right)
            continue
        exprs[name] = _inline(value, exprs)
    w3 = _subscript_of(last.value.right, params)
    got = _products(_inline(last.value.left, exprs), aliases, named, params)
    if w3 is None or got is None:
        return None
    act, products = got
    if len(products) > 2 or len({ast.dump(l) for l, _ in products}) != 1:
        return None
    left = products[0][0]
    ldims, w3dims = _dims(left), _dims(w3)
    if not _full(ldims[-1]) or len(w3dims) < 2:
        return None
    f_window = w3dims[-2]  # the hidden block: the down weights' contraction dim
    if not isinstance(f_window, ast.Slice):
        return None
    widx = None
    for _, w in products:
        wd = _dims(w)
        if len(wd) < 2 or not _full(wd[-2]) or _text(wd[-1]) != _text(f_window):
            return None
        if widx is not None and [_text(d) for d in wd[:-2]] != widx:
            return None
        widx = [_text(d) for d in wd[:-2]]
    if len(products) == 2 and products[0][1].value.id == products[1][1].value.id:
        return None
    # names the activation reads: the products, and prologue values (dtypes, constants)
    free = {n.id for n in ast.walk(act) if isinstance(n, ast.Name)}
    if any(n in params or n in aliases or n in named or n == acc for n in free if not n.startswith("ak_p")):
        return None
    # shapes and dtypes from the plan: the hidden activations' (rows, bf) and dtype, the down product's left
    scope = plan.scopes["body0"]
    new, leaf = scope.values.get(acc), scope.carried_in.get(acc)
    if not (isinstance(new, jaxlite.Sym) and new.node.op == "add"):
        return None
    x, y = new.node.args
    outer = y if x is leaf else x if y is leaf else None
    if not (isinstance(outer, jaxlite.Node) and outer.op == "dot"):
        return None
    h_dtype, p_shape = outer.args[0].dtype, tuple(outer.args[0].shape)
    if len(p_shape) != 2 or h_dtype.name not in ("bfloat16", "float32"):
        return None
    lparam = params.index(left.value.id)
    wparam = params.index(products[0][1].value.id)
    lshape, wshape = tuple(plan.inputs[lparam].shape), tuple(plan.inputs[wparam].shape)
    D = lshape[-1]
    tk = next((t for t in (512, 256, 128, 64) if D % t == 0 and D // t >= 2), None)
    if tk is None:
        return None
    h_shape = lshape[:-1] + (wshape[-1],)
    return _sources(plan, red, acc, act, products, left, w3, f_window, widx or [], tk, h_shape, h_dtype, p_shape)


def _loop_header(loop: Any, indent: str) -> List[str]:
    out = [f"{indent}for {loop.var} in range({', '.join(_text(b) for b in loop.bounds)}):"]
    if loop.mask is not None:
        out += [f"{indent}    if {_text(loop.mask)}:", f"{indent}        continue"]
    return out


def _sources(plan: Plan, red: Reduction, acc: str, act: ast.expr, products, left: ast.Subscript, w3: ast.Subscript,
             f_window: ast.Slice, widx: List[str], tk: int, h_shape: Tuple[int, ...], h_dtype: jaxlite.DType,
             p_shape: Tuple[int, ...]) -> ChainMatch:
    nest = plan.nest
    gate_name, down_name = f"{nest.name}_gate", f"{nest.name}_down"
    sig = list(nest.params)
    tun = f", {nest.tunable}={_text(nest.function.args.defaults[-1])}" if nest.tunable else ""
    rows = [_text(d) for d in _dims(left)[:-1]]
    fw = _text(f_window)
    prologue = [f"    {ast.unparse(s)}" for s in nest.prologue if s not in nest.allocations.values()]

    # The gate kernel: one tile per (hidden block, outer tile), the feature dim as its reduction loop. The
    # hidden blocks are the outermost loop (the mask goes inside), so a mask that reads only the outer
    # tiles' loops gives step tables of one pattern over those tiles, repeated per hidden block.
    g: List[str] = [f"def {gate_name}({', '.join(sig)}{tun}):"] + prologue
    g.append(f"    {H} = jnp.zeros({tuple(h_shape)}, jnp.{h_dtype.name})")
    g += _loop_header(red.loop, "    ")[:1]
    ind = "        "
    for loop in nest.parallel:
        g += _loop_header(loop, ind)
        ind += "    "
    for k in range(len(products)):
        g.append(f"{ind}ak_p{k} = jnp.zeros({p_shape}, jnp.float32)")
    g.append(f"{ind}for ak_k in range(0, {_feature_dim(plan, left)}, {tk}):")
    if red.loop.mask is not None:
        g += [f"{ind}    if {_text(red.loop.mask)}:", f"{ind}        continue"]
    kwin = f"ak_k : ak_k + {tk}"
    for k, (l, w) in enumerate(products):
        lt = _window(l.value.id, rows + [kwin])
        wt = _window(w.value.id, widx + [kwin, fw])
        g.append(f"{ind}    ak_p{k} += {lt} @ {wt}")
    g.append(f"{ind}{H} = {H}.at[{', '.join(rows + [fw])}].set({ast.unparse(act)})")
    g.append(f"    return {H}")

    # The down kernel: the original nest, its reduction body the product of h's block with w3's.
    fdef = copy.deepcopy(nest.function)
    fdef.decorator_list = []
    fdef.name = down_name
    fdef.args.args.insert(0, ast.arg(arg=H))
    target = red.loop.node
    new_body = [ast.parse(f"{acc} += {_window(H, rows + [fw])} @ {_text(w3)}").body[0]]
    for node in ast.walk(fdef):
        if isinstance(node, ast.For) and node.lineno == target.lineno and node.col_offset == target.col_offset:
            head = [s for s in node.body if isinstance(s, ast.If) and s is node.body[0] and red.loop.mask is not None]
            node.body = head + new_body
            break
    else:
        raise KernelError(f"{nest.name}: internal: the reduction loop of the chain was not found")
    if isinstance(fdef.body[0], ast.Expr) and isinstance(fdef.body[0].value, ast.Constant):
        fdef.body.pop(0)
    ast.fix_missing_locations(fdef)
    down = ast.unparse(fdef)
    return ChainMatch("\n".join(g) + "\n", down + "\n", gate_name, down_name, h_shape, h_dtype, len(products))


def _feature_dim(plan: Plan, left: ast.Subscript) -> int:
    """The left operand array's last dim: the feature dim the gate kernel's reduction loop walks."""
    return int(plan.inputs[plan.nest.params.index(left.value.id)].shape[-1])


def _function(source: str, name: str, plan: Plan) -> Any:
    """`source` made a function whose globals are the original kernel's (its helpers, jax, jnp), registered
    with linecache so the planner (and its errors) can read its lines."""
    filename = f"<tilejax-chain-{name}-{next(_names)}>"
    linecache.cache[filename] = (len(source), None, source.splitlines(True), filename)
    skip = set(plan.nest.params) | ({plan.nest.tunable} if plan.nest.tunable else set())
    skip |= {t.id for s in plan.nest.prologue for t in ast.walk(s) if isinstance(t, ast.Name) and isinstance(t.ctx, ast.Store)}
    env = {k: v for k, v in plan.env.items() if k not in skip}
    exec(compile(source, filename, "exec"), env)
    return env[name]


def _plan(source: str, name: str, plan: Plan, inputs: List[Spec]) -> Tuple[Plan, Schedule]:
    fn = _function(source, name, plan)
    sub = make_plan(parse(fn), fn, inputs, plan.tunable)
    return sub, make_schedule(sub)


def lower(plan: Plan, sch: Schedule, pipeline: Pipeline, c: ChainMatch, name: str, trace: bool = False) -> Program:
    """The chain as one program: the gate kernel's launches (step builder, then kernel) writing h, then the
    down kernel's reading it."""
    from . import gemm

    inputs = list(plan.inputs)
    gplan, gsch = _plan(c.gate_source, c.gate_name, plan, inputs)
    dplan, dsch = _plan(c.down_source, c.down_name, plan, [Spec(c.h_shape, c.h_dtype)] + inputs)
    gm, dm = gemm.match(gplan), gemm.match(dplan)
    if gm is None or dm is None or (c.products == 2 and gm.b2 is None):
        raise KernelError(f"{plan.nest.name}: the chain's kernels don't take the matmul family's form")
    gate = gemm.lower(gplan, gsch, pipeline, gm, f"{name}_gate", trace=trace)
    down = gemm.lower(dplan, dsch, pipeline, dm, f"{name}_down", trace=trace)
    return compose(plan, gate, down, c, name, trace)


def compose(plan: Plan, gate: Program, down: Program, c: ChainMatch, name: str, trace: bool) -> Program:
    """One program of the two: a source with the prelude once and each kernel's LDS arrays its own; the gate
    kernel's output and the down kernel's first input are the workspace h; each part's tables and workspaces
    keep their names with the gate's prefixed `g_` (the down kernel's keep theirs, so the program's step
    tables are the down kernel's, one step per hidden block of every tile a mask leaves, as in the nest as
    written); with trace regions both kernels' workgroups write one trace buffer, the gate's first."""
    grid_g = gate.notes["grid"] if trace else 0
    workspace: Dict[str, int] = {H: math.prod(c.h_shape) * c.h_dtype.itemsize}

    def remap(args: List[Arg], part: str) -> List[Arg]:
        out = []
        for a in args:
            if part == "gate":
                if a.kind == "output":
                    out.append(Arg("workspace", H, a.ctype.replace("const ", ""), a.name))
                elif a.kind in ("table", "state"):
                    out.append(Arg(a.kind, f"g_{a.key}", a.ctype, a.name))
                elif a.kind == "workspace":
                    out.append(Arg("workspace", TRACE if a.key == TRACE else f"g_{a.key}", a.ctype, a.name))
                else:
                    out.append(a)
            else:
                if a.kind == "input":
                    out.append(Arg("workspace", H, a.ctype, a.name) if a.key == 0 else Arg("input", a.key - 1, a.ctype, a.name))
                elif a.kind == "workspace" and a.key == TRACE:
                    out.append(Arg("workspace", (TRACE, grid_g * TRACE_FIELDS * 8), a.ctype, a.name))
                else:
                    out.append(a)
        return out

    launches = [Launch(l.symbol, remap(l.args, "gate"), l.grid, l.block, l.lds) for l in gate.launches]
    launches += [Launch(l.symbol, remap(l.args, "down"), l.grid, l.block, l.lds) for l in down.launches]
    tables = {f"g_{k}": v for k, v in gate.tables.items()}
    tables.update(down.tables)
    state = {f"g_{k}": v for k, v in gate.state.items()}
    state.update(down.state)
    for k, n in gate.workspace.items():
        if k != TRACE:
            workspace[f"g_{k}"] = n
    for k, n in down.workspace.items():
        if k != TRACE:
            workspace[k] = n
    if trace:
        workspace[TRACE] = (grid_g + down.notes["grid"]) * TRACE_FIELDS * 8
    # one translation unit: the down kernel's source without the prelude, its LDS arrays renamed
    down_src = down.source.replace(PRELUDE, "", 1)
    down_src = re.sub(r"\bak_s([ab])(\d+)\b", r"ak_d\1\2", down_src)
    notes = {**down.notes, "family": "gemm", "chain": True, "products": c.products, "gate": dict(gate.notes),
             "down": dict(down.notes), "trace_workgroups": grid_g + down.notes["grid"] if trace else 0,
             "trace_slots": max(gate.notes["grid"], down.notes["grid"]), "slices_per_step": 1}
    return Program(name=name, source=gate.source + "\n" + down_src, launches=launches, outputs=list(down.outputs),
                   inputs=[(spec.shape, spec.dtype) for spec in plan.inputs], tables=tables, workspace=workspace,
                   state=state, lds_bytes=max(gate.lds_bytes, down.lds_bytes), protocol=gate.protocol, notes=notes,
                   parts=(gate, down))
