"""Parse a kernel function into its loop nest. Syntax only: plan.py resolves it for concrete shapes.

The language is the reference's (src/autokernel/parse.py:1-35):

    def f(x, y, tiles=Tiles()):                    # input arrays; optionally last, a tunable
        <prologue>                                 # assignments on shapes, run when the kernel is planned
        out = jnp.zeros((M, N), dtype)             # each output allocated once
        for i in range(0, M, tiles.tm):            # parallel loops: each iteration stores its own tiles
            for j in range(0, N, TN):
                if <mask>:                         # optional: skip this output tile
                    continue
                <segment>                          # straight-line code, once per tile
                for k in range(0, K, TK):          # reduction loops, one after another (phases)
                    if <mask>:                     #   optional: skip this step (may read index arrays)
                        continue
                    <body>
                <segment>
                out = out.at[i : i + TM, j : j + TN].set(value)
        return out

Repeat loops (a loop around reduction loops) and inputs gathered across chips parse in the reference; the
gfx950 backend does not lower them yet, so they are rejected here with a KernelError naming the line.
"""

from __future__ import annotations

import ast
import inspect
import textwrap
from dataclasses import dataclass, field
from typing import Callable, Dict, Iterable, List, Optional, Tuple

from .errors import KernelError
from .tilecode import Store, as_store, assigned, element_reads, flatten, reads

__all__ = ["Loop", "Nest", "parse"]

_PROLOGUE_STATEMENTS = (ast.Assign, ast.AnnAssign, ast.AugAssign, ast.Assert, ast.Pass)


@dataclass(frozen=True)
class Loop:
    """`for var in range(*bounds):`, possibly opening with `if mask: continue`."""

    var: str
    bounds: Tuple[ast.expr, ...]
    mask: Optional[ast.expr]
    node: ast.For


@dataclass(frozen=True)
class Nest:
    """A kernel function's loop nest, as written."""

    name: str
    filename: str
    function: ast.FunctionDef
    params: Tuple[str, ...]  # the input arrays
    tunable: Optional[str]  # the last parameter, if it has a default
    prologue: Tuple[ast.stmt, ...]
    allocations: Dict[str, ast.Assign]  # output -> its allocation
    outputs: Tuple[str, ...]
    parallel: Tuple[Loop, ...]  # outermost first
    reductions: Tuple[Loop, ...]
    bodies: Tuple[Tuple[ast.stmt, ...], ...]
    segments: Tuple[Tuple[ast.stmt, ...], ...]  # before, between and after the reduction loops
    stores: Dict[str, Store]
    stored_in: Dict[str, Optional[int]]  # output -> the reduction loop storing it per step (None: per tile)
    _store_nodes: Dict[int, Store] = field(default_factory=dict, repr=False)

    def __post_init__(self) -> None:
        self._store_nodes.update({id(s.node): s for s in self.stores.values()})

    @property
    def inputs(self) -> Tuple[str, ...]:
        return self.params

    @property
    def tile(self) -> Tuple[ast.stmt, ...]:
        """Everything a tile runs, in order: segments with the reduction bodies between them."""
        out = self.segments[0]
        for body, segment in zip(self.bodies, self.segments[1:]):
            out += body + segment
        return out

    @property
    def loops(self) -> Tuple[Loop, ...]:
        return self.parallel + self.reductions

    @property
    def runtime_masks(self) -> bool:
        """Do masks read elements of index arrays (so the spec only runs eagerly, as in the reference)?"""
        return any(loop.mask is not None and element_reads(loop.mask, self.params) for loop in self.reductions)

    def store(self, stmt: ast.stmt) -> Optional[Store]:
        return self._store_nodes.get(id(stmt))

    def error(self, message: str, node: Optional[ast.AST] = None) -> KernelError:
        return _error(self.name, self.filename, message, node)


def _error(name: str, filename: str, message: str, node: Optional[ast.AST]) -> KernelError:
    return KernelError(f"{name}: {message}", filename=filename, node=node)


def parse(fn: Callable) -> Nest:
    """The loop nest of kernel function `fn`; KernelError naming the line it can't compile."""
    name = getattr(fn, "__name__", repr(fn))
    try:
        lines, first_line = inspect.getsourcelines(fn)
        filename = inspect.getsourcefile(fn) or fn.__code__.co_filename
    except (OSError, TypeError) as e:
        raise KernelError(f"{name}: can't read its source; kernels are compiled from a function's Python source") from e
    tree = ast.parse(textwrap.dedent("".join(lines)))
    ast.increment_lineno(tree, first_line - 1)
    fdef = tree.body[0]
    if not isinstance(fdef, ast.FunctionDef):
        raise _error(name, filename, "a kernel is a function defined with `def`", fdef)
    return _Parser(name, filename, fdef).parse()


class _Parser:
    def __init__(self, name: str, filename: str, fdef: ast.FunctionDef) -> None:
        self.name, self.filename, self.fdef = name, filename, fdef

    def error(self, message: str, node: Optional[ast.AST] = None) -> KernelError:
        return _error(self.name, self.filename, message, node)

    def parse(self) -> Nest:
        params, tunable = self._params()
        body = self.fdef.body
        if isinstance(body[0], ast.Expr) and isinstance(body[0].value, ast.Constant):
            body = body[1:]  # the docstring
        at = next((i for i, stmt in enumerate(body) if isinstance(stmt, ast.For)), None)
        if at is None:
            raise self.error("a kernel is a loop nest over output tiles, but there is no `for` loop", self.fdef)
        prologue = tuple(body[:at])
        for stmt in prologue:
            if not isinstance(stmt, _PROLOGUE_STATEMENTS):
                raise self.error("statements before the loop nest compute shapes: assignments and asserts", stmt)
            value = getattr(stmt, "value", None)
            if isinstance(value, ast.Call) and _function_name(value.func) == "all_gather":
                raise self.error("inputs gathered across chips are not lowered for a single MI355X", stmt)
        if len(body) != at + 2 or not isinstance(body[at + 1], ast.Return):
            node = body[at + 1] if len(body) > at + 1 else body[at]
            raise self.error("the loop nest must be followed by `return` of the outputs, and nothing else", node)
        outputs = self._outputs(body[at + 1])  # type: ignore[arg-type]
        allocations = self._allocations(prologue, outputs, body[at + 1])
        parallel, tile = self._parallel_loops(body[at])  # type: ignore[arg-type]
        reductions, bodies, segments = self._split_tile(tile)
        stores, stored_in = self._stores(bodies, segments, outputs)
        nest = Nest(
            name=self.name, filename=self.filename, function=self.fdef, params=params, tunable=tunable,
            prologue=prologue, allocations=allocations, outputs=outputs, parallel=parallel,
            reductions=reductions, bodies=bodies, segments=segments, stores=stores, stored_in=stored_in,
        )
        self._check_names(nest)
        return nest

    def _params(self) -> Tuple[Tuple[str, ...], Optional[str]]:
        args = self.fdef.args
        names = tuple(a.arg for a in [*args.posonlyargs, *args.args])
        if args.vararg or args.kwarg or args.kwonlyargs or len(args.defaults) > 1:
            raise self.error(
                "a kernel's parameters are its input arrays, then optionally a tunable with a default, `tiles=Tiles()`",
                args,
            )
        return (names[:-1], names[-1]) if args.defaults else (names, None)

    def _outputs(self, ret: ast.Return) -> Tuple[str, ...]:
        value = ret.value
        elts = value.elts if isinstance(value, ast.Tuple) else [value]
        if not elts or not all(isinstance(e, ast.Name) for e in elts):
            raise self.error("return the outputs by name: `return out` or `return out1, out2`", ret)
        names = tuple(e.id for e in elts)  # type: ignore[union-attr]
        if len(set(names)) != len(names):
            raise self.error("each output is returned once", ret)
        return names

    def _allocations(self, prologue: Tuple[ast.stmt, ...], outputs: Tuple[str, ...], ret: ast.stmt) -> Dict[str, ast.Assign]:
        allocations: Dict[str, ast.Assign] = {}
        for stmt in prologue:
            if isinstance(stmt, ast.Assign):
                targets = stmt.targets
            elif isinstance(stmt, (ast.AnnAssign, ast.AugAssign)):
                targets = [stmt.target]
            else:
                continue
            for name in sorted({n.id for t in targets for n in ast.walk(t) if isinstance(n, ast.Name)} & set(outputs)):
                single = isinstance(stmt, ast.Assign) and len(targets) == 1 and isinstance(targets[0], ast.Name)
                if name in allocations or not single:
                    raise self.error(f"allocate output `{name}` once, as `{name} = jnp.zeros(...)`", stmt)
                allocations[name] = stmt  # type: ignore[assignment]
        for name in outputs:
            if name not in allocations:
                raise self.error(f"output `{name}` must be allocated before the loops: `{name} = jnp.zeros(...)`", ret)
        return allocations

    def _loop(self, node: ast.For) -> Tuple[Loop, List[ast.stmt]]:
        call = node.iter
        if not (
            isinstance(node.target, ast.Name)
            and isinstance(call, ast.Call)
            and isinstance(call.func, ast.Name)
            and call.func.id == "range"
            and 1 <= len(call.args) <= 3
            and not call.keywords
        ):
            raise self.error("loops are `for v in range(start, stop, step)`", node)
        if node.orelse:
            raise self.error("loops can't have an `else` block", node)
        body, mask = list(node.body), None
        first = body[0]
        if isinstance(first, ast.If) and not first.orelse and [type(s) for s in first.body] == [ast.Continue]:
            mask, body = first.test, body[1:]
        if not body:
            raise self.error("the loop has nothing to run", node)
        return Loop(node.target.id, tuple(call.args), mask, node), body

    def _parallel_loops(self, node: ast.For) -> Tuple[Tuple[Loop, ...], List[ast.stmt]]:
        loops = []
        while True:
            loop, body = self._loop(node)
            loops.append(loop)
            if len(body) == 1 and isinstance(body[0], ast.For):
                node = body[0]
                continue
            return tuple(loops), body

    def _split_tile(self, tile: List[ast.stmt]):
        reductions: List[Loop] = []
        bodies: List[Tuple[ast.stmt, ...]] = []
        segments: List[Tuple[ast.stmt, ...]] = []
        segment: List[ast.stmt] = []
        for stmt in tile:
            if not isinstance(stmt, ast.For):
                segment.append(stmt)
                continue
            loop, body = self._loop(stmt)
            if any(isinstance(s, ast.For) for s in body):
                raise self.error(
                    "repeat loops (a loop around reduction loops) are not lowered by the gfx950 backend yet", stmt
                )
            self._check_statements(body)
            reductions.append(loop)
            bodies.append(tuple(body))
            segments.append(tuple(segment))
            segment = []
        self._check_statements(segment)
        segments.append(tuple(segment))
        for done in segments[:-1]:
            self._check_statements(done)
        return tuple(reductions), tuple(bodies), tuple(segments)

    def _check_statements(self, stmts: Iterable[ast.stmt]) -> None:
        for stmt in stmts:
            if isinstance(stmt, ast.For):
                raise self.error("loops nest only as parallel loops around reduction loops", stmt)
            if isinstance(stmt, ast.Assign):
                if len(stmt.targets) != 1 or not _names_only(stmt.targets[0]):
                    raise self.error("tile code assigns names: `a = ...` or `a, b = ...`", stmt)
            elif isinstance(stmt, ast.AugAssign):
                if not isinstance(stmt.target, ast.Name):
                    raise self.error("tile code augments names: `a += ...`", stmt)
            elif isinstance(stmt, ast.With):
                if any(item.optional_vars or not isinstance(item.context_expr, ast.Call) for item in stmt.items):
                    raise self.error("tile code opens only `with jax.named_scope(name):` blocks", stmt)
                self._check_statements(stmt.body)
            else:
                raise self.error(
                    "tile code is assignments, output stores and `with jax.named_scope(...)` blocks; "
                    "use jnp.where instead of `if`",
                    stmt,
                )
            for node in ast.walk(stmt):
                if isinstance(node, ast.NamedExpr):
                    raise self.error("tile code can't assign inside expressions (`:=`)", node)

    def _stores(self, bodies, segments, outputs):
        for stmt in flatten([s for part in segments[:-1] for s in part]):
            store = as_store(stmt)
            if store and store.output in outputs:
                raise self.error(
                    "store outputs after the reduction loops (a tile per tile), or in the body of a reduction loop "
                    "(a tile per step)",
                    stmt,
                )
        places = [(None, segments[-1])] + [(r, body) for r, body in enumerate(bodies)]
        stores: Dict[str, Store] = {}
        stored_in: Dict[str, Optional[int]] = {}
        for r, stmts in places:
            for stmt in flatten(stmts):
                store = as_store(stmt)
                if store and store.output in outputs:
                    if store.output in stores:
                        raise self.error(f"output `{store.output}` is stored twice in a tile", stmt)
                    stores[store.output], stored_in[store.output] = store, r
        for name in outputs:
            if name not in stores:
                raise self.error(f"no tile stores output `{name}`: `{name} = {name}.at[...].set(...)`")
        return stores, stored_in

    def _check_names(self, nest: Nest) -> None:
        params, outputs = set(nest.params), set(nest.outputs)
        for stmt in flatten(nest.tile):
            store = nest.store(stmt)
            parts: List[ast.AST] = [*store.index, store.value] if store else (
                [item.context_expr for item in stmt.items] if isinstance(stmt, ast.With) else [stmt])
            for part in parts:
                bases = {id(n.value) for n in ast.walk(part)
                         if isinstance(n, ast.Subscript) and isinstance(n.value, ast.Name) and n.value.id in params}
                fields = {id(n.value) for n in ast.walk(part)
                          if isinstance(n, ast.Attribute) and isinstance(n.value, ast.Name) and n.value.id == nest.tunable}
                for n in ast.walk(part):
                    if not isinstance(n, ast.Name):
                        continue
                    if n.id in params and id(n) not in bases:
                        raise self.error(f"`{n.id}` is an input: kernel code reads tiles of it, `{n.id}[...]`", n)
                    if n.id == nest.tunable and id(n) not in fields:
                        raise self.error(f"`{n.id}` is the kernel's tunable: tile code reads its fields, `{n.id}.x`", n)
                    if n.id in outputs:
                        what = "can't be read" if store else f"are written as `{n.id} = {n.id}.at[...].set(...)`"
                        raise self.error(f"output `{n.id}`'s tiles {what}", n)
        loop_vars = {loop.var for loop in nest.loops}
        parallel_vars = [loop.var for loop in nest.parallel]
        for depth, loop in enumerate(nest.loops):
            if loop.mask is None:
                continue
            reduction = depth >= len(parallel_vars)
            visible = {*parallel_vars, loop.var} if reduction else set(parallel_vars[: depth + 1])
            elements = {id(n.value) for n in element_reads(loop.mask, params)} if reduction else set()
            arrays = [n.id for n in ast.walk(loop.mask)
                      if isinstance(n, ast.Name) and n.id in params | outputs and id(n) not in elements]
            if arrays and reduction:
                raise self.error(
                    "a reduction loop's mask reads loop variables, constants and elements of index arrays "
                    f"(`lengths[b]`), not `{arrays[0]}` itself",
                    loop.mask,
                )
            if arrays:
                raise self.error(
                    f"masks are evaluated when the kernel is built, on loop variables and constants: this one reads "
                    f"`{arrays[0]}`",
                    loop.mask,
                )
            inner = reads(loop.mask) & (loop_vars - visible)
            if inner:
                raise self.error(f"a mask reads its own and enclosing loops' variables, not `{sorted(inner)[0]}`", loop.mask)
        written = assigned(nest.tile)
        for loop in nest.loops:
            if loop.var in written:
                raise self.error(f"loop variable `{loop.var}` can't be assigned in the tile", loop.node)
        for r, reduction in enumerate(nest.reductions):
            elsewhere = [s for b, body in enumerate(nest.bodies) if b != r for s in body]
            for stmt in flatten([*elsewhere, *(s for segment in nest.segments for s in segment)]):
                if reduction.var in reads(stmt):
                    raise self.error(f"`{reduction.var}` is only defined inside its reduction loop", stmt)


def _function_name(func: ast.expr) -> Optional[str]:
    return func.id if isinstance(func, ast.Name) else func.attr if isinstance(func, ast.Attribute) else None


def _names_only(target: ast.expr) -> bool:
    if isinstance(target, (ast.Tuple, ast.List)):
        return all(_names_only(e) for e in target.elts)
    return isinstance(target, ast.Name)
