"""Read a kernel function's source into its loop nest. Syntax only: plan.py resolves it for concrete shapes.

The language is the reference's (src/autokernel/parse.py:1-35):

    def f(x, y, tiles=Tiles()):                    # input arrays; optionally last, a tunable
        <prologue>                                 # assignments on shapes, run when the kernel is planned
        out = jnp.zeros((M, N), dtype)             # each output allocated once
        for i in range(0, M, tiles.tm):            # parallel loops: each iteration stores its own tiles
            for j in range(0, N, TN):
                if <mask>:                         # optional: skip this output tile
                    continue
                <code>                             # straight-line code, once per tile
                for k in range(0, K, TK):          # reduction loops, one after another (phases)
                    if <mask>:                     #   optional: skip this step (may read index arrays)
                        continue
                    <body>
                <code>
                out = out.at[i : i + TM, j : j + TN].set(value)
        return out

A loop around reduction loops is a repeat loop: its reduction loops' steps, iteration after iteration.

Here the tile is read as a tree: a sequence of parts, each straight-line `Code`, a `Reduction` loop with its
body, or a `RepeatLoop` holding code and reductions of its own. The flat views the planner reads (the
reduction loops in order, their bodies, the code between them) are derived from it.
"""

from __future__ import annotations

import ast
import inspect
import textwrap
from dataclasses import dataclass, field
from typing import Callable, Dict, Iterable, List, Optional, Sequence, Tuple, Union

from .errors import KernelError
from .syntax import Store, bound, element_reads, in_order, store_of, used

__all__ = ["Code", "Loop", "Nest", "Reduction", "RepeatLoop", "parse"]

_PROLOGUE_KINDS = (ast.Assign, ast.AnnAssign, ast.AugAssign, ast.Assert, ast.Pass)


@dataclass(frozen=True)
class Loop:
    """`for var in range(*bounds):`, with the mask of an opening `if mask: continue`, if any."""

    var: str
    bounds: Tuple[ast.expr, ...]
    mask: Optional[ast.expr]
    node: ast.For


@dataclass(frozen=True)
class Code:
    """Straight-line tile statements."""

    stmts: Tuple[ast.stmt, ...]


@dataclass(frozen=True)
class Reduction:
    """A reduction loop: `body` runs once per step."""

    loop: Loop
    body: Tuple[ast.stmt, ...]


@dataclass(frozen=True)
class RepeatLoop:
    """A loop around reduction loops: `parts` (code and reductions) run once per iteration."""

    loop: Loop
    parts: Tuple[Union[Code, Reduction], ...]


Part = Union[Code, Reduction, RepeatLoop]


def _reductions_of(parts: Iterable[Part]) -> List[Reduction]:
    out: List[Reduction] = []
    for part in parts:
        if isinstance(part, Reduction):
            out.append(part)
        elif isinstance(part, RepeatLoop):
            out.extend(p for p in part.parts if isinstance(p, Reduction))
    return out


@dataclass(frozen=True)
class Nest:
    """A kernel function's loop nest, as written."""

    name: str
    filename: str
    function: ast.FunctionDef
    params: Tuple[str, ...]  # the input arrays
    tunable: Optional[str]  # the last parameter, when it has a default
    prologue: Tuple[ast.stmt, ...]
    allocations: Dict[str, ast.Assign]  # output -> the prologue statement allocating it
    outputs: Tuple[str, ...]
    parallel: Tuple[Loop, ...]  # outermost first
    parts: Tuple[Part, ...]  # the tile, as a tree
    stores: Dict[str, Store]
    stored_in: Dict[str, Optional[int]]  # output -> the reduction storing it once per step (None: per tile)
    _by_node: Dict[int, Store] = field(default_factory=dict, repr=False, compare=False)

    def __post_init__(self) -> None:
        for store in self.stores.values():
            self._by_node[id(store.node)] = store

    # Flat views of the tile -----------------------------------------------------------------------------

    @property
    def inputs(self) -> Tuple[str, ...]:
        return self.params

    @property
    def reductions(self) -> Tuple[Loop, ...]:
        """The reduction loops, in the order they run (a repeat loop's in place)."""
        return tuple(r.loop for r in _reductions_of(self.parts))

    @property
    def bodies(self) -> Tuple[Tuple[ast.stmt, ...], ...]:
        return tuple(r.body for r in _reductions_of(self.parts))

    @property
    def repeats(self) -> Tuple[RepeatLoop, ...]:
        return tuple(p for p in self.parts if isinstance(p, RepeatLoop))

    @property
    def segments(self) -> Tuple[Tuple[ast.stmt, ...], ...]:
        """The straight-line code before, between and after the reduction loops: one more than there are
        reductions (a repeat loop's own code joins the segment next to it)."""
        out: List[List[ast.stmt]] = [[]]
        for part in self.parts:
            inner = part.parts if isinstance(part, RepeatLoop) else (part,)
            for p in inner:
                if isinstance(p, Code):
                    out[-1].extend(p.stmts)
                else:
                    out.append([])
        return tuple(tuple(s) for s in out)

    @property
    def tile(self) -> Tuple[ast.stmt, ...]:
        """Every statement a tile runs, in the order written (reduction bodies in place of their loops)."""
        out: List[ast.stmt] = []

        def add(parts: Iterable[Part]) -> None:
            for p in parts:
                if isinstance(p, Code):
                    out.extend(p.stmts)
                elif isinstance(p, Reduction):
                    out.extend(p.body)
                else:
                    add(p.parts)

        add(self.parts)
        return tuple(out)

    @property
    def loops(self) -> Tuple[Loop, ...]:
        return self.parallel + self.reductions + tuple(r.loop for r in self.repeats)

    @property
    def runtime_masks(self) -> bool:
        """Do reduction masks read elements of index arrays (so the spec itself only runs eagerly)?"""
        return any(loop.mask is not None and element_reads(loop.mask, self.params) for loop in self.reductions)

    def store(self, stmt: ast.stmt) -> Optional[Store]:
        return self._by_node.get(id(stmt))

    def error(self, message: str, node: Optional[ast.AST] = None) -> KernelError:
        return KernelError(f"{self.name}: {message}", filename=self.filename, node=node)


def parse(fn: Callable) -> Nest:
    """The loop nest of kernel function `fn`; KernelError naming the line it can't compile."""
    name = getattr(fn, "__name__", repr(fn))
    try:
        source, first = inspect.getsourcelines(fn)
        filename = inspect.getsourcefile(fn) or fn.__code__.co_filename
    except (OSError, TypeError) as e:
        raise KernelError(f"{name}: can't read its source; kernels are compiled from a function's Python source") from e
    reader = _Reader(name, filename)
    if name == "<lambda>":
        raise KernelError(f"{name}: a kernel is a function defined with `def`")
    try:
        module = ast.parse(textwrap.dedent("".join(source)))
    except SyntaxError as e:  # the source lines of something that isn't a whole `def`
        raise KernelError(f"{name}: a kernel is a function defined with `def`") from e
    ast.increment_lineno(module, first - 1)
    fdef = module.body[0]
    if not isinstance(fdef, ast.FunctionDef):
        raise reader.fail("a kernel is a function defined with `def`", fdef)
    return reader.read(fdef)


class _Reader:
    """Reads one kernel function; every method raises KernelError on what the language doesn't allow."""

    def __init__(self, name: str, filename: str) -> None:
        self.name, self.filename = name, filename

    def fail(self, message: str, node: Optional[ast.AST] = None) -> KernelError:
        return KernelError(f"{self.name}: {message}", filename=self.filename, node=node)

    def read(self, fdef: ast.FunctionDef) -> Nest:
        params, tunable = self.signature(fdef.args)
        stmts = list(fdef.body)
        if isinstance(stmts[0], ast.Expr) and isinstance(stmts[0].value, ast.Constant):
            stmts.pop(0)  # the docstring
        nest_at = next((k for k, s in enumerate(stmts) if isinstance(s, ast.For)), -1)
        if nest_at < 0:
            raise self.fail("a kernel is a loop nest over output tiles, but there is no `for` loop", fdef)
        prologue, rest = stmts[:nest_at], stmts[nest_at:]
        self.check_prologue(prologue)
        if len(rest) != 2 or not isinstance(rest[1], ast.Return):
            raise self.fail("the loop nest must be followed by `return` of the outputs, and nothing else",
                            rest[1] if len(rest) > 1 else rest[0])
        outputs = self.returned(rest[1])  # type: ignore[arg-type]
        allocations = self.allocations(prologue, outputs, rest[1])
        parallel, tile = self.parallel_loops(rest[0])  # type: ignore[arg-type]
        parts = self.tile_parts(tile, inside_repeat=False)
        stores, stored_in = self.stores(parts, outputs)
        nest = Nest(self.name, self.filename, fdef, params, tunable, tuple(prologue), allocations, outputs,
                    parallel, parts, stores, stored_in)
        _NameRules(nest).check()
        return nest

    # The function's parameters, prologue and outputs ----------------------------------------------------

    def signature(self, args: ast.arguments) -> Tuple[Tuple[str, ...], Optional[str]]:
        if args.vararg or args.kwarg or args.kwonlyargs or len(args.defaults) > 1:
            raise self.fail(
                "a kernel's parameters are its input arrays, then optionally a tunable with a default, `tiles=Tiles()`",
                args)
        names = [a.arg for a in args.posonlyargs + args.args]
        if args.defaults:
            return tuple(names[:-1]), names[-1]
        return tuple(names), None

    def check_prologue(self, prologue: Sequence[ast.stmt]) -> None:
        for stmt in prologue:
            if not isinstance(stmt, _PROLOGUE_KINDS):
                raise self.fail("statements before the loop nest compute shapes: assignments and asserts", stmt)
            call = getattr(stmt, "value", None)
            if isinstance(call, ast.Call):
                f = call.func
                called = f.id if isinstance(f, ast.Name) else f.attr if isinstance(f, ast.Attribute) else None
                if called == "all_gather":
                    raise self.fail("inputs gathered across chips are not lowered for a single MI355X", stmt)

    def returned(self, ret: ast.Return) -> Tuple[str, ...]:
        value = ret.value
        items = value.elts if isinstance(value, ast.Tuple) else [value]
        names = [v.id for v in items if isinstance(v, ast.Name)]
        if not items or len(names) != len(items):
            raise self.fail("return the outputs by name: `return out` or `return out1, out2`", ret)
        if len(set(names)) < len(names):
            raise self.fail("each output is returned once", ret)
        return tuple(names)

    def allocations(self, prologue: Sequence[ast.stmt], outputs: Tuple[str, ...],
                    ret: ast.stmt) -> Dict[str, ast.Assign]:
        found: Dict[str, ast.Assign] = {}
        for stmt in prologue:
            written = bound([stmt]) & set(outputs)
            for name in sorted(written):
                plain = (isinstance(stmt, ast.Assign) and len(stmt.targets) == 1
                         and isinstance(stmt.targets[0], ast.Name))
                if name in found or not plain:
                    raise self.fail(f"allocate output `{name}` once, as `{name} = jnp.zeros(...)`", stmt)
                found[name] = stmt  # type: ignore[assignment]
        missing = [name for name in outputs if name not in found]
        if missing:
            raise self.fail(f"output `{missing[0]}` must be allocated before the loops: `{missing[0]} = jnp.zeros(...)`",
                            ret)
        return found

    # Loops ----------------------------------------------------------------------------------------------

    def loop(self, node: ast.For) -> Tuple[Loop, List[ast.stmt]]:
        """`node` as a Loop, and its body after the mask."""
        it = node.iter
        is_range = (isinstance(it, ast.Call) and isinstance(it.func, ast.Name) and it.func.id == "range"
                    and not it.keywords and 1 <= len(it.args) <= 3)
        if not (isinstance(node.target, ast.Name) and is_range):
            raise self.fail("loops are `for v in range(start, stop, step)`", node)
        if node.orelse:
            raise self.fail("loops can't have an `else` block", node)
        body = list(node.body)
        mask = None
        head = body[0]
        if (isinstance(head, ast.If) and not head.orelse and len(head.body) == 1
                and isinstance(head.body[0], ast.Continue)):
            mask = head.test
            body = body[1:]
        if not body:
            raise self.fail("the loop has nothing to run", node)
        return Loop(node.target.id, tuple(it.args), mask, node), body  # type: ignore[attr-defined]

    def parallel_loops(self, node: ast.For) -> Tuple[Tuple[Loop, ...], List[ast.stmt]]:
        """The perfectly nested loops over output tiles, and the innermost one's body (the tile)."""
        found: List[Loop] = []
        body: List[ast.stmt] = [node]
        while len(body) == 1 and isinstance(body[0], ast.For):
            loop, body = self.loop(body[0])
            found.append(loop)
        return tuple(found), body

    def tile_parts(self, stmts: Sequence[ast.stmt], inside_repeat: bool) -> Tuple[Part, ...]:
        parts: List[Part] = []
        straight: List[ast.stmt] = []

        def close() -> None:
            if straight or not parts or not isinstance(parts[-1], Code):
                self.check_tile_statements(straight)
                parts.append(Code(tuple(straight)))
                straight.clear()

        for stmt in stmts:
            if not isinstance(stmt, ast.For):
                straight.append(stmt)
                continue
            close()
            loop, body = self.loop(stmt)
            if any(isinstance(s, ast.For) for s in body):
                if inside_repeat:
                    raise self.fail("repeat loops don't nest: a repeat loop holds reduction loops", stmt)
                if loop.mask is not None:
                    raise self.fail("a repeat loop (around reduction loops) can't be masked", loop.mask)
                parts.append(RepeatLoop(loop, self.tile_parts(body, inside_repeat=True)))  # type: ignore[arg-type]
            else:
                self.check_tile_statements(body)
                parts.append(Reduction(loop, tuple(body)))
        close()
        return tuple(parts)

    def check_tile_statements(self, stmts: Iterable[ast.stmt]) -> None:
        for stmt in stmts:
            if isinstance(stmt, ast.For):
                raise self.fail("loops nest only as parallel loops around reduction (and repeat) loops", stmt)
            if isinstance(stmt, ast.Assign):
                if len(stmt.targets) != 1 or not _only_names(stmt.targets[0]):
                    raise self.fail("tile code assigns names: `a = ...` or `a, b = ...`", stmt)
            elif isinstance(stmt, ast.AugAssign):
                if not isinstance(stmt.target, ast.Name):
                    raise self.fail("tile code augments names: `a += ...`", stmt)
            elif isinstance(stmt, ast.With):
                if any(i.optional_vars is not None or not isinstance(i.context_expr, ast.Call) for i in stmt.items):
                    raise self.fail("tile code opens only `with jax.named_scope(name):` blocks", stmt)
                self.check_tile_statements(stmt.body)
            else:
                raise self.fail("tile code is assignments, output stores and `with jax.named_scope(...)` blocks; "
                                "use jnp.where instead of `if`", stmt)
            walrus = next((n for n in ast.walk(stmt) if isinstance(n, ast.NamedExpr)), None)
            if walrus is not None:
                raise self.fail("tile code can't assign inside expressions (`:=`)", walrus)

    # Output stores --------------------------------------------------------------------------------------

    def stores(self, parts: Tuple[Part, ...], outputs: Tuple[str, ...]
               ) -> Tuple[Dict[str, Store], Dict[str, Optional[int]]]:
        """Each output's store and where it is: in the code after the last reduction loop (once per tile), or
        in a reduction loop's body outside repeat loops (once per step)."""
        wanted = set(outputs)
        allowed: List[Tuple[Optional[int], Sequence[ast.stmt]]] = []
        elsewhere: List[ast.stmt] = []
        r = 0
        for k, part in enumerate(parts):
            if isinstance(part, Reduction):
                allowed.append((r, part.body))
                r += 1
            elif isinstance(part, RepeatLoop):
                inner = [s for p in part.parts for s in (p.body if isinstance(p, Reduction) else p.stmts)]
                elsewhere.extend(inner)
                r += sum(isinstance(p, Reduction) for p in part.parts)
            elif k == len(parts) - 1:
                allowed.append((None, part.stmts))
            else:
                elsewhere.extend(part.stmts)
        for stmt in in_order(elsewhere):
            s = store_of(stmt)
            if s is not None and s.output in wanted:
                raise self.fail("store outputs after the reduction loops (a tile per tile), or in the body of a "
                                "reduction loop (a tile per step)", stmt)
        stores: Dict[str, Store] = {}
        stored_in: Dict[str, Optional[int]] = {}
        for place, stmts in sorted(allowed, key=lambda a: -1 if a[0] is None else a[0]):
            for stmt in in_order(stmts):
                s = store_of(stmt)
                if s is None or s.output not in wanted:
                    continue
                if s.output in stores:
                    raise self.fail(f"output `{s.output}` is stored twice in a tile", stmt)
                stores[s.output], stored_in[s.output] = s, place
        for name in outputs:
            if name not in stores:
                raise self.fail(f"no tile stores output `{name}`: `{name} = {name}.at[...].set(...)`")
        return stores, stored_in


class _NameRules:
    """What tile code and masks may name: inputs only through subscripts, the tunable only through its
    fields, outputs only as store targets; masks only their own and enclosing loops' variables (and
    elements of index arrays, in a reduction's mask); loop variables are never assigned, and a reduction's
    variable is used only in its own body."""

    def __init__(self, nest: Nest) -> None:
        self.nest = nest
        self.params, self.outputs = set(nest.params), set(nest.outputs)

    def check(self) -> None:
        self.tile_names()
        self.masks()
        self.loop_variables()

    def _parts_of(self, stmt: ast.stmt) -> List[ast.AST]:
        store = self.nest.store(stmt)
        if store is not None:
            return [*store.index, store.value]
        if isinstance(stmt, ast.With):
            return [item.context_expr for item in stmt.items]
        return [stmt]

    def tile_names(self) -> None:
        nest = self.nest
        for stmt in in_order(nest.tile):
            is_store = nest.store(stmt) is not None
            for part in self._parts_of(stmt):
                subscripted, attributed = set(), set()
                for n in ast.walk(part):
                    if isinstance(n, ast.Subscript) and isinstance(n.value, ast.Name):
                        subscripted.add(id(n.value))
                    elif isinstance(n, ast.Attribute) and isinstance(n.value, ast.Name):
                        attributed.add(id(n.value))
                for n in ast.walk(part):
                    if not isinstance(n, ast.Name):
                        continue
                    if n.id in self.params and id(n) not in subscripted:
                        raise nest.error(f"`{n.id}` is an input: kernel code reads tiles of it, `{n.id}[...]`", n)
                    if n.id == nest.tunable and id(n) not in attributed:
                        raise nest.error(f"`{n.id}` is the kernel's tunable: tile code reads its fields, `{n.id}.x`", n)
                    if n.id in self.outputs:
                        what = "can't be read" if is_store else f"are written as `{n.id} = {n.id}.at[...].set(...)`"
                        raise nest.error(f"output `{n.id}`'s tiles {what}", n)

    def masks(self) -> None:
        nest = self.nest
        outer = [loop.var for loop in nest.parallel]
        every = {loop.var for loop in nest.loops}
        repeat_var = {}
        for rep in nest.repeats:
            for p in rep.parts:
                if isinstance(p, Reduction):
                    repeat_var[p.loop.var] = rep.loop.var
        for depth, loop in enumerate(nest.parallel):
            if loop.mask is not None:
                self._mask(loop, set(outer[: depth + 1]), every, reduction=False)
        for loop in nest.reductions:
            if loop.mask is not None:
                visible = {*outer, loop.var}
                if loop.var in repeat_var:
                    visible.add(repeat_var[loop.var])
                self._mask(loop, visible, every, reduction=True)

    def _mask(self, loop: Loop, visible: set, every: set, reduction: bool) -> None:
        nest, mask = self.nest, loop.mask
        assert mask is not None
        elements = {id(n.value) for n in element_reads(mask, self.params)} if reduction else set()
        named = [n.id for n in ast.walk(mask) if isinstance(n, ast.Name)
                 and n.id in self.params | self.outputs and id(n) not in elements]
        if named and reduction:
            raise nest.error("a reduction loop's mask reads loop variables, constants and elements of index arrays "
                             f"(`lengths[b]`), not `{named[0]}` itself", mask)
        if named:
            raise nest.error("masks are evaluated when the kernel is built, on loop variables and constants: this one "
                             f"reads `{named[0]}`", mask)
        other = used(mask) & (every - visible)
        if other:
            raise nest.error(f"a mask reads its own and enclosing loops' variables, not `{min(other)}`", mask)

    def loop_variables(self) -> None:
        nest = self.nest
        assigned = bound(nest.tile)
        for loop in nest.loops:
            if loop.var in assigned:
                raise nest.error(f"loop variable `{loop.var}` can't be assigned in the tile", loop.node)
        reductions = _reductions_of(nest.parts)
        straight = [s for seg in nest.segments for s in seg]
        straight += [s for rep in nest.repeats for p in rep.parts if isinstance(p, Code) for s in p.stmts]
        for r, red in enumerate(reductions):
            others = [s for k, o in enumerate(reductions) if k != r for s in o.body]
            for stmt in in_order(others + straight):
                if red.loop.var in used(stmt):
                    raise nest.error(f"`{red.loop.var}` is only defined inside its reduction loop", stmt)
        for rep in nest.repeats:
            inside = {id(s) for p in rep.parts for s in in_order(p.body if isinstance(p, Reduction) else p.stmts)}
            for stmt in in_order(nest.tile):
                if id(stmt) not in inside and rep.loop.var in used(stmt):
                    raise nest.error(f"`{rep.loop.var}` is only defined inside its repeat loop", stmt)


def _only_names(target: ast.expr) -> bool:
    if isinstance(target, (ast.Tuple, ast.List)):
        return all(_only_names(t) for t in target.elts)
    return isinstance(target, ast.Name)
