"""Resolve a parsed loop nest for concrete input shapes: what the kernel copies, keeps and computes.

Same model as the reference's planner (src/autokernel/plan.py:241-431): the prologue runs on the inputs'
shapes; loop ranges are evaluated; every tile read becomes a `Tile` of `Window`s with a `Kind` (STREAM:
moves every step of its phase; TILE: once per output tile; ONCE: never); inputs read element by element
are index arrays; reduction loops become phases (one of one iteration, unmasked, is inlined); values a tile
carries between steps are found by name analysis; and the tile code is traced once with symbolic values.

The trace gives the types (as the reference's `jax.make_jaxpr` trace does) and, here, also the tile code's
IR (jaxlite `Node`s) per scope, which the gfx950 lowering (codegen/) reads: the code at a tile's first
step (`seg0`), each phase's body (`body<p>`) and the code at its last step (`end<p>`).
"""

from __future__ import annotations

import ast
import builtins
import copy
import enum
import inspect
import itertools
from dataclasses import dataclass, field
from typing import Any, Callable, Dict, List, Mapping, Optional, Sequence, Set, Tuple

from . import jaxlite, mxu
from .errors import KernelError
from .jaxlite import DType, Node, Sym
from .parse import Loop, Nest
from .tilecode import as_store, assigned, element_reads, first_reads, flatten, reads, subscript_dims

__all__ = ["Carried", "Index", "Kind", "Operand", "Output", "Phase", "Plan", "Range", "Scope", "Spec", "Tile",
           "Window", "make_plan"]

READ, INDEX, STORE = "__tilejax_read__", "__tilejax_index__", "__tilejax_store__"


@dataclass(frozen=True)
class Spec:
    """An input's shape and dtype: what a kernel is built for."""

    shape: Tuple[int, ...]
    dtype: DType

    @property
    def ndim(self) -> int:
        return len(self.shape)


@dataclass(frozen=True)
class Range:
    """A loop's iterations: `start + block * step` for block in `range(count)`; `runtime` if its mask reads
    index arrays (evaluated when the kernel runs)."""

    var: str
    start: int
    step: int
    count: int
    mask: Optional[ast.expr]
    runtime: bool = False

    def value(self, block: int) -> int:
        return self.start + block * self.step


@dataclass(frozen=True)
class Window:
    """How a tile indexes one array dim: from `offset` (plus the value of `loop`), `size` elements; `size`
    None is an integer index dropping the dim. `index` is an element of an index array chosen when the
    kernel runs (a runtime window), moved by `index_loops`; it is clamped into the dim, as JAX clamps."""

    loop: Optional[str]
    offset: int
    size: Optional[int]
    index: Optional[ast.Subscript] = None
    index_loops: frozenset = frozenset()


@dataclass(frozen=True)
class Tile:
    """A window of an array that the kernel reads from (or writes to) HBM."""

    array: str
    windows: Tuple[Window, ...]
    dtype: DType
    text: str

    @property
    def shape(self) -> Tuple[int, ...]:
        return tuple(w.size for w in self.windows if w.size is not None)

    @property
    def loops(self) -> frozenset:
        return frozenset(w.loop for w in self.windows if w.loop).union(*(w.index_loops for w in self.windows))


class Kind(enum.Enum):
    STREAM = "stream"  # moves every step (of its phase): a ring of LDS slots, fetched ahead
    TILE = "tile"  # moves once per output tile
    ONCE = "once"  # never moves: fetched once


@dataclass(frozen=True)
class Operand:
    name: str  # unique: "x", or "x2" for a second window of x
    param: int
    tile: Tile
    kind: Kind
    phase: Optional[int] = None


@dataclass(frozen=True)
class Index:
    """An index array: an int32 input read element by element."""

    name: str
    param: int
    shape: Tuple[int, ...]
    dtype: DType


@dataclass(frozen=True)
class Phase:
    range: Range
    body: Tuple[ast.stmt, ...]


@dataclass(frozen=True)
class Output:
    name: str
    shape: Tuple[int, ...]
    dtype: DType
    fill: Any  # the allocation's value (0 for jnp.zeros)
    tile: Tile
    value: Tuple[Tuple[int, ...], DType]  # the stored value's shape and dtype
    phase: Optional[int] = None


@dataclass(frozen=True)
class Carried:
    name: str
    shape: Tuple[int, ...]
    dtype: DType


@dataclass
class Scope:
    """One scope of traced tile code: the Nodes it made, the names it leaves bound, and its stores."""

    name: str
    nodes: List[Node]
    values: Dict[str, Any]  # name -> Sym or Python value, after the scope ran
    carried_in: Dict[str, Node]  # name -> the "carried" leaf it read
    stores: Dict[str, Any] = field(default_factory=dict)  # output -> the stored value (Sym or scalar)


@dataclass
class Plan:
    nest: Nest
    inputs: Tuple[Spec, ...]
    tunable: Any
    parallel: Tuple[Range, ...]
    reductions: Tuple[Range, ...]
    phases: Tuple[Phase, ...]
    segments: Tuple[Tuple[ast.stmt, ...], ...]  # code at a tile's first step, then after each phase
    operands: Tuple[Operand, ...]
    indices: Tuple[Index, ...]
    outputs: Tuple[Output, ...]
    carried: Dict[str, Carried]
    scopes: Dict[str, Scope]
    env: Dict[str, Any]
    constants: Dict[str, Any]
    repeats: Tuple[Any, ...] = ()

    @property
    def single_step(self) -> bool:
        return not self.phases

    @property
    def loops(self) -> Tuple[Range, ...]:
        return self.parallel + self.reductions

    @property
    def instances(self) -> Tuple[Tuple[int, int], ...]:
        """A tile's phases in the order its steps run them: (phase, iteration of its repeat loop)."""
        return tuple((p, 0) for p in range(len(self.phases)))

    @property
    def runtime(self) -> bool:
        return any(phase.range.runtime for phase in self.phases)

    @property
    def cursor(self) -> bool:
        """Must the kernel find its steps as it runs (runtime loop bounds)? Not lowered by this backend."""
        return False

    @property
    def either(self) -> bool:
        """May the kernel find its steps either way: from step tables the device makes of its runtime masks
        before it runs, or with a cursor as it runs (src/autokernel/plan.py:318-322)? Tuning tries both."""
        return self.runtime and not self.cursor

    def operand(self, name: str) -> Operand:
        return next(op for op in self.operands if op.name == name)

    def index(self, name: str) -> Index:
        return next(ix for ix in self.indices if ix.name == name)

    def eval(self, node: ast.expr, values: Optional[Mapping[str, Any]] = None) -> Any:
        return evaluate(self.nest, self.env, node, values)


def evaluate(nest: Nest, env: Dict[str, Any], node: ast.expr, values: Optional[Mapping[str, Any]] = None) -> Any:
    try:
        code = compile(ast.Expression(node), nest.filename, "eval")
        return eval(code, env, dict(values or {}))
    except Exception as e:
        raise nest.error(f"can't evaluate `{ast.unparse(node)}` when planning: {e!r}", node) from e


def make_plan(nest: Nest, fn: Callable, inputs: Sequence[Spec], tunable: Any = None) -> Plan:
    """Resolve `nest` (parsed from `fn`) for inputs of these shapes and dtypes and the tunable's values."""
    return _Planner(nest, fn, tuple(inputs), tunable).plan()


class _Planner:
    def __init__(self, nest: Nest, fn: Callable, inputs: Tuple[Spec, ...], tunable: Any) -> None:
        self.nest, self.fn, self.inputs = nest, fn, inputs
        closure = inspect.getclosurevars(fn).nonlocals
        self.env: Dict[str, Any] = {"__builtins__": builtins, **fn.__globals__, **closure}
        with jaxlite.default_device("meta"):
            for name, spec in zip(nest.params, inputs):
                self.env[name] = jaxlite.zeros(spec.shape, spec.dtype)
        if nest.tunable:
            self.env[nest.tunable] = tunable
        self.tunable = tunable
        self.ranges: Dict[str, Range] = {}

    def error(self, message: str, node: Optional[ast.AST] = None) -> KernelError:
        return self.nest.error(message, node)

    def eval(self, node: ast.expr, values: Optional[Mapping[str, Any]] = None) -> Any:
        return evaluate(self.nest, self.env, node, values)

    def plan(self) -> Plan:
        outputs = self._prologue()
        indices = self._index_arrays()
        self.indices = {ix.name: ix for ix in indices}
        parallel = tuple(self._range(loop) for loop in self.nest.parallel)
        reductions = tuple(self._range(loop) for loop in self.nest.reductions)
        self.ranges = {r.var: r for r in (*parallel, *reductions)}
        self._check_element_bounds()
        phases, segments, bound = self._phases(reductions)
        operands, by_node = self._operands(phases, segments)
        self.operands = operands
        output_tiles = {name: self._output_tile(name, *outputs[name][:2], parallel) for name in self.nest.outputs}
        for name in self.nest.outputs:
            if self.nest.stored_in[name] is not None:
                raise self.error("outputs stored per step are not lowered by the gfx950 backend yet",
                                 self.nest.stores[name].node)
        self._check_reads_before_assignment()
        scopes, carried = self._trace(phases, segments, bound, by_node)
        outs = []
        for name in self.nest.outputs:
            shape, dt, fill = outputs[name]
            value = scopes["last"].stores[name]
            vshape, vdt = (tuple(value.shape), value.dtype) if isinstance(value, jaxlite.Array) else ((), dt)
            self._check_store(output_tiles[name], vshape)
            outs.append(Output(name, shape, dt, fill, output_tiles[name], (vshape, vdt)))
        return Plan(
            nest=self.nest, inputs=self.inputs, tunable=self.tunable, parallel=parallel, reductions=reductions,
            phases=phases, segments=segments, operands=operands, indices=indices, outputs=tuple(outs),
            carried=carried, scopes=scopes, env=self.env, constants=self._constants(),
        )

    # ------------------------------------------------------------------ prologue and outputs

    def _prologue(self) -> Dict[str, Tuple[Tuple[int, ...], DType, Any]]:
        allocation_of = {id(stmt): name for name, stmt in self.nest.allocations.items()}
        outputs = {}
        with jaxlite.default_device("meta"):
            for stmt in self.nest.prologue:
                name = allocation_of.get(id(stmt))
                if name is not None:
                    outputs[name] = self._allocation(name, stmt.value)  # type: ignore[attr-defined]
                    self.env[name] = jaxlite.zeros(*outputs[name][:2])
                    continue
                try:
                    exec(compile(ast.Module([stmt], []), self.nest.filename, "exec"), self.env)
                except KernelError:
                    raise
                except Exception as e:
                    raise self.error(f"the prologue runs on the inputs' shapes and dtypes, and failed: {e!r}", stmt) from e
        return outputs

    def _allocation(self, name: str, call: ast.expr) -> Tuple[Tuple[int, ...], DType, Any]:
        usage = f"allocate output `{name}` with jnp.zeros(shape, dtype) or jnp.full(shape, value, dtype)"
        if isinstance(call, ast.Name) and call.id in self.nest.params:
            raise self.error(f"outputs updated in place (`{name} = {call.id}`) are not lowered by the gfx950 backend yet", call)
        if not isinstance(call, ast.Call):
            raise self.error(usage, call)
        func = self.eval(call.func)
        if func is not jaxlite.zeros and func is not jaxlite.full:
            raise self.error(usage, call)
        args = [self.eval(a) for a in call.args]
        kwargs = {k.arg: self.eval(k.value) for k in call.keywords if k.arg}
        try:
            value = func(*args, **kwargs)
        except Exception as e:
            raise self.error(f"{usage}: {e!r}", call) from e
        fill = 0 if func is jaxlite.zeros else (args[1] if len(args) > 1 else kwargs.get("fill_value"))
        if not isinstance(fill, (int, float, bool)):
            raise self.error(f"output `{name}` is filled with a scalar constant, not {type(fill).__name__}", call)
        return tuple(value.shape), value.dtype, fill

    # ------------------------------------------------------------------ loops

    def _range(self, loop: Loop) -> Range:
        if loop.mask is not None and element_reads(loop.mask, assigned(self.nest.tile)):
            raise self.error("a mask can't read values the tile code computes (it is evaluated before the kernel runs)",
                             loop.mask)
        if any(element_reads(b, self.indices) for b in loop.bounds):
            raise self.error("loops with runtime bounds (a cursor) are not lowered by the gfx950 backend yet", loop.node)
        bounds = [self.eval(b) for b in loop.bounds]
        if not all(isinstance(b, int) for b in bounds):
            raise self.error(f"loop bounds are ints when planning, got {bounds}", loop.node)
        if len(bounds) == 3 and bounds[2] <= 0:
            raise self.error(f"`{loop.var}` steps by {bounds[2]}: loops count up", loop.node)
        r = range(*bounds)
        if not r:
            raise self.error(f"`{loop.var}` loops over {r}, which is empty", loop.node)
        if (r.stop - r.start) % r.step:
            raise self.error(f"`{loop.var}` loops over {r}: the range must be a whole number of steps of {r.step}", loop.node)
        if r.start % r.step:
            raise self.error(f"`{loop.var}` loops over {r}: it must start at a multiple of its step", loop.node)
        runtime = loop.mask is not None and bool(element_reads(loop.mask, self.indices))
        if runtime and loop in self.nest.parallel:
            raise self.error("a tile mask can't read index arrays: mask the reduction loop's steps instead", loop.mask)
        return Range(loop.var, r.start, r.step, len(r), loop.mask, runtime)

    def _phases(self, reductions: Tuple[Range, ...]):
        """The reduction loops that take steps and the code around them; a loop of one iteration and no mask
        joins the code around it, its variable bound to its value (`bound`)."""
        nest = self.nest
        phases: List[Phase] = []
        segments: List[List[ast.stmt]] = [list(nest.segments[0])]
        bound: Dict[str, int] = {}
        for r, body, after in zip(reductions, nest.bodies, nest.segments[1:]):
            if r.count == 1 and r.mask is None:
                bound[r.var] = r.start
                segments[-1] += list(body) + list(after)
                continue
            phases.append(Phase(r, tuple(body)))
            segments.append(list(after))
        return tuple(phases), tuple(tuple(s) for s in segments), bound

    # ------------------------------------------------------------------ index arrays

    def _index_arrays(self) -> Tuple[Index, ...]:
        nest, params = self.nest, set(self.nest.params)
        trees: List[ast.AST] = [*nest.tile, *(loop.mask for loop in nest.reductions if loop.mask is not None)]
        trees += [bound for loop in nest.loops for bound in loop.bounds]
        elements = [n for tree in trees for n in element_reads(tree, params)]
        found = []
        for p, name in enumerate(nest.params):
            mine = [n for n in elements if n.value.id == name]  # type: ignore[attr-defined]
            if not mine:
                continue
            ids = {id(n) for n in mine}
            tiles = [n for tree in trees for n in ast.walk(tree)
                     if isinstance(n, ast.Subscript) and isinstance(n.value, ast.Name) and n.value.id == name
                     and id(n) not in ids]
            if tiles:
                raise self.error(
                    f"`{name}` is read element by element (an index array) and as tiles: read it one way or the other",
                    tiles[0],
                )
            spec = self.inputs[p]
            if spec.dtype != jaxlite.int32:
                raise self.error(f"`{name}` is read element by element, an index array: it must be int32, not "
                                 f"{spec.dtype.name}", mine[0])
            for node in mine:
                if len(subscript_dims(node)) != len(spec.shape):
                    raise self.error(f"{ast.unparse(node)}: index every one of {name}'s {len(spec.shape)} dims", node)
            found.append(Index(name, p, tuple(spec.shape), spec.dtype))
        return tuple(found)

    def _check_element_bounds(self) -> None:
        """Index array elements are read at indices inside the arrays, for every loop value."""
        trees: List[ast.AST] = [*self.nest.tile, *(l.mask for l in self.nest.reductions if l.mask is not None)]
        for tree in trees:
            for node in element_reads(tree, self.indices):
                ix = self.indices[node.value.id]  # type: ignore[attr-defined]
                for expr, dim in zip(subscript_dims(node), ix.shape):
                    loops = [self.ranges[v] for v in sorted(reads(expr) & self.ranges.keys())]
                    for values in itertools.product(*(range(r.count) for r in loops)):
                        at = {r.var: r.value(b) for r, b in zip(loops, values)}
                        value = self.eval(expr, at)
                        if not 0 <= value < dim:
                            raise self.error(f"{ast.unparse(node)}: reads element {value} of a dim of {dim}", node)

    # ------------------------------------------------------------------ tiles

    def _window(self, index: ast.expr, dim: int, text: str) -> Window:
        usage = (f"{text}: each index is `v:v + size` or `v` for a loop variable v, `:`, constants "
                 "(`start:stop`, an int), or an element of an index array (`w[ids[e], :]`)")
        loop_vars = reads(index) & self.ranges.keys()
        if isinstance(index, ast.Subscript) and isinstance(index.value, ast.Name) and index.value.id in self.indices:
            if any(isinstance(i, ast.Slice) for i in subscript_dims(index)):
                raise self.error(f"{text}: windows gathered through index-array slices are not lowered yet", index)
            return Window(None, 0, None, index, frozenset(loop_vars))
        if isinstance(index, ast.Slice):
            lower, upper = index.lower, index.upper
            if index.step is not None:
                raise self.error(usage, index)
            if isinstance(lower, ast.Name) and lower.id in self.ranges:
                if not (isinstance(upper, ast.BinOp) and isinstance(upper.op, ast.Add)
                        and ast.dump(upper.left) == ast.dump(lower) and not reads(upper.right) & self.ranges.keys()):
                    raise self.error(usage, index)
                return self._checked(Window(lower.id, 0, self._int(upper.right, text)), dim, text, index)
            if loop_vars:
                raise self.error(usage, index)
            start = 0 if lower is None else self._int(lower, text)
            stop = dim if upper is None else self._int(upper, text)
            return self._checked(Window(None, start, stop - start), dim, text, index)
        if isinstance(index, ast.Name) and index.id in self.ranges:
            return self._checked(Window(index.id, 0, None), dim, text, index)
        if loop_vars:
            raise self.error(usage, index)
        return self._checked(Window(None, self._int(index, text), None), dim, text, index)

    def _int(self, node: ast.expr, text: str) -> int:
        value = self.eval(node)
        if not isinstance(value, int):
            raise self.error(f"{text}: tile bounds are ints when planning, not {value!r}", node)
        return int(value)

    def _checked(self, window: Window, dim: int, text: str, node: ast.AST) -> Window:
        if window.size is not None and window.size <= 0:
            raise self.error(f"{text}: a slice takes at least one element", node)
        first = window.offset
        last = window.offset + (window.size or 1)
        if window.loop:
            r = self.ranges[window.loop]
            first += r.start
            last += r.value(r.count - 1)
        if first < 0 or last > dim:
            raise self.error(f"{text}: reads elements {first} to {last - 1} of a dim of {dim}", node)
        return window

    def _tile(self, array: str, shape: Tuple[int, ...], dt: DType, index: Sequence[ast.expr], node: ast.AST) -> Tile:
        text = f"{array}[{', '.join(ast.unparse(i) for i in index)}]"
        if len(index) != len(shape):
            raise self.error(f"{text}: index every one of {array}'s {len(shape)} dims", node)
        windows = tuple(self._window(i, d, text) for i, d in zip(index, shape))
        sliced = [w.size is not None for w in windows]
        if not any(sliced):
            raise self.error(f"{text}: a tile keeps at least one dim (slice it, `v:v + 1`)", node)
        if not all(sliced[sliced.index(True):]):
            raise self.error(f"{text}: integer indices go before every sliced dim", node)
        return Tile(array, windows, dt, text)

    def _operands(self, phases: Tuple[Phase, ...], segments: Tuple[Tuple[ast.stmt, ...], ...]):
        operands: List[Operand] = []
        by_key: Dict[str, Operand] = {}
        by_node: Dict[int, Operand] = {}
        params = {name: i for i, name in enumerate(self.nest.params)}
        subscripts = [n for stmt in self.nest.tile for n in ast.walk(stmt) if isinstance(n, ast.Subscript)]
        for node in sorted(subscripts, key=lambda n: (n.lineno, n.col_offset)):
            if not isinstance(node.value, ast.Name) or node.value.id in self.indices:
                continue
            param = params.get(node.value.id)
            if param is None:
                continue
            spec = self.inputs[param]
            tile = self._tile(node.value.id, spec.shape, spec.dtype, subscript_dims(node), node)
            moving = {v for v in tile.loops if v in self.ranges and self.ranges[v].count > 1}
            phase = next((p for p, ph in enumerate(phases) if ph.range.var in moving), None)
            key = ast.dump(node)
            if key in by_key:
                by_node[_pos(node)] = by_key[key]
                continue
            if not moving:
                kind = Kind.ONCE
            elif phase is not None or not phases:
                kind = Kind.STREAM
            else:
                kind = Kind.TILE
            taken = {*self.nest.params, *(op.name for op in operands)}
            name = tile.array if tile.array not in {op.tile.array for op in operands} else _fresh(tile.array, taken)
            operand = Operand(name, param, tile, kind, phase)
            operands.append(operand)
            by_key[key] = by_node[_pos(node)] = operand
        return tuple(operands), by_node

    def _output_tile(self, name: str, shape: Tuple[int, ...], dt: DType, parallel: Tuple[Range, ...]) -> Tile:
        store = self.nest.stores[name]
        tile = self._tile(name, shape, dt, store.index, store.node)
        if any(w.index is not None for w in tile.windows):
            raise self.error(f"{tile.text}: stores at windows an index array chooses are not lowered yet", store.node)
        uses = [w.loop for w in tile.windows if w.loop]
        for r in parallel:
            if uses.count(r.var) != 1:
                raise self.error(
                    f"{tile.text}: every parallel loop places each output tile, so `{r.var}` indexes exactly one dim "
                    "of the output", store.node)
        for window, dim in zip(tile.windows, shape):
            r = self.ranges.get(window.loop) if window.loop else None
            if r is None:
                if window.offset != 0 or window.size != dim:
                    raise self.error(f"{tile.text}: dims no loop places are stored whole, with `:`", store.node)
            elif (window.size or 1) != r.step or r.start != 0 or r.count * r.step != dim:
                raise self.error(f"{tile.text}: loop `{r.var}` must cover the dim of {dim} exactly, one step per tile",
                                 store.node)
        return tile

    def _check_store(self, tile: Tile, vshape: Tuple[int, ...]) -> None:
        import numpy as np

        node = self.nest.stores[tile.array].node
        try:
            ok = np.broadcast_shapes(vshape, tile.shape) == tile.shape
        except ValueError:
            ok = False
        if not ok:
            raise self.error(f"{tile.text}: can't store a value of shape {vshape} in a {tile.shape} tile", node)

    def _check_reads_before_assignment(self) -> None:
        nest = self.nest
        early = (first_reads(nest.tile) & assigned(nest.tile)) - set(nest.outputs)
        for stmt in flatten(nest.tile):
            names = sorted(reads(stmt) & early)
            if names:
                raise self.error(
                    f"`{names[0]}` is read before the tile assigns it: nothing carries over from one tile to the next", stmt)

    def _constants(self) -> Dict[str, Any]:
        nest = self.nest
        own = assigned(nest.tile) | {r.var for r in nest.loops} | set(nest.params) | set(nest.outputs)
        names = set().union(*(reads(stmt) for stmt in flatten(nest.tile))) - own
        return {name: self.env[name] for name in sorted(names) if name in self.env}

    # ------------------------------------------------------------------ the trace

    def _rewrite(self, stmts: Sequence[ast.stmt], by_node: Dict[int, Operand]) -> List[ast.stmt]:
        """The tile code as the trace runs it: tile reads, index-array elements and stores as calls of the
        tracer, and `@` as the matrix-core product."""
        indices, outputs = set(self.indices), set(self.nest.outputs)
        nest = self.nest

        class Rewrite(ast.NodeTransformer):
            def visit_Subscript(self, node: ast.Subscript) -> ast.expr:
                op = by_node.get(_pos(node))
                if op is not None:
                    return ast.copy_location(ast.Call(ast.Name(READ, ast.Load()), [ast.Constant(op.name)], []), node)
                if isinstance(node.value, ast.Name) and node.value.id in indices:
                    dims = [self.visit(d) for d in subscript_dims(node)]
                    return ast.copy_location(ast.Call(ast.Name(INDEX, ast.Load()),
                                                      [ast.Constant(node.value.id), ast.Tuple(dims, ast.Load())], []), node)
                self.generic_visit(node)
                return node

            def visit_Assign(self, node: ast.Assign) -> ast.stmt:
                store = as_store(node)
                if store is not None and store.output in outputs:
                    value = self.visit(copy.deepcopy(store.value))
                    call = ast.Call(ast.Name(STORE, ast.Load()), [ast.Constant(store.output), value], [])
                    return ast.copy_location(ast.Expr(call), node)
                self.generic_visit(node)
                return node

        out = []
        for stmt in stmts:
            new = Rewrite().visit(copy.deepcopy(stmt))
            out.append(mxu.rewrite_matmuls(new))
        return [ast.fix_missing_locations(s) for s in out]

    def _trace(self, phases, segments, bound, by_node):
        """Trace the tile's scopes in the order they run; find the carried values and their types."""
        nest = self.nest
        order: List[Tuple[str, Tuple[ast.stmt, ...]]] = [("seg0", segments[0])]
        for p, phase in enumerate(phases):
            order += [(f"body{p}", phase.body), (f"end{p}", segments[p + 1])]
        made: Set[str] = set()
        carried_names: Set[str] = set()
        for _, stmts in order:
            carried_names |= first_reads(stmts) & made
            made |= assigned(stmts)
        carried_names -= set(nest.outputs)
        types: Dict[str, Tuple[Tuple[int, ...], DType]] = {}
        scopes: Dict[str, Scope] = {}

        def run(name: str, stmts: Tuple[ast.stmt, ...], carried_in: Dict[str, Tuple[Tuple[int, ...], Any]]) -> Scope:
            with jaxlite.trace() as tr:
                locals_: Dict[str, Any] = {}
                for var in self.ranges:
                    locals_[var] = jaxlite.leaf("loop", (), jaxlite.int32, var=var)
                for var, value in bound.items():
                    locals_[var] = value
                leaves = {}
                for cname, (shape, dt) in carried_in.items():
                    if isinstance(dt, DType):
                        sym = jaxlite.leaf("carried", shape, dt, name=cname)
                        locals_[cname], leaves[cname] = sym, sym.node
                    else:  # a Python number carried as itself
                        locals_[cname] = dt
                stores: Dict[str, Any] = {}
                scope_env = dict(self.env)
                scope_env.update(mxu.FUNCTIONS)
                scope_env[READ] = lambda op: self._load(op)
                scope_env[INDEX] = lambda arr, idx: self._index_load(arr, idx)
                scope_env[STORE] = lambda out, value: stores.__setitem__(out, value)
                code = self._rewrite(stmts, by_node)
                for stmt in code:
                    try:
                        exec(compile(ast.Module([stmt], []), nest.filename, "exec"), scope_env, locals_)
                    except KernelError:
                        raise
                    except Exception as e:
                        raise self.error(f"tile code failed when traced with symbolic tiles: {e!r}", stmt) from e
                values = {k: v for k, v in locals_.items() if k not in self.ranges and k not in bound}
                return Scope(name, list(tr.nodes), values, leaves, stores)

        def type_of(v: Any) -> Tuple[Tuple[int, ...], Any]:
            if isinstance(v, jaxlite.Array):
                return tuple(v.shape), v.dtype
            if isinstance(v, (int, float, bool)):
                return (), v  # a Python number: carried as the number until an array replaces it
            raise self.error(f"a carried value must be an array or a number, not {type(v).__name__}")

        for idx, (name, stmts) in enumerate(order):
            needed = {c: types[c] for c in (first_reads(stmts) & carried_names) if c in types}
            scope = run(name, stmts, needed)
            if name.startswith("body"):
                # Carried values keep one type: run the body again from what it leaves until they agree.
                for _ in range(3):
                    after = {c: type_of(scope.values[c]) for c in needed if c in scope.values}
                    changed = {c: t for c, t in after.items() if _type_key(t) != _type_key(needed[c])}
                    if not changed:
                        break
                    for c, t in changed.items():
                        if isinstance(needed[c][1], DType) and isinstance(t[1], DType) and needed[c][0] != t[0]:
                            raise self.error(f"carried value `{c}` changes shape between steps: {needed[c][0]} -> {t[0]}",
                                             phases[int(name[4:])].body[0])
                        needed[c] = t
                    scope = run(name, stmts, needed)
                else:
                    raise self.error("a carried value's type doesn't settle", phases[int(name[4:])].body[0])
            scopes[name] = scope
            for k, v in scope.values.items():
                if k in carried_names:
                    types[k] = type_of(v)
        scopes["last"] = scopes[order[-1][0]]
        carried = {}
        for c in sorted(carried_names):
            if c in types:
                shape, dt = types[c]
                if isinstance(dt, DType):
                    carried[c] = Carried(c, shape, dt)
        return scopes, carried

    def _load(self, name: str) -> Sym:
        op = next(o for o in self.operands if o.name == name)
        return jaxlite.leaf("load", op.tile.shape, op.tile.dtype, operand=name)

    def _index_load(self, array: str, index: Tuple[Any, ...]) -> Any:
        ix = self.indices[array]
        node = jaxlite.Node("index", tuple(i.node if isinstance(i, Sym) else i for i in index), {"array": array},
                            (), jaxlite.int32)
        if jaxlite._TRACE is not None:
            jaxlite._TRACE.nodes.append(node)
        import torch

        return Sym(torch.empty((), dtype=torch.int32, device="meta"), node)


def _pos(node: ast.AST) -> Tuple[int, int, int, int]:
    return (node.lineno, node.col_offset, node.end_lineno or 0, node.end_col_offset or 0)  # type: ignore[attr-defined]


def _type_key(t: Tuple[Tuple[int, ...], Any]) -> Any:
    shape, dt = t
    return (shape, dt.name) if isinstance(dt, DType) else ("py", type(dt).__name__)


def _fresh(base: str, taken: Set[str]) -> str:
    n = 2
    while f"{base}{n}" in taken:
        n += 1
    return f"{base}{n}"
