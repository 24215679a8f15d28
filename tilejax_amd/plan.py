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

import numpy as np

from . import jaxlite
from .errors import KernelError
from .jaxlite import DType, Node, Sym
from .parse import Loop, Nest
from .syntax import bound, element_reads, in_order, index_dims, store_of, used, used_before_bound

__all__ = ["Carried", "Index", "Kind", "NeedsWalk", "Operand", "Output", "Phase", "Plan", "Range", "Scope", "Spec",
           "Tile", "Window", "make_plan"]

READ, INDEX, STORE = "__tilejax_read__", "__tilejax_index__", "__tilejax_store__"


class NeedsWalk(KernelError):
    """A nest the step planner doesn't take but the walk planner (walk.py) may: repeat loops, runtime loop
    bounds, outputs updated in place or stored per step or where index arrays say, gathered and ragged
    windows, windows and bounds the tile code computes. Its message is the step planner's reason."""


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
    # A plan of the tile as written (walk.py), for nests without the phases-of-steps form: its blocks, the
    # values kept between them, every loop's bounds, the tile reads and output stores, in-place outputs.
    walk: bool = False
    tree: Tuple[Any, ...] = ()
    kept: Dict[str, Carried] = field(default_factory=dict)
    bounds: Dict[str, Any] = field(default_factory=dict)
    accesses: Dict[str, Any] = field(default_factory=dict)
    placed: Dict[str, Any] = field(default_factory=dict)
    aliases: Dict[str, int] = field(default_factory=dict)  # output -> the input it updates in place

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


SHAPE_ATTRIBUTES = frozenset({"shape", "dtype", "ndim", "size"})


def _data_read(stmt: ast.stmt, params: Sequence[str]) -> Optional[ast.Name]:
    """The first use of an input array in `stmt` that needs its data (anything but its shape, dtype, ndim,
    size or len), or None."""
    parent: Dict[ast.AST, ast.AST] = {}
    for node in ast.walk(stmt):
        for child in ast.iter_child_nodes(node):
            parent[child] = node
    for node in ast.walk(stmt):
        if not (isinstance(node, ast.Name) and node.id in params and isinstance(node.ctx, ast.Load)):
            continue
        up = parent.get(node)
        if isinstance(up, ast.Attribute) and up.attr in SHAPE_ATTRIBUTES:
            continue
        if isinstance(up, ast.Call) and isinstance(up.func, ast.Name) and up.func.id == "len" and node in up.args:
            continue
        return node
    return None


def _check_named_scopes(nest: Nest, envs: "_Env") -> None:
    """Every `with` in the tile opens `jax.named_scope(name)` with one string."""
    for node in ast.walk(nest.function):
        if not isinstance(node, ast.With):
            continue
        for item in node.items:
            call = item.context_expr
            ok = isinstance(call, ast.Call) and len(call.args) == 1 and not call.keywords
            try:
                ok = ok and envs.eval(call.func) is jaxlite.named_scope and isinstance(envs.eval(call.args[0]), str)
            except KernelError:
                ok = False
            if not ok:
                raise nest.error("tile code opens only `with jax.named_scope(name):` blocks, `name` a string", node)


def make_plan(nest: Nest, fn: Callable, inputs: Sequence[Spec], tunable: Any = None) -> Plan:
    """Resolve `nest` (parsed from `fn`) for inputs of these shapes and dtypes and the tunable's values: a
    plan of phases and steps when the nest has that form, else a plan of the tile as written (walk.py)."""
    try:
        return _Planner(nest, fn, tuple(inputs), tunable).plan()
    except NeedsWalk:
        from .walk import plan_walk

        return plan_walk(nest, fn, tuple(inputs), tunable)


class _Env:
    """Where plan-time code runs: the function's globals and closure, the tunable, and the inputs as meta
    arrays (shapes and dtypes, no data). Every failure becomes a KernelError naming the line."""

    def __init__(self, nest: Nest, fn: Callable, inputs: Tuple[Spec, ...], tunable: Any) -> None:
        self.nest = nest
        scope: Dict[str, Any] = {"__builtins__": builtins}
        scope.update(fn.__globals__)
        scope.update(inspect.getclosurevars(fn).nonlocals)
        with jaxlite.default_device("meta"):
            scope.update({name: jaxlite.zeros(s.shape, s.dtype) for name, s in zip(nest.params, inputs)})
        if nest.tunable:
            scope[nest.tunable] = tunable
        self.scope = scope

    def eval(self, node: ast.expr, values: Optional[Mapping[str, Any]] = None) -> Any:
        return evaluate(self.nest, self.scope, node, values)

    def run(self, stmt: ast.stmt) -> None:
        data = _data_read(stmt, self.nest.params)
        if data is not None:
            raise self.nest.error(f"the prologue runs on the inputs' shapes and dtypes: it can't read `{data.id}`'s data "
                                  "(only its .shape, .dtype, .ndim, .size or len)", stmt)
        try:
            with jaxlite.default_device("meta"):
                exec(compile(ast.Module([stmt], []), self.nest.filename, "exec"), self.scope)
        except KernelError:
            raise
        except Exception as e:
            raise self.nest.error(f"the prologue runs on the inputs' shapes and dtypes, and failed: {e!r}", stmt) from e

    def integer(self, node: ast.expr, text: str) -> int:
        value = self.eval(node)
        if not isinstance(value, int):
            raise self.nest.error(f"{text}: tile bounds are ints when planning, not {value!r}", node)
        return int(value)


def _allocation(env: _Env, name: str, call: ast.expr) -> Tuple[Tuple[int, ...], DType, Any]:
    """An output's (shape, dtype, fill) from its allocation, `jnp.zeros(shape, dtype)` or `jnp.full(...)`."""
    nest = env.nest
    usage = (f"allocate output `{name}` with jnp.zeros(shape, dtype) or jnp.full(shape, value, dtype), or as an "
             f"input updated in place (`{name} = x`)")
    if isinstance(call, ast.Name) and call.id in nest.params:
        raise NeedsWalk(f"output `{name}` updates `{call.id}` in place", filename=nest.filename, node=call)
    maker = env.eval(call.func) if isinstance(call, ast.Call) else None
    if maker is not jaxlite.zeros and maker is not jaxlite.full:
        raise nest.error(usage, call)
    args = [env.eval(a) for a in call.args]  # type: ignore[attr-defined]
    kwargs = {k.arg: env.eval(k.value) for k in call.keywords if k.arg}  # type: ignore[attr-defined]
    try:
        with jaxlite.default_device("meta"):
            made = maker(*args, **kwargs)
    except Exception as e:
        raise nest.error(f"{usage}: {e!r}", call) from e
    if maker is jaxlite.zeros:
        fill: Any = 0
    else:
        fill = args[1] if len(args) > 1 else kwargs.get("fill_value")
    if not isinstance(fill, (int, float, bool)):
        raise nest.error(f"output `{name}` is filled with a scalar constant, not {type(fill).__name__}", call)
    return tuple(made.shape), made.dtype, fill


def _loop_range(env: _Env, loop: Loop, parallel: bool, indices: Mapping[str, Any]) -> Range:
    """A loop's iterations, evaluated when planning: a nonempty `range` of whole steps from a multiple of its
    step; `runtime` when its mask reads index-array elements."""
    nest = env.nest
    computed = bound(nest.tile)
    if loop.mask is not None and element_reads(loop.mask, computed):
        raise nest.error("a mask can't read values the tile code computes (it is evaluated before the kernel runs)",
                         loop.mask)
    if any(element_reads(b, indices) or used(b) & computed for b in loop.bounds):
        raise NeedsWalk(f"`{loop.var}`'s bounds are read when the kernel runs", filename=nest.filename, node=loop.node)
    values = [env.eval(b) for b in loop.bounds]
    if any(not isinstance(v, int) for v in values):
        raise nest.error(f"loop bounds are ints when planning, got {values}", loop.node)
    start, stop, step = (0, values[0], 1) if len(values) == 1 else (*values, 1)[:3]
    if step <= 0:
        raise nest.error(f"`{loop.var}` steps by {step}: loops count up", loop.node)
    span = range(start, stop, step)
    problems = [
        (len(span) == 0, f"`{loop.var}` loops over {span}, which is empty"),
        ((stop - start) % step != 0, f"`{loop.var}` loops over {span}: the range must be a whole number of steps of {step}"),
        (start % step != 0, f"`{loop.var}` loops over {span}: it must start at a multiple of its step"),
    ]
    for bad, message in problems:
        if bad:
            raise nest.error(message, loop.node)
    runtime = loop.mask is not None and bool(element_reads(loop.mask, indices))
    if runtime and parallel:
        raise nest.error("a tile mask can't read index arrays: mask the reduction loop's steps instead", loop.mask)
    return Range(loop.var, start, step, len(span), loop.mask, runtime)


def _is_rows_call(env: "_Env", index: ast.expr) -> bool:
    """Is `index` a call of `tilejax_amd.rows` (a ragged window of rows)?"""
    if not (isinstance(index, ast.Call) and isinstance(index.func, (ast.Name, ast.Attribute))):
        return False
    from .ragged import rows

    try:
        return env.eval(index.func) is rows
    except KernelError:
        return False


class _Windows:
    """Reads the index expressions of tile reads and stores into Windows. A dim's index is one of:
    `v : v + n` (a loop variable v, n an int: moves with v), `v` (an integer index moving with v), constants
    (`a : b`, `:`, an int), or an element of an index array (`w[ids[e], ...]`: chosen when the kernel runs).
    Every window is checked to stay inside its dim for every value its loop takes."""

    def __init__(self, env: _Env, ranges: Mapping[str, Range], indices: Mapping[str, Any]) -> None:
        self.env, self.ranges, self.indices = env, ranges, indices

    def _fail(self, text: str, node: ast.AST) -> KernelError:
        return self.env.nest.error(
            f"{text}: each index is `v:v + size` or `v` for a loop variable v, `:`, constants (`start:stop`, an int), "
            "or an element of an index array (`w[ids[e], :]`)", node)

    def _loop_name(self, node: Optional[ast.expr]) -> Optional[str]:
        return node.id if isinstance(node, ast.Name) and node.id in self.ranges else None

    def window(self, index: ast.expr, dim: int, text: str) -> Window:
        movers = used(index) & set(self.ranges)
        nest = self.env.nest
        gathered = (isinstance(index, ast.Subscript) and isinstance(index.value, ast.Name)
                    and index.value.id in nest.params and any(isinstance(d, ast.Slice) for d in index_dims(index)))
        if gathered or _is_rows_call(self.env, index) or used(index) & bound(nest.tile):
            raise NeedsWalk(f"{text}: a window the kernel finds as it runs", filename=nest.filename, node=index)
        if isinstance(index, ast.Subscript) and isinstance(index.value, ast.Name) and index.value.id in self.indices:
            return Window(None, 0, None, index, frozenset(movers))
        if isinstance(index, ast.Slice):
            return self._slice(index, dim, text, movers)
        var = self._loop_name(index)
        if var is not None:
            return self._inside(Window(var, 0, None), dim, text, index)
        if movers:
            raise self._fail(text, index)
        return self._inside(Window(None, self.env.integer(index, text), None), dim, text, index)

    def _slice(self, index: ast.Slice, dim: int, text: str, movers: Set[str]) -> Window:
        if index.step is not None:
            raise self._fail(text, index)
        lo, hi = index.lower, index.upper
        var = self._loop_name(lo)
        if var is not None:
            ok = (isinstance(hi, ast.BinOp) and isinstance(hi.op, ast.Add) and self._loop_name(hi.left) == var
                  and not used(hi.right) & set(self.ranges))
            if not ok:
                raise self._fail(text, index)
            return self._inside(Window(var, 0, self.env.integer(hi.right, text)), dim, text, index)  # type: ignore[union-attr]
        if movers:
            raise self._fail(text, index)
        first = self.env.integer(lo, text) if lo is not None else 0
        stop = self.env.integer(hi, text) if hi is not None else dim
        return self._inside(Window(None, first, stop - first), dim, text, index)

    def _inside(self, w: Window, dim: int, text: str, node: ast.AST) -> Window:
        if w.size is not None and w.size <= 0:
            raise self.env.nest.error(f"{text}: a slice takes at least one element", node)
        width = w.size if w.size is not None else 1
        lowest, highest = w.offset, w.offset + width
        if w.loop:
            r = self.ranges[w.loop]
            lowest, highest = lowest + r.value(0), highest + r.value(r.count - 1)
        if lowest < 0 or highest > dim:
            raise self.env.nest.error(f"{text}: reads elements {lowest} to {highest - 1} of a dim of {dim}", node)
        return w

    def tile(self, array: str, shape: Tuple[int, ...], dt: DType, index: Sequence[ast.expr], node: ast.AST) -> Tile:
        text = f"{array}[{', '.join(ast.unparse(i) for i in index)}]"
        if len(index) != len(shape):
            raise self.env.nest.error(f"{text}: index every one of {array}'s {len(shape)} dims", node)
        windows = tuple(self.window(i, d, text) for i, d in zip(index, shape))
        kept = [w.size is not None for w in windows]
        if True not in kept:
            raise self.env.nest.error(f"{text}: a tile keeps at least one dim (slice it, `v:v + 1`)", node)
        if False in kept[kept.index(True):]:
            raise self.env.nest.error(f"{text}: integer indices go before every sliced dim", node)
        return Tile(array, windows, dt, text)


class _Planner:
    def __init__(self, nest: Nest, fn: Callable, inputs: Tuple[Spec, ...], tunable: Any) -> None:
        self.nest, self.fn, self.inputs, self.tunable = nest, fn, inputs, tunable
        self.envs = _Env(nest, fn, inputs, tunable)
        self.env = self.envs.scope
        _check_named_scopes(nest, self.envs)
        self.ranges: Dict[str, Range] = {}
        self.indices: Dict[str, Index] = {}

    def error(self, message: str, node: Optional[ast.AST] = None) -> KernelError:
        return self.nest.error(message, node)

    def eval(self, node: ast.expr, values: Optional[Mapping[str, Any]] = None) -> Any:
        return self.envs.eval(node, values)

    def plan(self) -> Plan:
        nest = self.nest
        if nest.repeats:
            raise NeedsWalk("repeat loops run as the tile is written", filename=nest.filename,
                            node=nest.repeats[0].loop.node)
        allocated = self._run_prologue()
        self.indices = {ix.name: ix for ix in self._index_arrays()}
        parallel = tuple(_loop_range(self.envs, loop, True, self.indices) for loop in nest.parallel)
        reductions = tuple(_loop_range(self.envs, loop, False, self.indices) for loop in nest.reductions)
        self.ranges = {r.var: r for r in parallel + reductions}
        self._check_element_bounds()
        windows = _Windows(self.envs, self.ranges, self.indices)
        self.windows = windows
        phases, segments, bound_vars = self._phases(reductions)
        operands, by_node = self._operands(phases, windows)
        self.operands = operands
        out_tiles = {name: self._output_tile(name, *allocated[name][:2], parallel, windows) for name in nest.outputs}
        per_step = [name for name in nest.outputs if nest.stored_in[name] is not None]
        if per_step:
            raise NeedsWalk("outputs stored per step", filename=nest.filename, node=nest.stores[per_step[0]].node)
        self._check_reads_before_assignment()
        scopes, carried = self._trace(phases, segments, bound_vars, by_node)
        outputs = tuple(self._output(name, allocated[name], out_tiles[name], scopes["last"].stores[name])
                        for name in nest.outputs)
        return Plan(nest=nest, inputs=self.inputs, tunable=self.tunable, parallel=parallel, reductions=reductions,
                    phases=phases, segments=segments, operands=operands, indices=tuple(self.indices.values()),
                    outputs=outputs, carried=carried, scopes=scopes, env=self.env, constants=self._constants())

    # ------------------------------------------------------------------ prologue and outputs

    def _run_prologue(self) -> Dict[str, Tuple[Tuple[int, ...], DType, Any]]:
        """Run the prologue on meta arrays; each output's (shape, dtype, fill) from its allocation."""
        which = {id(stmt): name for name, stmt in self.nest.allocations.items()}
        found: Dict[str, Tuple[Tuple[int, ...], DType, Any]] = {}
        for stmt in self.nest.prologue:
            name = which.get(id(stmt))
            if name is None:
                self.envs.run(stmt)
                continue
            found[name] = _allocation(self.envs, name, stmt.value)  # type: ignore[attr-defined]
            with jaxlite.default_device("meta"):
                self.env[name] = jaxlite.zeros(found[name][0], found[name][1])
        return found

    def _output(self, name: str, allocated: Tuple[Tuple[int, ...], DType, Any], tile: Tile, value: Any) -> Output:
        shape, dt, fill = allocated
        if isinstance(value, jaxlite.Array):
            vshape, vdt = tuple(value.shape), value.dtype
        elif isinstance(value, (bool, int, float)):
            vshape, vdt = (), dt
        else:
            raise self.error(f"{tile.text}: a stored value must be an array or a number, not {type(value).__name__}",
                             self.nest.stores[name].node)
        try:
            fits = np.broadcast_shapes(vshape, tile.shape) == tile.shape
        except ValueError:
            fits = False
        if not fits:
            raise self.error(f"{tile.text}: can't store a value of shape {vshape} in a {tile.shape} tile",
                             self.nest.stores[name].node)
        return Output(name, shape, dt, fill, tile, (vshape, vdt))

    # ------------------------------------------------------------------ loops

    def _phases(self, reductions: Tuple[Range, ...]):
        """The reduction loops that take steps, and the code at a tile's first step and after each of them. A
        loop of one iteration with no mask takes no step: its body joins the code around it, with its
        variable bound to its one value (returned as `bound`)."""
        nest = self.nest
        phases: List[Phase] = []
        code: List[List[ast.stmt]] = [list(nest.segments[0])]
        bound_vars: Dict[str, int] = {}
        for r, body, after in zip(reductions, nest.bodies, nest.segments[1:]):
            if r.count == 1 and r.mask is None:
                bound_vars[r.var] = r.start
                code[-1] += [*body, *after]
            else:
                phases.append(Phase(r, tuple(body)))
                code.append(list(after))
        return tuple(phases), tuple(tuple(c) for c in code), bound_vars

    # ------------------------------------------------------------------ index arrays

    def _index_arrays(self) -> Tuple[Index, ...]:
        """The inputs read element by element (in tile code, reduction masks or loop bounds): int32 arrays the
        kernel reads when it runs, each indexed in every dim and never also read as tiles."""
        nest = self.nest
        places: List[ast.AST] = list(nest.tile)
        places += [loop.mask for loop in nest.reductions if loop.mask is not None]
        places += [b for loop in nest.loops for b in loop.bounds]
        found = []
        for p, name in enumerate(nest.params):
            elements = [n for place in places for n in element_reads(place, {name})]
            if not elements:
                continue
            element_ids = {id(n) for n in elements}
            as_tiles = next((n for place in places for n in ast.walk(place)
                             if isinstance(n, ast.Subscript) and isinstance(n.value, ast.Name)
                             and n.value.id == name and id(n) not in element_ids), None)
            if as_tiles is not None:
                raise self.error(f"`{name}` is read element by element (an index array) and as tiles: read it one way "
                                 "or the other", as_tiles)
            spec = self.inputs[p]
            if spec.dtype != jaxlite.int32:
                raise self.error(f"`{name}` is read element by element, an index array: it must be int32, not "
                                 f"{spec.dtype.name}", elements[0])
            short = next((n for n in elements if len(index_dims(n)) != len(spec.shape)), None)
            if short is not None:
                raise self.error(f"{ast.unparse(short)}: index every one of {name}'s {len(spec.shape)} dims", short)
            found.append(Index(name, p, tuple(spec.shape), spec.dtype))
        return tuple(found)

    def _check_element_bounds(self) -> None:
        """Every index-array element the tile code or a reduction mask reads is inside its array, for every value
        of the loops its index expressions read."""
        nest = self.nest
        computed = bound(nest.tile) - set(self.ranges)
        places: List[ast.AST] = [*nest.tile, *(loop.mask for loop in nest.reductions if loop.mask is not None)]
        for place in places:
            for node in element_reads(place, self.indices):
                shape = self.indices[node.value.id].shape  # type: ignore[attr-defined]
                for expr, dim in zip(index_dims(node), shape):
                    if used(expr) & computed:  # an element the tile code picks: read as the tile runs
                        raise NeedsWalk(f"{ast.unparse(node)}: an element index the tile code computes",
                                        filename=nest.filename, node=node)
                    loops = [self.ranges[v] for v in sorted(used(expr) & set(self.ranges))]
                    for blocks in itertools.product(*(range(r.count) for r in loops)):
                        at = self.eval(expr, {r.var: r.value(b) for r, b in zip(loops, blocks)})
                        if not 0 <= at < dim:
                            raise self.error(f"{ast.unparse(node)}: reads element {at} of a dim of {dim}", node)

    # ------------------------------------------------------------------ tiles

    def _operands(self, phases: Tuple[Phase, ...], windows: _Windows):
        """Every tile read of an input, in source order: the same read text is one operand. Its kind follows
        the loops that move it: none (ONCE), a phase's loop (STREAM), or only parallel loops (TILE; STREAM when
        nothing takes steps)."""
        params = {name: k for k, name in enumerate(self.nest.params)}
        reads = sorted((n for stmt in self.nest.tile for n in ast.walk(stmt)
                        if isinstance(n, ast.Subscript) and isinstance(n.value, ast.Name)
                        and n.value.id in params and n.value.id not in self.indices),
                       key=lambda n: (n.lineno, n.col_offset))
        operands: List[Operand] = []
        same_text: Dict[str, Operand] = {}
        by_node: Dict[Tuple[int, int, int, int], Operand] = {}
        for node in reads:
            key = ast.dump(node)
            if key in same_text:
                by_node[_pos(node)] = same_text[key]
                continue
            array = node.value.id  # type: ignore[attr-defined]
            spec = self.inputs[params[array]]
            tile = windows.tile(array, spec.shape, spec.dtype, index_dims(node), node)
            moving = {v for v in tile.loops if v in self.ranges and self.ranges[v].count > 1}
            phase = next((k for k, ph in enumerate(phases) if ph.range.var in moving), None)
            if not moving:
                kind = Kind.ONCE
            elif phase is not None or not phases:
                kind = Kind.STREAM
            else:
                kind = Kind.TILE
            name = array
            if any(op.tile.array == array for op in operands):
                name = _fresh(array, {*self.nest.params, *(op.name for op in operands)})
            op = Operand(name, params[array], tile, kind, phase)
            operands.append(op)
            same_text[key] = by_node[_pos(node)] = op
        return tuple(operands), by_node

    def _output_tile(self, name: str, shape: Tuple[int, ...], dt: DType, parallel: Tuple[Range, ...],
                     windows: _Windows) -> Tile:
        """The window an output's store writes: every parallel loop places it along exactly one dim, covering
        that dim one step per tile; dims no loop places are written whole."""
        store = self.nest.stores[name]
        tile = windows.tile(name, shape, dt, store.index, store.node)
        if any(w.index is not None for w in tile.windows):
            raise NeedsWalk(f"{tile.text}: a store at a window an index array chooses", filename=self.nest.filename,
                            node=store.node)
        placing = [w.loop for w in tile.windows if w.loop]
        for r in parallel:
            if placing.count(r.var) != 1:
                raise self.error(f"{tile.text}: every parallel loop places each output tile, so `{r.var}` indexes "
                                 "exactly one dim of the output", store.node)
        for w, dim in zip(tile.windows, shape):
            r = self.ranges.get(w.loop) if w.loop else None
            if r is None and (w.offset != 0 or w.size != dim):
                raise self.error(f"{tile.text}: dims no loop places are stored whole, with `:`", store.node)
            if r is not None and ((w.size or 1) != r.step or r.start != 0 or r.count * r.step != dim):
                raise self.error(f"{tile.text}: loop `{r.var}` must cover the dim of {dim} exactly, one step per tile",
                                 store.node)
        return tile

    def _check_reads_before_assignment(self) -> None:
        """Nothing carries from one tile to the next: a name the tile assigns can't be read before that."""
        tile = self.nest.tile
        too_early = (used_before_bound(tile) & bound(tile)) - set(self.nest.outputs)
        if not too_early:
            return
        for stmt in in_order(tile):
            hit = used(stmt) & too_early
            if hit:
                raise self.error(f"`{min(hit)}` is read before the tile assigns it: nothing carries over from one tile "
                                 "to the next", stmt)

    def _constants(self) -> Dict[str, Any]:
        """The module and closure values the tile code reads, as they are when planning."""
        nest = self.nest
        own = bound(nest.tile) | {loop.var for loop in nest.loops} | set(nest.params) | set(nest.outputs)
        wanted: Set[str] = set()
        for stmt in in_order(nest.tile):
            wanted |= used(stmt)
        return {name: self.env[name] for name in sorted(wanted - own) if name in self.env}

    # ------------------------------------------------------------------ the trace

    def _rewrite(self, stmts: Sequence[ast.stmt], by_node: Dict[int, Operand]) -> List[ast.stmt]:
        """The tile code as the trace runs it: tile reads, index-array elements and stores as calls of the
        tracer (`@` keeps its text: the trace runs under jaxlite.matrix_units())."""
        indices, outputs = set(self.indices), set(self.nest.outputs)
        nest = self.nest

        class Rewrite(ast.NodeTransformer):
            def visit_Subscript(self, node: ast.Subscript) -> ast.expr:
                op = by_node.get(_pos(node))
                if op is not None:
                    return ast.copy_location(ast.Call(ast.Name(READ, ast.Load()), [ast.Constant(op.name)], []), node)
                if isinstance(node.value, ast.Name) and node.value.id in indices:
                    dims = [self.visit(d) for d in index_dims(node)]
                    return ast.copy_location(ast.Call(ast.Name(INDEX, ast.Load()),
                                                      [ast.Constant(node.value.id), ast.Tuple(dims, ast.Load())], []), node)
                self.generic_visit(node)
                return node

            def visit_Assign(self, node: ast.Assign) -> ast.stmt:
                store = store_of(node)
                if store is not None and store.output in outputs:
                    value = self.visit(copy.deepcopy(store.value))
                    call = ast.Call(ast.Name(STORE, ast.Load()), [ast.Constant(store.output), value], [])
                    return ast.copy_location(ast.Expr(call), node)
                self.generic_visit(node)
                return node

        out = []
        for stmt in stmts:
            new = Rewrite().visit(copy.deepcopy(stmt))
            out.append(new)
        return [ast.fix_missing_locations(s) for s in out]

    def _trace(self, phases, segments, bound_vars, by_node):
        """Trace the tile's scopes in the order they run; find the carried values and their types."""
        nest = self.nest
        order: List[Tuple[str, Tuple[ast.stmt, ...]]] = [("seg0", segments[0])]
        for p, phase in enumerate(phases):
            order += [(f"body{p}", phase.body), (f"end{p}", segments[p + 1])]
        made: Set[str] = set()
        carried_names: Set[str] = set()
        for _, stmts in order:
            carried_names |= used_before_bound(stmts) & made
            made |= bound(stmts)
        carried_names -= set(nest.outputs)
        types: Dict[str, Tuple[Tuple[int, ...], DType]] = {}
        scopes: Dict[str, Scope] = {}

        def run(name: str, stmts: Tuple[ast.stmt, ...], carried_in: Dict[str, Tuple[Tuple[int, ...], Any]]) -> Scope:
            return self._run_scope(name, stmts, carried_in, set(self.ranges), bound_vars, by_node)

        def type_of(v: Any, c: str = "", stmts: Sequence[ast.stmt] = ()) -> Tuple[Tuple[int, ...], Any]:
            if isinstance(v, jaxlite.Array):
                return tuple(v.shape), v.dtype
            if isinstance(v, (int, float, bool)):
                return (), v  # a Python number: carried as the number until an array replaces it
            raise self.error(f"a carried value must be an array or a number: this code makes `{c}` not an array "
                             f"({type(v).__name__})", stmts[0] if stmts else None)

        for idx, (name, stmts) in enumerate(order):
            needed = {c: types[c] for c in (used_before_bound(stmts) & carried_names) if c in types}
            scope = run(name, stmts, needed)
            if name.startswith("body"):
                # Carried values keep one type: run the body again from what it leaves until they agree.
                for _ in range(3):
                    after = {c: type_of(scope.values[c], c, stmts) for c in needed if c in scope.values}
                    changed = {c: t for c, t in after.items() if _type_key(t) != _type_key(needed[c])}
                    if not changed:
                        break
                    for c, t in changed.items():
                        if isinstance(needed[c][1], DType) and isinstance(t[1], DType):
                            if needed[c][0] != t[0]:
                                raise self.error(f"carried value `{c}` changes shape between steps: {needed[c][0]} -> "
                                                 f"{t[0]}", phases[int(name[4:])].body[0])
                            raise self.error(f"carried value `{c}` keeps one type: a step starts with it as "
                                             f"{needed[c][1].name}{list(needed[c][0])} and leaves {t[1].name}"
                                             f"{list(t[0])}", phases[int(name[4:])].body[0])
                        needed[c] = t  # (a Python number becomes the array it meets)
                    scope = run(name, stmts, needed)
                else:
                    raise self.error("a carried value's type doesn't settle", phases[int(name[4:])].body[0])
                still = sorted(c for c, t in needed.items() if not isinstance(t[1], DType))
                if still:
                    raise self.error(f"carried value `{still[0]}` stays a Python number through the loop's steps, so it "
                                     "must be an array (start it with jnp.zeros or jnp.full)", phases[int(name[4:])].body[0])
            scopes[name] = scope
            for k, v in scope.values.items():
                if k in carried_names:
                    types[k] = type_of(v, k, stmts)
        scopes["last"] = scopes[order[-1][0]]
        carried = {}
        for c in sorted(carried_names):
            if c in types:
                shape, dt = types[c]
                if isinstance(dt, DType):
                    carried[c] = Carried(c, shape, dt)
        return scopes, carried

    def _run_scope(self, name: str, stmts: Sequence[ast.stmt], carried_in: Dict[str, Tuple[Tuple[int, ...], Any]],
                   loop_vars: Set[str], bound_vars: Mapping[str, Any], by_node: Mapping[Any, Any]) -> Scope:
        """Trace `stmts` with symbolic loop variables and carried values of the given types (a Python number
        carried as itself): the Nodes they make, the names they leave bound, their output stores."""
        with jaxlite.trace() as tr, jaxlite.matrix_units():
            locals_: Dict[str, Any] = {}
            for var in loop_vars:
                locals_[var] = jaxlite.leaf("loop", (), jaxlite.int32, var=var)
            for var, value in bound_vars.items():
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
            scope_env[READ] = lambda op: self._load(op)
            scope_env[INDEX] = lambda arr, idx: self._index_load(arr, idx)
            scope_env[STORE] = lambda out, value: stores.__setitem__(out, value)
            code = self._rewrite(stmts, by_node)
            # one namespace, as a function's: comprehensions and lambdas in tile code see its names
            namespace = scope_env
            namespace.update(locals_)
            for stmt in code:
                try:
                    exec(compile(ast.Module([stmt], []), self.nest.filename, "exec"), namespace)
                except KernelError:
                    raise
                except Exception as e:
                    raise self.error(f"tile code failed when traced with symbolic tiles: {e!r}", stmt) from e
            names = (set(locals_) | bound(stmts)) - set(loop_vars) - set(bound_vars)
            values = {k: namespace[k] for k in names if k in namespace}
            return Scope(name, list(tr.nodes), values, leaves, stores)

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
