"""Plans of a tile as written: for loop nests the step planner (plan.py) doesn't take.

The step planner turns a tile into phases of steps, the form the matmul, flash and decode kernels run. Some
nests don't have that form, and the reference's planner takes them (src/autokernel/plan.py:241-431):

- repeat loops, a loop around reduction loops (tests/test_repeat_loops.py of the reference);
- loop bounds read when the kernel runs: from index arrays (`range(0, lengths[b], 128)`, a runtime count of
  tiles `range(n[0])`) or from index arrays the tile code computes (`range(0, n[0] * D, D)`,
  tests/test_runtime_ranges.py, tests/test_computed_indices.py);
- outputs updated in place (`new = pool`) and stored where index arrays say (`new.at[slots[b], ...]`),
  outputs stored once per step (tests/test_in_place.py);
- windows gathered through index-array slices (`pages[table[b * 4 : b * 4 + 2], :, :]`) and ragged rows
  (`q[rows(start, stop, 16), :, :]`), and windows placed by values the tile code computes.

Such a nest is planned here as the tile is written: a tree of blocks (straight-line code, reduction loops,
repeat loops) each traced once with symbolic values, like the step planner's scopes; the values that live
from one block into another (or from one iteration into the next) are `kept`, each with one type; loop
bounds, masks and window starts stay Python expressions, which the kernel evaluates as it runs (over loop
variables, constants, elements of index arrays and of kept int32 arrays). The generic gfx950 kernel walks
the tree (codegen/generic.py).
"""

from __future__ import annotations

import ast
import itertools
import math
from dataclasses import dataclass
from typing import Any, Callable, Dict, List, Optional, Sequence, Set, Tuple, Union

import numpy as np

from . import jaxlite
from .errors import KernelError
from .jaxlite import DType
from .parse import Code, Nest, Reduction, RepeatLoop
from .plan import (Carried, Index, Output, Plan, Range, Scope, Spec, Tile, Window, _allocation, _is_rows_call,
                   _Planner, _pos, _type_key)
from .syntax import bound, element_reads, index_dims, used, used_before_bound

__all__ = ["Access", "Block", "Bound", "Dim", "plan_walk"]

_MAX_CHECKED = 4096  # loop-value combinations a window's bounds are checked over when planning


@dataclass(frozen=True)
class Bound:
    """A loop's `range(start, stop, step)`: start and stop ints, or expressions the kernel evaluates as it
    runs; `mask`, if any, skips an iteration (a tile, for a parallel loop)."""

    var: str
    start: Union[int, ast.expr]
    stop: Union[int, ast.expr]
    step: int
    mask: Optional[ast.expr]
    node: ast.For

    @property
    def static(self) -> bool:
        return isinstance(self.start, int) and isinstance(self.stop, int)

    @property
    def count(self) -> int:
        """Iterations (a static range only)."""
        return max(0, -(-(self.stop - self.start) // self.step))  # type: ignore[operator]


@dataclass(frozen=True)
class Dim:
    """How a read or store indexes one dim of an array. `size` elements from `start` (an int, or an
    expression the kernel evaluates), or, `size` None, the one element `start` (the dim dropped). With
    `gather`, `ids[a : a + n]`, element e is at `ids[a + e]`; with `stop` (a ragged window, `rows`), a store
    writes only the elements before it. The kernel clamps what it evaluates into the dim, as JAX clamps."""

    size: Optional[int]
    start: Union[int, ast.expr] = 0
    stop: Optional[ast.expr] = None
    gather: Optional[ast.Subscript] = None


@dataclass(frozen=True)
class Access:
    """A tile read of an input, or an output's store: each dim's window."""

    name: str  # unique per read text: "x", "x2" for a second window of x
    array: str
    param: Optional[int]  # the input read (None for an output)
    dims: Tuple[Dim, ...]
    dtype: DType
    text: str

    @property
    def shape(self) -> Tuple[int, ...]:
        return tuple(d.size for d in self.dims if d.size is not None)


@dataclass
class Block:
    """A piece of the tile: straight-line `code`, a reduction `loop` (its body's trace), or a `repeat` loop
    of blocks. `binds` are the kept values it assigns."""

    kind: str
    scope: Optional[Scope] = None
    loop: Optional[str] = None
    children: Tuple["Block", ...] = ()
    binds: Tuple[str, ...] = ()


def plan_walk(nest: Nest, fn: Callable, inputs: Tuple[Spec, ...], tunable: Any) -> Plan:
    return _WalkPlanner(nest, fn, inputs, tunable).plan()


def _value_type(v: Any) -> Optional[Tuple[Tuple[int, ...], Any]]:
    if isinstance(v, jaxlite.Array):
        return tuple(v.shape), v.dtype
    if isinstance(v, (int, float, bool)):
        return (), v
    return None


class _WalkPlanner(_Planner):
    def plan(self) -> Plan:
        nest = self.nest
        self.aliases: Dict[str, int] = {}
        allocated = self._allocations()
        self.computed = bound(nest.tile) - set(nest.outputs)
        self.indices = {ix.name: ix for ix in self._walk_index_arrays()}
        for name, p in self.aliases.items():
            if nest.params[p] in self.indices:
                raise self.error(f"output `{name}` updates `{nest.params[p]}` in place, but `{nest.params[p]}` is an "
                                 "index array", nest.allocations[name])
        self.bounds: Dict[str, Bound] = {}
        for depth, loop in enumerate(nest.parallel):
            self.bounds[loop.var] = self._bound(loop, parallel=True, outermost=depth == 0)
        for loop in nest.reductions + tuple(r.loop for r in nest.repeats):
            self.bounds[loop.var] = self._bound(loop, parallel=False, outermost=False)
        self.ranges = {v: Range(v, b.start, b.step, b.count, b.mask) for v, b in self.bounds.items()  # type: ignore[arg-type]
                       if b.static}
        accesses, by_node = self._accesses()
        self.accesses = accesses
        placed = {name: self._placed(name, *allocated[name][:2]) for name in nest.outputs}
        self._check_reads_before_assignment()
        tree, kept, stores = self._trace_tree(by_node)
        outputs = []
        for name in nest.outputs:
            shape, dt, fill = allocated[name]
            acc = placed[name]
            value = stores[name]
            vtype = _value_type(value)
            try:
                fits = vtype is not None and np.broadcast_shapes(vtype[0], acc.shape) == acc.shape
            except ValueError:
                fits = False
            if not fits:
                raise self.error(f"{acc.text}: can't store a value of shape {vtype[0] if vtype else '?'} in a "
                                 f"{acc.shape} tile", nest.stores[name].node)
            vdt = vtype[1] if isinstance(vtype[1], DType) else dt  # type: ignore[index]
            tile = Tile(name, tuple(Window(None, 0, d.size) for d in acc.dims), dt, acc.text)
            outputs.append(Output(name, shape, dt, fill, tile, (vtype[0], vdt)))  # type: ignore[index]
        parallel = tuple(self._range(self.bounds[loop.var]) for loop in nest.parallel)
        reductions = tuple(self._range(self.bounds[loop.var]) for loop in nest.reductions)
        return Plan(nest=nest, inputs=self.inputs, tunable=self.tunable, parallel=parallel, reductions=reductions,
                    phases=(), segments=((),), operands=(), indices=tuple(self.indices.values()), outputs=tuple(outputs),
                    carried={}, scopes={}, env=self.env, constants=self._constants(), walk=True, tree=tree, kept=kept,
                    bounds=dict(self.bounds), accesses=accesses, placed=placed, aliases=dict(self.aliases))

    # ------------------------------------------------------------------ prologue

    def _allocations(self) -> Dict[str, Tuple[Tuple[int, ...], DType, Any]]:
        """Run the prologue; each output's (shape, dtype, fill), fill None for an input updated in place."""
        nest = self.nest
        which = {id(stmt): name for name, stmt in nest.allocations.items()}
        found: Dict[str, Tuple[Tuple[int, ...], DType, Any]] = {}
        for stmt in nest.prologue:
            name = which.get(id(stmt))
            if name is None:
                self.envs.run(stmt)
                continue
            value = stmt.value  # type: ignore[attr-defined]
            if isinstance(value, ast.Name) and value.id in nest.params:
                p = nest.params.index(value.id)
                spec = self.inputs[p]
                self.aliases[name] = p
                found[name] = (tuple(spec.shape), spec.dtype, None)
            else:
                found[name] = _allocation(self.envs, name, value)
            with jaxlite.default_device("meta"):
                self.env[name] = jaxlite.zeros(found[name][0], found[name][1])
        return found

    def _walk_index_arrays(self) -> Tuple[Index, ...]:
        """The inputs read element by element (in tile code, masks, loop bounds) or gathered through slices
        in another array's window: int32 arrays the kernel reads as it runs, indexed in every dim, never read
        as tiles too."""
        nest = self.nest
        places: List[ast.AST] = list(nest.tile)
        places += [loop.mask for loop in nest.loops if loop.mask is not None]
        places += [b for loop in nest.loops for b in loop.bounds]
        params = set(nest.params)
        gathers: Dict[str, List[ast.Subscript]] = {}
        for place in places:
            for n in ast.walk(place):
                if isinstance(n, ast.Subscript) and isinstance(n.value, ast.Name) and n.value.id in params:
                    for d in index_dims(n):
                        if (isinstance(d, ast.Subscript) and isinstance(d.value, ast.Name) and d.value.id in params
                                and any(isinstance(x, ast.Slice) for x in index_dims(d))):
                            gathers.setdefault(d.value.id, []).append(d)
        found = []
        for p, name in enumerate(nest.params):
            elements = [n for place in places for n in element_reads(place, {name})] + gathers.get(name, [])
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

    # ------------------------------------------------------------------ loops

    def _runtime_names(self) -> Set[str]:
        return {loop.var for loop in self.nest.loops} | set(self.indices) | self.computed

    def _static(self, node: ast.expr) -> bool:
        """Does `node` read nothing the kernel learns as it runs (loop variables, index arrays, tile values)?"""
        return not used(node) & self._runtime_names()

    def _bound(self, loop: Any, parallel: bool, outermost: bool) -> Bound:
        nest = self.nest
        if loop.mask is not None:
            if element_reads(loop.mask, self.computed) or used(loop.mask) & self.computed:
                raise self.error("a mask can't read values the tile code computes (it is evaluated before the kernel "
                                 "runs)", loop.mask)
            if parallel and element_reads(loop.mask, self.indices):
                raise self.error("a tile mask can't read index arrays: mask the reduction loop's steps instead",
                                 loop.mask)
        args: List[Union[int, ast.expr]] = list(loop.bounds)
        if len(args) == 1:
            args = [0, args[0]]
        if len(args) == 2:
            args.append(1)
        start, stop, step_node = args
        if isinstance(step_node, int):
            step = step_node
        elif self._static(step_node):
            step = self.envs.integer(step_node, f"`{loop.var}`'s step")
        else:
            raise self.error(f"`{loop.var}` steps by an int known when planning", loop.node)
        if step <= 0:
            raise self.error(f"`{loop.var}` steps by {step}: loops count up", loop.node)
        values: List[Union[int, ast.expr]] = []
        for b in (start, stop):
            if isinstance(b, int) or not self._static(b):
                values.append(b)
            else:
                values.append(self.envs.integer(b, f"`{loop.var}`'s bounds"))
        exprs = [b for b in (start, stop) if not isinstance(b, int)]
        if parallel and not all(isinstance(v, int) for v in values):
            loop_reads = set().union(*(used(b) for b in exprs)) & {lp.var for lp in nest.loops}
            if not outermost or loop_reads or set().union(*(used(b) for b in exprs)) & self.computed:
                raise self.error("a parallel loop's bounds are known when planning, except the outermost one's, which "
                                 "may read index arrays (a count of tiles found as the kernel runs)", loop.node)
        b = Bound(loop.var, values[0], values[1], step, loop.mask, loop.node)
        if b.static:
            span = range(b.start, b.stop, step)  # type: ignore[arg-type]
            if len(span) == 0 and parallel:
                raise self.error(f"`{loop.var}` loops over {span}, which is empty", loop.node)
        return b

    @staticmethod
    def _range(b: Bound) -> Range:
        if b.static:
            return Range(b.var, b.start, b.step, max(b.count, 1), b.mask)  # type: ignore[arg-type]
        return Range(b.var, 0, b.step, 1, b.mask, runtime=True)

    # ------------------------------------------------------------------ windows

    def _accesses(self) -> Tuple[Dict[str, Access], Dict[Tuple[int, int, int, int], Access]]:
        """Every tile read of an input, in source order: the same read text is one access."""
        nest = self.nest
        params = {name: k for k, name in enumerate(nest.params)}
        reads = sorted((n for stmt in nest.tile for n in ast.walk(stmt)
                        if isinstance(n, ast.Subscript) and isinstance(n.value, ast.Name)
                        and n.value.id in params and n.value.id not in self.indices),
                       key=lambda n: (n.lineno, n.col_offset))
        found: Dict[str, Access] = {}
        same: Dict[str, Access] = {}
        by_node: Dict[Tuple[int, int, int, int], Access] = {}
        for node in reads:
            key = ast.dump(node)
            if key in same:
                by_node[_pos(node)] = same[key]
                continue
            array = node.value.id  # type: ignore[attr-defined]
            spec = self.inputs[params[array]]
            name = array if not any(a.array == array for a in found.values()) else self._fresh(array, found)
            acc = self._access(name, array, params[array], spec.shape, spec.dtype, index_dims(node), node)
            found[name] = same[key] = by_node[_pos(node)] = acc
        return found, by_node

    def _fresh(self, base: str, taken: Dict[str, Access]) -> str:
        n = 2
        while f"{base}{n}" in taken or f"{base}{n}" in self.nest.params:
            n += 1
        return f"{base}{n}"

    def _access(self, name: str, array: str, param: Optional[int], shape: Sequence[int], dt: DType,
                index: Sequence[ast.expr], node: ast.AST) -> Access:
        text = f"{array}[{', '.join(ast.unparse(i) for i in index)}]"
        if len(index) != len(shape):
            raise self.error(f"{text}: index every one of {array}'s {len(shape)} dims", node)
        dims = tuple(self._dim(i, n, text) for i, n in zip(index, shape))
        # Index arrays (ragged rows, gathers) follow NumPy's rules in JAX: with integer indices they broadcast
        # as one block, whose dims go first unless the block is contiguous. The kernel reads each index along
        # its own dim, which agrees only for one array index next to every integer index.
        arrays = [k for k, d in enumerate(dims) if d.stop is not None or d.gather is not None]
        if len(arrays) > 1:
            raise self.error(f"{text}: a window is placed through one `rows` or index-array slice", node)
        if arrays:
            block = sorted(arrays + [k for k, d in enumerate(dims) if d.size is None])
            if block[-1] - block[0] + 1 != len(block):
                raise self.error(f"{text}: `rows` (or an index-array slice) goes right after the integer indices, with "
                                 "no slice between them (NumPy and JAX would put its rows first)", node)
        kept = [d.size is not None for d in dims]
        if True not in kept:
            raise self.error(f"{text}: a tile keeps at least one dim (slice it, `v:v + 1`)", node)
        return Access(name, array, param, dims, dt, text)

    def _dim(self, index: ast.expr, n: int, text: str) -> Dim:
        usage = (f"{text}: each index is a slice `e : e + size` (size an int when planning), `:`, constants, an "
                 "integer expression, `rows(start, stop, size)`, or an index array's slice `ids[a : a + size]`")
        if isinstance(index, ast.Slice):
            if index.step is not None:
                raise self.error(usage, index)
            lo, hi = index.lower, index.upper
            if lo is None and hi is None:
                return Dim(n, 0)
            if (lo is not None and isinstance(hi, ast.BinOp) and isinstance(hi.op, ast.Add)
                    and ast.dump(hi.left) == ast.dump(lo) and self._static(hi.right)):
                size = self.envs.integer(hi.right, text)
                return self._checked(Dim(size, self._start(lo, text)), n, text, index)
            if (lo is None or self._static(lo)) and (hi is None or self._static(hi)):
                first = 0 if lo is None else self.envs.integer(lo, text)
                stop = n if hi is None else self.envs.integer(hi, text)
                return self._checked(Dim(stop - first, first), n, text, index)
            raise self.error(usage, index)
        if _is_rows_call(self.envs, index):
            call: ast.Call = index  # type: ignore[assignment]
            if len(call.args) != 3 or call.keywords:
                raise self.error("rows takes (start, stop, size)", index)
            if not self._static(call.args[2]):
                raise self.error(f"{text}: rows' size is an int when planning", index)
            size = self.envs.integer(call.args[2], text)
            if size <= 0 or size > n:
                raise self.error(f"{text}: rows of {size} in a dim of {n}", index)
            return Dim(size, self._start(call.args[0], text), stop=call.args[1])
        if isinstance(index, ast.Subscript) and isinstance(index.value, ast.Name) and index.value.id in self.indices:
            sliced = [d for d in index_dims(index) if isinstance(d, ast.Slice)]
            if sliced:
                return Dim(self._gathered(sliced, text), 0, gather=index)
        if isinstance(index, (ast.Slice, ast.Tuple)):
            raise self.error(usage, index)
        return self._checked(Dim(None, self._start(index, text)), n, text, index)

    def _gathered(self, sliced: List[ast.Slice], text: str) -> int:
        """How many elements `ids[..., a : a + n]` gathers (n an int when planning)."""
        usage = f"{text}: a window gathered through an index array slices one of its dims, `ids[a : a + n]`"
        s = sliced[0]
        ok = (len(sliced) == 1 and s.step is None and s.lower is not None and isinstance(s.upper, ast.BinOp)
              and isinstance(s.upper.op, ast.Add) and ast.dump(s.upper.left) == ast.dump(s.lower)
              and self._static(s.upper.right))
        if not ok:
            raise self.error(usage, s)
        return self.envs.integer(s.upper.right, text)  # type: ignore[union-attr]

    def _start(self, node: ast.expr, text: str) -> Union[int, ast.expr]:
        return self.envs.integer(node, text) if self._static(node) else node

    def _checked(self, d: Dim, n: int, text: str, node: ast.AST) -> Dim:
        """A window inside its dim for every value of the static loops its start reads (when planning); starts
        that read what the kernel learns as it runs are clamped by the kernel."""
        width = 1 if d.size is None else d.size
        if width <= 0:
            raise self.error(f"{text}: a slice takes at least one element", node)
        if isinstance(d.start, int):
            starts = [d.start]
        else:
            names = used(d.start)
            loops = [self.bounds[v] for v in sorted(names & set(self.bounds))]
            if names & (set(self.indices) | self.computed) or not all(b.static for b in loops):
                return d
            if math.prod(b.count for b in loops) > _MAX_CHECKED:
                return d
            starts = []
            for values in itertools.product(*(range(b.start, b.stop, b.step) for b in loops)):  # type: ignore[arg-type]
                starts.append(self.envs.eval(d.start, dict(zip((b.var for b in loops), values))))
        for s in starts:
            if not isinstance(s, int) or s < 0 or s + width > n:
                lo, hi = min(starts), max(starts) + width
                raise self.error(f"{text}: reads elements {lo} to {hi - 1} of a dim of {n}", node)
        return d

    def _placed(self, name: str, shape: Tuple[int, ...], dt: DType) -> Access:
        """Where an output's store writes. A window an index array places (an element, a gather, ragged rows)
        may leave parts of the output no tile stores: only an input updated in place keeps its values there."""
        store = self.nest.stores[name]
        acc = self._access(name, name, None, shape, dt, store.index, store.node)
        indexed = set(self.indices) | self.computed
        for d in acc.dims:
            placed_by_index = (d.gather is not None or d.stop is not None
                               or (not isinstance(d.start, int) and bool(used(d.start) & indexed)))
            if placed_by_index and name not in self.aliases:
                raise self.error(f"{acc.text}: an index array places this tile, so no tile might store the rest of "
                                 f"`{name}`: allocate it as an input updated in place (`{name} = x`), whose values the "
                                 "rest keeps", store.node)
        return acc

    # ------------------------------------------------------------------ the trace

    def _load(self, name: str) -> jaxlite.Sym:
        acc = self.accesses[name]
        return jaxlite.leaf("load", acc.shape, acc.dtype, operand=name)

    def _trace_tree(self, by_node: Dict[Tuple[int, int, int, int], Access]
                    ) -> Tuple[Tuple[Block, ...], Dict[str, Carried], Dict[str, Any]]:
        """Trace every block of the tile in the order it runs, settling the types of values kept from one
        block (or iteration) to the next; the kept values' types, and each output's stored value."""
        nest = self.nest
        leaves: List[Sequence[ast.stmt]] = []

        def collect(parts: Sequence[Any]) -> None:
            for p in parts:
                if isinstance(p, Code):
                    leaves.append(p.stmts)
                elif isinstance(p, Reduction):
                    leaves.append(p.body)
                else:
                    collect(p.parts)

        collect(nest.parts)
        loop_vars = {loop.var for loop in nest.loops}
        read_early = set().union(*(used_before_bound(b) for b in leaves)) if leaves else set()
        for loop in nest.loops:  # bounds are evaluated before the loop runs: what they read is kept
            read_early |= set().union(*(used(b) for b in loop.bounds))
        made = set().union(*(bound(b) for b in leaves)) if leaves else set()
        kept_names = (read_early & made) - set(nest.outputs) - loop_vars
        # A window placed by an element of an array the tile computes reads the array as the kernel keeps it:
        # computed in an earlier part of the tile (before the loop that reads the window), not the same one.
        for leaf in leaves:
            here = bound(leaf)
            for stmt in leaf:
                for node in ast.walk(stmt):
                    acc = by_node.get(_pos(node)) if isinstance(node, ast.Subscript) else None
                    if acc is None:
                        continue
                    for d in acc.dims:
                        exprs = [e for e in (d.stop, d.gather) if e is not None]
                        if not isinstance(d.start, int):
                            exprs.append(d.start)
                        late = sorted(set().union(*(used(e) for e in exprs)) & here) if exprs else []
                        if late:
                            raise self.error(f"{acc.text}: a window is placed by `{late[0]}`, which the same part of "
                                             f"the tile computes: compute it before the loop that reads the window",
                                             node)
        types: Dict[str, Tuple[Tuple[int, ...], Any]] = {}
        stores: Dict[str, Any] = {}
        counter = itertools.count()

        def type_of(v: Any, c: str) -> Tuple[Tuple[int, ...], Any]:
            t = _value_type(v)
            if t is None:
                raise self.error(f"`{c}` is kept from one part of the tile to the next, so it must be an array or a "
                                 f"number, not {type(v).__name__}")
            return t

        def scope_of(stmts: Sequence[ast.stmt], carried: Dict[str, Tuple[Tuple[int, ...], Any]]) -> Scope:
            return self._run_scope(f"block{next(counter)}", stmts, carried, loop_vars, {}, by_node)

        def binds_of(stmts: Sequence[ast.stmt]) -> Tuple[str, ...]:
            return tuple(sorted(bound(stmts) & kept_names))

        def leave(scope: Scope, stmts: Sequence[ast.stmt]) -> None:
            for c in binds_of(stmts):
                if c in scope.values:
                    types[c] = type_of(scope.values[c], c)
            stores.update(scope.stores)

        def code(stmts: Sequence[ast.stmt]) -> Block:
            needed = {c: types[c] for c in used_before_bound(stmts) & kept_names if c in types}
            scope = scope_of(stmts, needed)
            leave(scope, stmts)
            return Block("code", scope=scope, binds=binds_of(stmts))

        def reduction(red: Reduction) -> Block:
            needed = {c: types[c] for c in used_before_bound(red.body) & kept_names if c in types}
            for _ in range(4):
                scope = scope_of(red.body, needed)
                after = {c: type_of(scope.values[c], c) for c in needed if c in scope.values}
                changed = {c: t for c, t in after.items() if _type_key(t) != _type_key(needed[c])}
                if not changed:
                    break
                self._settle(needed, changed, red.loop.node)
            else:
                raise self.error("a carried value's type doesn't settle", red.loop.node)
            types.update(needed)
            leave(scope, red.body)
            return Block("loop", scope=scope, loop=red.loop.var, binds=binds_of(red.body))

        def repeat(rep: RepeatLoop) -> Block:
            entry = dict(types)
            for _ in range(4):
                types.clear()
                types.update(entry)
                children = tuple(part(p) for p in rep.parts)
                changed = {c: t for c, t in types.items() if c in entry and _type_key(t) != _type_key(entry[c])}
                if not changed:
                    break
                self._settle(entry, changed, rep.loop.node)
            else:
                raise self.error("a carried value's type doesn't settle", rep.loop.node)
            return Block("repeat", loop=rep.loop.var, children=children)

        def part(p: Any) -> Block:
            if isinstance(p, Code):
                return code(p.stmts)
            if isinstance(p, Reduction):
                return reduction(p)
            return repeat(p)

        tree = tuple(part(p) for p in nest.parts)
        kept = self._kept(tree, kept_names)
        missing = [name for name in nest.outputs if name not in stores]
        if missing:
            raise self.error(f"no tile stores output `{missing[0]}`")
        return tree, kept, stores

    def _settle(self, entry: Dict[str, Tuple[Tuple[int, ...], Any]], changed: Dict[str, Tuple[Tuple[int, ...], Any]],
                node: ast.AST) -> None:
        for c, t in changed.items():
            old = entry[c]
            if isinstance(old[1], DType) and isinstance(t[1], DType) and old[0] != t[0]:
                raise self.error(f"carried value `{c}` changes shape between steps: {old[0]} -> {t[0]}", node)
            entry[c] = t

    def _kept(self, tree: Tuple[Block, ...], names: Set[str]) -> Dict[str, Carried]:
        """Each kept array's one type: every block that reads or assigns it agrees (a name only ever a Python
        number is carried as that number and kept nowhere)."""
        seen: Dict[str, Dict[Any, Tuple[Tuple[int, ...], DType]]] = {}

        def visit(blocks: Sequence[Block]) -> None:
            for b in blocks:
                if b.kind == "repeat":
                    visit(b.children)
                    continue
                scope = b.scope
                assert scope is not None
                for c, leaf in scope.carried_in.items():
                    seen.setdefault(c, {})[(tuple(leaf.shape), leaf.dtype.name)] = (tuple(leaf.shape), leaf.dtype)
                for c in b.binds:
                    v = scope.values.get(c)
                    if isinstance(v, jaxlite.Array):
                        seen.setdefault(c, {})[(tuple(v.shape), v.dtype.name)] = (tuple(v.shape), v.dtype)

        visit(tree)
        kept = {}
        for c in sorted(names):
            kinds = seen.get(c, {})
            if len(kinds) > 1:
                raise self.error(f"`{c}` is kept from one part of the tile to the next with two types: "
                                 + ", ".join(f"{s} {d.name}" for s, d in kinds.values()))
            if kinds:
                shape, dt = next(iter(kinds.values()))
                kept[c] = Carried(c, shape, dt)
        return kept


def static_steps(plan: Plan, limit: int = 1 << 20) -> Optional[int]:
    """How many reduction-loop iterations every tile takes in all (static bounds and masks only), or None."""
    if not all(b.static for b in plan.bounds.values()):
        return None
    nest = plan.nest
    total = 0
    parallel = [plan.bounds[loop.var] for loop in nest.parallel]

    def holds(mask: Optional[ast.expr], values: Dict[str, int]) -> bool:
        return mask is not None and bool(plan.eval(mask, values))

    def walk(blocks: Sequence[Block], values: Dict[str, int]) -> int:
        n = 0
        for b in blocks:
            if b.kind == "code":
                continue
            bd = plan.bounds[b.loop]  # type: ignore[index]
            for v in range(bd.start, bd.stop, bd.step):  # type: ignore[arg-type]
                values[bd.var] = v
                if b.kind == "repeat":
                    n += walk(b.children, values)
                elif not holds(bd.mask, values):
                    n += 1
        return n

    try:
        for tile in itertools.product(*(range(b.start, b.stop, b.step) for b in parallel)):  # type: ignore[arg-type]
            values = {b.var: v for b, v in zip(parallel, tile)}
            if any(holds(b.mask, values) for b in parallel):
                continue
            total += walk(plan.tree, values)
            if total > limit:
                return None
    except (KernelError, RuntimeError, TypeError):
        return None  # a mask reading an index array: known only when the kernel runs
    return total
