"""Name analysis of kernel code, over Python's `ast`.

Tile code is straight-line: assignments, augmented assignments, output stores and `with` blocks of those
(parse.py enforces it), so "in the order it runs" is the order it is written, a `with` block's statements
running where the block stands. The questions the compiler asks of it:

- which names an expression uses (`used`), honouring the scopes Python gives lambdas and comprehensions;
- which names statements bind (`bound`), and which they use before binding them (`used_before_bound`);
- which subscripts read one element of an array (`element_reads`: integer indices only, `lengths[b]`);
- whether a statement is an output store, `out = out.at[index].set(value)` (`store_of`).

The rules are those of the reference's tile code (src/autokernel/tilecode.py:17-136); this module is the
backend's own implementation of them.
"""

from __future__ import annotations

import ast
from dataclasses import dataclass
from typing import AbstractSet, FrozenSet, Iterable, Iterator, List, Optional, Set, Tuple

__all__ = ["Store", "bound", "element_reads", "index_dims", "in_order", "store_of", "used",
           "used_before_bound"]


@dataclass(frozen=True)
class Store:
    """`out = out.at[index].set(value)`: one tile of an output written."""

    output: str
    index: Tuple[ast.expr, ...]
    value: ast.expr
    node: ast.Assign


def index_dims(sub: ast.Subscript) -> List[ast.expr]:
    """The per-dimension index expressions of a subscript (`a[i, j:k]` -> [i, j:k])."""
    s = sub.slice
    return list(s.elts) if isinstance(s, ast.Tuple) else [s]


def store_of(stmt: ast.stmt) -> Optional[Store]:
    """`stmt` as an output store, or None. The shape is fixed: one name target, assigned the result of
    `<same name>.at[<index>].set(<value>)` with one positional argument."""
    if not isinstance(stmt, ast.Assign) or len(stmt.targets) != 1:
        return None
    target, call = stmt.targets[0], stmt.value
    if not isinstance(target, ast.Name) or not isinstance(call, ast.Call):
        return None
    if len(call.args) != 1 or call.keywords:
        return None
    method = call.func
    if not isinstance(method, ast.Attribute) or method.attr != "set":
        return None
    at_index = method.value
    if not isinstance(at_index, ast.Subscript):
        return None
    at = at_index.value
    if not (isinstance(at, ast.Attribute) and at.attr == "at" and isinstance(at.value, ast.Name)):
        return None
    if at.value.id != target.id:
        return None
    return Store(target.id, tuple(index_dims(at_index)), call.args[0], stmt)


def in_order(stmts: Iterable[ast.stmt]) -> Iterator[ast.stmt]:
    """Every statement in the order it runs: a `with` statement, then its body's statements."""
    stack: List[Iterator[ast.stmt]] = [iter(stmts)]
    while stack:
        stmt = next(stack[-1], None)
        if stmt is None:
            stack.pop()
            continue
        yield stmt
        if isinstance(stmt, ast.With):
            stack.append(iter(stmt.body))


def _target_names(target: ast.AST) -> Set[str]:
    return {n.id for n in ast.walk(target) if isinstance(n, ast.Name)}


def _free(node: ast.AST, hidden: FrozenSet[str], out: Set[str]) -> None:
    """Add to `out` the names `node` loads that are not `hidden` by an enclosing lambda or comprehension."""
    if isinstance(node, ast.Name):
        if not isinstance(node.ctx, ast.Store) and node.id not in hidden:
            out.add(node.id)
        return
    if isinstance(node, ast.Lambda):
        a = node.args
        for d in [*a.defaults, *a.kw_defaults]:
            if d is not None:
                _free(d, hidden, out)
        params = {p.arg for p in [*a.posonlyargs, *a.args, *a.kwonlyargs]}
        params |= {p.arg for p in (a.vararg, a.kwarg) if p is not None}
        _free(node.body, hidden | params, out)
        return
    if isinstance(node, (ast.ListComp, ast.SetComp, ast.GeneratorExp, ast.DictComp)):
        inner = hidden
        for k, gen in enumerate(node.generators):
            # The first iterable is evaluated outside the comprehension; the rest see earlier targets.
            _free(gen.iter, hidden if k == 0 else inner, out)
            inner = inner | _target_names(gen.target)
            for cond in gen.ifs:
                _free(cond, inner, out)
        parts = (node.key, node.value) if isinstance(node, ast.DictComp) else (node.elt,)
        for part in parts:
            _free(part, inner, out)
        return
    for child in ast.iter_child_nodes(node):
        _free(child, hidden, out)


def used(node: ast.AST) -> Set[str]:
    """The names `node` reads. For a statement, only what it evaluates: an assignment's value (`a += b`
    reads `a` too), a `with` statement's context expressions (not its body)."""
    out: Set[str] = set()
    if isinstance(node, ast.Assign):
        _free(node.value, frozenset(), out)
    elif isinstance(node, ast.AugAssign):
        _free(node.value, frozenset(), out)
        out |= _target_names(node.target)
    elif isinstance(node, ast.AnnAssign):
        if node.value is not None:
            _free(node.value, frozenset(), out)
    elif isinstance(node, ast.With):
        for item in node.items:
            _free(item.context_expr, frozenset(), out)
    else:
        _free(node, frozenset(), out)
    return out


def _binds(stmt: ast.stmt) -> Set[str]:
    if isinstance(stmt, ast.Assign):
        return set().union(*(_target_names(t) for t in stmt.targets))
    if isinstance(stmt, (ast.AugAssign, ast.AnnAssign)):
        return _target_names(stmt.target)
    return set()


def bound(stmts: Iterable[ast.stmt]) -> Set[str]:
    """The names `stmts` bind (in `with` bodies too)."""
    names: Set[str] = set()
    for stmt in in_order(stmts):
        names |= _binds(stmt)
    return names


def used_before_bound(stmts: Iterable[ast.stmt]) -> Set[str]:
    """The names `stmts` read at a point where they have not bound them yet."""
    seen: Set[str] = set()
    early: Set[str] = set()
    for stmt in in_order(stmts):
        early |= used(stmt) - seen
        seen |= _binds(stmt)
    return early


def element_reads(node: ast.AST, arrays: AbstractSet[str] | Iterable[str]) -> List[ast.Subscript]:
    """The subscripts in `node` that read one element of one of `arrays`: every index an expression, none a
    slice (`lengths[b]`, `tables[b, p]`), in walk order."""
    names = arrays if isinstance(arrays, (set, frozenset)) else set(arrays)
    found = []
    for n in ast.walk(node):
        if isinstance(n, ast.Subscript) and isinstance(n.value, ast.Name) and n.value.id in names:
            if all(not isinstance(d, ast.Slice) for d in index_dims(n)):
                found.append(n)
    return found
