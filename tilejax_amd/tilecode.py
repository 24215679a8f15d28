"""Name analysis of tile code: the statements a tile runs, the names they read and assign, output stores.

Tile statements are assignments, augmented assignments, output stores and `with jax.named_scope(...)`
blocks of those (parse.py checks), so every analysis here is straight-line. Same rules as the reference's
tilecode (src/autokernel/tilecode.py:17-136).
"""

from __future__ import annotations

import ast
from dataclasses import dataclass
from typing import Iterable, Iterator, List, Optional, Set, Tuple

__all__ = ["Store", "as_store", "assigned", "element_reads", "first_reads", "flatten", "reads"]


@dataclass(frozen=True)
class Store:
    """`out = out.at[index].set(value)`: writing a tile of an output."""

    output: str
    index: Tuple[ast.expr, ...]
    value: ast.expr
    node: ast.Assign


def as_store(stmt: ast.stmt) -> Optional[Store]:
    """The output store `stmt` is, or None."""
    if not (isinstance(stmt, ast.Assign) and len(stmt.targets) == 1 and isinstance(stmt.targets[0], ast.Name)):
        return None
    call = stmt.value
    if not (isinstance(call, ast.Call) and len(call.args) == 1 and not call.keywords):
        return None
    func = call.func
    if not (isinstance(func, ast.Attribute) and func.attr == "set" and isinstance(func.value, ast.Subscript)):
        return None
    at = func.value.value
    if not (isinstance(at, ast.Attribute) and at.attr == "at" and isinstance(at.value, ast.Name)):
        return None
    if at.value.id != stmt.targets[0].id:
        return None
    index = func.value.slice
    dims = tuple(index.elts) if isinstance(index, ast.Tuple) else (index,)
    return Store(at.value.id, dims, call.args[0], stmt)


def subscript_dims(node: ast.Subscript) -> List[ast.expr]:
    return list(node.slice.elts) if isinstance(node.slice, ast.Tuple) else [node.slice]


def element_reads(node: ast.AST, arrays: Iterable[str]) -> List[ast.Subscript]:
    """Reads of single elements of `arrays` in `node`: subscripts without slices, `lengths[b]`."""
    names = set(arrays)
    return [
        n
        for n in ast.walk(node)
        if isinstance(n, ast.Subscript)
        and isinstance(n.value, ast.Name)
        and n.value.id in names
        and not any(isinstance(i, ast.Slice) for i in subscript_dims(n))
    ]


def flatten(stmts: Iterable[ast.stmt]) -> Iterator[ast.stmt]:
    """`stmts` in the order they run, each `with` block followed by its statements."""
    for stmt in stmts:
        yield stmt
        if isinstance(stmt, ast.With):
            yield from flatten(stmt.body)


class _Reads(ast.NodeVisitor):
    def __init__(self) -> None:
        self.names: Set[str] = set()

    def visit_Name(self, node: ast.Name) -> None:
        self.names.add(node.id)

    def visit_Lambda(self, node: ast.Lambda) -> None:
        for default in [*node.args.defaults, *[d for d in node.args.kw_defaults if d is not None]]:
            self.visit(default)
        params = {a.arg for a in ast.walk(node.args) if isinstance(a, ast.arg)}
        self.names |= reads(node.body) - params

    def _comprehension(self, node: ast.AST) -> None:
        bound: Set[str] = set()
        inner: Set[str] = set()
        for gen in node.generators:  # type: ignore[attr-defined]
            bound |= {n.id for n in ast.walk(gen.target) if isinstance(n, ast.Name)}
            inner |= reads(gen.iter)
            for cond in gen.ifs:
                inner |= reads(cond)
        parts = (node.key, node.value) if isinstance(node, ast.DictComp) else (node.elt,)  # type: ignore[attr-defined]
        for part in parts:
            inner |= reads(part)
        self.names |= inner - bound

    visit_ListComp = visit_SetComp = visit_GeneratorExp = visit_DictComp = _comprehension


def reads(node: ast.AST) -> Set[str]:
    """The names an expression reads (a statement: its own expressions; `a += b` reads `a` too)."""
    visitor = _Reads()
    if isinstance(node, ast.With):
        for item in node.items:
            visitor.visit(item.context_expr)
    elif isinstance(node, ast.AugAssign):
        visitor.visit(node.value)
        visitor.names.add(node.target.id)  # type: ignore[union-attr]
    elif isinstance(node, ast.Assign):
        visitor.visit(node.value)
    else:
        visitor.visit(node)
    return visitor.names


def _assigns(stmt: ast.stmt) -> Set[str]:
    if isinstance(stmt, ast.Assign):
        return {n.id for t in stmt.targets for n in ast.walk(t) if isinstance(n, ast.Name)}
    if isinstance(stmt, ast.AugAssign):
        return {stmt.target.id}  # type: ignore[union-attr]
    return set()


def assigned(stmts: Iterable[ast.stmt]) -> Set[str]:
    """The names `stmts` assign."""
    return {name for stmt in flatten(stmts) for name in _assigns(stmt)}


def first_reads(stmts: Iterable[ast.stmt]) -> Set[str]:
    """The names `stmts` read before assigning them."""
    needed: Set[str] = set()
    done: Set[str] = set()
    for stmt in flatten(stmts):
        needed |= reads(stmt) - done
        done |= _assigns(stmt)
    return needed
