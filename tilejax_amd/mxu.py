"""What `@` means in kernel code: a matrix-core product accumulating in f32 (i32 for integers).

Plain JAX rounds `bf16 @ bf16` to bf16; an MFMA accumulates in f32, and so do kernels. The kernel, the
plan's type trace and the reference all compute `@` with these functions, so they agree. Same meaning as
the reference's (src/autokernel/mxu.py:21-43): mixed operand types are promoted first; f32 operands keep
full precision; `a @ b.T` contracts both last dims, the lowering reading `b` transposed in place.
"""

from __future__ import annotations

import ast
from typing import Any

from .jaxlite import Array, jnp, matmul, matmul_nt, promote_types

__all__ = ["DOT", "DOT_NT", "FUNCTIONS", "rewrite_matmuls"]

DOT = "_mxu_dot"
DOT_NT = "_mxu_dot_nt"


def _mxu_operands(x: Any, y: Any):
    if x.dtype != y.dtype:
        common = promote_types(x.dtype, y.dtype)
        x, y = x.astype(common), y.astype(common)
    acc = jnp.int32 if x.dtype.kind in "iu" else jnp.float32
    return x, y, acc


def _mxu_dot(x: Any, y: Any) -> Array:
    """`x @ y`, accumulating in f32 (i32 for integers)."""
    x, y, acc = _mxu_operands(x, y)
    return matmul(x, y, preferred_element_type=acc)


def _mxu_dot_nt(x: Any, y: Any) -> Array:
    """`x @ y.T`: for two matrices, contract both last dims."""
    if x.ndim != 2 or y.ndim != 2:
        return _mxu_dot(x, y.T)
    x, y, acc = _mxu_operands(x, y)
    return matmul_nt(x, y, preferred_element_type=acc)


FUNCTIONS = {DOT: _mxu_dot, DOT_NT: _mxu_dot_nt}


class _MatmulRewriter(ast.NodeTransformer):
    def visit_BinOp(self, node: ast.BinOp) -> ast.expr:
        self.generic_visit(node)
        if not isinstance(node.op, ast.MatMult):
            return node
        right = node.right
        if isinstance(right, ast.Attribute) and right.attr == "T":
            call = _call(DOT_NT, node.left, right.value)
        else:
            call = _call(DOT, node.left, right)
        return ast.copy_location(call, node)

    def visit_AugAssign(self, node: ast.AugAssign) -> ast.stmt:
        self.generic_visit(node)
        if not isinstance(node.op, ast.MatMult):
            return node
        target = ast.Name(node.target.id, ast.Store())  # type: ignore[union-attr]
        product = self.visit_BinOp(ast.BinOp(ast.Name(node.target.id, ast.Load()), ast.MatMult(), node.value))  # type: ignore[union-attr]
        return ast.copy_location(ast.Assign([target], product), node)


def _call(name: str, *args: ast.expr) -> ast.Call:
    return ast.Call(ast.Name(name, ast.Load()), list(args), [])


def rewrite_matmuls(tree: ast.AST) -> ast.AST:
    """`tree` with `a @ b` a call of `_mxu_dot`, `a @ b.T` of `_mxu_dot_nt` (in place; returned)."""
    tree = _MatmulRewriter().visit(tree)
    ast.fix_missing_locations(tree)
    return tree
