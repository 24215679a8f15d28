"""The reference a kernel is checked against: the kernel function itself, run as plain (jaxlite) JAX.

As in the reference (src/autokernel/reference.py:25-47), the only change to the user's function is that
`@` means what it means in the kernel (mxu.py): a product accumulating in f32. One more change here, for
speed and not meaning: output stores `out = out.at[...].set(v)` write into the output's own buffer. An
output is allocated fresh in the prologue (`jnp.zeros`/`jnp.full`) and tile code never reads it
(parse.py), so no one can see the difference; a functional copy per tile would make the 8192^2 reference
copy the whole output once per tile.
"""

from __future__ import annotations

import ast
import copy
from typing import Any, Callable

from . import jaxlite, mxu
from .parse import Nest
from .tilecode import as_store

__all__ = ["make_reference"]

_STORE = "__tilejax_store_into__"
_INDEX = "__tilejax_index_of__"


class _IndexOf:
    def __getitem__(self, index: Any) -> Any:
        return index


class _InPlaceStores(ast.NodeTransformer):
    def __init__(self, outputs: set) -> None:
        self.outputs = outputs

    def visit_Assign(self, node: ast.Assign) -> ast.stmt:
        store = as_store(node)
        if store is None or store.output not in self.outputs:
            self.generic_visit(node)
            return node
        index = node.value.func.value.slice  # type: ignore[attr-defined]
        call = ast.Call(
            ast.Name(_STORE, ast.Load()),
            [ast.Name(store.output, ast.Load()), ast.Subscript(ast.Name(_INDEX, ast.Load()), index, ast.Load()),
             self.visit(store.value)],
            [],
        )
        return ast.copy_location(ast.Assign([ast.Name(store.output, ast.Store())], call), node)


def make_reference(nest: Nest, fn: Callable) -> Callable[..., Any]:
    """`fn` over jaxlite arrays with `@` as the matrix-core product, reading the module's and closure's
    values as they are now (as the kernel built now does)."""
    fdef = copy.deepcopy(nest.function)
    fdef.decorator_list = []
    fdef.args.defaults = []
    at = next(i for i, stmt in enumerate(fdef.body) if isinstance(stmt, ast.For))
    loop = _InPlaceStores(set(nest.outputs)).visit(fdef.body[at])
    fdef.body[at] = mxu.rewrite_matmuls(loop)
    free = fn.__code__.co_freevars
    maker = ast.FunctionDef(
        name="__make__",
        args=ast.arguments([], [ast.arg(name) for name in free], None, [], [], None, []),
        body=[fdef, ast.Return(ast.Name(fdef.name, ast.Load()))],
        decorator_list=[],
        returns=None,
    )
    module = ast.fix_missing_locations(ast.Module([ast.copy_location(maker, fdef)], []))
    namespace = {**fn.__globals__, **mxu.FUNCTIONS, _STORE: jaxlite.store_, _INDEX: _IndexOf()}
    exec(compile(module, nest.filename, "exec"), namespace)
    cells = [cell.cell_contents for cell in fn.__closure__ or ()]
    return namespace["__make__"](*cells)
