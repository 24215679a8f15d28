"""`kernel.reference`: what a kernel computes, by running its loop nest as plain (jaxlite) JAX.

The reference (src/autokernel/reference.py:25-47) defines it as the user's function with one change: `@`
means what it means in the kernel, a product accumulating in f32. Here that function is run by a small
interpreter of the parsed nest rather than recompiled: the prologue, then every tile of the parallel loops
(tile masks skip tiles), and in each tile its code and reduction loops in order (step masks skip steps),
all under `jaxlite.matrix_units()`, so `@` accumulates in f32 and `a @ b.T` contracts both last dims.

One thing differs from running the function, for speed and not meaning: an output store
`out = out.at[index].set(value)` writes into the output's own buffer. An output is allocated fresh in the
prologue (an input updated in place, `new = pool`, is copied first) and tile code never reads it (parse.py
checks), so no one can see the difference; a functional copy per tile would copy a whole 8192^2 output once
per tile.

Module and closure values are read as they are when the reference is made (when the kernel is built for a
signature), as the kernel's constants are.
"""

from __future__ import annotations

import ast
import builtins
import inspect
from typing import Any, Callable, Dict, List, Optional, Sequence, Union

from . import jaxlite
from .parse import Code, Loop, Nest, Reduction, RepeatLoop
from .syntax import store_of

__all__ = ["make_reference"]

_KEY = "__tilejax_index_key__"


class _Key:
    """`KEY[index]` is `index`: how a store's index expression (slices and all) is evaluated."""

    def __getitem__(self, index: Any) -> Any:
        return index


class _Run:
    """Statements compiled once: straight-line code as one code object, an output store as its index and
    value expressions, a `with` block as its context expression and its body's steps."""

    def __init__(self, stmts: Sequence[ast.stmt], outputs: set, filename: str) -> None:
        self.steps: List[Any] = []
        pending: List[ast.stmt] = []

        def flush() -> None:
            if pending:
                module = ast.fix_missing_locations(ast.Module(list(pending), []))
                self.steps.append(("exec", compile(module, filename, "exec")))
                pending.clear()

        for stmt in stmts:
            store = store_of(stmt)
            if store is not None and store.output in outputs:
                flush()
                # `KEY[<the store's index>]` evaluates to the index itself (slices included)
                dims = list(store.index)
                key = dims[0] if len(dims) == 1 else ast.Tuple(dims, ast.Load())
                index = ast.copy_location(ast.Subscript(ast.Name(_KEY, ast.Load()), key, ast.Load()), stmt)
                index = ast.fix_missing_locations(index)
                value = ast.fix_missing_locations(ast.Expression(store.value))
                self.steps.append(("store", store.output,
                                   compile(ast.Expression(index), filename, "eval"),
                                   compile(value, filename, "eval")))
            elif isinstance(stmt, ast.With) and any(store_of(s) for s in ast.walk(stmt) if isinstance(s, ast.stmt)):
                flush()
                contexts = [compile(ast.fix_missing_locations(ast.Expression(i.context_expr)), filename, "eval")
                            for i in stmt.items]
                self.steps.append(("with", contexts, _Run(stmt.body, outputs, filename)))
            else:
                pending.append(stmt)
        flush()

    def __call__(self, env: Dict[str, Any]) -> None:
        for step in self.steps:
            kind = step[0]
            if kind == "exec":
                exec(step[1], env)
            elif kind == "store":
                _, name, index, value = step
                jaxlite.store_(env[name], eval(index, env), eval(value, env))
            else:
                _, contexts, body = step
                managers = [eval(c, env) for c in contexts]
                for m in managers:
                    m.__enter__()
                try:
                    body(env)
                finally:
                    for m in reversed(managers):
                        m.__exit__(None, None, None)


class _LoopCode:
    """A loop's bounds and mask, compiled."""

    def __init__(self, loop: Loop, filename: str) -> None:
        self.var = loop.var
        self.bounds = [compile(ast.fix_missing_locations(ast.Expression(b)), filename, "eval") for b in loop.bounds]
        self.mask = None
        if loop.mask is not None:
            self.mask = compile(ast.fix_missing_locations(ast.Expression(loop.mask)), filename, "eval")

    def values(self, env: Dict[str, Any]) -> range:
        return range(*(int(eval(b, env)) for b in self.bounds))

    def skips(self, env: Dict[str, Any]) -> bool:
        return self.mask is not None and bool(eval(self.mask, env))


class _Interpreter:
    def __init__(self, nest: Nest, fn: Callable) -> None:
        self.nest = nest
        outputs = set(nest.outputs)
        f = nest.filename
        scope: Dict[str, Any] = {"__builtins__": builtins}
        scope.update(fn.__globals__)
        scope.update(inspect.getclosurevars(fn).nonlocals)
        scope[_KEY] = _Key()
        self.scope = scope
        self.prologue = _Run(nest.prologue, set(), f)
        self.parallel = [_LoopCode(loop, f) for loop in nest.parallel]
        self.parts: List[Any] = [self._part(p, outputs, f) for p in nest.parts]

    def _part(self, part: Union[Code, Reduction, RepeatLoop], outputs: set, f: str) -> Any:
        if isinstance(part, Code):
            return ("code", _Run(part.stmts, outputs, f))
        if isinstance(part, Reduction):
            return ("reduce", _LoopCode(part.loop, f), _Run(part.body, outputs, f))
        return ("repeat", _LoopCode(part.loop, f), [self._part(p, outputs, f) for p in part.parts])

    def _run_parts(self, parts: Sequence[Any], env: Dict[str, Any]) -> None:
        for part in parts:
            if part[0] == "code":
                part[1](env)
                continue
            loop = part[1]
            for value in loop.values(env):
                env[loop.var] = value
                if part[0] == "reduce":
                    if not loop.skips(env):
                        part[2](env)
                else:
                    self._run_parts(part[2], env)

    def _tiles(self, depth: int, env: Dict[str, Any]) -> None:
        if depth == len(self.parallel):
            self._run_parts(self.parts, dict(env))
            return
        loop = self.parallel[depth]
        for value in loop.values(env):
            env[loop.var] = value
            if not loop.skips(env):
                self._tiles(depth + 1, env)

    def __call__(self, *args: Any) -> Any:
        nest = self.nest
        env = dict(self.scope)
        env.update(zip(nest.params, args))
        if nest.tunable:
            env[nest.tunable] = args[len(nest.params)] if len(args) > len(nest.params) else None
        with jaxlite.matrix_units():
            self.prologue(env)
            inputs = {id(a) for a in args}
            for name in nest.outputs:  # an input updated in place: its own copy (the input stays as it was)
                if id(env[name]) in inputs:
                    env[name] = jaxlite.Array(env[name].t.clone())
            self._tiles(0, env)
        outs = tuple(env[name] for name in nest.outputs)
        return outs if len(outs) > 1 else outs[0]


def make_reference(nest: Nest, fn: Callable) -> Callable[..., Any]:
    """The loop nest of `fn` as a function over jaxlite arrays (then the tunable, if it has one), with `@` on
    matrix units, reading the module's and closure's values as they are now."""
    return _Interpreter(nest, fn)
