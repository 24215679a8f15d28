"""Tile code as C expressions: pointwise emission of traced IR, integer expressions of loop values, and
interval analysis of conditions over a rectangle of a tile.

A pointwise value of a tile is computed element by element where the element lives (a register of the
MFMA accumulator layout, or a lane's share of a row): each Node becomes one C local, named `v<id>`, of the
C type of its dtype. bf16 and f16 intermediates are kept in float registers but rounded to their type
after every operation, so the kernel computes what the traced code computes. Leaves are supplied by the
caller (`leaves`): the accumulator element, the row/column of the element, loop values, index elements.
"""

from __future__ import annotations

import ast
import math
import struct
from typing import Any, Callable, Dict, List, Optional, Sequence, Set, Tuple

from ..errors import KernelError
from .. import jaxlite
from ..jaxlite import DType, Node

__all__ = ["CExpr", "Emitter", "int_expr", "literal", "nodes_between", "depends_on"]


def literal(value: Any, dt: Optional[DType] = None) -> str:
    """A C literal for a Python number (as a float, int or bool constant)."""
    if isinstance(value, bool):
        return "true" if value else "false"
    if dt is not None and dt.kind == "u":
        return f"{int(value)}u"
    if dt is not None and dt.kind in "iu":
        return f"{int(value)}"
    if isinstance(value, int) and (dt is None or dt.kind in "iub"):
        return f"{value}"
    value = float(value)
    if math.isnan(value):
        return "__builtin_nanf(\"\")"
    if math.isinf(value):
        return "__builtin_inff()" if value > 0 else "(-__builtin_inff())"
    bits = struct.unpack("<I", struct.pack("<f", value))[0]
    return f"__builtin_bit_cast(float, 0x{bits:08x}u) /* {value!r} */"


def ctype(dt: DType) -> str:
    if dt.kind == "f":
        return "double" if dt.itemsize == 8 else "float"
    if dt.kind == "b":
        return "bool"
    if dt.kind == "u":
        return "unsigned" if dt.itemsize <= 4 else "unsigned long long"
    return "int" if dt.itemsize <= 4 else "long long"


def _rounded(expr: str, dt: DType) -> str:
    """`expr` (a float) rounded to `dt`'s precision when `dt` is narrower than f32."""
    if dt.name == "bfloat16":
        return f"ak_round_bf16({expr})"
    if dt.name == "float16":
        return f"ak_round_f16({expr})"
    return expr


def depends_on(node: Node, targets: Set[int]) -> bool:
    """Does `node` read (transitively) any Node whose id is in `targets`?"""
    seen: Set[int] = set()
    stack = [node]
    while stack:
        n = stack.pop()
        if n.id in seen:
            continue
        seen.add(n.id)
        if n.id in targets:
            return True
        stack.extend(n.inputs())
    return False


def nodes_between(root: Node) -> List[Node]:
    """The Nodes `root` reads (transitively) and itself, in an order where each follows its inputs."""
    order: List[Node] = []
    seen: Set[int] = set()

    def visit(n: Node) -> None:
        if n.id in seen:
            return
        seen.add(n.id)
        for i in n.inputs():
            visit(i)
        order.append(n)

    visit(root)
    return order


_BINARY = {"add": "+", "subtract": "-", "multiply": "*", "bitwise_and": "&", "bitwise_or": "|", "bitwise_xor": "^",
           "left_shift": "<<", "right_shift": ">>"}
_COMPARE = {"less": "<", "less_equal": "<=", "greater": ">", "greater_equal": ">=", "equal": "==", "not_equal": "!="}


class CExpr:
    """A C expression and its dtype (or a Python scalar: weakly typed)."""

    def __init__(self, text: str, dt: Optional[DType], scalar: Any = None) -> None:
        self.text, self.dtype, self.scalar = text, dt, scalar


class Emitter:
    """Emit the pointwise computation of Nodes as C statements.

    `leaves(node)` gives the C expression of a leaf (or of any Node the caller computes itself), or None.
    `shape` is the shape of the values being computed: a Node of a different shape must broadcast to it.
    """

    def __init__(self, leaves: Callable[[Node], Optional[str]], shape: Sequence[int], prefix: str = "v") -> None:
        self.leaves, self.shape, self.prefix = leaves, tuple(shape), prefix
        self.lines: List[str] = []
        self.done: Dict[int, str] = {}
        # values are numbered in the order they are emitted (not by Node id, which depends on what was traced
        # before), so one nest's source is the same text in every process
        self.count = 0

    def value(self, arg: Any, want: Optional[DType] = None) -> str:
        if isinstance(arg, Node):
            return self.emit(arg)
        if isinstance(arg, (bool, int, float)):
            return literal(arg, want)
        raise KernelError(f"the gfx950 lowering can't compute {arg!r} in tile code")

    def emit(self, node: Node) -> str:
        """The C name of `node`'s value at the current element (emitting what it needs first)."""
        if node.id in self.done:
            return self.done[node.id]
        leaf = self.leaves(node)
        if leaf is not None:
            self.done[node.id] = leaf
            return leaf
        text = self._op(node)
        name = f"{self.prefix}_{self.count}"
        self.count += 1
        self.lines.append(f"const {ctype(node.dtype)} {name} = {text};")
        self.done[node.id] = name
        return name

    def _args_dtype(self, node: Node) -> DType:
        return node.dtype

    def _op(self, n: Node) -> str:
        op, a, dt = n.op, n.args, n.dtype
        if op in _BINARY:
            x, y = self.value(a[0], dt), self.value(a[1], dt)
            if dt.kind == "f":
                return _rounded(f"(({ctype(dt)}){x} {_BINARY[op]} ({ctype(dt)}){y})", dt)
            return f"(({ctype(dt)}){x} {_BINARY[op]} ({ctype(dt)}){y})"
        if op in _COMPARE:
            return f"({self.value(a[0])} {_COMPARE[op]} {self.value(a[1])})"
        if op == "divide":
            x, y = self.value(a[0], dt), self.value(a[1], dt)
            return _rounded(f"(({ctype(dt)}){x} / ({ctype(dt)}){y})", dt)
        if op == "floor_divide":
            x, y = self.value(a[0], dt), self.value(a[1], dt)
            if dt.kind in "iu":
                return f"ak_floordiv({x}, {y})"
            return _rounded(f"floorf(({ctype(dt)}){x} / ({ctype(dt)}){y})", dt)
        if op == "remainder":
            x, y = self.value(a[0], dt), self.value(a[1], dt)
            if dt.kind in "iu":
                return f"ak_floormod({x}, {y})"
            raise KernelError("float remainders are not lowered for gfx950")
        if op in ("maximum", "minimum"):
            fn = "fmaxf" if op == "maximum" else "fminf"
            x, y = self.value(a[0], dt), self.value(a[1], dt)
            if dt.kind == "f":
                return _rounded(f"ak_{op}(({ctype(dt)}){x}, ({ctype(dt)}){y})", dt)
            return f"(({x}) {'>' if op == 'maximum' else '<'} ({y}) ? ({x}) : ({y}))"
        if op in ("logical_and", "logical_or"):
            return f"({self.value(a[0])} {'&&' if op == 'logical_and' else '||'} {self.value(a[1])})"
        if op == "logical_not":
            return f"(!{self.value(a[0])})"
        if op == "invert":
            return f"(~{self.value(a[0])})" if dt.kind != "b" else f"(!{self.value(a[0])})"
        if op == "negative":
            return f"(-{self.value(a[0], dt)})"
        if op == "abs":
            return f"fabsf({self.value(a[0], dt)})" if dt.kind == "f" else f"abs({self.value(a[0])})"
        if op == "where":
            c, x, y = self.value(a[0]), self.value(a[1], dt), self.value(a[2], dt)
            return f"({c} ? ({ctype(dt)})({x}) : ({ctype(dt)})({y}))"
        if op == "astype":
            x = self.value(a[0])
            src = a[0].dtype if isinstance(a[0], Node) else None
            if dt.kind == "f":
                return _rounded(f"({ctype(dt)})({x})", dt)
            if dt.kind == "b":
                return f"(({x}) != 0)"
            return f"({ctype(dt)})({x})"
        if op in ("exp", "exp2", "log", "sqrt", "rsqrt", "tanh", "sigmoid", "reciprocal", "square", "sign"):
            x = self.value(a[0], dt)
            fn = {"exp": "ak_exp", "exp2": "ak_exp2", "log": "__logf", "sqrt": "sqrtf", "rsqrt": "ak_rsqrt",
                  "tanh": "tanhf", "sigmoid": "ak_sigmoid", "reciprocal": "ak_rcp", "square": "ak_square",
                  "sign": "ak_sign"}[op]
            return _rounded(f"{fn}((float)({x}))", dt)
        if op == "tile":
            x = a[0]
            if isinstance(x, Node) and _broadcasts(x.shape, self.shape, tile=a[1]):
                return self.value(x)
            raise KernelError("jnp.tile of a value that varies along a tiled dim is not pointwise")
        if op == "broadcast_to":
            return self.value(a[0])
        if op == "reshape" and isinstance(a[0], Node) and _same_elements(a[0].shape, n.shape):
            return self.value(a[0])
        raise KernelError(f"the gfx950 lowering has no pointwise form of `{op}` here")


def _same_elements(a: Tuple[int, ...], b: Tuple[int, ...]) -> bool:
    """Reshapes that only add or drop dims of one keep every element where it is."""
    return [d for d in a if d != 1] == [d for d in b if d != 1]


def _broadcasts(shape: Tuple[int, ...], target: Tuple[int, ...], tile: Any = None) -> bool:
    return all(s == 1 or s == t for s, t in zip(shape[::-1], target[::-1]))


def int_expr(node: ast.expr, names: Callable[[str], Optional[str]], index: Callable[[ast.Subscript], str]) -> str:
    """C for an integer Python expression of loop variables, constants and index-array elements (masks,
    runtime window indices): `//` and `%` are floor division and modulo, as in Python."""

    def go(n: ast.expr) -> str:
        if isinstance(n, ast.Constant) and isinstance(n.value, (bool, int)):
            return literal(n.value)
        if isinstance(n, ast.Name):
            got = names(n.id)
            if got is None:
                raise KernelError(f"`{n.id}` can't be read here by the gfx950 lowering")
            return got
        if isinstance(n, ast.Subscript):
            return index(n)
        if isinstance(n, ast.BinOp):
            x, y = go(n.left), go(n.right)
            if isinstance(n.op, ast.FloorDiv):
                return f"ak_floordiv({x}, {y})"
            if isinstance(n.op, ast.Mod):
                return f"ak_floormod({x}, {y})"
            ops = {ast.Add: "+", ast.Sub: "-", ast.Mult: "*", ast.BitAnd: "&", ast.BitOr: "|", ast.BitXor: "^",
                   ast.LShift: "<<", ast.RShift: ">>"}
            if type(n.op) in ops:
                return f"({x} {ops[type(n.op)]} {y})"
        if isinstance(n, ast.UnaryOp):
            x = go(n.operand)
            if isinstance(n.op, ast.USub):
                return f"(-{x})"
            if isinstance(n.op, ast.Not):
                return f"(!{x})"
            if isinstance(n.op, ast.UAdd):
                return x
        if isinstance(n, ast.Compare):
            ops = {ast.Lt: "<", ast.LtE: "<=", ast.Gt: ">", ast.GtE: ">=", ast.Eq: "==", ast.NotEq: "!="}
            parts, left = [], go(n.left)
            for op, right in zip(n.ops, n.comparators):
                r = go(right)
                if type(op) not in ops:
                    break
                parts.append(f"({left} {ops[type(op)]} {r})")
                left = r
            else:
                return "(" + " && ".join(parts) + ")"
        if isinstance(n, ast.BoolOp):
            joiner = " && " if isinstance(n.op, ast.And) else " || "
            return "(" + joiner.join(go(v) for v in n.values) + ")"
        if isinstance(n, ast.IfExp):
            return f"({go(n.test)} ? {go(n.body)} : {go(n.orelse)})"
        if isinstance(n, ast.Call) and isinstance(n.func, ast.Name) and n.func.id in ("min", "max") and len(n.args) == 2:
            return f"{'ak_imin' if n.func.id == 'min' else 'ak_imax'}({go(n.args[0])}, {go(n.args[1])})"
        raise KernelError(f"`{ast.unparse(n)}` isn't an integer expression the gfx950 lowering can compute")

    return go(node)


# --------------------------------------------------------------------------------------------- intervals


class Interval:
    """What a value can be over a rectangle of a tile: an integer range, a known/unknown bool, or unknown;
    `data` marks values that depend on the tile's computed data (not just positions and loop values)."""

    def __init__(self, lo: Any = None, hi: Any = None, data: bool = False, const: Any = None) -> None:
        self.lo, self.hi, self.data, self.const = lo, hi, data, const

    @property
    def known(self) -> bool:
        return self.lo is not None and self.lo == self.hi


def intervals(root: Node, leaves: Callable[[Node], Optional[Interval]]) -> Interval:
    """Interval semantics of `root`: integer arithmetic, comparisons, logic and `where` exactly; anything
    else unknown (data-dependent if its inputs are)."""
    memo: Dict[int, Interval] = {}

    def val(a: Any) -> Interval:
        if isinstance(a, Node):
            return go(a)
        if isinstance(a, (bool, int, float)):
            return Interval(a, a, const=a)
        return Interval()

    def go(n: Node) -> Interval:
        if n.id in memo:
            return memo[n.id]
        got = leaves(n)
        if got is None:
            args = [val(a) for a in n.args if isinstance(a, (Node, bool, int, float))]
            data = any(x.data for x in args)
            got = Interval(data=data)
            op = n.op
            if op in ("add", "subtract", "multiply") and len(args) == 2 and all(x.lo is not None for x in args):
                x, y = args
                if op == "add":
                    got = Interval(x.lo + y.lo, x.hi + y.hi, data)
                elif op == "subtract":
                    got = Interval(x.lo - y.hi, x.hi - y.lo, data)
                else:
                    c = [x.lo * y.lo, x.lo * y.hi, x.hi * y.lo, x.hi * y.hi]
                    got = Interval(min(c), max(c), data)
            elif op in _COMPARE and all(x.lo is not None for x in args):
                x, y = args
                always = {"less": x.hi < y.lo, "less_equal": x.hi <= y.lo, "greater": x.lo > y.hi,
                          "greater_equal": x.lo >= y.hi, "equal": x.known and y.known and x.lo == y.lo,
                          "not_equal": x.hi < y.lo or x.lo > y.hi}[op]
                never = {"less": x.lo >= y.hi, "less_equal": x.lo > y.hi, "greater": x.hi <= y.lo,
                         "greater_equal": x.hi < y.lo, "equal": x.hi < y.lo or x.lo > y.hi,
                         "not_equal": x.known and y.known and x.lo == y.lo}[op]
                got = Interval(True, True, data) if always else Interval(False, False, data) if never else Interval(False, True, data)
            elif op in ("logical_and", "bitwise_and") and n.dtype.kind == "b" and all(x.lo is not None for x in args):
                got = Interval(args[0].lo and args[1].lo, args[0].hi and args[1].hi, data)
            elif op in ("logical_or", "bitwise_or") and n.dtype.kind == "b" and all(x.lo is not None for x in args):
                got = Interval(args[0].lo or args[1].lo, args[0].hi or args[1].hi, data)
            elif op in ("logical_not", "invert") and n.dtype.kind == "b" and args[0].lo is not None:
                got = Interval(not args[0].hi, not args[0].lo, data)
            elif op == "where":
                c, x, y = (val(a) for a in n.args[:3])
                if c.known and not c.data:
                    got = x if c.lo else y
                else:
                    got = Interval(data=c.data or x.data or y.data)
            elif op in ("astype", "tile", "broadcast_to") and isinstance(n.args[0], Node):
                inner = go(n.args[0])
                got = Interval(data=inner.data, const=inner.const if n.dtype.kind == "f" else None)
                if n.dtype.kind in "iu" and inner.lo is not None and not isinstance(inner.lo, float):
                    got = Interval(inner.lo, inner.hi, inner.data)
                if inner.const is not None:
                    got.const = inner.const
        memo[n.id] = got
        return got

    return go(root)


# --------------------------------------------------------------------------------------------- elements


class ElementEmitter:
    """One element of a traced tile value as a C expression, at C index expressions: the per-element view
    of code that moves data around (reshape, concatenate, slices, jnp.tile, broadcasts) as well as computing
    it pointwise. `leaves(node, idx)` gives the expression of a leaf the caller provides (an input tile, a
    carried value, ...), or None.

    Branches stay branches: `where` and `concatenate` become C conditionals, so only the chosen operand is
    evaluated when the kernel runs."""

    MAX_CHARS = 1 << 20

    def __init__(self, leaves: Callable[[Node, Tuple[str, ...]], Optional[str]]) -> None:
        self.leaves = leaves

    def at(self, node: Any, idx: Sequence[str]) -> str:
        text = self._at(node, tuple(idx))
        if len(text) > self.MAX_CHARS:
            raise KernelError("an element of this tile code is too large an expression to generate")
        return text

    def _val(self, arg: Any, idx: Tuple[str, ...], shape: Tuple[int, ...], dt: Optional[DType] = None) -> str:
        if isinstance(arg, Node):
            return self._at(arg, _broadcast_index(arg.shape, shape, idx))
        if isinstance(arg, (bool, int, float)):
            return literal(arg, dt)
        if isinstance(arg, jaxlite.Array) and arg.ndim == 0 and arg.t.device.type != "meta":
            return literal(arg.t.item(), arg.dtype)  # a concrete scalar made in tile code (`jnp.uint32(...)`)
        raise KernelError(f"the gfx950 lowering can't compute {arg!r} per element")

    def _at(self, n: Node, idx: Tuple[str, ...]) -> str:
        leaf = self.leaves(n, idx)
        if leaf is not None:
            return leaf
        op, a, dt, shape = n.op, n.args, n.dtype, tuple(n.shape)
        ct = ctype(dt)
        if op == "iota":
            return f"({idx[n.kwargs['dimension']]})"
        if op == "full":
            return literal(n.kwargs["value"], dt)
        if op in _BINARY:
            x, y = self._val(a[0], idx, shape, dt), self._val(a[1], idx, shape, dt)
            return _rounded(f"(({ct})({x}) {_BINARY[op]} ({ct})({y}))", dt) if dt.kind == "f" else \
                f"(({ct})({x}) {_BINARY[op]} ({ct})({y}))"
        if op in _COMPARE:
            return f"(({self._val(a[0], idx, shape)}) {_COMPARE[op]} ({self._val(a[1], idx, shape)}))"
        if op == "divide":
            x, y = self._val(a[0], idx, shape, dt), self._val(a[1], idx, shape, dt)
            return _rounded(f"(({ct})({x}) / ({ct})({y}))", dt)
        if op in ("maximum", "minimum"):
            x, y = self._val(a[0], idx, shape, dt), self._val(a[1], idx, shape, dt)
            if dt.kind == "f":
                return _rounded(f"ak_{op}(({ct})({x}), ({ct})({y}))", dt)
            return f"((({x}) {'>' if op == 'maximum' else '<'} ({y})) ? ({x}) : ({y}))"
        if op in ("logical_and", "logical_or"):
            j = " && " if op == "logical_and" else " || "
            return f"(({self._val(a[0], idx, shape)}){j}({self._val(a[1], idx, shape)}))"
        if op in ("logical_not",) or (op == "invert" and dt.kind == "b"):
            return f"(!({self._val(a[0], idx, shape)}))"
        if op == "negative":
            return f"(-({self._val(a[0], idx, shape, dt)}))"
        if op == "where":
            c = self._val(a[0], idx, shape)
            return f"(({c}) ? ({ct})({self._val(a[1], idx, shape, dt)}) : ({ct})({self._val(a[2], idx, shape, dt)}))"
        if op == "astype":
            x = self._val(a[0], idx, shape)
            if dt.kind == "f":
                return _rounded(f"({ct})({x})", dt)
            if dt.kind == "b":
                return f"(({x}) != 0)"
            return f"({ct})({x})"
        if op in ("exp", "log", "sqrt", "rsqrt", "reciprocal", "square", "sigmoid", "abs"):
            x = self._val(a[0], idx, shape, dt)
            fn = {"exp": "ak_exp", "log": "__logf", "sqrt": "sqrtf", "rsqrt": "ak_rsqrt", "reciprocal": "ak_rcp",
                  "square": "ak_square", "sigmoid": "ak_sigmoid", "abs": "fabsf"}[op]
            return _rounded(f"{fn}((float)({x}))", dt)
        if op == "broadcast_to":
            return self._val(a[0], idx, shape)
        if op == "tile":
            src = a[0]
            inner = tuple(idx[len(idx) - len(src.shape) + k] if len(src.shape) else "0" for k in range(len(src.shape)))
            inner = tuple(f"(({i}) % {s})" if s != 1 else "0" for i, s in zip(inner, src.shape))
            return self._at(src, inner)
        if op == "reshape":
            src = a[0]
            flat = "0"
            for i, s in zip(idx, shape):
                flat = f"(({flat}) * {s} + ({i}))"
            inner, rest = [], flat
            st = strides_of(src.shape)
            for s, d in zip(st, src.shape):
                inner.append(f"((({rest}) / {s}) % {d})" if d != 1 else "0")
            return self._at(src, tuple(inner))
        if op == "concatenate":
            pieces, axis = a[0], n.kwargs["axis"]
            axis = axis % len(shape)
            out, start = None, 0
            branches = []
            for p in pieces:
                size = p.shape[axis]
                sub = tuple(f"(({i}) - {start})" if k == axis and start else i for k, i in enumerate(idx))
                branches.append((start, start + size, self._at(p, sub)))
                start += size
            expr = f"({ct})({branches[-1][2]})"
            for lo, hi, text in reversed(branches[:-1]):
                expr = f"((({idx[axis]}) < {hi}) ? ({ct})({text}) : {expr})"
            return expr
        if op == "getitem":
            src, key = a[0], a[1]
            key = key if isinstance(key, tuple) else (key,)
            inner, k_out = [], 0
            for k, d in enumerate(src.shape):
                sel = key[k] if k < len(key) else slice(None)
                if isinstance(sel, slice):
                    start, _, step = sel.indices(d)
                    i = idx[k_out]
                    inner.append(f"({start} + ({i}) * {step})" if (start or step != 1) else i)
                    k_out += 1
                elif isinstance(sel, int):
                    inner.append(str(sel % d))
                else:
                    raise KernelError("only static slices and integers index tile values per element")
            return self._at(src, tuple(inner))
        if op == "scatter_set":
            # x.at[key].set(v): inside the region the key selects, v (broadcast to the region), else x. Integer
            # keys the kernel computes select their one element; one out of the dim selects nothing (JAX drops
            # updates out of the array).
            src, key, val = a[0], a[1], a[2]
            key = key if isinstance(key, tuple) else (key,)
            conds, vidx, vshape = [], [], []
            for k, d in enumerate(src.shape):
                sel = key[k] if k < len(key) else slice(None)
                i = idx[k]
                if isinstance(sel, slice):
                    start, stop, step = sel.indices(d)
                    if (start, stop, step) != (0, d, 1):
                        c = f"({i}) >= {start} && ({i}) < {stop}"
                        conds.append(f"({c} && ((({i}) - {start}) % {step}) == 0)" if step != 1 else f"({c})")
                    vidx.append(f"((({i}) - {start}) / {step})" if (start or step != 1) else i)
                    vshape.append(len(range(start, stop, step)))
                elif isinstance(sel, int):
                    conds.append(f"(({i}) == {sel % d})")
                elif isinstance(sel, Node) and sel.shape == () and sel.dtype.kind in "iu":
                    conds.append(f"(({i}) == (int)({self._at(sel, ())}))")
                else:
                    raise KernelError("x.at[...].set per element takes static slices, integers and scalar integers")
            inside = " && ".join(conds) or "true"
            v = self._val(val, tuple(vidx), tuple(vshape), dt)
            return f"(({inside}) ? ({ct})({v}) : ({ct})({self._at(src, idx)}))"
        if op == "transpose":
            perm = n.kwargs.get("axes") or tuple(reversed(range(len(shape))))
            inner = [None] * len(perm)
            for out_k, in_k in enumerate(perm):
                inner[in_k] = idx[out_k]
            return self._at(a[0], tuple(inner))
        raise KernelError(f"the gfx950 lowering has no per-element form of `{op}` in tile setup or epilogue code")


def strides_of(shape: Sequence[int]) -> List[int]:
    out, n = [], 1
    for d in reversed(tuple(shape)):
        out.append(n)
        n *= d
    return list(reversed(out))


def _broadcast_index(shape: Sequence[int], target: Sequence[int], idx: Tuple[str, ...]) -> Tuple[str, ...]:
    """The index into an operand of `shape` broadcast (numpy rules) to `target` at index `idx`."""
    shape, target = tuple(shape), tuple(target)
    lead = len(target) - len(shape)
    if lead < 0:
        raise KernelError(f"can't broadcast {shape} to {target}")
    return tuple("0" if s == 1 and t != 1 else idx[lead + k] for k, (s, t) in enumerate(zip(shape, target[lead:])))
