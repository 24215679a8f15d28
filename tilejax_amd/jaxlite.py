"""A small stand-in for the parts of `jax` and `jax.numpy` that kernel specs are written in, over PyTorch.

The reference's specs are plain JAX loop nests (e.g. examples/matmul.py:22-35 of the reference). JAX is
not part of this stack, so a spec imports `from tilejax_amd.jaxlite import jax, jnp` instead and keeps
its text: `jnp.zeros`, `x[i : i + tm, k : k + tk] @ y[...]`, `out.at[...].set(...)`, `jnp.where`,
`jax.lax.broadcasted_iota`, `jax.nn.silu`, ... Arrays are immutable values (`.at[].set` copies), as in JAX.

Three ways the same functions run:

- concretely, on torch tensors (CPU or GPU): `kernel.fn` and `kernel.reference`;
- on torch "meta" tensors, shapes and dtypes only: the prologue when a kernel is planned;
- symbolically: while `trace()` is active, calls on `Sym` values record `Node`s (the tile code's IR,
  which the gfx950 lowering reads) and compute their types on meta tensors with the same functions, so
  the plan's types and the concrete run's can't disagree.

Type promotion is torch's, which agrees with JAX's for what specs do (Python scalars are weak: `bf16 * 2.0`
stays bf16; `bf16 + f32` is f32; comparisons give bool).
"""

from __future__ import annotations

import contextlib
import itertools
import math
import types
from typing import Any, Callable, Dict, Iterator, List, Optional, Sequence, Tuple

import numpy as np
import torch

__all__ = ["Array", "DType", "Node", "Sym", "jax", "jnp", "trace"]


# --------------------------------------------------------------------------------------------- dtypes


class DType:
    """A dtype, named as NumPy/JAX name it; also callable as a scalar constructor."""

    __slots__ = ("name", "torch", "kind", "itemsize")

    def __init__(self, name: str, torch_dtype: torch.dtype, kind: str, itemsize: int) -> None:
        self.name, self.torch, self.kind, self.itemsize = name, torch_dtype, kind, itemsize

    def __repr__(self) -> str:
        return f"dtype('{self.name}')"

    def __str__(self) -> str:
        return self.name

    def __eq__(self, other: Any) -> bool:
        try:
            return dtype(other).name == self.name
        except TypeError:
            return False

    def __hash__(self) -> int:
        return hash(self.name)

    def __call__(self, value: Any) -> "Array":
        return asarray(value, self)

    @property
    def type(self) -> "DType":
        return self


float32 = DType("float32", torch.float32, "f", 4)
float64 = DType("float64", torch.float64, "f", 8)
bfloat16 = DType("bfloat16", torch.bfloat16, "f", 2)
float16 = DType("float16", torch.float16, "f", 2)
int32 = DType("int32", torch.int32, "i", 4)
int64 = DType("int64", torch.int64, "i", 8)
int16 = DType("int16", torch.int16, "i", 2)
int8 = DType("int8", torch.int8, "i", 1)
uint8 = DType("uint8", torch.uint8, "u", 1)
uint32 = DType("uint32", torch.uint32, "u", 4)
bool_ = DType("bool", torch.bool, "b", 1)
_DTYPES = {d.name: d for d in (float32, float64, bfloat16, float16, int32, int64, int16, int8, uint8, uint32, bool_)}
_BY_TORCH = {d.torch: d for d in _DTYPES.values()}


def dtype(value: Any) -> DType:
    """The DType of a name, DType, torch or NumPy dtype, or Python type."""
    if isinstance(value, DType):
        return value
    if isinstance(value, torch.dtype):
        return _BY_TORCH[value]
    if value is float:
        return float32
    if value is int:
        return int32
    if value is bool:
        return bool_
    name = value if isinstance(value, str) else getattr(value, "name", None)
    if name is None and isinstance(value, type) and issubclass(value, np.generic):
        name = np.dtype(value).name
    if name in _DTYPES:
        return _DTYPES[name]
    raise TypeError(f"not a dtype: {value!r}")


def issubdtype(a: Any, b: Any) -> bool:
    kind = dtype(a).kind
    return {"floating": kind == "f", "inexact": kind == "f", "integer": kind in "iu", "bool": kind == "b",
            "signedinteger": kind == "i", "unsignedinteger": kind == "u"}[b]


floating, inexact, integer, signedinteger, unsignedinteger = "floating", "inexact", "integer", "signedinteger", "unsignedinteger"


def promote_types(a: Any, b: Any) -> DType:
    return _BY_TORCH[torch.promote_types(dtype(a).torch, dtype(b).torch)]


# --------------------------------------------------------------------------------------------- the IR


class Node:
    """One operation of traced tile code: `op` applied to `args` (Nodes, Python values, tuples of them)."""

    _ids = itertools.count()

    def __init__(self, op: str, args: tuple, kwargs: dict, shape: tuple, dt: DType) -> None:
        self.op, self.args, self.kwargs, self.shape, self.dtype = op, args, kwargs, tuple(shape), dt
        self.id = next(Node._ids)

    def inputs(self) -> List["Node"]:
        """The Nodes this one reads, in argument order."""
        out: List[Node] = []

        def walk(v: Any) -> None:
            if isinstance(v, Node):
                out.append(v)
            elif isinstance(v, (tuple, list)):
                for x in v:
                    walk(x)
            elif isinstance(v, slice):
                walk(v.start), walk(v.stop), walk(v.step)

        walk(self.args)
        walk(tuple(self.kwargs.values()))
        return out

    def __repr__(self) -> str:
        def show(v: Any) -> str:
            if isinstance(v, Node):
                return f"%{v.id}"
            if isinstance(v, (tuple, list)):
                return "(" + ", ".join(show(x) for x in v) + ")"
            return repr(v)

        kw = "".join(f", {k}={show(v)}" for k, v in self.kwargs.items())
        return f"%{self.id} = {self.op}({', '.join(show(a) for a in self.args)}{kw}) : {self.dtype.name}{list(self.shape)}"


class _Trace:
    def __init__(self) -> None:
        self.nodes: List[Node] = []


_TRACE: Optional[_Trace] = None


@contextlib.contextmanager
def trace() -> Iterator[_Trace]:
    """Record the operations on `Sym` values made inside the block."""
    global _TRACE
    previous, _TRACE = _TRACE, _Trace()
    try:
        yield _TRACE
    finally:
        _TRACE = previous


def leaf(op: str, shape: Sequence[int], dt: Any, **attrs: Any) -> "Sym":
    """A symbolic value not computed from others: a tile read, a loop variable, a carried value, ..."""
    dt = dtype(dt)
    node = Node(op, (), attrs, tuple(shape), dt)
    if _TRACE is not None:
        _TRACE.nodes.append(node)
    return Sym(torch.empty(tuple(shape), dtype=dt.torch, device="meta"), node)


def _has_sym(v: Any) -> bool:
    if isinstance(v, Sym):
        return True
    if isinstance(v, (tuple, list)):
        return any(_has_sym(x) for x in v)
    if isinstance(v, slice):
        return _has_sym(v.start) or _has_sym(v.stop) or _has_sym(v.step)
    return False


def _metas(v: Any) -> Any:
    if isinstance(v, Sym):
        return Array(v.t)
    if isinstance(v, tuple):
        return tuple(_metas(x) for x in v)
    if isinstance(v, list):
        return [_metas(x) for x in v]
    if isinstance(v, slice):
        return slice(_metas(v.start), _metas(v.stop), _metas(v.step))
    return v


def _nodes(v: Any) -> Any:
    if isinstance(v, Sym):
        return v.node
    if isinstance(v, (tuple, list)):
        return tuple(_nodes(x) for x in v)
    if isinstance(v, slice):
        return slice(_nodes(v.start), _nodes(v.stop), _nodes(v.step))
    if isinstance(v, Array):  # a concrete array met in traced code: a constant
        return v
    return v


def _op(name: str) -> Callable[[Callable], Callable]:
    """Make a function traceable: called with `Sym` arguments it records a Node named `name` whose type
    is what the function gives on meta tensors."""

    def wrap(fn: Callable) -> Callable:
        def traced(*args: Any, **kwargs: Any) -> Any:
            if not (_has_sym(args) or _has_sym(tuple(kwargs.values()))):
                return fn(*args, **kwargs)
            meta = fn(*_metas(args), **{k: _metas(v) for k, v in kwargs.items()})
            if not isinstance(meta, Array):
                raise TypeError(f"{name} gave {type(meta).__name__} on symbolic values")
            node = Node(name, _nodes(args), {k: _nodes(v) for k, v in kwargs.items()}, meta.shape, meta.dtype)
            if _TRACE is not None:
                _TRACE.nodes.append(node)
            return Sym(meta.t, node)

        traced.__name__ = fn.__name__
        traced.__doc__ = fn.__doc__
        traced.__wrapped__ = fn  # type: ignore[attr-defined]
        return traced

    return wrap


# --------------------------------------------------------------------------------------------- arrays

_DEVICE: List[Any] = ["cpu"]


@contextlib.contextmanager
def default_device(device: Any) -> Iterator[None]:
    """Where `jnp.zeros` and the like allocate inside the block (a spec's inputs' device, or "meta")."""
    _DEVICE.append(device)
    try:
        yield
    finally:
        _DEVICE.pop()


def _t(v: Any, like: Optional[torch.Tensor] = None) -> Any:
    """A torch tensor for an Array, else the value itself (Python scalars stay weak)."""
    if isinstance(v, Array):
        return v.t
    if isinstance(v, np.ndarray):
        return torch.from_numpy(v)
    if isinstance(v, np.generic):
        return v.item()
    return v


def _device_of(*vs: Any) -> Any:
    for v in vs:
        if isinstance(v, Array):
            return v.t.device
        if isinstance(v, (tuple, list)):
            d = _device_of(*v)
            if d is not None:
                return d
    return None


def _scalar_tensor(v: Any, like: torch.Tensor) -> torch.Tensor:
    """A Python scalar as a 0-d tensor of the type torch gives it next to `like` (weak promotion)."""
    return torch.tensor(v, dtype=torch.result_type(like, v), device=like.device)


def _pair(a: Any, b: Any) -> Tuple[torch.Tensor, torch.Tensor]:
    ta, tb = _t(a), _t(b)
    if not isinstance(ta, torch.Tensor) and not isinstance(tb, torch.Tensor):
        ta = torch.tensor(ta, device=_DEVICE[-1])
    if not isinstance(ta, torch.Tensor):
        ta = _scalar_tensor(ta, tb)
    if not isinstance(tb, torch.Tensor):
        tb = _scalar_tensor(tb, ta)
    return ta, tb


class Array:
    """An immutable array value (a torch tensor inside), with the JAX methods specs use."""

    __slots__ = ("t",)
    __array_priority__ = 100  # NumPy scalars defer to our operators

    def __init__(self, t: torch.Tensor) -> None:
        self.t = t

    @property
    def shape(self) -> Tuple[int, ...]:
        return tuple(self.t.shape)

    @property
    def dtype(self) -> DType:
        return _BY_TORCH[self.t.dtype]

    @property
    def ndim(self) -> int:
        return self.t.dim()

    @property
    def size(self) -> int:
        return self.t.numel()

    def __len__(self) -> int:
        return self.shape[0]

    def __repr__(self) -> str:
        return f"Array({self.t!r})"

    def astype(self, dt: Any) -> "Array":
        return astype(self, dt)

    @property
    def T(self) -> "Array":
        return transpose(self)

    def reshape(self, *shape: Any) -> "Array":
        if len(shape) == 1 and isinstance(shape[0], (tuple, list)):
            shape = tuple(shape[0])
        return reshape(self, tuple(shape))

    def __getitem__(self, index: Any) -> "Array":
        return getitem(self, index)

    @property
    def at(self) -> "_At":
        return _At(self)

    def sum(self, axis: Any = None, keepdims: bool = False, dtype: Any = None) -> "Array":
        return sum(self, axis=axis, keepdims=keepdims, dtype=dtype)

    def max(self, axis: Any = None, keepdims: bool = False) -> "Array":
        return max(self, axis=axis, keepdims=keepdims)

    def min(self, axis: Any = None, keepdims: bool = False) -> "Array":
        return min(self, axis=axis, keepdims=keepdims)

    def mean(self, axis: Any = None, keepdims: bool = False) -> "Array":
        return mean(self, axis=axis, keepdims=keepdims)

    def any(self, axis: Any = None, keepdims: bool = False) -> "Array":
        return any_(self, axis=axis, keepdims=keepdims)

    def __add__(self, o: Any) -> "Array":
        return add(self, o)

    def __radd__(self, o: Any) -> "Array":
        return add(o, self)

    def __sub__(self, o: Any) -> "Array":
        return subtract(self, o)

    def __rsub__(self, o: Any) -> "Array":
        return subtract(o, self)

    def __mul__(self, o: Any) -> "Array":
        return multiply(self, o)

    def __rmul__(self, o: Any) -> "Array":
        return multiply(o, self)

    def __truediv__(self, o: Any) -> "Array":
        return divide(self, o)

    def __rtruediv__(self, o: Any) -> "Array":
        return divide(o, self)

    def __floordiv__(self, o: Any) -> "Array":
        return floor_divide(self, o)

    def __rfloordiv__(self, o: Any) -> "Array":
        return floor_divide(o, self)

    def __mod__(self, o: Any) -> "Array":
        return remainder(self, o)

    def __pow__(self, o: Any) -> "Array":
        return power(self, o)

    def __neg__(self) -> "Array":
        return negative(self)

    def __pos__(self) -> "Array":
        return self

    def __abs__(self) -> "Array":
        return abs(self)

    def __matmul__(self, o: Any) -> "Array":
        return _at_operator(self, o)

    def __rmatmul__(self, o: Any) -> "Array":
        return _at_operator(o, self)

    def __and__(self, o: Any) -> "Array":
        return bitwise_and(self, o)

    def __rand__(self, o: Any) -> "Array":
        return bitwise_and(o, self)

    def __or__(self, o: Any) -> "Array":
        return bitwise_or(self, o)

    def __ror__(self, o: Any) -> "Array":
        return bitwise_or(o, self)

    def __invert__(self) -> "Array":
        return invert(self)

    def __lshift__(self, o: Any) -> "Array":
        return left_shift(self, o)

    def __rshift__(self, o: Any) -> "Array":
        return right_shift(self, o)

    def __lt__(self, o: Any) -> "Array":
        return less(self, o)

    def __le__(self, o: Any) -> "Array":
        return less_equal(self, o)

    def __gt__(self, o: Any) -> "Array":
        return greater(self, o)

    def __ge__(self, o: Any) -> "Array":
        return greater_equal(self, o)

    def __eq__(self, o: Any) -> "Array":  # type: ignore[override]
        return equal(self, o)

    def __ne__(self, o: Any) -> "Array":  # type: ignore[override]
        return not_equal(self, o)

    __hash__ = None  # type: ignore[assignment]

    def __bool__(self) -> bool:
        return bool(self.t.item())

    def __int__(self) -> int:
        return int(self.t.item())

    def __index__(self) -> int:
        if self.dtype.kind not in "iub":
            raise TypeError("only integer arrays can index")
        return int(self.t.item())

    def __float__(self) -> float:
        return float(self.t.item())

    def __array__(self, dt: Any = None, copy: Any = None) -> np.ndarray:
        t = self.t.detach().cpu()
        if t.dtype == torch.bfloat16:
            t = t.float()
        out = t.numpy()
        return out if dt is None else out.astype(dt)


class Sym(Array):
    """A symbolic array in traced tile code: its type (a meta tensor) and the Node that computes it."""

    __slots__ = ("node",)

    def __init__(self, meta: torch.Tensor, node: Node) -> None:
        super().__init__(meta)
        self.node = node

    def __repr__(self) -> str:
        return f"Sym({self.node!r})"

    def __bool__(self) -> bool:
        raise TypeError("tile code can't branch on a value the kernel computes: use jnp.where")

    def __int__(self) -> int:
        raise TypeError("tile code can't use a value the kernel computes as a Python int")

    __index__ = __int__  # type: ignore[assignment]

    def __float__(self) -> float:
        raise TypeError("tile code can't use a value the kernel computes as a Python float")

    def __array__(self, dt: Any = None, copy: Any = None) -> np.ndarray:
        raise TypeError("a symbolic tile value has no data")


class _At:
    def __init__(self, array: Array) -> None:
        self.array = array

    def __getitem__(self, index: Any) -> "_AtIndex":
        return _AtIndex(self.array, index)


class _AtIndex:
    def __init__(self, array: Array, index: Any) -> None:
        self.array, self.index = array, index

    def set(self, value: Any, mode: Any = None) -> Array:
        return scatter_set(self.array, self.index, value)

    def add(self, value: Any, mode: Any = None) -> Array:
        return scatter_add(self.array, self.index, value)


def _index(index: Any) -> Any:
    """An index with arrays of one element as ints (JAX clamps out-of-range integer indices: so do we)."""
    if isinstance(index, tuple):
        return tuple(_index(i) for i in index)
    if isinstance(index, slice):
        return slice(_index(index.start), _index(index.stop), _index(index.step))
    if isinstance(index, Array):
        if index.ndim == 0:
            if index.t.device.type == "meta":
                return 0  # a traced scalar index: the result's type doesn't depend on its value
            return int(index)
        return index.t.long()
    return index


def _clamped(index: Any, shape: Tuple[int, ...]) -> Any:
    """Integer indices (and integer index arrays) clamped into their dims, as JAX clamps reads: negative
    ones count from the end first."""
    idx = index if isinstance(index, tuple) else (index,)
    out, dim = [], 0
    for i in idx:
        if i is None:
            out.append(i)
            continue
        if i is Ellipsis:
            out.append(i)
            dim += len(shape) - (len(idx) - 1)
            continue
        if isinstance(i, int) and dim < len(shape):
            n = shape[dim]
            i = n + i if i < 0 else i
            i = 0 if i < 0 else (n - 1 if i >= n else i)
        elif isinstance(i, torch.Tensor) and i.dtype != torch.bool and dim < len(shape) and i.device.type != "meta":
            n = shape[dim]
            i = torch.where(i < 0, i + n, i).clamp(0, n - 1)
        out.append(i)
        dim += 1
    return tuple(out)


def _set(target: torch.Tensor, index: Any, value: Any) -> None:
    """`target[index] = value` as JAX updates: a negative integer index counts from the end, and an update
    at an index still out of its dim is dropped, for a single integer index (a whole update) as for the
    entries of one integer index array (a gathered or ragged window)."""
    idx = index if isinstance(index, tuple) else (index,)
    v = value.to(target.dtype) if isinstance(value, torch.Tensor) else value
    plain = all(i is not None and i is not Ellipsis for i in idx)
    if plain and target.device.type != "meta":
        for k, i in enumerate(idx):
            scalar = isinstance(i, int) and not isinstance(i, bool)
            scalar = scalar or (isinstance(i, torch.Tensor) and i.ndim == 0 and i.dtype != torch.bool
                                and not i.dtype.is_floating_point and i.device.type != "meta")
            if scalar and k < target.ndim:
                n = target.shape[k]
                at = int(i)
                if not -n <= at < n:
                    return  # the update falls outside the array: JAX drops it
    arrays = [k for k, i in enumerate(idx) if isinstance(i, torch.Tensor) and i.dtype != torch.bool and i.ndim > 0]
    if len(arrays) == 1 and plain and idx[arrays[0]].ndim == 1 and target.device.type != "meta":
        k = arrays[0]
        n = target.shape[k]
        i = torch.where(idx[k] < 0, idx[k] + n, idx[k])
        keep = (i >= 0) & (i < n)
        if not bool(keep.all()):
            # the dropped entries write a spare row past the end, which is then cut off
            spare = torch.cat([target, target.narrow(k, 0, 1)], k)
            moved = list(_clamped(idx, tuple(spare.shape)))
            moved[k] = torch.where(keep, i, n)
            spare[tuple(moved)] = v
            target.copy_(spare.narrow(k, 0, n))
            return
    target[_clamped(idx, tuple(target.shape))] = v


@_op("getitem")
def getitem(x: Array, index: Any) -> Array:
    return Array(x.t[_clamped(_index(index), x.shape)])


@_op("scatter_set")
def scatter_set(x: Array, index: Any, value: Any) -> Array:
    out = x.t.clone()
    _set(out, _index(index), _t(value))
    return Array(out)


@_op("scatter_add")
def scatter_add(x: Array, index: Any, value: Any) -> Array:
    out = x.t.clone()
    out[_clamped(_index(index), x.shape)] += _t(value)
    return Array(out)


def store_(x: Array, index: Any, value: Any) -> Array:
    """`x.at[index].set(value)` writing into `x`'s own buffer: what `kernel.reference` does for output
    stores (an output is never read by tile code, so no one sees the buffer change)."""
    _set(x.t, _index(index), _t(value))
    return x


# --------------------------------------------------------------------------------------------- creation


def _shape(shape: Any) -> Tuple[int, ...]:
    if isinstance(shape, (int, np.integer)):
        return (int(shape),)
    return tuple(int(s) for s in shape)


def zeros(shape: Any, dtype: Any = None) -> Array:
    dt = float32 if dtype is None else globals()["dtype"](dtype)
    if _TRACE is not None:
        return leaf("full", _shape(shape), dt, value=0)
    return Array(torch.zeros(_shape(shape), dtype=dt.torch, device=_DEVICE[-1]))


def ones(shape: Any, dtype: Any = None) -> Array:
    dt = float32 if dtype is None else globals()["dtype"](dtype)
    if _TRACE is not None:
        return leaf("full", _shape(shape), dt, value=1)
    return Array(torch.ones(_shape(shape), dtype=dt.torch, device=_DEVICE[-1]))


def full(shape: Any, fill_value: Any, dtype: Any = None) -> Array:
    if dtype is None:
        dt = float32 if isinstance(fill_value, float) else (bool_ if isinstance(fill_value, bool) else int32)
    else:
        dt = globals()["dtype"](dtype)
    if _TRACE is not None and isinstance(fill_value, (int, float, bool)):
        return leaf("full", _shape(shape), dt, value=fill_value)
    return Array(torch.full(_shape(shape), fill_value, dtype=dt.torch, device=_DEVICE[-1]))


def zeros_like(x: Array, dtype: Any = None) -> Array:
    return zeros(x.shape, x.dtype if dtype is None else dtype)


def asarray(value: Any, dtype: Any = None) -> Array:
    if isinstance(value, Array):
        return value if dtype is None else value.astype(dtype)
    if isinstance(value, torch.Tensor):
        t = value
    elif isinstance(value, np.ndarray):
        t = torch.from_numpy(np.ascontiguousarray(value))
    else:
        t = torch.tensor(value)
    if dtype is not None:
        t = t.to(globals()["dtype"](dtype).torch)
    elif t.dtype == torch.int64:
        t = t.to(torch.int32)
    elif t.dtype == torch.float64 and not isinstance(value, (torch.Tensor, np.ndarray)):
        t = t.to(torch.float32)
    return Array(t)


array = asarray


def arange(start: int, stop: Optional[int] = None, step: int = 1, dtype: Any = None) -> Array:
    if stop is None:
        start, stop = 0, start
    dt = int32 if dtype is None else globals()["dtype"](dtype)
    if _TRACE is not None and all(isinstance(v, int) for v in (start, stop, step)):
        # traced tile code: an iota node (the kernels compute each element's value), not a constant array
        n = len(range(start, stop, step))
        return leaf("iota", (n,), dt, dimension=0) * step + start
    return Array(torch.arange(start, stop, step, dtype=dt.torch, device=_DEVICE[-1]))


def broadcasted_iota(dt: Any, shape: Any, dimension: int) -> Array:
    """jax.lax.broadcasted_iota: each element's index along `dimension`."""
    shape = _shape(shape)
    dt = dtype(dt)
    if _TRACE is not None:
        return leaf("iota", shape, dt, dimension=int(dimension))
    view = [1] * len(shape)
    view[dimension] = shape[dimension]
    r = torch.arange(shape[dimension], dtype=dt.torch, device=_DEVICE[-1]).reshape(view)
    return Array(r.expand(shape).contiguous())


# --------------------------------------------------------------------------------------------- elementwise


def _binary(name: str, fn: Callable[[torch.Tensor, torch.Tensor], torch.Tensor]) -> Callable:
    @_op(name)
    def op(a: Any, b: Any) -> Array:
        ta, tb = _pair(a, b)
        if torch.uint32 in (ta.dtype, tb.dtype):
            # torch computes few ops on uint32: in int64, then wrapped back to 32 bits (comparisons stay bool)
            wide = fn(ta.to(torch.int64), tb.to(torch.int64))
            return Array(wide if wide.dtype == torch.bool else (wide & 0xFFFFFFFF).to(torch.uint32))
        return Array(fn(ta, tb))

    op.__name__ = name
    return op


add = _binary("add", torch.add)
subtract = _binary("subtract", torch.sub)
multiply = _binary("multiply", torch.mul)
maximum = _binary("maximum", torch.maximum)
minimum = _binary("minimum", torch.minimum)
less = _binary("less", torch.lt)
less_equal = _binary("less_equal", torch.le)
greater = _binary("greater", torch.gt)
greater_equal = _binary("greater_equal", torch.ge)
equal = _binary("equal", torch.eq)
not_equal = _binary("not_equal", torch.ne)
bitwise_and = _binary("bitwise_and", torch.bitwise_and)
bitwise_or = _binary("bitwise_or", torch.bitwise_or)
bitwise_xor = _binary("bitwise_xor", torch.bitwise_xor)
left_shift = _binary("left_shift", torch.bitwise_left_shift)
right_shift = _binary("right_shift", torch.bitwise_right_shift)
power = _binary("power", torch.pow)
logical_and = _binary("logical_and", torch.logical_and)
logical_or = _binary("logical_or", torch.logical_or)


@_op("divide")
def divide(a: Any, b: Any) -> Array:
    ta, tb = _pair(a, b)
    if not ta.is_floating_point() and not tb.is_floating_point():
        ta = ta.to(torch.float32)
    return Array(torch.div(ta, tb))


@_op("floor_divide")
def floor_divide(a: Any, b: Any) -> Array:
    ta, tb = _pair(a, b)
    return Array(torch.div(ta, tb, rounding_mode="floor"))


@_op("remainder")
def remainder(a: Any, b: Any) -> Array:
    ta, tb = _pair(a, b)
    return Array(torch.remainder(ta, tb))


def _unary(name: str, fn: Callable[[torch.Tensor], torch.Tensor], floats: bool = False) -> Callable:
    @_op(name)
    def op(x: Any) -> Array:
        t = _t(x)
        if not isinstance(t, torch.Tensor):
            t = torch.tensor(t, device=_DEVICE[-1])
        if floats and not t.is_floating_point():
            t = t.to(torch.float32)
        return Array(fn(t))

    op.__name__ = name
    return op


negative = _unary("negative", torch.neg)
exp = _unary("exp", torch.exp, True)
exp2 = _unary("exp2", torch.exp2, True)
log = _unary("log", torch.log, True)
sqrt = _unary("sqrt", torch.sqrt, True)
rsqrt = _unary("rsqrt", torch.rsqrt, True)
tanh = _unary("tanh", torch.tanh, True)
abs = _unary("abs", torch.abs)
square = _unary("square", torch.square)
sign = _unary("sign", torch.sign)
invert = _unary("invert", torch.bitwise_not)
logical_not = _unary("logical_not", torch.logical_not)
reciprocal = _unary("reciprocal", torch.reciprocal, True)


@_op("bitcast_convert_type")
def bitcast_convert_type(x: Any, new_dtype: Any) -> Array:
    """x's bits as `new_dtype` of the same width (jax.lax.bitcast_convert_type; widths that differ are the
    packing helpers' business, tilejax_amd.pairs / unpairs)."""
    t, dt = _t(x), dtype(new_dtype)
    if t.element_size() != dt.itemsize:
        raise TypeError(f"bitcast_convert_type between widths {t.element_size()} and {dt.itemsize} is not supported")
    return Array(t.contiguous().view(dt.torch))


@_op("pairs")
def pairs(x: Any) -> Array:
    """A 16-bit tile (..., 2, d) as uint32 words (..., d): x[..., 0, i] in each word's low half, x[..., 1, i]
    in its high half."""
    t = _t(x)
    if t.element_size() != 2:
        raise TypeError(f"pairs takes a 16-bit tile of pairs of rows (..., 2, d), not {_BY_TORCH[t.dtype].name}")
    if t.dim() < 2 or t.shape[-2] != 2:
        raise TypeError(f"pairs takes a 16-bit tile of pairs of rows (..., 2, d), not shape {tuple(t.shape)}")
    return Array(t.transpose(-1, -2).contiguous().view(torch.uint32).squeeze(-1))


@_op("unpairs")
def unpairs(words: Any, new_dtype: Any) -> Array:
    """`pairs` undone: uint32 words (..., d) as a tile (..., 2, d) of the 16-bit `new_dtype`."""
    t, dt = _t(words), dtype(new_dtype)
    if t.dtype != torch.uint32 or dt.itemsize != 2:
        have = _BY_TORCH[t.dtype].name if t.dtype in _BY_TORCH else str(t.dtype)
        raise TypeError(f"unpairs takes uint32 words and a 16-bit dtype, not {have} and {dt.name}")
    return Array(t.contiguous().view(dt.torch).reshape(*t.shape, 2).transpose(-1, -2))


@_op("astype")
def astype(x: Any, dt: Any) -> Array:
    t = _t(x)
    if not isinstance(t, torch.Tensor):
        t = torch.tensor(t, device=_DEVICE[-1])
    return Array(t.to(dtype(dt).torch))


@_op("where")
def where(condition: Any, x: Any, y: Any) -> Array:
    c = _t(condition)
    if not isinstance(c, torch.Tensor):
        c = torch.tensor(c, device=_device_of(x, y) or _DEVICE[-1])
    tx, ty = _pair(x, y)
    dt = torch.result_type(_t(x) if isinstance(x, Array) else tx, _t(y) if isinstance(y, Array) else ty)
    if isinstance(x, Array) and not isinstance(y, Array):
        dt = torch.result_type(tx, _t(y))
    elif isinstance(y, Array) and not isinstance(x, Array):
        dt = torch.result_type(ty, _t(x))
    return Array(torch.where(c.to(torch.bool), tx.to(dt), ty.to(dt)))


def select(pred: Any, on_true: Any, on_false: Any) -> Array:
    return where(pred, on_true, on_false)


@_op("clip")
def clip(x: Any, lo: Any = None, hi: Any = None) -> Array:
    return Array(torch.clamp(_t(x), _t(lo), _t(hi)))


# --------------------------------------------------------------------------------------------- reductions


def _axes(axis: Any, ndim: int) -> Optional[Tuple[int, ...]]:
    if axis is None:
        return None
    axes = (axis,) if isinstance(axis, int) else tuple(axis)
    return tuple(a % ndim for a in axes)


@_op("reduce_max")
def max(x: Any, axis: Any = None, keepdims: bool = False) -> Array:
    t = _t(x)
    axes = _axes(axis, t.dim())
    return Array(torch.amax(t, dim=axes if axes is not None else tuple(range(t.dim())), keepdim=keepdims))


@_op("reduce_min")
def min(x: Any, axis: Any = None, keepdims: bool = False) -> Array:
    t = _t(x)
    axes = _axes(axis, t.dim())
    return Array(torch.amin(t, dim=axes if axes is not None else tuple(range(t.dim())), keepdim=keepdims))


@_op("reduce_sum")
def sum(x: Any, axis: Any = None, keepdims: bool = False, dtype: Any = None) -> Array:
    t = _t(x)
    axes = _axes(axis, t.dim())
    want = globals()["dtype"](dtype).torch if dtype is not None else (
        torch.int32 if not t.is_floating_point() else t.dtype)
    acc = torch.float32 if t.is_floating_point() and t.element_size() < 4 else None
    dims = axes if axes is not None else tuple(range(t.dim()))
    out = torch.sum(t, dim=dims, keepdim=keepdims, dtype=acc) if dims else t.clone()
    return Array(out.to(want))


@_op("reduce_mean")
def mean(x: Any, axis: Any = None, keepdims: bool = False) -> Array:
    t = _t(x)
    axes = _axes(axis, t.dim())
    src = t if t.is_floating_point() else t.to(torch.float32)
    dims = axes if axes is not None else tuple(range(t.dim()))
    acc = torch.float32 if src.element_size() < 4 else None
    return Array(torch.mean(src, dim=dims, keepdim=keepdims, dtype=acc).to(src.dtype))


@_op("reduce_any")
def any_(x: Any, axis: Any = None, keepdims: bool = False) -> Array:
    t = _t(x).to(torch.bool)
    axes = _axes(axis, t.dim())
    if axes is None:
        return Array(t.any())
    out = t
    for a in sorted(axes, reverse=True):
        out = out.any(dim=a, keepdim=keepdims)
    return Array(out)


@_op("argmax")
def argmax(x: Any, axis: Any = None, keepdims: bool = False) -> Array:
    return Array(torch.argmax(_t(x), dim=axis, keepdim=keepdims).to(torch.int32))


# --------------------------------------------------------------------------------------------- shapes


@_op("reshape")
def reshape(x: Any, shape: Any) -> Array:
    return Array(_t(x).reshape(_shape(shape) if not isinstance(shape, int) else (shape,)))


@_op("transpose")
def transpose(x: Any, axes: Any = None) -> Array:
    t = _t(x)
    return Array(t.permute(*(axes if axes is not None else reversed(range(t.dim())))))


@_op("tile")
def tile(x: Any, reps: Any) -> Array:
    return Array(torch.tile(_t(x), _shape(reps)))


@_op("concatenate")
def concatenate(xs: Any, axis: int = 0) -> Array:
    return Array(torch.cat([_t(x) for x in xs], dim=axis))


@_op("stack")
def stack(xs: Any, axis: int = 0) -> Array:
    return Array(torch.stack([_t(x) for x in xs], dim=axis))


@_op("broadcast_to")
def broadcast_to(x: Any, shape: Any) -> Array:
    return Array(_t(x).expand(_shape(shape)).contiguous())


@_op("pad")
def pad(x: Any, pad_width: Any) -> Array:
    t = _t(x)
    flat = []
    for lo, hi in reversed([tuple(p) for p in pad_width]):
        flat += [lo, hi]
    return Array(torch.nn.functional.pad(t, flat))


@_op("repeat")
def repeat(x: Any, repeats: int, axis: Any = None) -> Array:
    return Array(torch.repeat_interleave(_t(x), repeats, dim=axis))


# --------------------------------------------------------------------------------------------- matmuls


def _acc_type(t: torch.Tensor) -> torch.dtype:
    if t.is_floating_point():
        return torch.float64 if t.dtype == torch.float64 else torch.float32
    return torch.int64


@_op("dot")
def matmul(a: Any, b: Any, preferred_element_type: Any = None, precision: Any = None) -> Array:
    """`a @ b`: computed with f32 accumulation; the result in `preferred_element_type`, else the operands'
    promoted type (plain JAX on a CPU rounds `bf16 @ bf16` to bf16 at the end)."""
    ta, tb = _t(a), _t(b)
    common = torch.promote_types(ta.dtype, tb.dtype)
    acc = _acc_type(ta.to(common) if ta.dtype != common else ta)
    if ta.device.type == "meta":
        out = torch.matmul(ta.to(acc), tb.to(acc))
    elif acc == torch.int64:
        out = torch.matmul(ta.to(torch.float64), tb.to(torch.float64)).round().to(torch.int64)
    else:
        out = torch.matmul(ta.to(acc), tb.to(acc))
    want = dtype(preferred_element_type).torch if preferred_element_type is not None else common
    return Array(out.to(want))


def dot(a: Any, b: Any, preferred_element_type: Any = None, precision: Any = None) -> Array:
    return matmul(a, b, preferred_element_type=preferred_element_type, precision=precision)


@_op("dot_nt")
def matmul_nt(a: Any, b: Any, preferred_element_type: Any = None) -> Array:
    """`a @ b.T` for two matrices, contracting both last dims (b read transposed in place)."""
    ta, tb = _t(a), _t(b)
    common = torch.promote_types(ta.dtype, tb.dtype)
    acc = _acc_type(ta.to(common) if ta.dtype != common else ta)
    out = torch.matmul(ta.to(acc), tb.to(acc).transpose(-1, -2))
    want = dtype(preferred_element_type).torch if preferred_element_type is not None else common
    return Array(out.to(want))


def dot_general(x: Any, y: Any, dimension_numbers: Any, preferred_element_type: Any = None, precision: Any = None) -> Array:
    (lc, rc), (lb, rb) = dimension_numbers
    if tuple(lb) == (0,) and tuple(rb) == (0,) and len(x.shape) == 3 and len(y.shape) == 3:
        # one leading batch dim: the batch's products, stacked
        inner = ((tuple(c - 1 for c in lc), tuple(c - 1 for c in rc)), ((), ()))
        return stack([dot_general(x[b], y[b], inner, preferred_element_type) for b in range(x.shape[0])])
    if tuple(lb) or tuple(rb) or len(x.shape) != 2 or len(y.shape) != 2:
        raise NotImplementedError("dot_general: two matrices, or a leading batch dim of two stacks of them")
    lc, rc = tuple(lc), tuple(rc)
    xx = x if lc == (1,) else transpose(x)
    if rc == (1,):
        return matmul_nt(xx, y, preferred_element_type=preferred_element_type)
    return matmul(xx, y, preferred_element_type=preferred_element_type)


# --------------------------------------------------------------------------------------------- `@` on matrix units

_MATRIX_UNITS: List[int] = [0]


@contextlib.contextmanager
def matrix_units() -> Iterator[None]:
    """Inside the block, the `@` operator means what a kernel's matrix units compute (the reference's
    src/autokernel/mxu.py:21-43): operands of different types are promoted to a common one, the product
    accumulates in f32 (i32 for integers) and stays f32 (f32 operands at full precision), and `a @ b.T` of
    two matrices contracts both last dims. Outside it `@` is plain JAX: `bf16 @ bf16` rounds to bf16. Only
    the operator changes: `jnp.matmul` and `jnp.dot` keep their meaning either way. `kernel.reference` and
    the planner's trace run the loop nest inside this block; `kernel.fn` runs outside it."""
    _MATRIX_UNITS[0] += 1
    try:
        yield
    finally:
        _MATRIX_UNITS[0] -= 1


def _transposed_matrix(v: Any) -> Optional["Sym"]:
    """For a traced `m.T` of a matrix m, m itself (so the product reads it transposed in place)."""
    if not (isinstance(v, Sym) and v.node.op == "transpose" and v.ndim == 2):
        return None
    axes = v.node.args[1] if len(v.node.args) > 1 else v.node.kwargs.get("axes")
    src = v.node.args[0]
    if axes not in (None, (1, 0), [1, 0]) or not isinstance(src, Node) or len(src.shape) != 2:
        return None
    return Sym(torch.empty(src.shape, dtype=src.dtype.torch, device="meta"), src)


def _at_operator(a: Any, b: Any) -> Array:
    if not _MATRIX_UNITS[0]:
        return matmul(a, b)
    ta, tb = asarray(a) if not isinstance(a, Array) else a, asarray(b) if not isinstance(b, Array) else b
    if ta.dtype != tb.dtype:
        common = promote_types(ta.dtype, tb.dtype)
        ta, tb = ta.astype(common), tb.astype(common)
    acc = int32 if ta.dtype.kind in "iu" else float32
    if ta.ndim == 2:
        source = _transposed_matrix(tb)
        if source is not None:
            return matmul_nt(ta, source, preferred_element_type=acc)
    return matmul(ta, tb, preferred_element_type=acc)


# --------------------------------------------------------------------------------------------- activations


def silu(x: Any) -> Array:
    return x * sigmoid(x)


@_op("sigmoid")
def sigmoid(x: Any) -> Array:
    t = _t(x)
    return Array(torch.sigmoid(t if t.is_floating_point() else t.to(torch.float32)))


def relu(x: Any) -> Array:
    return maximum(x, 0)


def gelu(x: Any, approximate: bool = True) -> Array:
    if approximate:
        return 0.5 * x * (1.0 + tanh(0.7978845608028654 * (x + 0.044715 * x * x * x)))
    return _gelu_exact(x)


@_op("gelu_exact")
def _gelu_exact(x: Any) -> Array:
    return Array(torch.nn.functional.gelu(_t(x)))


def softmax(x: Any, axis: int = -1) -> Array:
    m = max(x, axis=axis, keepdims=True)
    e = exp(x - m)
    return e / sum(e, axis=axis, keepdims=True)


# --------------------------------------------------------------------------------------------- namespaces


class Precision:
    DEFAULT, HIGH, HIGHEST = "default", "high", "highest"


@contextlib.contextmanager
def named_scope(name: str) -> Iterator[None]:
    yield


def _namespace(name: str, **members: Any) -> types.SimpleNamespace:
    ns = types.SimpleNamespace(**members)
    ns.__name__ = name
    return ns


jnp = _namespace(
    "jnp",
    float32=float32, float64=float64, bfloat16=bfloat16, float16=float16, int32=int32, int64=int64,
    int16=int16, int8=int8, uint8=uint8, uint32=uint32, bool_=bool_, dtype=dtype, issubdtype=issubdtype,
    promote_types=promote_types, floating=floating, inexact=inexact, integer=integer,
    signedinteger=signedinteger, unsignedinteger=unsignedinteger,
    zeros=zeros, ones=ones, full=full, zeros_like=zeros_like, asarray=asarray, array=array, arange=arange,
    add=add, subtract=subtract, multiply=multiply, divide=divide, floor_divide=floor_divide,
    remainder=remainder, maximum=maximum, minimum=minimum, less=less, less_equal=less_equal,
    greater=greater, greater_equal=greater_equal, equal=equal, not_equal=not_equal, power=power,
    logical_and=logical_and, logical_or=logical_or, logical_not=logical_not,
    negative=negative, exp=exp, exp2=exp2, log=log, sqrt=sqrt, tanh=tanh, abs=abs, square=square,
    sign=sign, reciprocal=reciprocal, where=where, clip=clip,
    max=max, min=min, sum=sum, mean=mean, any=any_, argmax=argmax,
    reshape=reshape, transpose=transpose, tile=tile, concatenate=concatenate, stack=stack,
    broadcast_to=broadcast_to, pad=pad, repeat=repeat, matmul=matmul, dot=dot,
    ndarray=Array, inf=float("inf"), nan=float("nan"),
)
lax = _namespace(
    "jax.lax", broadcasted_iota=broadcasted_iota, rsqrt=rsqrt, dot_general=dot_general,
    Precision=Precision, exp=exp, max=maximum, min=minimum, select=select, bitcast_convert_type=bitcast_convert_type,
    div=lambda a, b: floor_divide(a, b), rem=remainder, tanh=tanh,
)
nn = _namespace("jax.nn", silu=silu, sigmoid=sigmoid, relu=relu, gelu=gelu, softmax=softmax)
jax = _namespace("jax", numpy=jnp, lax=lax, nn=nn, named_scope=named_scope, Array=Array)
