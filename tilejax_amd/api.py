"""`@tilejax_amd.kernel`: a Python loop nest over tiles, compiled to one persistent HIP kernel for gfx950.

Same surface as the reference's api.py (src/autokernel/api.py:36-391): a `Kernel` caches builds per input
signature; called without its tunable it is tuned on the GPU (tune.py) and remembers the result; `.fn`
is the function itself, `.reference` the function with `@` accumulating in f32, `.verify` compares the
two, `.source` is the generated HIP C++, `.tuning` what tuning tried and chose.

Inputs and outputs are torch tensors on the GPU (the spec itself runs over jaxlite arrays, wrapped and
unwrapped at this boundary). There is no CPU fallback: a kernel call without a GPU, or without the
built runtime library, raises KernelError.
"""

from __future__ import annotations

import functools
import itertools
import math
from dataclasses import dataclass, field
from typing import Any, Callable, Dict, Optional, Tuple

import numpy as np
import torch

from . import jaxlite
from .errors import KernelError
from .parse import Nest, parse
from .pipeline import Pipeline
from .plan import Plan, Spec, make_plan
from .reference import make_reference
from .schedule import Schedule, make_schedule
from .tunable import is_tunable, neighbours

__all__ = ["Kernel", "Lowered", "compare", "kernel"]

Signature = Tuple[Tuple[Tuple[int, ...], jaxlite.DType], ...]


@dataclass(frozen=True)
class Lowered:
    """A kernel generated for one input signature and schedule: its plan, schedule and HIP source."""

    plan: Plan
    schedule: Schedule
    config: Any  # tune.Config
    source: str
    trace: bool
    program: Any = field(repr=False)  # codegen.Program: the launches and how to pack their arguments

    @property
    def pipeline(self) -> Pipeline:
        return self.config.pipeline

    @property
    def steps(self) -> int:
        return self.schedule.steps

    @property
    def tiles(self) -> int:
        return self.schedule.tiles

    @property
    def total_tiles(self) -> int:
        return self.schedule.total_tiles

    @property
    def lds_bytes(self) -> int:
        return self.program.lds_bytes

    def run(self, *arrays: Any) -> Any:
        """The kernel on torch tensors already on the GPU; the outputs (one tensor, or a tuple)."""
        return self.program(*arrays)


def _tensor(x: Any) -> torch.Tensor:
    if isinstance(x, jaxlite.Array):
        return x.t
    if isinstance(x, torch.Tensor):
        return x
    if isinstance(x, np.ndarray):
        return jaxlite.asarray(x).t
    raise KernelError(f"kernel inputs are torch tensors (or jaxlite arrays), not {type(x).__name__}")


class Kernel:
    """A loop nest compiled to a persistent gfx950 kernel. Call it like the function it was made from."""

    def __init__(self, fn: Callable[..., Any]) -> None:
        self.fn = _SpecFunction(fn)
        self.nest: Nest = parse(fn)
        self._raw = fn
        functools.update_wrapper(self, fn)
        self.default_tunable = fn.__defaults__[-1] if self.nest.tunable else None
        if self.nest.tunable and not is_tunable(self.default_tunable):
            raise self.nest.error(
                f"`{self.nest.tunable}`'s default must be a @tilejax_amd.tunable, not {self.default_tunable!r}",
                self.nest.function.args,
            )
        self._builds: Dict[Tuple[Signature, Any], Tuple[Plan, Schedule]] = {}
        self._references: Dict[Signature, Callable[..., Any]] = {}
        self._lowered: Dict[Tuple[Signature, Any, bool], Lowered] = {}
        self._tunings: Dict[Signature, Any] = {}

    def __repr__(self) -> str:
        return f"<tilejax_amd.Kernel {self.nest.name}>"

    def __call__(self, *args: Any) -> Any:
        arrays, _ = self._split(args)
        return self.lower(*args).run(*(_tensor(a) for a in arrays))

    def lower(self, *args: Any) -> Lowered:
        """The kernel for inputs like these (tensors, or (shape, dtype) pairs), and the tunable if given."""
        from .tune import Config

        arrays, tunable = self._split(args)
        signature = self.signature(*arrays)
        if tunable is None:
            return self.lowered(signature, self.tuning(*arrays).config)
        plan, schedule = self.build(signature, tunable)
        from .codegen import default_pipeline

        return self.lowered(signature, Config(tunable, default_pipeline(plan, schedule)))

    def source(self, *args: Any) -> str:
        """The generated HIP source for inputs like these."""
        return self.lower(*args).source

    def reference(self, *args: Any) -> Any:
        """What the kernel computes: the loop nest run as plain (jaxlite) JAX with `@` accumulating in f32,
        on the inputs' device."""
        arrays, tunable = self._split(args)
        signature = self.signature(*arrays)
        if self.nest.tunable:
            tunable = tunable if tunable is not None else self.lower(*arrays).config.tunable
        self.build(signature, tunable if tunable is not None else self.default_tunable)
        reference = self._references[signature]
        tensors = [_tensor(a) for a in arrays]
        with jaxlite.default_device(tensors[0].device):
            wrapped = [jaxlite.Array(t) for t in tensors]
            out = reference(*wrapped, tunable) if self.nest.tunable else reference(*wrapped)
        return tuple(o.t for o in out) if isinstance(out, tuple) else out.t

    def verify(self, *args: Any, rtol: Optional[float] = None, atol: Optional[float] = None) -> float:
        """Run the kernel and its reference; AssertionError unless they agree within the dtypes' tolerances
        (or `rtol`/`atol`). Returns the largest absolute difference."""
        arrays, tunable = self._split(args)
        if self.nest.tunable:
            arrays = (*arrays, tunable if tunable is not None else self.lower(*arrays).config.tunable)
        got, want = self(*arrays), self.reference(*arrays)
        dtypes = tuple(dt for _, dt in self.signature(*arrays[: len(self.nest.inputs)]))
        got, want = (got, want) if isinstance(got, tuple) else ((got,), (want,))
        return max(compare(f"{self.nest.name} output {name!r}", g, w, rtol, atol, dtypes)
                   for name, g, w in zip(self.nest.outputs, got, want))

    def tuning(self, *arrays: Any) -> Any:
        """The schedule for inputs like these: tuned on the GPU when first asked (tune.py)."""
        from .tune import tune

        signature = self.signature(*arrays)
        if signature not in self._tunings:
            self._tunings[signature] = tune(self, signature, arrays)
        return self._tunings[signature]

    # ------------------------------------------------------------------ building (used by tune.py too)

    def signature(self, *arrays: Any) -> Signature:
        """The inputs' shapes and dtypes."""
        signature = []
        for name, x in zip(self.nest.inputs, arrays):
            if isinstance(x, tuple) and len(x) == 2 and isinstance(x[0], tuple):
                signature.append((tuple(int(s) for s in x[0]), jaxlite.dtype(x[1])))
                continue
            if not (hasattr(x, "shape") and hasattr(x, "dtype")) or not tuple(x.shape):
                raise KernelError(f"{self.nest.name}: input `{name}` must be an array, got {type(x).__name__}")
            signature.append((tuple(int(s) for s in x.shape), jaxlite.dtype(x.dtype)))
        return tuple(signature)

    def default_config(self, signature: Signature) -> Any:
        """The tunable's defaults with their default buffering, or the nearest tunable that builds."""
        from .codegen import default_pipeline
        from .tune import Config

        def make(t: Any) -> Any:
            plan, schedule = self.build(signature, t)
            config = Config(t, default_pipeline(plan, schedule))
            self.lowered(signature, config)  # (it must lower, too)
            return config

        try:
            return make(self.default_tunable)
        except KernelError:
            if self.default_tunable is None:
                raise
            found = _nearest(self.default_tunable, make)
            if found is None:
                raise
            return found

    def build(self, signature: Signature, tunable: Any) -> Tuple[Plan, Schedule]:
        key = (signature, tunable)
        if signature not in self._references:
            self._references[signature] = make_reference(self.nest, self._raw)
        if key not in self._builds:
            specs = [Spec(shape, dt) for shape, dt in signature]
            plan = make_plan(self.nest, self._raw, specs, tunable)
            self._builds[key] = (plan, make_schedule(plan))
        return self._builds[key]

    def lowered(self, signature: Signature, config: Any, trace: bool = False) -> Lowered:
        """The kernel for this signature and schedule."""
        from . import codegen

        key = (signature, config, trace)
        if key not in self._lowered:
            plan, schedule = self.build(signature, config.tunable)
            if config.cursor and not plan.either:
                raise KernelError(f"{self.nest.name}: only a kernel with runtime masks finds its steps with a cursor")
            program = codegen.generate(plan, schedule, config.pipeline, trace=trace, cursor=config.cursor)
            self._lowered[key] = Lowered(plan, schedule, config, program.source, trace, program)
        return self._lowered[key]

    def _split(self, args: Tuple[Any, ...]) -> Tuple[Tuple[Any, ...], Any]:
        n = len(self.nest.inputs)
        if self.nest.tunable and len(args) == n + 1:
            tunable = args[-1]
            if type(tunable) is not type(self.default_tunable):
                raise KernelError(
                    f"{self.nest.name}: `{self.nest.tunable}` must be a {type(self.default_tunable).__name__}, "
                    f"not {type(tunable).__name__}")
            return args[:-1], tunable
        if len(args) != n:
            more = f", then optionally `{self.nest.tunable}`" if self.nest.tunable else ""
            raise KernelError(f"{self.nest.name} takes {n} input arrays ({', '.join(self.nest.inputs)}){more}; got {len(args)}")
        return args, None


class _SpecFunction:
    """`kernel.fn`: the function as written, over torch tensors (wrapped as jaxlite arrays inside)."""

    def __init__(self, fn: Callable[..., Any]) -> None:
        self.__wrapped__ = fn
        functools.update_wrapper(self, fn)

    def __call__(self, *args: Any) -> Any:
        device = next((a.device for a in args if isinstance(a, torch.Tensor)), "cpu")
        wrapped = [jaxlite.Array(a) if isinstance(a, torch.Tensor) else a for a in args]
        with jaxlite.default_device(device):
            out = self.__wrapped__(*wrapped)
        if isinstance(out, tuple):
            return tuple(o.t if isinstance(o, jaxlite.Array) else o for o in out)
        return out.t if isinstance(out, jaxlite.Array) else out


def _nearest(tunable: Any, make: Callable[[Any], Any]) -> Any:
    seen, frontier = {tunable}, [tunable]
    while frontier:
        later = []
        for t in frontier:
            for n in neighbours(t):
                if n in seen:
                    continue
                seen.add(n)
                try:
                    return make(n)
                except KernelError:
                    later.append(n)
        frontier = later
    return None


COMPARE_CHUNK = 1 << 22


def compare(what: str, got: Any, want: Any, rtol: Optional[float] = None, atol: Optional[float] = None,
            inputs: Tuple[Any, ...] = ()) -> float:
    """The largest absolute difference between `got` and `want`; AssertionError beyond `rtol`/`atol`
    (default: exact for integers; 1e-4 for f32; for 16-bit results, or f32 from 16-bit inputs, 2e-2 and
    an atol of 2e-2 of the largest |want|), as the reference's compare (src/autokernel/api.py:320-364)."""
    want_dt = jaxlite.dtype(want.dtype)
    narrow = any(jaxlite.dtype(d).kind == "f" and jaxlite.dtype(d).itemsize <= 2 for d in inputs)
    if want_dt.kind != "f":
        default = 0.0
    elif want_dt.itemsize <= 2 or narrow:
        default = 2e-2
    else:
        default = 1e-4
    rtol = default if rtol is None else rtol
    g_all = _tensor(got).reshape(-1)
    w_all = _tensor(want).reshape(-1)
    chunks = range(0, w_all.numel(), COMPARE_CHUNK)
    if atol is None:
        scale = 1.0
        if default >= 2e-2:
            for start in chunks:
                w = w_all[start:start + COMPARE_CHUNK].double()
                finite = w[torch.isfinite(w)]
                if finite.numel():
                    scale = max(scale, float(finite.abs().max()))
        atol = default * scale
    error, differ = 0.0, 0
    for start in chunks:
        g = g_all[start:start + COMPARE_CHUNK].double().to(w_all.device)
        w = w_all[start:start + COMPARE_CHUNK].double()
        same = (g == w) | (torch.isnan(g) & torch.isnan(w))
        diff = torch.where(same, torch.zeros_like(g), (g - w).abs())
        diff = torch.nan_to_num(diff, nan=float("inf"))
        if diff.numel():
            error = max(error, float(diff.max()))
        close = torch.isclose(g, w, rtol=rtol, atol=atol, equal_nan=True)
        differ += int((~close).sum())
    if differ:
        raise AssertionError(f"{what}: the kernel and its reference differ in {differ} of {w_all.numel()} elements "
                             f"(largest difference {error:.3g}; rtol={rtol}, atol={atol:.3g})")
    return error


def kernel(fn: Callable[..., Any]) -> Kernel:
    """Compile a Python loop nest over tiles into one persistent gfx950 kernel (see Kernel)."""
    return Kernel(fn)
