"""`@tilejax_amd.kernel`: a Python loop nest over tiles, compiled to one persistent HIP kernel for gfx950.

The surface is the reference's (src/autokernel/api.py:36-391): a `Kernel` builds once per input signature
(shapes and dtypes); called without its tunable it is tuned on the GPU (tune.py) and remembers the result;
`.fn` is the function as written, `.reference` what the kernel computes (the nest run with `@` on matrix
units, reference.py), `.verify` compares the two, `.source` is the generated HIP C++, `.tuning` is what
tuning tried and chose.

Inputs and outputs are torch tensors on the GPU; the spec itself runs over jaxlite arrays, wrapped and
unwrapped here. There is no CPU fallback: calling a kernel without a GPU, or without the built runtime
library, raises KernelError.
"""

from __future__ import annotations

import collections
import functools
from dataclasses import dataclass, field
from typing import Any, Callable, Dict, Iterable, Optional, Tuple

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
    """One generated kernel: for a signature and a schedule, its plan, step schedule, HIP source and the
    program (launches, argument packing) that runs it."""

    plan: Plan
    schedule: Schedule
    config: Any  # tune.Config
    source: str
    trace: bool  # generated with trace regions, for the profiler
    program: Any = field(repr=False)

    @property
    def pipeline(self) -> Pipeline:
        return self.config.pipeline

    @property
    def steps(self) -> int:
        return self.schedule.steps

    @property
    def tiles(self) -> int:
        """Output tiles the kernel computes (tiles a mask skips excluded)."""
        return self.schedule.tiles

    @property
    def total_tiles(self) -> int:
        return self.schedule.total_tiles

    @property
    def lds_bytes(self) -> int:
        """LDS the kernel's own buffers take per workgroup."""
        return self.program.lds_bytes

    def run(self, *arrays: Any) -> Any:
        """The kernel on torch tensors already on the GPU: its output, or a tuple of them."""
        return self.program(*arrays)


def _as_tensor(x: Any) -> torch.Tensor:
    if isinstance(x, torch.Tensor):
        return x
    if isinstance(x, jaxlite.Array):
        return x.t
    if isinstance(x, np.ndarray):
        return jaxlite.asarray(x).t
    raise KernelError(f"kernel inputs are torch tensors (or jaxlite arrays), not {type(x).__name__}")


class _Signature:
    """What a kernel has built for one signature: its reference, plans per tunable, lowered kernels per
    schedule, and its tuning once asked."""

    __slots__ = ("reference", "plans", "lowered", "tuning")

    def __init__(self, reference: Callable[..., Any]) -> None:
        self.reference = reference
        self.plans: Dict[Any, Tuple[Plan, Schedule]] = {}
        self.lowered: Dict[Tuple[Any, bool], Lowered] = {}
        self.tuning: Any = None


class Kernel:
    """A loop nest compiled to a persistent gfx950 kernel. Call it like the function it was made from.

    Given its tunable (`matmul(x, y, MatmulTiles(tm=256))`) it uses it; without, it is tuned on the GPU for
    the inputs' signature when first called with it. A kernel is built when first called for a signature
    and schedule, reading the module and closure values its code uses at that moment."""

    def __init__(self, fn: Callable[..., Any]) -> None:
        self.nest: Nest = parse(fn)
        self.fn = _AsWritten(fn)
        self._source_fn = fn
        functools.update_wrapper(self, fn)
        defaults = fn.__defaults__ or ()
        self.default_tunable = defaults[-1] if self.nest.tunable else None
        if self.nest.tunable and not is_tunable(self.default_tunable):
            raise self.nest.error(
                f"`{self.nest.tunable}`'s default must be a @tilejax_amd.tunable, not {self.default_tunable!r}",
                self.nest.function.args)
        self._signatures: Dict[Signature, _Signature] = {}

    def __repr__(self) -> str:
        return f"<tilejax_amd.Kernel {self.nest.name}>"

    # Calling ------------------------------------------------------------------------------------------------

    def __call__(self, *args: Any) -> Any:
        arrays, _ = self._arguments(args)
        return self.lower(*args).run(*map(_as_tensor, arrays))

    def lower(self, *args: Any) -> Lowered:
        """The kernel for inputs like these (tensors, or (shape, dtype) pairs), and the tunable if given."""
        from .codegen import default_pipeline
        from .tune import Config

        arrays, tunable = self._arguments(args)
        signature = self.signature(*arrays)
        if tunable is None:
            return self.lowered(signature, self.tuning(*arrays).config)
        plan, schedule = self.build(signature, tunable)
        return self.lowered(signature, Config(tunable, default_pipeline(plan, schedule)))

    def source(self, *args: Any) -> str:
        """The generated HIP source for inputs like these."""
        return self.lower(*args).source

    def reference(self, *args: Any) -> Any:
        """What the kernel computes: the loop nest run as plain (jaxlite) JAX with `@` on matrix units, on
        the inputs' device. Without a tunable, at the one tuning chooses."""
        arrays, tunable = self._arguments(args)
        signature = self.signature(*arrays)
        if self.nest.tunable and tunable is None:
            tunable = self.lower(*arrays).config.tunable
        self.build(signature, tunable if tunable is not None else self.default_tunable)
        run = self._signatures[signature].reference
        tensors = [_as_tensor(a) for a in arrays]
        with jaxlite.default_device(tensors[0].device):
            out = run(*(jaxlite.Array(t) for t in tensors), *((tunable,) if self.nest.tunable else ()))
        if isinstance(out, tuple):
            return tuple(o.t for o in out)
        return out.t

    def verify(self, *args: Any, rtol: Optional[float] = None, atol: Optional[float] = None) -> float:
        """Run the kernel and its reference on the same inputs; AssertionError unless every output agrees
        within the dtypes' tolerances (or `rtol`/`atol`). Returns the largest absolute difference."""
        arrays, tunable = self._arguments(args)
        if self.nest.tunable:
            if tunable is None:
                tunable = self.lower(*arrays).config.tunable
            arrays = (*arrays, tunable)
        got, want = self(*arrays), self.reference(*arrays)
        if not isinstance(got, tuple):
            got, want = (got,), (want,)
        input_types = [dt for _, dt in self.signature(*arrays[: len(self.nest.inputs)])]
        return max(compare(f"{self.nest.name} output {name!r}", g, w, rtol, atol, tuple(input_types))
                   for name, g, w in zip(self.nest.outputs, got, want))

    def tuning(self, *arrays: Any) -> Any:
        """The schedule for inputs like these, tuned on the GPU the first time it is asked (tune.py)."""
        from .tune import tune

        signature = self.signature(*arrays)
        entry = self._entry(signature)
        if entry.tuning is None:
            entry.tuning = tune(self, signature, arrays)
        return entry.tuning

    # Building (tune.py uses these too) ---------------------------------------------------------------------

    def signature(self, *arrays: Any) -> Signature:
        """The inputs' shapes and dtypes; an input may be given as a (shape, dtype) pair."""
        out = []
        for name, x in zip(self.nest.inputs, arrays):
            if isinstance(x, tuple) and len(x) == 2 and isinstance(x[0], tuple):
                out.append((tuple(int(n) for n in x[0]), jaxlite.dtype(x[1])))
            elif hasattr(x, "shape") and hasattr(x, "dtype") and tuple(x.shape):
                out.append((tuple(int(n) for n in x.shape), jaxlite.dtype(x.dtype)))
            else:
                raise KernelError(f"{self.nest.name}: input `{name}` must be an array, got {type(x).__name__}")
        return tuple(out)

    def default_config(self, signature: Signature) -> Any:
        """The tunable's defaults with their default buffering; if those don't build for this signature, the
        nearest tunable (fewest moves) that does."""
        from .codegen import default_pipeline
        from .tune import Config

        def config_for(t: Any) -> Any:
            plan, schedule = self.build(signature, t)
            config = Config(t, default_pipeline(plan, schedule))
            self.lowered(signature, config)  # it has to lower, too
            return config

        try:
            return config_for(self.default_tunable)
        except KernelError:
            if self.default_tunable is None:
                raise
            found = _closest_that_builds(self.default_tunable, config_for)
            if found is None:
                raise
            return found

    def build(self, signature: Signature, tunable: Any) -> Tuple[Plan, Schedule]:
        """The plan and step schedule for this signature and tunable."""
        entry = self._entry(signature)
        if tunable not in entry.plans:
            plan = make_plan(self.nest, self._source_fn, [Spec(s, dt) for s, dt in signature], tunable)
            entry.plans[tunable] = (plan, make_schedule(plan))
        return entry.plans[tunable]

    def lowered(self, signature: Signature, config: Any, trace: bool = False) -> Lowered:
        """The kernel for this signature and schedule (with trace regions when `trace`)."""
        from . import codegen

        entry = self._entry(signature)
        key = (config, trace)
        if key not in entry.lowered:
            plan, schedule = self.build(signature, config.tunable)
            if config.cursor and not plan.either:
                raise KernelError(f"{self.nest.name}: only a kernel with runtime masks finds its steps with a cursor")
            program = codegen.generate(plan, schedule, config.pipeline, trace=trace, cursor=config.cursor,
                                       hardware=dict(getattr(config, "hardware", ())))
            entry.lowered[key] = Lowered(plan, schedule, config, program.source, trace, program)
        return entry.lowered[key]

    def _entry(self, signature: Signature) -> _Signature:
        entry = self._signatures.get(signature)
        if entry is None:
            entry = self._signatures[signature] = _Signature(make_reference(self.nest, self._source_fn))
        return entry

    def _arguments(self, args: Tuple[Any, ...]) -> Tuple[Tuple[Any, ...], Any]:
        """(the input arrays, the tunable or None)."""
        nest, n = self.nest, len(self.nest.inputs)
        if len(args) == n:
            return args, None
        if nest.tunable and len(args) == n + 1:
            given = args[-1]
            if type(given) is not type(self.default_tunable):
                raise KernelError(f"{nest.name}: `{nest.tunable}` must be a {type(self.default_tunable).__name__}, "
                                  f"not {type(given).__name__}")
            return args[:-1], given
        also = f", then optionally `{nest.tunable}`" if nest.tunable else ""
        raise KernelError(f"{nest.name} takes {n} input arrays ({', '.join(nest.inputs)}){also}; got {len(args)}")


class _AsWritten:
    """`kernel.fn`: the function exactly as written (plain JAX: `bf16 @ bf16` rounds to bf16), on torch
    tensors, wrapped as jaxlite arrays inside."""

    def __init__(self, fn: Callable[..., Any]) -> None:
        self.__wrapped__ = fn
        functools.update_wrapper(self, fn)

    @property
    def __globals__(self) -> Dict[str, Any]:  # the function's own globals, as on the plain function
        return self.__wrapped__.__globals__

    @property
    def __code__(self) -> Any:
        return self.__wrapped__.__code__

    def __call__(self, *args: Any) -> Any:
        device = next((a.device for a in args if isinstance(a, torch.Tensor)), "cpu")
        with jaxlite.default_device(device):
            out = self.__wrapped__(*(jaxlite.Array(a) if isinstance(a, torch.Tensor) else a for a in args))
        unwrap = lambda o: o.t if isinstance(o, jaxlite.Array) else o  # noqa: E731
        return tuple(map(unwrap, out)) if isinstance(out, tuple) else unwrap(out)


def _closest_that_builds(start: Any, make: Callable[[Any], Any]) -> Any:
    """Breadth first over neighbours from `start` (itself excluded): the first tunable `make` turns into a
    config without a KernelError, or None."""
    queue = collections.deque(neighbours(start))
    seen = {start, *queue}
    while queue:
        t = queue.popleft()
        try:
            return make(t)
        except KernelError:
            pass
        for n in neighbours(t):
            if n not in seen:
                seen.add(n)
                queue.append(n)
    return None


COMPARE_CHUNK = 1 << 22  # elements compared at a time (float64 copies of a whole large output don't fit)


def _default_tolerance(want: Any, inputs: Iterable[Any]) -> Tuple[float, bool]:
    """(rtol, whether atol scales with the largest |want|): exact for integers; 1e-4 for f32; 2e-2, scaled,
    for 16-bit results and for f32 results of 16-bit inputs, whose intermediates round at every step."""
    dt = jaxlite.dtype(want.dtype)
    if dt.kind != "f":
        return 0.0, False
    sixteen = dt.itemsize <= 2 or any(jaxlite.dtype(d).kind == "f" and jaxlite.dtype(d).itemsize <= 2 for d in inputs)
    return (2e-2, True) if sixteen else (1e-4, False)


def compare(what: str, got: Any, want: Any, rtol: Optional[float] = None, atol: Optional[float] = None,
            inputs: Tuple[Any, ...] = ()) -> float:
    """The largest absolute difference between `got` and `want`; AssertionError where they differ beyond
    `rtol`/`atol`. Defaults as the reference's compare (src/autokernel/api.py:320-364): exact for integers,
    1e-4 for f32, and for 16-bit results (or f32 from 16-bit inputs) 2e-2 with an atol of 2e-2 of the
    largest finite |want|. NaN matches NaN."""
    default_rtol, scaled = _default_tolerance(want, inputs)
    rtol = default_rtol if rtol is None else rtol
    g_flat, w_flat = _as_tensor(got).reshape(-1), _as_tensor(want).reshape(-1)
    n = w_flat.numel()
    spans = [(k, min(k + COMPARE_CHUNK, n)) for k in range(0, n, COMPARE_CHUNK)]
    if atol is None:
        largest = 1.0
        if scaled:
            for a, b in spans:
                w = w_flat[a:b].double()
                w = w[torch.isfinite(w)]
                if w.numel():
                    largest = max(largest, float(w.abs().max()))
        atol = default_rtol * largest
    worst, bad = 0.0, 0
    for a, b in spans:
        g = g_flat[a:b].double().to(w_flat.device)
        w = w_flat[a:b].double()
        both_nan = torch.isnan(g) & torch.isnan(w)
        diff = torch.nan_to_num(torch.where((g == w) | both_nan, torch.zeros_like(g), (g - w).abs()), nan=float("inf"))
        if diff.numel():
            worst = max(worst, float(diff.max()))
        bad += int((~torch.isclose(g, w, rtol=rtol, atol=atol, equal_nan=True)).sum())
    if bad:
        raise AssertionError(f"{what}: the kernel and its reference differ in {bad} of {n} elements "
                             f"(largest difference {worst:.3g}; rtol={rtol}, atol={atol:.3g})")
    return worst


def kernel(fn: Callable[..., Any]) -> Kernel:
    """Compile a Python loop nest over tiles into one persistent gfx950 kernel (see Kernel)."""
    return Kernel(fn)
