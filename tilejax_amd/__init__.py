"""tilejax_amd: plain-JAX loop nests over tiles, compiled to persistent HIP kernels for one MI355X.

The API of the reference's `autokernel` package (src/autokernel/__init__.py:32-62), MI355X-native:

- `@tilejax_amd.kernel` compiles a loop nest over output tiles into one persistent gfx950 kernel; call it
  like the function. Its last parameter may be a tunable (`@tilejax_amd.tunable`); pass one and it is
  used, leave it out and the kernel is tuned on the GPU.
- `kernel.fn` is the function as written; `kernel.reference` the same with `@` accumulating in f32;
  `kernel.verify(...)` compares the kernel with it; `kernel.source(...)` is the generated HIP C++;
  `kernel.tuning(...)` is what tuning tried and chose.
- `tilejax_amd.profile(kernel, ...)` says where a kernel's time goes (device time, step count, bottleneck).

Specs are written over `tilejax_amd.jaxlite` (`from tilejax_amd.jaxlite import jax, jnp`).
"""

from __future__ import annotations

from typing import Any

from .api import Kernel, Lowered, compare, kernel
from .errors import KernelError
from .packing import pairs, unpairs
from .pipeline import Pipeline
from .ragged import rows
from .tunable import choice, tunable

__all__ = [
    "Config",
    "Kernel",
    "KernelError",
    "KernelProfile",
    "Lowered",
    "Pipeline",
    "Trial",
    "Tuning",
    "choice",
    "compare",
    "enable_profiling",
    "kernel",
    "pairs",
    "profile",
    "rows",
    "tunable",
    "unpairs",
]

__version__ = "0.1.0"


def __getattr__(name: str) -> Any:
    if name in ("Config", "Trial", "Tuning"):
        from . import tune

        return getattr(tune, name)
    if name in ("KernelProfile", "enable_profiling"):
        from . import profiling

        return getattr(profiling, name)
    raise AttributeError(name)


def profile(kernel: Kernel, *args: Any, runs: int = 5) -> Any:
    """Where `kernel`'s time goes on the GPU for these inputs (and tunable, if given)."""
    from . import profiling

    return profiling.profile(kernel, args, runs=runs)
