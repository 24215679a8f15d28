"""Shared helpers: kernels from source strings (registered with linecache so errors can quote their lines),
input specs, and seeded inputs."""

from __future__ import annotations

import itertools
import linecache
import textwrap
from typing import Any, Tuple

import torch

import tilejax_amd
from tilejax_amd import jaxlite
from tilejax_amd.jaxlite import jax, jnp

_sources = itertools.count()


def make_kernel(source: str, **namespace: Any) -> tilejax_amd.Kernel:
    """The kernel of the last function a source string defines; `namespace` holds its globals (jax and jnp
    are there already)."""
    source = textwrap.dedent(source)
    filename = f"<tilejax-test-{next(_sources)}>"
    linecache.cache[filename] = (len(source), None, source.splitlines(True), filename)
    env = {"jax": jax, "jnp": jnp, **namespace}
    exec(compile(source, filename, "exec"), env)
    fns = [v for v in env.values() if callable(v) and getattr(getattr(v, "__code__", None), "co_filename", "") == filename]
    return tilejax_amd.kernel(fns[-1])


def spec(*shape: int, dtype: Any = jaxlite.float32) -> Tuple[Tuple[int, ...], Any]:
    """An input of this shape and dtype, without data: what `lower` and `build` take."""
    return (tuple(shape), jaxlite.dtype(dtype))


def rand(shape, seed: int = 0, dtype: torch.dtype = torch.float32) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(dtype)


def schedule_of(kernel: tilejax_amd.Kernel, *inputs: Any, tunable: Any = None):
    return kernel.build(kernel.signature(*inputs), tunable)[1]
