"""Causal matmul, `tril(x @ y)`, skipping every output tile above the diagonal.

The spec of the reference's examples/causal_matmul.py:23-40. Tiles above the diagonal are skipped by the
mask (written with the zeros of jnp.zeros); tiles on it are computed, then the entries above the diagonal
zeroed by jnp.where.
"""

import tilejax_amd as autokernel
from tilejax_amd.jaxlite import jax, jnp

from .matmul import MatmulTiles


@autokernel.kernel
def causal_matmul(x, y, tiles=MatmulTiles()):
    M, K = x.shape
    N = y.shape[1]
    tm, tn, tk = min(tiles.tm, M), min(tiles.tn, N), min(tiles.tk, K)
    dtype = x.dtype
    out = jnp.zeros((M, N), dtype)
    for i in range(0, M, tm):
        for j in range(0, N, tn):
            if j > i + tm - 1:  # the whole tile is above the diagonal
                continue
            acc = jnp.zeros((tm, tn), jnp.float32)
            for k in range(0, K, tk):
                acc += x[i : i + tm, k : k + tk] @ y[k : k + tk, j : j + tn]
            rows = i + jax.lax.broadcasted_iota(jnp.int32, (tm, tn), 0)
            cols = j + jax.lax.broadcasted_iota(jnp.int32, (tm, tn), 1)
            out = out.at[i : i + tm, j : j + tn].set(jnp.where(cols <= rows, acc, 0.0).astype(dtype))
    return out
