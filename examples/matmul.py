"""Matmul, `x @ y`, as plain loops over tiles, its tile sizes left to the autotuner.

The spec of the reference's examples/matmul.py:13-35, in this package's JAX stand-in (jaxlite): the
same loop nest, the same tunable.
"""

import tilejax_amd as autokernel
from tilejax_amd.jaxlite import jnp


@autokernel.tunable
class MatmulTiles:
    """(tm, tn) output tiles, each summing tk-deep products."""

    tm: int = autokernel.choice(128, 256, 512, 1024, 2048, default=512)
    tn: int = autokernel.choice(128, 256, 512, 1024, 2048, default=512)
    tk: int = autokernel.choice(128, 256, 512, 1024, 2048, default=512)


@autokernel.kernel
def matmul(x, y, tiles=MatmulTiles()):
    M, K = x.shape
    N = y.shape[1]
    tm, tn, tk = min(tiles.tm, M), min(tiles.tn, N), min(tiles.tk, K)
    dtype = x.dtype
    out = jnp.zeros((M, N), dtype)
    for i in range(0, M, tm):
        for j in range(0, N, tn):
            acc = jnp.zeros((tm, tn), jnp.float32)
            for k in range(0, K, tk):
                acc += x[i : i + tm, k : k + tk] @ y[k : k + tk, j : j + tn]
            out = out.at[i : i + tm, j : j + tn].set(acc.astype(dtype))
    return out
