"""RMSNorm fused with the projection after it: `rmsnorm(x) @ w`.

    rmsnorm(x) = x / sqrt(mean(x**2, axis=-1) + eps) * gamma

The spec of the reference's examples/rmsnorm_matmul.py:21-46, in this package's JAX stand-in: the row
scale commutes with the matmul, `rmsnorm(x) @ w = (1 / rms(x)) * ((x * gamma) @ w)`, so one reduction over
the model dimension accumulates both `(x * gamma) @ w` and each row's sum of squares (lane-wide, (tm, 128)),
and the tile is scaled once at the end.
"""

import tilejax_amd as autokernel
from tilejax_amd.jaxlite import jax, jnp

EPS = 1e-6
LANES = 128


@autokernel.tunable
class NormMatmulTiles:
    """(tm, tn) output tiles, each summing tk-deep products (and tm rows' squares) over the model dim."""

    tm: int = autokernel.choice(128, 256, 512, 1024, 2048, default=512)
    tn: int = autokernel.choice(128, 256, 512, 1024, 2048, default=512)
    tk: int = autokernel.choice(128, 256, 512, 1024, 2048, default=512)


@autokernel.kernel
def rmsnorm_matmul(x, gamma, w, tiles=NormMatmulTiles()):
    M, D = x.shape
    N = w.shape[1]
    tm, tn, tk = min(tiles.tm, M), min(tiles.tn, N), min(tiles.tk, D)
    dtype = x.dtype
    out = jnp.zeros((M, N), dtype)
    for i in range(0, M, tm):
        for j in range(0, N, tn):
            acc = jnp.zeros((tm, tn), jnp.float32)  # (x * gamma) @ w
            sum_sq = jnp.zeros((tm, LANES), jnp.float32)  # each row's sum of squares, lane-wide
            for k in range(0, D, tk):
                xk = x[i : i + tm, k : k + tk].astype(jnp.float32)
                sum_sq += jnp.sum(xk * xk, axis=1, keepdims=True)
                acc += (xk * gamma[0:1, k : k + tk].astype(jnp.float32)).astype(dtype) @ w[k : k + tk, j : j + tn]
            scale = jax.lax.rsqrt(sum_sq / D + EPS)
            out = out.at[i : i + tm, j : j + tn].set((acc * jnp.tile(scale, (1, tn // LANES))).astype(dtype))
    return out
