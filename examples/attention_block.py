"""A transformer block's attention half and feed-forward in one loop nest: causal multi-head attention, the
post-attention RMSNorm, then the feed-forward projections.

    a   = [softmax(q_h @ k_h.T + causal mask) @ v_h for every head h], side by side    (B, S, D = H * Dh)
    h   = a * rsqrt(mean(a^2) + eps) * gamma
    out = gelu(h @ w_up) @ w_down

The spec of the reference's examples/attention_block.py:47-80, over this package's JAX stand-in. The
parallel loops walk (batch, query block); each tile runs two reduction loops in turn: the attention over
key blocks (those wholly in the query block's future skipped), every head at once through per-head lists
of products, then the feed-forward over blocks of hidden units. Neither the attention output nor the
hidden activations leave the tile. It has no matmul-family or flash-family shape, so it lowers to the
generic kernel (tilejax_amd/codegen/generic.py).
"""

import tilejax_amd as autokernel
from tilejax_amd.jaxlite import jax, jnp

EPS = 1e-6
LANES = 128
MASK_VALUE = -1e30  # finite, so exp(old max - new max) never computes -inf + inf


@autokernel.tunable
class BlockTiles:
    """Queries per tile, keys per attention step, hidden units per feed-forward step."""

    block_q: int = autokernel.choice(64, 128, 256, 512, 1024, default=256)
    block_kv: int = autokernel.choice(64, 128, 256, 512, 1024, default=256)
    block_f: int = autokernel.choice(256, 512, 1024, 2048, 4096, 8192, 16384, default=1024)


def widen(stat, n):
    """A lane-wide (..., 128) statistic as (..., n): repeated across lanes, or its first n lanes."""
    return jnp.tile(stat, (1,) * (stat.ndim - 1) + (n // LANES,)) if n >= LANES else stat[..., :n]


@autokernel.kernel
def attention_block(q, k, v, gamma, w_up, w_down, tiles=BlockTiles()):
    B, H, S, Dh = q.shape
    D, F = H * Dh, w_up.shape[1]
    bq, bk, bf = min(tiles.block_q, S), min(tiles.block_kv, S), min(tiles.block_f, F)
    dtype = q.dtype
    out = jnp.zeros((B, S, D), dtype)
    for b in range(B):
        for i in range(0, S, bq):
            row_max = jnp.full((H, bq, LANES), MASK_VALUE, jnp.float32)
            row_sum = jnp.zeros((H, bq, LANES), jnp.float32)
            acc = jnp.zeros((H, bq, Dh), jnp.float32)
            for j in range(0, S, bk):  # the attention, every head at once
                if j > i + bq - 1:
                    continue
                qt, kt, vt = q[b, :, i : i + bq, :], k[b, :, j : j + bk, :], v[b, :, j : j + bk, :]
                rows = i + jax.lax.broadcasted_iota(jnp.int32, (bq, bk), 0)
                cols = j + jax.lax.broadcasted_iota(jnp.int32, (bq, bk), 1)
                s = jnp.stack([jnp.where(cols <= rows, qt[h] @ kt[h].T, MASK_VALUE) for h in range(H)])
                max_new = jnp.maximum(row_max, jnp.max(s, axis=2, keepdims=True))
                p = jnp.exp(s - widen(max_new, bk))
                alpha = jnp.exp(row_max - max_new)
                row_sum = alpha * row_sum + jnp.sum(p, axis=2, keepdims=True)
                pv = jnp.stack([p[h].astype(dtype) @ vt[h] for h in range(H)])
                acc = widen(alpha, Dh) * acc + pv
                row_max = max_new
            heads = acc / widen(row_sum, Dh)
            a = jnp.concatenate([heads[h] for h in range(H)], axis=1)  # (bq, D)
            normed = (a * jax.lax.rsqrt(jnp.mean(a * a, axis=1, keepdims=True) + EPS) * gamma[0:1, :]).astype(dtype)
            y = jnp.zeros((bq, D), jnp.float32)
            for f in range(0, F, bf):  # the feed-forward, bf hidden units at a time
                hidden = jax.nn.gelu(normed @ w_up[:, f : f + bf])
                y += hidden.astype(dtype) @ w_down[f : f + bf, :]
            out = out.at[b, i : i + bq, :].set(y.astype(dtype))
    return out
