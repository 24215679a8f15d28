"""Causal multi-head attention, flash-attention style, skipping key blocks in the future of a query block.

    out[b, h] = softmax(q[b, h] @ k[b, h].T + causal mask) @ v[b, h]

The spec of the reference's examples/causal_attention.py:25-63: q is pre-scaled by 1/sqrt(head_dim); for
each query block the key/value blocks stream by with a running row max, row sum and accumulator (the
online softmax), normalised once at the end. The reduction mask skips key blocks wholly in the future.
The row statistics are lane-wide, (block_q, 128), a row's value repeated in every lane, as written there.
"""

import tilejax_amd as autokernel
from tilejax_amd.jaxlite import jax, jnp

LANES = 128
MASK_VALUE = -1e30  # finite, so exp(old max - new max) never computes -inf + inf


@autokernel.tunable
class AttentionBlocks:
    """Queries and keys per block."""

    block_q: int = autokernel.choice(128, 256, 512, 1024, default=512)
    block_kv: int = autokernel.choice(128, 256, 512, 1024, default=512)


@autokernel.kernel
def causal_attention(q, k, v, blocks=AttentionBlocks()):
    B, H, S, D = q.shape
    bq, bk = min(blocks.block_q, S), min(blocks.block_kv, S)
    dtype = q.dtype
    out = jnp.zeros((B, H, S, D), dtype)
    for b in range(B):
        for h in range(H):
            for i in range(0, S, bq):
                row_max = jnp.full((bq, LANES), MASK_VALUE, jnp.float32)
                row_sum = jnp.zeros((bq, LANES), jnp.float32)  # of exp(s - row_max)
                acc = jnp.zeros((bq, D), jnp.float32)  # sum of exp(s - row_max) @ v
                for j in range(0, S, bk):
                    if j > i + bq - 1:  # every key is in the future of every query
                        continue
                    s = q[b, h, i : i + bq, :] @ k[b, h, j : j + bk, :].T
                    rows = i + jax.lax.broadcasted_iota(jnp.int32, (bq, bk), 0)
                    cols = j + jax.lax.broadcasted_iota(jnp.int32, (bq, bk), 1)
                    s = jnp.where(cols <= rows, s, MASK_VALUE)
                    max_new = jnp.maximum(row_max, jnp.max(s, axis=1, keepdims=True))
                    p = jnp.exp(s - jnp.tile(max_new, (1, bk // LANES)))
                    alpha = jnp.exp(row_max - max_new)
                    row_sum = alpha * row_sum + jnp.sum(p, axis=1, keepdims=True)
                    acc = jnp.tile(alpha, (1, D // LANES)) * acc + p.astype(dtype) @ v[b, h, j : j + bk, :]
                    row_max = max_new
                out = out.at[b, h, i : i + bq, :].set((acc / jnp.tile(row_sum, (1, D // LANES))).astype(dtype))
    return out
