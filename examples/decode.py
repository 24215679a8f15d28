"""Paged grouped-query decode attention: one new token per sequence against a paged KV cache.

    out[b, t, h] = softmax(q[b, t, h] @ K[b, kv(h), :n].T) @ V[b, kv(h), :n],   n = lengths[b]

The spec of BASELINE.json config 5, the reference's `paged_gqa_decode` (examples/decode.py:199-223, with the
helpers at :92-172) in this package's JAX stand-in: the cache is vLLM's paged layout (kv_cache.py), pages
(num_pages, page_size, Hkv * Dh) with sequence b's i-th page at `block_tables[b, i]`; the reduction loop
walks a sequence's pages under the runtime mask `p * P >= lengths[b]`, reading the page through a runtime
window. All query heads go through one matmul against each page: the query rows are spread
block-diagonally over the kv heads' column blocks once per sequence (`block_diagonal`), and each row's own
block of the accumulator is picked at the end (`own_blocks`). Row statistics are lane-wide (rows, 128).
"""

import tilejax_amd as autokernel
from tilejax_amd.jaxlite import jax, jnp

LANES = 128
MASK_VALUE = -1e30  # finite, so exp(old max - new max) never computes -inf + inf


def widen(stat, n):
    """A lane-wide (rows, 128) row statistic as (rows, n): repeated across lanes, or its first n lanes."""
    return jnp.tile(stat, (1, n // LANES)) if n >= LANES else stat[:, :n]


def _dot(a, b):
    """a @ b accumulating in f32, as `@` in kernel code means."""
    return jnp.dot(a, b, preferred_element_type=jnp.float32)


def query_rows(qt):
    """A sequence's queries (T, H, d) as rows (T * H, d), row t * H + h being token t's head h."""
    t, h, d = qt.shape
    return qt.astype(jnp.float32).reshape(t * h, d)


def _blocks_below(x, size, count):
    """x // size for int32 x in [0, size * count), by comparisons."""
    out = jnp.zeros(x.shape, jnp.int32)
    for k in range(1, count):
        out += (x >= k * size).astype(jnp.int32)
    return out


def row_index(n_rows, heads, kv_heads):
    """For query rows, lane-wide (n_rows, 128) int32: each row's token, and its kv head h // (heads / kv_heads)."""
    rows = jax.lax.broadcasted_iota(jnp.int32, (n_rows, LANES), 0)
    token = _blocks_below(rows, heads, n_rows // heads)
    return token, _blocks_below(rows - token * heads, heads // kv_heads, kv_heads)


def block_diagonal(rows, group, kv_heads, dtype):
    """Query rows (R, Dh) spread over the kv heads' column blocks, (R, kv_heads * Dh): a row keeps its
    values in the block of its kv head and is 0 elsewhere."""
    group = widen(group, rows.shape[1])
    return jnp.concatenate([jnp.where(group == g, rows, 0.0) for g in range(kv_heads)], axis=1).astype(dtype)


def own_blocks(acc, group, kv_heads):
    """Each row's own kv head's column block of `acc` (R, kv_heads * Dh): (R, Dh)."""
    dh = acc.shape[1] // kv_heads
    group = widen(group, dh)
    out = acc[:, :dh]
    for g in range(1, kv_heads):
        out = jnp.where(group == g, acc[:, g * dh : (g + 1) * dh], out)
    return out


def visible(token, bk, j, length, new_tokens):
    """Which (query row, cache position) pairs attend for a cache block at position j."""
    cols = j + jax.lax.broadcasted_iota(jnp.int32, (token.shape[0], bk), 1)
    if new_tokens == 1:
        return cols < length
    return cols <= length - new_tokens + widen(token, bk)


def online_softmax(s, v, ok, row_max, row_sum, acc):
    """One online-softmax step over scores `s` (R, bk), masked where not `ok`, against values `v` (bk, Dv)."""
    bk, dv = s.shape[1], v.shape[1]
    s = jnp.where(ok, s, MASK_VALUE)
    max_new = jnp.maximum(row_max, jnp.max(s, axis=1, keepdims=True))
    p = jnp.exp(s - widen(max_new, bk))
    alpha = jnp.exp(row_max - max_new)
    row_sum = alpha * row_sum + jnp.sum(p, axis=1, keepdims=True)
    acc = widen(alpha, dv) * acc + _dot(p.astype(v.dtype), v)
    return max_new, row_sum, acc


def finish(acc, row_sum, shape, dtype):
    """The normalized output (T * H, d) as `shape`; rows that saw no key (an empty sequence) are 0."""
    out = acc * widen(1.0 / jnp.maximum(row_sum, 1e-30), acc.shape[1])
    return out.reshape(shape).astype(dtype)


@autokernel.tunable
class DecodeTiles:
    """Cache positions per step."""

    block_kv: int = autokernel.choice(128, 256, 512, 1024, 2048, default=512)


@autokernel.kernel
def gqa_decode(q, k_cache, v_cache, lengths, tiles=DecodeTiles()):
    """GQA decode attention over a contiguous cache: q (B, T, H, Dh), caches (B, S_max, Hkv * Dh)
    (the reference's examples/decode.py:175-196)."""
    B, T, H, Dh = q.shape
    S, W = k_cache.shape[1], k_cache.shape[2]
    Hkv, R = W // Dh, T * H
    bk, dtype = min(tiles.block_kv, S), q.dtype
    out = jnp.zeros((B, T, H, Dh), dtype)
    for b in range(B):
        token, group = row_index(R, H, Hkv)
        qt = block_diagonal(query_rows(q[b, :, :, :]), group, Hkv, dtype)  # once per sequence
        row_max = jnp.full((R, LANES), MASK_VALUE, jnp.float32)
        row_sum = jnp.zeros((R, LANES), jnp.float32)
        acc = jnp.zeros((R, W), jnp.float32)  # every kv head's values; a row keeps its own block
        for j in range(0, S, bk):
            if j >= lengths[b]:  # past the sequence's end: decided on the device, before the kernel runs
                continue
            s = qt @ k_cache[b, j : j + bk, :].T
            ok = visible(token, bk, j, lengths[b], T)
            row_max, row_sum, acc = online_softmax(s, v_cache[b, j : j + bk, :], ok, row_max, row_sum, acc)
        out = out.at[b, :, :, :].set(finish(own_blocks(acc, group, Hkv), row_sum, (T, H, Dh), dtype))
    return out


@autokernel.kernel
def paged_gqa_decode(q, k_pages, v_pages, block_tables, lengths):
    """GQA decode attention over a paged cache: q (B, T, H, Dh), pages (num_pages, page_size, Hkv * Dh),
    sequence b's pages listed in block_tables[b, :]."""
    B, T, H, Dh = q.shape
    P, W = k_pages.shape[1], k_pages.shape[2]
    pages = block_tables.shape[1]
    Hkv, R = W // Dh, T * H
    dtype = q.dtype
    out = jnp.zeros((B, T, H, Dh), dtype)
    for b in range(B):
        token, group = row_index(R, H, Hkv)
        qt = block_diagonal(query_rows(q[b, :, :, :]), group, Hkv, dtype)
        row_max = jnp.full((R, LANES), MASK_VALUE, jnp.float32)
        row_sum = jnp.zeros((R, LANES), jnp.float32)
        acc = jnp.zeros((R, W), jnp.float32)
        for p in range(pages):
            if p * P >= lengths[b]:
                continue
            s = qt @ k_pages[block_tables[b, p], :, :].T  # a runtime window: the page is chosen on the device
            ok = visible(token, P, p * P, lengths[b], T)
            vt = v_pages[block_tables[b, p], :, :]
            row_max, row_sum, acc = online_softmax(s, vt, ok, row_max, row_sum, acc)
        out = out.at[b, :, :, :].set(finish(own_blocks(acc, group, Hkv), row_sum, (T, H, Dh), dtype))
    return out
