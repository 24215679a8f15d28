"""Ragged paged attention's cache write and decode attention (vLLM's RPA v3 ABI), as tilejax_amd kernels.

The specs of the reference's examples/ragged_paged_attention.py:31-142 (`rpa_write`, `make_decode`), over this
package's JAX stand-in. The cache is (pages, page_size, Hkv, 2, D): each kv head's key and value side by side,
read as 32-bit words with `tilejax_amd.pairs` (key in the low half) and written back with `unpairs`.

- `rpa_write` stores the step's new keys and values into the cache in place, a tile per run of a sequence's
  new tokens that lands in one page: ragged rows (`rows`), a runtime count of tiles, a scatter through the
  page table.
- `make_decode(scale)` is the decode sequences' attention, a tile per sequence: its pages are a loop whose
  count is read as the kernel runs, each page's keys and values split out of the words, every query head
  against every kv head's keys masked to its own kv head (GQA), an online softmax. The output is q updated in
  place: a decode token's row becomes its attention output, every other row stays its query.

Neither has a kernel family's shape: both lower to the generic kernel walking the tile as written.
"""

from __future__ import annotations

import tilejax_amd
from tilejax_amd.jaxlite import jax, jnp

LANES = 128
MASK_VALUE = -1e30  # finite: exp(old max - new max) never computes -inf + inf


def key_value_words(k, v):
    """Keys and values (..., D) bf16 as the cache's (key | value << 16) words: a bf16 is the high half of
    the f32 it widens to."""
    bits = lambda x: jax.lax.bitcast_convert_type(x.astype(jnp.float32), jnp.uint32)  # noqa: E731
    return (bits(k) >> 16) | (bits(v) & jnp.uint32(0xFFFF0000))


def keys_values(words):
    """A page's words (positions, Hkv, D) as keys and values (positions * Hkv, D) bf16, row t * Hkv + g
    position t's kv head g."""
    w = words.reshape(-1, words.shape[-1])
    k = jax.lax.bitcast_convert_type(w << 16, jnp.float32)
    v = jax.lax.bitcast_convert_type(w & jnp.uint32(0xFFFF0000), jnp.float32)
    return k.astype(jnp.bfloat16), v.astype(jnp.bfloat16)


def own_heads(heads, kv_heads, positions, start, length):
    """Which (query head, column) pairs attend (column t * kv_heads + g: position start + t's kv head g): a
    query head's own kv head, at positions before `length`."""
    shape = (heads, positions * kv_heads)
    col = jax.lax.broadcasted_iota(jnp.int32, shape, 1)
    head = jax.lax.broadcasted_iota(jnp.int32, shape, 0)
    return ((col % kv_heads) == head // (heads // kv_heads)) & (start + col // kv_heads < length)


def online_softmax(s, v, row_max, row_sum, acc):
    """One online-softmax step: scores s (R, n) against values v (n, D); lane-wide running max and sum
    (R, 128) and the accumulator (R, D)."""
    n, d = s.shape[1], v.shape[1]
    max_new = jnp.maximum(row_max, jnp.max(s, axis=1, keepdims=True))
    p = jnp.exp(s - jnp.tile(max_new, (1, n // LANES)))
    alpha = jnp.exp(row_max - max_new)
    row_sum = alpha * row_sum + jnp.sum(p, axis=1, keepdims=True)
    acc = jnp.tile(alpha, (1, d // LANES)) * acc + p.astype(v.dtype) @ v
    return max_new, row_sum, acc


@tilejax_amd.kernel
def rpa_write(kv_cache, keys, values, page_indices, write_page, write_rows, write_first, write_stop, n_writes):
    """The cache with the new keys and values (T, Hkv, D) written in place: run w's tokens from
    write_rows[w] go to positions write_first[w] .. write_stop[w] of page page_indices[write_page[w]]."""
    ps, dtype = kv_cache.shape[1], kv_cache.dtype
    out = kv_cache
    for w in range(n_writes[0]):  # the runs, counted as the kernel runs
        k = keys[tilejax_amd.rows(write_rows[w], write_rows[w] + write_stop[w] - write_first[w], ps), :, :]
        v = values[tilejax_amd.rows(write_rows[w], write_rows[w] + write_stop[w] - write_first[w], ps), :, :]
        out = out.at[page_indices[write_page[w]], tilejax_amd.rows(write_first[w], write_stop[w], ps), :, :, :].set(
            tilejax_amd.unpairs(key_value_words(k, v), dtype)
        )
    return out


def make_decode(sm_scale: float) -> tilejax_amd.Kernel:
    """The decode sequences' attention, a tile per sequence (s < distribution[0] is token s)."""

    @tilejax_amd.kernel
    def rpa_decode(q, kv_cache, kv_lens, page_indices, distribution):
        T, H, D = q.shape
        ps, Hkv = kv_cache.shape[1], kv_cache.shape[2]
        S = kv_lens.shape[0]
        pps = page_indices.shape[0] // S
        dtype = q.dtype
        out = q
        for s in range(min(S, T)):
            qs = q[s, :, :]
            row_max = jnp.full((H, LANES), MASK_VALUE, jnp.float32)
            row_sum = jnp.zeros((H, LANES), jnp.float32)
            acc = jnp.zeros((H, D), jnp.float32)
            for p in range((kv_lens[s] + ps - 1) // ps if s < distribution[0] else 0):  # its pages, as it runs
                k, v = keys_values(tilejax_amd.pairs(kv_cache[page_indices[s * pps + p], :, :, :, :]))
                scores = (qs @ k.T) * sm_scale  # every query head against every kv head's keys
                ok = own_heads(H, Hkv, ps, p * ps, kv_lens[s])
                row_max, row_sum, acc = online_softmax(jnp.where(ok, scores, MASK_VALUE), v, row_max, row_sum, acc)
            o = acc * jnp.tile(1.0 / jnp.maximum(row_sum, 1e-30), (1, D // LANES))
            out = out.at[s, :, :].set(jnp.where(s < distribution[0], o.astype(dtype), qs))
        return out

    return rpa_decode


# --------------------------------------------------------------------------- prefill and mixed: a block of queries

BLOCK_Q = 256  # query tokens per tile


@tilejax_amd.tunable
class PrefillTiles:
    pages: int = tilejax_amd.choice(1, 2, 4, 8, default=4)  # cache pages per step


def head_rows(qb, kv_heads):
    """A block of queries (BQ, H, D) as each kv head's rows (Hkv, BQ * G, D), row t * G + i being token t's
    query head g * G + i (G = H / Hkv, as GQA groups heads)."""
    bq, h, d = qb.shape
    g = h // kv_heads
    return jnp.stack([qb[:, i * g : (i + 1) * g, :].reshape(bq * g, d) for i in range(kv_heads)])


def token_heads(rows, heads):
    """`head_rows` undone: (Hkv, BQ * G, D) -> (BQ, H, D)."""
    kv_heads, n, d = rows.shape
    g = heads // kv_heads
    return jnp.concatenate([rows[i].reshape(n // g, g, d) for i in range(kv_heads)], axis=1)


def visible(heads, rows, cols, first_row, first_col, stop):
    """Which (row, column) pairs attend: row t * G + i (a query at position first_row + t) sees position
    first_col + c if it is no later than its own and before `stop`."""
    shape = (1, rows, cols)
    pos = first_row + jax.lax.broadcasted_iota(jnp.int32, shape, 1) // heads
    col = first_col + jax.lax.broadcasted_iota(jnp.int32, shape, 2)
    return (col <= pos) & (col < stop)


def online_softmax_heads(s, v, row_max, row_sum, acc):
    """`online_softmax` for every kv head at once: s (Hkv, R, n), v (Hkv, n, D), stats (Hkv, R, 128)."""
    n, d = s.shape[-1], v.shape[-1]
    max_new = jnp.maximum(row_max, jnp.max(s, axis=-1, keepdims=True))
    p = jnp.exp(s - jnp.tile(max_new, (1, 1, n // LANES)))
    alpha = jnp.exp(row_max - max_new)
    row_sum = alpha * row_sum + jnp.sum(p, axis=-1, keepdims=True)
    pv = jax.lax.dot_general(p.astype(v.dtype), v, (((2,), (1,)), ((0,), (0,))), preferred_element_type=jnp.float32)
    return max_new, row_sum, jnp.tile(alpha, (1, 1, d // LANES)) * acc + pv


def make_prefill(sm_scale: float, block_q: int = BLOCK_Q) -> tilejax_amd.Kernel:
    """The attention of the sequences with several new tokens (RPA's prefill and mixed cases), a tile per
    block of a sequence's queries: tile k < n_tiles[0] is queries tile_rows[k] .. tile_rows[k + 1] of a
    sequence whose pages start at page_indices[tile_page[k]], its first query at position tile_pos[k],
    attending positions before tile_stop[k]. The output is q updated in place."""

    @tilejax_amd.kernel
    def rpa_prefill(q, kv_cache, page_indices, tile_page, tile_rows, tile_pos, tile_stop, n_tiles,
                    tiles=PrefillTiles()):
        _, H, D = q.shape
        ps, Hkv = kv_cache.shape[1], kv_cache.shape[2]
        G, NP, BQ = H // Hkv, tiles.pages, block_q
        dtype = q.dtype
        out = q
        for k in range(n_tiles[0]):  # the tiles, counted as the kernel runs
            qh = head_rows(q[tilejax_amd.rows(tile_rows[k], tile_rows[k + 1], BQ), :, :], Hkv)
            row_max = jnp.full((Hkv, BQ * G, LANES), MASK_VALUE, jnp.float32)
            row_sum = jnp.zeros((Hkv, BQ * G, LANES), jnp.float32)
            acc = jnp.zeros((Hkv, BQ * G, D), jnp.float32)
            for j in range(0, tile_stop[k], NP * ps):  # NP pages a step, up to the tile's last query
                words = tilejax_amd.pairs(
                    kv_cache[page_indices[tile_page[k] + j // ps : tile_page[k] + j // ps + NP], :, :, :, :]
                )  # the step's pages as words (NP, ps, Hkv, D)
                kv = [keys_values(words[:, :, g, :]) for g in range(Hkv)]
                k_heads = jnp.stack([k_ for k_, _ in kv])  # (Hkv, NP * ps, D)
                v_heads = jnp.stack([v_ for _, v_ in kv])
                s = jax.lax.dot_general(qh, k_heads, (((2,), (2,)), ((0,), (0,))), preferred_element_type=jnp.float32)
                ok = visible(G, BQ * G, NP * ps, tile_pos[k], j, tile_stop[k])
                row_max, row_sum, acc = online_softmax_heads(
                    jnp.where(ok, s * sm_scale, MASK_VALUE), v_heads, row_max, row_sum, acc
                )
            o = acc * jnp.tile(1.0 / jnp.maximum(row_sum, 1e-30), (1, 1, D // LANES))
            out = out.at[tilejax_amd.rows(tile_rows[k], tile_rows[k + 1], BQ), :, :].set(token_heads(o, H).astype(dtype))
        return out

    return rpa_prefill
