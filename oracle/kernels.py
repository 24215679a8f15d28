"""TEST INFRASTRUCTURE ONLY. The spec kernels restated as loops over tiles on CPU torch tensors.

Each function follows one of the reference's examples loop for loop, with `@` accumulating bf16
products in f32 (src/autokernel/mxu.py:21-43), and rounds where the spec rounds (`.astype(dtype)`).
Sizes here must be ones a CPU finishes in seconds; the GPU tests compare against these on the same
seeded inputs.
"""

from __future__ import annotations

import math
from typing import Optional

import numpy as np
import torch

LANES = 128
MASK_VALUE = -1e30


def _f32(x: torch.Tensor) -> torch.Tensor:
    return x.detach().to("cpu", torch.float32)


def matmul(x: torch.Tensor, y: torch.Tensor, tm: int = 512, tn: int = 512, tk: int = 512) -> torch.Tensor:
    """examples/matmul.py:22-35: out[i, j] tile = bf16(sum_k x[i, k] @ y[k, j]), f32 accumulation."""
    M, K = x.shape
    N = y.shape[1]
    tm, tn, tk = min(tm, M), min(tn, N), min(tk, K)
    xf, yf = _f32(x), _f32(y)
    out = torch.zeros((M, N), dtype=x.dtype)
    for i in range(0, M, tm):
        for j in range(0, N, tn):
            acc = torch.zeros((tm, tn), dtype=torch.float32)
            for k in range(0, K, tk):
                acc += xf[i:i + tm, k:k + tk] @ yf[k:k + tk, j:j + tn]
            out[i:i + tm, j:j + tn] = acc.to(x.dtype)
    return out


def causal_matmul(x: torch.Tensor, y: torch.Tensor, tm: int = 512, tn: int = 512, tk: int = 512) -> torch.Tensor:
    """examples/causal_matmul.py:23-40: tiles wholly above the diagonal (j > i + tm - 1) keep the zeros of
    the allocation; computed tiles are zeroed above the diagonal by `where(cols <= rows, acc, 0)`."""
    M, K = x.shape
    N = y.shape[1]
    tm, tn, tk = min(tm, M), min(tn, N), min(tk, K)
    xf, yf = _f32(x), _f32(y)
    out = torch.zeros((M, N), dtype=x.dtype)
    for i in range(0, M, tm):
        for j in range(0, N, tn):
            if j > i + tm - 1:
                continue
            acc = torch.zeros((tm, tn), dtype=torch.float32)
            for k in range(0, K, tk):
                acc += xf[i:i + tm, k:k + tk] @ yf[k:k + tk, j:j + tn]
            rows = i + torch.arange(tm).reshape(-1, 1)
            cols = j + torch.arange(tn).reshape(1, -1)
            out[i:i + tm, j:j + tn] = torch.where(cols <= rows, acc, torch.zeros(())).to(x.dtype)
    return out


def causal_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, bq: int = 512, bk: int = 512) -> torch.Tensor:
    """examples/causal_attention.py:37-63: online softmax over key blocks not wholly in the future; scores
    s = q @ k.T in f32, masked with -1e30 above the diagonal; p cast to bf16 before `p @ v` (f32 acc). The
    (b, h) loops of the spec run as batch dims of each tile's products: every (b, h) is independent."""
    B, H, S, D = q.shape
    bq, bk = min(bq, S), min(bk, S)
    dtype = q.dtype
    qf, kf, vf = (_f32(t).reshape(B * H, S, D) for t in (q, k, v))
    out = torch.zeros((B * H, S, D), dtype=dtype)
    for i in range(0, S, bq):
        row_max = torch.full((B * H, bq, 1), MASK_VALUE)
        row_sum = torch.zeros((B * H, bq, 1))
        acc = torch.zeros((B * H, bq, D))
        rows = i + torch.arange(bq).reshape(-1, 1)
        for j in range(0, S, bk):
            if j > i + bq - 1:
                continue
            s = qf[:, i:i + bq] @ kf[:, j:j + bk].transpose(1, 2).contiguous()
            cols = j + torch.arange(bk).reshape(1, -1)
            s = torch.where(cols <= rows, s, torch.tensor(MASK_VALUE))
            max_new = torch.maximum(row_max, s.max(dim=2, keepdim=True).values)
            p = torch.exp(s - max_new)
            alpha = torch.exp(row_max - max_new)
            row_sum = alpha * row_sum + p.sum(dim=2, keepdim=True)
            acc = alpha * acc + p.to(dtype).float() @ vf[:, j:j + bk]
            row_max = max_new
        out[:, i:i + bq] = (acc / row_sum).to(dtype)
    return out.reshape(B, H, S, D)


def attention_float64(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> np.ndarray:
    """Causal softmax(q k^T) v in float64: what the reference's own tests compare attention against
    (tests/test_examples.py:71-77 of the reference)."""
    qd, kd, vd = (t.detach().cpu().double() for t in (q, k, v))
    S = q.shape[2]
    s = qd @ kd.transpose(-1, -2)
    mask = torch.ones(S, S, dtype=torch.bool).tril()
    s = s.masked_fill(~mask, float("-inf"))
    return (torch.softmax(s, dim=-1) @ vd).numpy()


def grouped_matmul(xs: torch.Tensor, w: torch.Tensor, group_expert: torch.Tensor, tn: int = 512,
                   tk: int = 512) -> torch.Tensor:
    """The grouped matmul of config 4 (examples/moe.py:167-187's runtime window `w[tile_expert[i // G]]`,
    in the single-matrix form of tests/test_index_arrays.py:109-125): each group of G rows through its
    expert's weights; groups with expert < 0 keep the zeros; the expert index is clamped into [0, E)."""
    M, K = xs.shape
    E, _, N = w.shape
    G = M // group_expert.shape[0]
    tn, tk = min(tn, N), min(tk, K)
    xf, wf = _f32(xs), _f32(w)
    ge = group_expert.cpu().numpy()
    out = torch.zeros((M, N), dtype=xs.dtype)
    for j in range(0, N, tn):
        for i in range(0, M, G):
            e = int(ge[i // G])
            if e < 0:
                continue
            e = min(max(e, 0), E - 1)
            acc = torch.zeros((G, tn))
            for k in range(0, K, tk):
                acc += xf[i:i + G, k:k + tk] @ wf[e, k:k + tk, j:j + tn]
            out[i:i + G, j:j + tn] = acc.to(xs.dtype)
    return out


def expert_ffn(xs: torch.Tensor, w_gate: torch.Tensor, w_up: torch.Tensor, w_down: torch.Tensor,
               tile_expert: torch.Tensor, bf: int = 256) -> torch.Tensor:
    """examples/moe.py:167-187 of the reference: per tile of G rows and per block of bf hidden units, the gate
    and up products in f32, silu(g) * u rounded to the input dtype, its product with the down block added in
    f32; tiles whose expert is negative keep the zeros; the expert index is clamped into [0, E)."""
    M, D = xs.shape
    E, _, F = w_gate.shape
    G = M // tile_expert.shape[0]
    bf = min(bf, F)
    xf, wg, wu, wd = _f32(xs), _f32(w_gate), _f32(w_up), _f32(w_down)
    te = tile_expert.cpu().numpy()
    out = torch.zeros((M, D), dtype=xs.dtype)
    for i in range(0, M, G):
        e = int(te[i // G])
        if e < 0:
            continue
        e = min(e, E - 1)
        acc = torch.zeros((G, D))
        for f in range(0, F, bf):
            g = xf[i:i + G] @ wg[e, :, f:f + bf]
            u = xf[i:i + G] @ wu[e, :, f:f + bf]
            hidden = (g * torch.sigmoid(g) * u).to(xs.dtype).float()
            acc += hidden @ wd[e, f:f + bf, :]
        out[i:i + G] = acc.to(xs.dtype)
    return out


def expert_ffn_float64(xs: torch.Tensor, w_gate: torch.Tensor, w_up: torch.Tensor, w_down: torch.Tensor,
                       tile_expert: torch.Tensor) -> np.ndarray:
    """The SwiGLU layer in float64 with nothing rounded: silu(x @ w_gate[e]) * (x @ w_up[e]) @ w_down[e] per
    tile of G rows, zeros for a negative expert."""
    M, D = xs.shape
    E = w_gate.shape[0]
    G = M // tile_expert.shape[0]
    x, wg, wu, wd = (t.detach().cpu().double() for t in (xs, w_gate, w_up, w_down))
    out = torch.zeros((M, D), dtype=torch.float64)
    for t, e in enumerate(tile_expert.cpu().tolist()):
        if e < 0:
            continue
        e = min(e, E - 1)
        rows = x[t * G:(t + 1) * G]
        g = rows @ wg[e]
        out[t * G:(t + 1) * G] = (g * torch.sigmoid(g) * (rows @ wu[e])) @ wd[e]
    return out.numpy()


def paged_gqa_decode(q: torch.Tensor, k_pages: torch.Tensor, v_pages: torch.Tensor, block_tables: torch.Tensor,
                     lengths: torch.Tensor) -> torch.Tensor:
    """examples/decode.py:199-223: query head h of new token t attends its kv head h // (H / Hkv) over the
    positions `visible` gives (decode.py:92-99: < lengths[b] for one new token; with T of them, token t sits
    at lengths[b] - T + t and sees the positions up to it), pages read through block_tables[b, p]
    (clamped) while p * P < lengths[b]; scores in f32, p rounded to bf16 before `p @ v`, one online-softmax
    step per page; empty sequences give zeros. Each query row's softmax is its own: the heads of one kv
    group, and the groups, run as batch rows of each page's products."""
    B, T, H, Dh = q.shape
    P, W = k_pages.shape[1], k_pages.shape[2]
    Hkv = W // Dh
    group = H // Hkv
    n_pages = k_pages.shape[0]
    qf, kf, vf = _f32(q), _f32(k_pages), _f32(v_pages)
    tables = block_tables.cpu().numpy()
    lens = lengths.cpu().numpy()
    out = torch.zeros((B, T, H, Dh), dtype=q.dtype)
    for b in range(B):
        L = int(lens[b])
        pages = [min(max(int(tables[b, p]), 0), n_pages - 1) for p in range(tables.shape[1]) if p * P < L]
        if not pages:
            continue
        for t in range(T):
            qq = qf[b, t].reshape(Hkv, group, Dh)
            row_max = torch.full((Hkv, group, 1), MASK_VALUE)
            row_sum = torch.zeros((Hkv, group, 1))
            acc = torch.zeros((Hkv, group, Dh))
            for n, page in enumerate(pages):
                kk = kf[page].reshape(P, Hkv, Dh).permute(1, 2, 0).contiguous()  # (Hkv, Dh, P)
                vv = vf[page].reshape(P, Hkv, Dh).permute(1, 0, 2).contiguous()  # (Hkv, P, Dh)
                s = qq @ kk
                pos = n * P + torch.arange(P)
                ok = pos < L if T == 1 else pos <= L - T + t
                s = torch.where(ok, s, torch.tensor(MASK_VALUE))
                m_new = torch.maximum(row_max, s.max(dim=2, keepdim=True).values)
                p = torch.exp(s - m_new)
                alpha = torch.exp(row_max - m_new)
                row_sum = alpha * row_sum + p.sum(dim=2, keepdim=True)
                acc = alpha * acc + p.to(q.dtype).float() @ vv
                row_max = m_new
            out[b, t] = (acc / torch.clamp(row_sum, min=1e-30)).reshape(H, Dh).to(q.dtype)
    return out


def gqa_float64(q: torch.Tensor, k_pages: torch.Tensor, v_pages: torch.Tensor, block_tables: torch.Tensor,
                lengths: torch.Tensor) -> np.ndarray:
    """GQA decode attention in float64 over the pages (tests/test_decode.py:62-76 of the reference): token t
    of sequence b sits at position lengths[b] - T + t and sees the positions up to it."""
    B, T, H, Dh = q.shape
    P, W = k_pages.shape[1], k_pages.shape[2]
    Hkv = W // Dh
    out = np.zeros((B, T, H, Dh))
    tables = block_tables.cpu().numpy()
    lens = lengths.cpu().numpy()
    kd, vd, qd = k_pages.double().cpu(), v_pages.double().cpu(), q.double().cpu()
    for b in range(B):
        L = int(lens[b])
        if L == 0:
            continue
        npages = -(-L // P)
        kk = torch.cat([kd[int(tables[b, p])] for p in range(npages)])[:L].reshape(L, Hkv, Dh)
        vv = torch.cat([vd[int(tables[b, p])] for p in range(npages)])[:L].reshape(L, Hkv, Dh)
        for t in range(T):
            seen = L - T + t + 1
            for h in range(H):
                g = h // (H // Hkv)
                s = kk[:seen, g] @ qd[b, t, h]
                out[b, t, h] = (torch.softmax(s, 0) @ vv[:seen, g]).numpy()
    return out


def contiguous_as_pages(cache: torch.Tensor, block: int):
    """A contiguous cache (B, S, W) as pages of `block` positions (B * S / block, block, W) and the page
    table (B, S / block) that lists sequence b's blocks in order: the paged spec over these pages reads
    exactly what the contiguous spec reads, block for block."""
    B, S, W = cache.shape
    n = S // block
    table = torch.arange(B * n, dtype=torch.int32).reshape(B, n)
    return cache.reshape(B * n, block, W), table


def gqa_decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, lengths: torch.Tensor,
               block_kv: int = 512) -> torch.Tensor:
    """examples/decode.py:175-196 of the reference: the contiguous cache's blocks
    of bk = min(block_kv, S) positions, skipped from lengths[b] on, are the paged spec's pages in order, so
    this is `paged_gqa_decode` over `contiguous_as_pages` (same blocks, same online-softmax steps)."""
    bk = min(block_kv, k_cache.shape[1])
    kp, table = contiguous_as_pages(k_cache, bk)
    vp, _ = contiguous_as_pages(v_cache, bk)
    return paged_gqa_decode(q, kp, vp, table, lengths)


def gqa_contiguous_float64(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                           lengths: torch.Tensor) -> np.ndarray:
    """GQA decode attention in float64 over a contiguous cache: softmax(q k[:seen].T) v[:seen] per head, token t
    seeing lengths[b] - T + t + 1 positions (the reference's tests/test_decode.py:62-76 `_gqa`); empty
    sequences give 0."""
    B, T, H, Dh = q.shape
    Hkv = k_cache.shape[2] // Dh
    out = np.zeros((B, T, H, Dh))
    kd, vd, qd = k_cache.double().cpu(), v_cache.double().cpu(), q.double().cpu()
    for b, n in enumerate(lengths.cpu().tolist()):
        if n == 0:
            continue
        kk, vv = kd[b, :n].reshape(n, Hkv, Dh), vd[b, :n].reshape(n, Hkv, Dh)
        for t in range(T):
            seen = n - T + t + 1
            for h in range(H):
                g = h // (H // Hkv)
                out[b, t, h] = (torch.softmax(kk[:seen, g] @ qd[b, t, h], 0) @ vv[:seen, g]).numpy()
    return out


def rmsnorm_matmul(x: torch.Tensor, gamma: torch.Tensor, w: torch.Tensor, tm: int = 512, tn: int = 512,
                   tk: int = 512, eps: float = 1e-6) -> torch.Tensor:
    """examples/rmsnorm_matmul.py:33-46 of the reference: per output tile, over tk-deep blocks of the model
    dim, acc += bf16(x * gamma) @ w (f32 accumulation) and each row's sum of squares of x (f32); then
    out = bf16(acc * rsqrt(sum_sq / D + eps))."""
    M, D = x.shape
    N = w.shape[1]
    tm, tn, tk = min(tm, M), min(tn, N), min(tk, D)
    xf, gf, wf = _f32(x), _f32(gamma), _f32(w)
    out = torch.zeros((M, N), dtype=x.dtype)
    for i in range(0, M, tm):
        for j in range(0, N, tn):
            acc = torch.zeros((tm, tn), dtype=torch.float32)
            sum_sq = torch.zeros((tm, 1), dtype=torch.float32)
            for k in range(0, D, tk):
                xk = xf[i:i + tm, k:k + tk]
                sum_sq += (xk * xk).sum(dim=1, keepdim=True)
                acc += (xk * gf[0:1, k:k + tk]).to(x.dtype).float() @ wf[k:k + tk, j:j + tn]
            out[i:i + tm, j:j + tn] = (acc * torch.rsqrt(sum_sq / D + eps)).to(x.dtype)
    return out


def rmsnorm_matmul_float64(x: torch.Tensor, gamma: torch.Tensor, w: torch.Tensor, eps: float = 1e-6) -> np.ndarray:
    """rmsnorm(x) @ w in float64: x / sqrt(mean(x^2, axis=-1) + eps) * gamma, then @ w."""
    xd, gd, wd = x.double().cpu(), gamma.double().cpu(), w.double().cpu()
    normed = xd / torch.sqrt((xd * xd).mean(dim=1, keepdim=True) + eps) * gd
    return (normed @ wd).numpy()


def _gelu_tanh(x: torch.Tensor) -> torch.Tensor:
    """The tanh form of GELU, as jax.nn.gelu computes it by default."""
    return 0.5 * x * (1.0 + torch.tanh(0.7978845608028654 * (x + 0.044715 * x * x * x)))


def attention_block(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, gamma: torch.Tensor, w_up: torch.Tensor,
                    w_down: torch.Tensor, bq: int = 256, bk: int = 256, bf: int = 1024,
                    eps: float = 1e-6) -> torch.Tensor:
    """examples/attention_block.py:47-80 of the reference: per (batch, query block) tile, the causal online
    softmax over key blocks for every head (p rounded to the inputs' dtype before `p @ v`), the heads side
    by side, RMSNorm rounded to the inputs' dtype, then over blocks of hidden units y += bf16(gelu(h @
    w_up[:, f]))) @ w_down[f]; products accumulate in f32; the tile stored in the inputs' dtype."""
    B, H, S, Dh = q.shape
    F = w_up.shape[1]
    bq, bk, bf = min(bq, S), min(bk, S), min(bf, F)
    dtype = q.dtype
    qf, kf, vf = _f32(q), _f32(k), _f32(v)
    gf, uf, df = _f32(gamma), _f32(w_up), _f32(w_down)
    out = torch.zeros((B, S, H * Dh), dtype=dtype)
    for b in range(B):
        for i in range(0, S, bq):
            row_max = torch.full((H, bq, 1), MASK_VALUE)
            row_sum = torch.zeros((H, bq, 1))
            acc = torch.zeros((H, bq, Dh))
            rows = i + torch.arange(bq).reshape(-1, 1)
            for j in range(0, S, bk):
                if j > i + bq - 1:
                    continue
                cols = j + torch.arange(bk).reshape(1, -1)
                s = torch.stack([torch.where(cols <= rows, qf[b, h, i:i + bq] @ kf[b, h, j:j + bk].T,
                                             torch.tensor(MASK_VALUE)) for h in range(H)])
                max_new = torch.maximum(row_max, s.max(dim=2, keepdim=True).values)
                p = torch.exp(s - max_new)
                alpha = torch.exp(row_max - max_new)
                row_sum = alpha * row_sum + p.sum(dim=2, keepdim=True)
                pv = torch.stack([p[h].to(dtype).float() @ vf[b, h, j:j + bk] for h in range(H)])
                acc = alpha * acc + pv
                row_max = max_new
            heads = acc / row_sum
            a = torch.cat([heads[h] for h in range(H)], dim=1)
            normed = (a * torch.rsqrt((a * a).mean(dim=1, keepdim=True) + eps) * gf[0:1]).to(dtype).float()
            y = torch.zeros((bq, H * Dh))
            for f in range(0, F, bf):
                hidden = _gelu_tanh(normed @ uf[:, f:f + bf])
                y += hidden.to(dtype).float() @ df[f:f + bf]
            out[b, i:i + bq] = y.to(dtype)
    return out


def attention_block_float64(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, gamma: torch.Tensor,
                            w_up: torch.Tensor, w_down: torch.Tensor, eps: float = 1e-6) -> np.ndarray:
    """The block in float64 with nothing rounded: causal attention per head, the heads side by side,
    RMSNorm, tanh-GELU feed-forward (the reference's tests/test_examples.py:168-177 check)."""
    a = torch.as_tensor(attention_float64(q, k, v))  # (B, H, S, Dh)
    B, H, S, Dh = a.shape
    a = a.permute(0, 2, 1, 3).reshape(B, S, H * Dh)
    normed = a / torch.sqrt((a * a).mean(dim=-1, keepdim=True) + eps) * gamma.double().cpu()
    up = normed @ w_up.double().cpu()
    return (_gelu_tanh(up) @ w_down.double().cpu()).numpy()
