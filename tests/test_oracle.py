"""The CPU oracle (oracle/kernels.py) pinned against what the mathematics fixes: each function is compared
with a float64 closed form (x @ y, tril, causal softmax, GQA softmax over the valid cache), on the special
cases the reference's tests hold (an empty sequence gives zeros, paged equals contiguous, out-of-range
expert indices clamp, groups with expert -1 keep the zeros), and checked to fail on a planted mistake."""

import numpy as np
import pytest
import torch

from helpers import rand
from oracle import kernels

BF = torch.bfloat16


def _close(got, want, rtol=2e-2, atol_frac=2e-2):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    atol = atol_frac * np.abs(want).max()
    np.testing.assert_allclose(got, want, rtol=rtol, atol=atol)


def test_matmul_is_x_at_y():
    x, y = rand((256, 384), 0, BF), rand((384, 256), 1, BF)
    want = x.double() @ y.double()
    _close(kernels.matmul(x, y, 128, 128, 128).double(), want)
    # f32 accumulation: within a bf16 rounding of the float64 product (2^-8 relative, plus cancellation)
    got = kernels.matmul(x, y, 128, 128, 128).double()
    assert ((got - want).abs() <= 2**-8 * want.abs() + 1e-2).all()


def test_matmul_oracle_catches_a_dropped_step():
    x, y = rand((256, 384), 0, BF), rand((384, 256), 1, BF)
    wrong = kernels.matmul(x[:, :256], y[:256], 128, 128, 128)  # one reduction step short
    with pytest.raises(AssertionError):
        _close(wrong.double(), x.double() @ y.double())


def test_causal_matmul_is_tril():
    x, y = rand((512, 256), 0, BF), rand((256, 512), 1, BF)
    got = kernels.causal_matmul(x, y, 128, 128, 128)
    _close(got.double(), torch.tril(x.double() @ y.double()))
    assert not got.float().triu(1).any()


def _attn_inputs(b, h, s, d):
    q, k, v = (rand((b, h, s, d), seed, BF) for seed in range(3))
    return (q.float() * d**-0.5).to(BF), k, v


@pytest.mark.parametrize("bq,bk", [(128, 128), (256, 128), (128, 256)])
def test_causal_attention_is_softmax_attention(bq, bk):
    q, k, v = _attn_inputs(1, 2, 512, 128)
    got = kernels.causal_attention(q, k, v, bq, bk)
    _close(got.double(), kernels.attention_float64(q, k, v), atol_frac=2e-2)


def test_attention_float64_reduces_to_the_first_value_row_for_the_first_query():
    q, k, v = _attn_inputs(1, 1, 64, 128)
    out = kernels.attention_float64(q, k, v)
    np.testing.assert_allclose(out[0, 0, 0], v[0, 0, 0].double().numpy(), rtol=1e-12)


def _paged(B=4, H=8, Hkv=2, D=128, P=16, pages=8, seed=0, lengths=(0, 1, 37, 128)):
    q = (rand((B, 1, H, D), seed, torch.float32) * D**-0.5).to(BF)
    n_pages = B * pages
    k_pages = rand((n_pages, P, Hkv * D), seed + 1, BF)
    v_pages = rand((n_pages, P, Hkv * D), seed + 2, BF)
    g = torch.Generator().manual_seed(seed + 3)
    table = torch.randperm(n_pages, generator=g).reshape(B, pages).to(torch.int32)
    return q, k_pages, v_pages, table, torch.tensor(lengths, dtype=torch.int32)


def test_paged_decode_is_gqa_softmax():
    q, kp, vp, table, lengths = _paged()
    got = kernels.paged_gqa_decode(q, kp, vp, table, lengths)
    want = kernels.gqa_float64(q, kp, vp, table, lengths)
    _close(got.double(), want)
    assert not got[0].float().any()  # an empty sequence gives zeros


def test_paged_decode_with_new_tokens_is_gqa_softmax():
    # two new tokens per sequence: token t sees the positions up to lengths[b] - 2 + t
    B, T, H, Hkv, D, P, pages = 3, 2, 8, 2, 128, 16, 8
    q = (rand((B, T, H, D), 7, torch.float32) * D**-0.5).to(BF)
    kp = rand((B * pages, P, Hkv * D), 8, BF)
    vp = rand((B * pages, P, Hkv * D), 9, BF)
    table = torch.randperm(B * pages, generator=torch.Generator().manual_seed(1)).reshape(B, pages).to(torch.int32)
    lengths = torch.tensor([2, 64, 100], dtype=torch.int32)
    got = kernels.paged_gqa_decode(q, kp, vp, table, lengths)
    want = kernels.gqa_float64(q, kp, vp, table, lengths)
    _close(got.double(), want)
    # the first token of a sequence of two sees one position: its value row
    np.testing.assert_allclose(want[0, 0, 0], vp[int(table[0, 0]), 0, :D].double().numpy(), rtol=1e-12)


def test_paged_decode_is_independent_of_the_page_layout():
    q, kp, vp, table, lengths = _paged()
    got = kernels.paged_gqa_decode(q, kp, vp, table, lengths)
    perm = torch.randperm(kp.shape[0], generator=torch.Generator().manual_seed(9))
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(perm.numel())
    again = kernels.paged_gqa_decode(q, kp[perm], vp[perm], inv[table.long()].to(torch.int32), lengths)
    assert torch.equal(got, again)


def test_gqa_float64_single_position_returns_its_value():
    q, kp, vp, table, _ = _paged(lengths=(1, 1, 1, 1))
    out = kernels.gqa_float64(q, kp, vp, table, torch.ones(4, dtype=torch.int32))
    for b in range(4):
        page = int(table[b, 0])
        np.testing.assert_allclose(out[b, 0, 0], vp[page, 0, :128].double().numpy(), rtol=1e-12)


def _contiguous(B=4, H=8, Hkv=2, D=128, S=256, seed=0, lengths=(0, 1, 100, 256)):
    q = (rand((B, 1, H, D), seed, torch.float32) * D**-0.5).to(BF)
    k = rand((B, S, Hkv * D), seed + 1, BF)
    v = rand((B, S, Hkv * D), seed + 2, BF)
    return q, k, v, torch.tensor(lengths, dtype=torch.int32)


@pytest.mark.parametrize("block_kv", [64, 128, 512])
def test_contiguous_decode_is_gqa_softmax(block_kv):
    q, k, v, lengths = _contiguous()
    got = kernels.gqa_decode(q, k, v, lengths, block_kv)
    _close(got.double(), kernels.gqa_contiguous_float64(q, k, v, lengths))
    assert not got[0].float().any()  # an empty sequence gives zeros


def test_contiguous_float64_agrees_with_the_paged_one():
    # the two float64 references, each from its own layout, on one cache
    q, k, v, lengths = _contiguous()
    kp, table = kernels.contiguous_as_pages(k, 32)
    vp, _ = kernels.contiguous_as_pages(v, 32)
    perm = torch.randperm(kp.shape[0], generator=torch.Generator().manual_seed(5))
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(perm.numel())
    np.testing.assert_allclose(kernels.gqa_float64(q, kp[perm], vp[perm], inv[table.long()].to(torch.int32), lengths),
                               kernels.gqa_contiguous_float64(q, k, v, lengths), rtol=1e-12, atol=1e-12)


def test_contiguous_float64_catches_an_off_by_one_length():
    q, k, v, lengths = _contiguous(lengths=(3, 50, 100, 200))
    want = kernels.gqa_contiguous_float64(q, k, v, lengths)
    wrong = kernels.gqa_contiguous_float64(q, k, v, lengths + 1)
    assert np.abs(want - wrong).max() > 1e-3


@pytest.mark.parametrize("tiles", [(128, 128, 128), (256, 128, 512)])
def test_rmsnorm_matmul_is_normalized_projection(tiles):
    x = rand((256, 512), 0, BF)
    gamma = (1 + 0.1 * rand((1, 512), 1, torch.float32)).to(BF)
    w = (rand((512, 256), 2, torch.float32) / 16).to(BF)
    got = kernels.rmsnorm_matmul(x, gamma, w, *tiles)
    _close(got.double(), kernels.rmsnorm_matmul_float64(x, gamma, w))


def test_rmsnorm_float64_is_the_plain_normalization():
    # rows of one repeated value v normalize to sign(v) (times gamma): mean(x^2) = v^2
    x = torch.full((4, 64), 3.0, dtype=torch.float64)
    x[1] = -0.5
    gamma = torch.ones((1, 64), dtype=torch.float64)
    w = torch.eye(64, dtype=torch.float64)
    got = kernels.rmsnorm_matmul_float64(x, gamma, w, eps=0.0)
    np.testing.assert_allclose(got[0], np.ones(64), rtol=1e-12)
    np.testing.assert_allclose(got[1], -np.ones(64), rtol=1e-12)


def test_rmsnorm_matmul_check_catches_a_planted_eps():
    # small activations (mean square 1e-4): the oracle run with a wrong eps fails the float64 comparison
    x = (rand((128, 256), 3, torch.float32) * 0.01).to(BF)
    gamma = torch.ones((1, 256), dtype=BF)
    w = (rand((256, 128), 4, torch.float32) / 16).to(BF)
    want = kernels.rmsnorm_matmul_float64(x, gamma, w)
    _close(kernels.rmsnorm_matmul(x, gamma, w, 128, 128, 128).double(), want)
    with pytest.raises(AssertionError):
        _close(kernels.rmsnorm_matmul(x, gamma, w, 128, 128, 128, eps=1e-3).double(), want)


def test_grouped_matmul_routes_groups_to_their_experts():
    G, E, K, N = 64, 3, 128, 256
    xs = rand((4 * G, K), 0, BF)
    w = rand((E, K, N), 1, BF)
    ge = torch.tensor([0, 2, -1, 9], dtype=torch.int32)  # -1: zeros; 9: clamped to expert E - 1
    got = kernels.grouped_matmul(xs, w, ge, tn=128, tk=64).double()
    for g, e in enumerate([0, 2, None, 2]):
        rows = slice(g * G, (g + 1) * G)
        if e is None:
            assert not got[rows].any()
        else:
            _close(got[rows], xs[rows].double() @ w[e].double())


def _expert_inputs(G=64, E=3, D=128, F=256):
    xs = rand((4 * G, D), 0, BF)
    return xs, rand((E, D, F), 1, BF) / 8, rand((E, D, F), 2, BF) / 8, rand((E, F, D), 3, BF) / 8


def test_expert_ffn_is_swiglu_per_tile():
    xs, wg, wu, wd = _expert_inputs()
    te = torch.tensor([0, 2, -1, 9], dtype=torch.int32)  # -1: zeros; 9: clamped to expert E - 1
    got = kernels.expert_ffn(xs, wg, wu, wd, te, bf=64).double()
    want = kernels.expert_ffn_float64(xs, wg, wu, wd, te)
    _close(got, want)
    assert not got[128:192].any()
    with pytest.raises(AssertionError):  # gate and up swapped: silu(u) * g
        _close(kernels.expert_ffn(xs, wu, wg, wd, te, bf=64).double(), want)


def test_expert_ffn_float64_is_silu_of_the_gate_when_up_is_one():
    """x = 1/D everywhere and w_up = 1 give up = 1; w_down = I leaves silu(gate) = g / (1 + e^-g)."""
    G, D = 64, 128
    xs = torch.full((G, D), 1.0 / D)
    wg = rand((1, D, D), 4) * 4
    wu, wd = torch.ones((1, D, D)), torch.eye(D)[None]
    g = (xs.double() @ wg[0].double()).numpy()
    want = g / (1 + np.exp(-g))
    np.testing.assert_allclose(kernels.expert_ffn_float64(xs, wg, wu, wd, torch.tensor([0], dtype=torch.int32)),
                               want, rtol=1e-12, atol=1e-12)
