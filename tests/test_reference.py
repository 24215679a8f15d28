"""`kernel.reference` (the nest interpreter, tilejax_amd/reference.py) on the CPU against the oracle's
restatement of each spec: the same loop nests on the same inputs, so within the parity bar of
tests/tolerance.py, and `@` there is the matrix units' (f32 accumulation) while `kernel.fn` is plain JAX."""

import torch

from examples.causal_attention import AttentionBlocks, causal_attention
from examples.causal_matmul import causal_matmul
from examples.decode import DecodeTiles, gqa_decode, paged_gqa_decode
from examples.matmul import MatmulTiles, matmul
from examples.moe import GroupTiles, grouped_matmul
from examples.rmsnorm_matmul import NormMatmulTiles, rmsnorm_matmul
from oracle import kernels
from tests.tolerance import check_bf16, matmul_floor, score_err, softmax_floor


def _bf16(*shape, seed=0, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16)


def test_matmul_and_causal():
    x, y = _bf16(256, 384, seed=1), _bf16(384, 256, seed=2)
    t = MatmulTiles(128, 128, 128)
    check_bf16("reference matmul", matmul.reference(x, y, t), kernels.matmul(x, y, 128, 128, 128), matmul_floor(x, y))
    got = causal_matmul.reference(x[:, :256], y[:256], t)
    check_bf16("reference causal", got, kernels.causal_matmul(x[:, :256], y[:256], 128, 128, 128),
               matmul_floor(x[:, :256], y[:256]))
    assert not got.float().triu(1).any()


def test_fn_rounds_each_product_where_the_reference_accumulates_in_f32():
    """`kernel.fn` is the function as written: `bf16 @ bf16` rounds each tile product to bf16 before `acc +=`;
    `kernel.reference` keeps the f32 sum. At 6 reduction steps the two differ, the reference is the closer."""
    x, y = _bf16(128, 768, seed=3), _bf16(768, 128, seed=4)
    t = MatmulTiles(128, 128, 128)
    exact = (x.double() @ y.double())
    ref, fn = matmul.reference(x, y, t).double(), matmul.fn(x, y, t).double()
    assert not torch.equal(ref, fn)
    assert (ref - exact).abs().mean() < (fn - exact).abs().mean()


def test_attention():
    q, k, v = _bf16(1, 2, 256, 128, seed=5, scale=128 ** -0.5), _bf16(1, 2, 256, 128, seed=6), _bf16(1, 2, 256, 128, seed=7)
    got = causal_attention.reference(q, k, v, AttentionBlocks(128, 128))
    want = kernels.causal_attention(q, k, v, 128, 128)
    weighted = torch.as_tensor(kernels.attention_float64(q, k, v.float().abs()))
    check_bf16("reference attention", got, want, softmax_floor(weighted, 256, score_err(q, k)))


def test_grouped_matmul_with_unused_and_clamped_experts():
    xs, w = _bf16(1024, 256, seed=8), _bf16(4, 256, 512, seed=9, scale=0.02)
    experts = [2, -1, 9, 0]
    ge = torch.tensor(experts, dtype=torch.int32)
    got = grouped_matmul.reference(xs, w, ge, GroupTiles(256, 128))
    want = kernels.grouped_matmul(xs, w, ge, 256, 128)
    floor = torch.cat([matmul_floor(xs[g * 256:(g + 1) * 256], w[min(max(e, 0), 3)]) for g, e in enumerate(experts)])
    check_bf16("reference grouped", got, want, floor)
    assert not got[256:512].float().any()


def test_paged_and_contiguous_decode():
    g = torch.Generator().manual_seed(10)
    B, pages = 3, 8
    q = (torch.randn(B, 1, 32, 128, generator=g) * 128 ** -0.5).to(torch.bfloat16)
    kp = torch.randn(B * pages, 16, 1024, generator=g).to(torch.bfloat16)
    vp = torch.randn(B * pages, 16, 1024, generator=g).to(torch.bfloat16)
    table = torch.randperm(B * pages, generator=g).reshape(B, pages).to(torch.int32)
    lengths = torch.tensor([0, 17, 128], dtype=torch.int32)
    got = paged_gqa_decode.reference(q, kp, vp, table, lengths)
    want = kernels.paged_gqa_decode(q, kp, vp, table, lengths)
    weighted = torch.as_tensor(kernels.gqa_float64(q, kp, vp.float().abs(), table, lengths))
    check_bf16("reference paged decode", got, want, softmax_floor(weighted, 128, score_err(q, kp)))
    assert not got[0].float().any()
    kc, vc = _bf16(B, 128, 1024, seed=11), _bf16(B, 128, 1024, seed=12)
    got = gqa_decode.reference(q, kc, vc, lengths, DecodeTiles(64))
    weighted = torch.as_tensor(kernels.gqa_contiguous_float64(q, kc, vc.float().abs(), lengths))
    check_bf16("reference contiguous decode", got, kernels.gqa_decode(q, kc, vc, lengths, 64),
               softmax_floor(weighted, 128, score_err(q, kc)))


def test_rmsnorm_matmul():
    x, gamma, w = _bf16(256, 256, seed=13), (1 + 0.1 * _bf16(1, 256, seed=14).float()).bfloat16(), _bf16(256, 256, seed=15)
    got = rmsnorm_matmul.reference(x, gamma, w, NormMatmulTiles(128, 128, 128))
    want = kernels.rmsnorm_matmul(x, gamma, w, 128, 128, 128)
    mag = torch.as_tensor(kernels.rmsnorm_matmul_float64(x.float().abs(), gamma.float().abs(), w.float().abs()))
    check_bf16("reference rmsnorm_matmul", got, want, 2 * 256 * 2.0 ** -24 * mag + 2.0 ** -8 * mag)
