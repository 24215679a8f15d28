"""Parity of GQA decode over a contiguous cache (the reference's `gqa_decode`, examples/decode.py:175-196)
with the CPU oracle on the same seeded inputs, with the paged kernel on the same cache cut into pages
(bit for bit, as the reference's tests/test_decode.py:202-212 asserts), of its device step tables with the
reference's table semantics, and at a cache the size of BASELINE.json config 5 with a float32 GPU reference on sampled
sequences.

Tolerance (tests/tolerance.py): bf16 outputs within 2 bf16 ulp of the expected value plus the softmax floor
(2^-8 + 2 n 2^-24 + 2 e_s) * softmax(s) @ |v| (the paged tests' bound: the kernel merges per-workgroup
partial softmaxes where the spec runs one pass per block, so p is rounded against other running maxima).
"""

import numpy as np
import pytest
import torch

from examples.decode import DecodeTiles, gqa_decode, paged_gqa_decode
from oracle import kernels
from oracle import schedule as oracle_schedule
from tests.tolerance import check_bf16, score_err, softmax_floor

pytestmark = pytest.mark.gpu


def _inputs(B, S, lengths, H=32, Hkv=8, D=128, seed=0):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(B, 1, H, D, generator=g) * D**-0.5).to(torch.bfloat16)
    k = torch.randn(B, S, Hkv * D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, S, Hkv * D, generator=g).to(torch.bfloat16)
    return q, k, v, torch.tensor(lengths, dtype=torch.int32)


def _close(what, got, want, q, k, v, lengths):
    """2 bf16 ulp plus the softmax floor of these inputs."""
    weighted = torch.as_tensor(kernels.gqa_contiguous_float64(q, k, v.float().abs(), lengths))
    floor = softmax_floor(weighted, int(lengths.max()), score_err(q, k))
    check_bf16(what, got.cpu(), torch.as_tensor(want).cpu(), floor)


@pytest.mark.parametrize("block_kv", [128, 256, 512])
def test_contiguous_decode_matches_oracle(block_kv):
    # an empty sequence, one with just the new token, a partial last block and a full cache
    ins = _inputs(4, 512, (0, 1, 300, 512))
    print(f"contiguous decode block_kv={block_kv}", flush=True)
    got = gqa_decode(*(t.cuda() for t in ins), DecodeTiles(block_kv))
    torch.cuda.synchronize()
    _close(f"contiguous decode block_kv={block_kv}", got, kernels.gqa_decode(*ins, block_kv), *ins)
    _close(f"contiguous decode block_kv={block_kv} vs float64", got, kernels.gqa_contiguous_float64(*ins), *ins)
    assert not got[0].float().any()  # the empty sequence


def test_paged_equals_contiguous_bit_for_bit():
    """The same cache as 128-position pages in a shuffled page table: the paged kernel reads exactly the
    blocks the contiguous one reads, in the same order, so the outputs agree exactly."""
    q, k, v, lengths = _inputs(4, 512, (0, 1, 300, 512), seed=1)
    kp, table = kernels.contiguous_as_pages(k, 128)
    vp, _ = kernels.contiguous_as_pages(v, 128)
    perm = torch.randperm(kp.shape[0], generator=torch.Generator().manual_seed(2))
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(perm.numel())
    table = inv[table.long()].to(torch.int32)
    print("paged (128-position pages) vs contiguous (block_kv 128)", flush=True)
    paged = paged_gqa_decode(q.cuda(), kp[perm].cuda(), vp[perm].cuda(), table.cuda(), lengths.cuda())
    contiguous = gqa_decode(q.cuda(), k.cuda(), v.cuda(), lengths.cuda(), DecodeTiles(128))
    assert torch.equal(paged, contiguous)


def test_contiguous_decode_step_tables():
    """The reference's count for lengths (0, 1, 300, 512) at block_kv 128 (tests/test_decode.py:195-199):
    the empty sequence takes one empty step, then 1 + 3 + 4 blocks."""
    lengths = (0, 1, 300, 512)
    ins = _inputs(4, 512, lengths)
    lowered = gqa_decode.lower(*ins, DecodeTiles(128))
    got = lowered.program.step_tables(*(t.cuda() for t in ins))
    step_tile, step_code, count = oracle_schedule.runtime_tables(
        [{"b": b} for b in range(4)], [("j", 0, 128, 4, lambda v: v["j"] >= lengths[v["b"]])])
    assert int(got["count"][0]) == count == 1 + 1 + 3 + 4
    np.testing.assert_array_equal(got["step_tile"].cpu().numpy(), step_tile)
    np.testing.assert_array_equal(got["step_code"].cpu().numpy(), step_code)


def test_contiguous_decode_large_cache_sampled():
    """64 sequences over an 8192-position cache (1 GiB per K and V, BASELINE.json config 5's shape without the
    page table), lengths uniform in [128, 8192], block_kv 512; every sequence against float32 on the GPU."""
    B, H, Hkv, D, S = 64, 32, 8, 128, 8192
    g = torch.Generator().manual_seed(0)
    lengths = torch.randint(128, S + 1, (B,), generator=g, dtype=torch.int32)
    q = (torch.randn(B, 1, H, D, generator=g) * D**-0.5).to(torch.bfloat16).cuda()
    k = torch.randn(B, S, Hkv * D, generator=g).to(torch.bfloat16).cuda()
    v = torch.randn(B, S, Hkv * D, generator=g).to(torch.bfloat16).cuda()
    print("contiguous decode 64 x 8192, block_kv 512", flush=True)
    got = gqa_decode(q, k, v, lengths.cuda(), DecodeTiles(512))
    e_s = score_err(q, k)
    for b in range(B):
        n = int(lengths[b])
        kk = k[b, :n].reshape(n, Hkv, D).float().permute(1, 2, 0).contiguous()  # (g, d, n)
        vv = v[b, :n].reshape(n, Hkv, D).float().permute(1, 0, 2).contiguous()  # (g, n, d)
        qq = q[b, 0].float().reshape(Hkv, H // Hkv, D)
        p = torch.softmax(torch.bmm(qq, kk), -1)
        want = torch.bmm(p, vv).reshape(H, D)
        floor = softmax_floor(torch.bmm(p, vv.abs()).reshape(H, D), n, e_s)
        check_bf16(f"contiguous decode sequence {b} (length {n})", got[b, 0], want, floor)


def test_contiguous_cursor_equals_step_tables():
    from tilejax_amd.tune import Config

    ins = _inputs(4, 512, (0, 1, 300, 512), seed=3)
    dev = [t.cuda() for t in ins]
    plain = gqa_decode.lower(*ins, DecodeTiles(128))
    cursor = gqa_decode.lowered(gqa_decode.signature(*ins), Config(DecodeTiles(128), plain.config.pipeline, True))
    print("contiguous decode cursor vs tables", flush=True)
    assert torch.equal(plain.run(*dev), cursor.run(*dev))


@pytest.mark.parametrize("t, heads, kv_heads, block_kv", [(1, 8, 2, 128), (1, 4, 4, 256), (3, 8, 2, 128),
                                                          (1, 4, 1, 128), (1, 12, 3, 256)])
def test_few_query_rows(t, heads, kv_heads, block_kv):
    """The reference's own cases (tests/test_decode.py:176-191): fewer than 32 query rows (t * heads), the
    kernels' rows past them zero; an empty sequence, one with just the new tokens, a partial block, a full
    cache. One and three KV heads (widths 128 and 384) take the decode kernel in four waves, the others in
    eight."""
    g = torch.Generator().manual_seed(4)
    q = (torch.randn(4, t, heads, 128, generator=g) * 128**-0.5).to(torch.bfloat16)
    k = torch.randn(4, 512, kv_heads * 128, generator=g).to(torch.bfloat16)
    v = torch.randn(4, 512, kv_heads * 128, generator=g).to(torch.bfloat16)
    lengths = torch.tensor([0, t, 300, 512], dtype=torch.int32)
    print(f"contiguous decode t={t} heads={heads}/{kv_heads} block_kv={block_kv}", flush=True)
    assert gqa_decode.lower(q, k, v, lengths, DecodeTiles(block_kv)).program.notes["family"] == "decode"
    got = gqa_decode(q.cuda(), k.cuda(), v.cuda(), lengths.cuda(), DecodeTiles(block_kv))
    torch.cuda.synchronize()
    what = f"contiguous decode t={t} heads={heads}/{kv_heads} block_kv={block_kv}"
    _close(what, got, kernels.gqa_decode(q, k, v, lengths, block_kv), q, k, v, lengths)
    _close(what + " vs float64", got, kernels.gqa_contiguous_float64(q, k, v, lengths), q, k, v, lengths)
    assert not got[0].float().any()
