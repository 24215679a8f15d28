"""Parity of the generated gfx950 flash-attention kernels with the CPU oracle (oracle/kernels.py, the spec's
loop nest with f32 accumulation) on the same seeded inputs, and at BASELINE.json config 3's shapes with a float32 torch
reference on the GPU (the attention kernel is floating point).

Tolerance: bf16 outputs within rtol 1e-2 of |want| plus 1e-2 of the output's largest magnitude (about
2 bf16 ulp): the kernel and the oracle differ in f32 summation order and in where the online softmax
rescales (the kernel steps through 64-key blocks, the spec through its own blocks). f32 q, k, v run on
the vector ALUs in f32: within 1e-4 of float64 (the reference's own tolerance, tests/test_examples.py:97-101).
"""

import pytest
import torch

from examples.causal_attention import AttentionBlocks, causal_attention
from oracle import kernels

pytestmark = pytest.mark.gpu


def _inputs(b, h, s, d, seed=0):
    gens = [torch.Generator().manual_seed(seed + i) for i in range(3)]
    q, k, v = (torch.randn(b, h, s, d, generator=g).to(torch.bfloat16) for g in gens)
    return (q.float() * d**-0.5).to(torch.bfloat16), k, v


def _close(got, want):
    got, want = got.float().cpu(), want.float().cpu()
    scale = want.abs().max().item()
    bad = (got - want).abs() > 1e-2 * want.abs() + 1e-2 * scale
    assert not bad.any(), f"{int(bad.sum())} of {want.numel()} differ; max |diff| {(got - want).abs().max().item()}"


@pytest.mark.parametrize("shape,blocks", [
    ((1, 2, 512, 128), AttentionBlocks(128, 128)),
    ((2, 2, 512, 128), AttentionBlocks(256, 128)),
    ((2, 2, 512, 128), AttentionBlocks(128, 128)),  # the reference's block shapes, tests/test_examples.py:80-88
    ((2, 2, 512, 128), AttentionBlocks(128, 256)),
    ((1, 2, 1024, 128), AttentionBlocks(256, 256)),
    ((1, 1, 1024, 128), AttentionBlocks(512, 512)),
])
def test_causal_attention_matches_oracle(shape, blocks):
    q, k, v = _inputs(*shape)
    print(f"attention {shape} {blocks}", flush=True)
    got = causal_attention(q.cuda(), k.cuda(), v.cuda(), blocks)
    torch.cuda.synchronize()
    _close(got, kernels.causal_attention(q, k, v, blocks.block_q, blocks.block_kv))


def _reference_f32(q, k, v):
    B, H, S, D = q.shape
    qf, vf = q.float().reshape(B * H, S, D), v.float().reshape(B * H, S, D)
    kt = k.float().reshape(B * H, S, D).transpose(-1, -2).contiguous()
    mask = torch.ones(S, S, dtype=torch.bool, device=q.device).tril()
    out = torch.empty(B * H, S, D, device=q.device)
    for i in range(0, B * H, 8):
        s = (qf[i:i + 8] @ kt[i:i + 8]).masked_fill(~mask, float("-inf"))
        out[i:i + 8] = torch.softmax(s, -1) @ vf[i:i + 8]
    return out.reshape(B, H, S, D)


@pytest.mark.parametrize("shape", [(4, 16, 2048, 128), (1, 16, 4096, 128)])
def test_causal_attention_baseline_shapes(shape):
    q, k, v = (t.cuda() for t in _inputs(*shape, seed=7))
    print(f"attention {shape} 512x512", flush=True)
    got = causal_attention(q, k, v, AttentionBlocks(512, 512))
    want = _reference_f32(q, k, v)
    torch.cuda.synchronize()
    _close(got, want)


def test_verify_against_the_spec_reference():
    q, k, v = _inputs(1, 2, 512, 128, seed=3)
    err = causal_attention.verify(q.cuda(), k.cuda(), v.cuda(), AttentionBlocks(128, 128))
    assert err < 0.1


@pytest.mark.parametrize("shape,blocks", [
    ((1, 1, 256, 128), AttentionBlocks(128, 128)),  # tests/test_examples.py:97-101 of the reference
    ((2, 2, 512, 128), AttentionBlocks(256, 128)),
    ((1, 2, 512, 128), AttentionBlocks(128, 256)),
])
def test_causal_attention_f32(shape, blocks):
    gens = [torch.Generator().manual_seed(20 + i) for i in range(3)]
    q, k, v = (torch.randn(*shape, generator=g) for g in gens)
    q = q * shape[-1] ** -0.5
    print(f"attention f32 {shape} {blocks}", flush=True)
    got = causal_attention(q.cuda(), k.cuda(), v.cuda(), blocks)
    torch.cuda.synchronize()
    assert got.dtype == torch.float32
    want = torch.as_tensor(kernels.attention_float64(q, k, v))
    diff = (got.double().cpu() - want).abs()
    assert diff.max().item() < 1e-4, diff.max().item()


def test_split_tiles_call_after_call():
    """(1, 2, 1024, 128) at 256 x 256 blocks cuts its longest tiles into chunks, which the merge kernel
    combines; three calls in a row give the same bits."""
    q, k, v = (t.cuda() for t in _inputs(1, 2, 1024, 128, seed=9))
    lowered = causal_attention.lower(q, k, v, AttentionBlocks(256, 256))
    assert lowered.program.notes["split_items"] > 0
    print("attention (1, 2, 1024, 128) split, three calls", flush=True)
    outs = [lowered.run(q, k, v) for _ in range(3)]
    torch.cuda.synchronize()
    _close(outs[0], kernels.causal_attention(q.cpu(), k.cpu(), v.cpu(), 256, 256))
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
