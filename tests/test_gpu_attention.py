"""Parity of the generated gfx950 flash-attention kernels with the CPU oracle (oracle/kernels.py, the spec's
loop nest with f32 accumulation) on the same seeded inputs, at every size including BASELINE.json config 3's
shapes, and there also with a float32 torch reference on the GPU.

Tolerance (tests/tolerance.py): bf16 outputs within 2 bf16 ulp of the expected value plus a floor of
(2^-8 + 2 S 2^-24 + 2 e_s) times softmax(s) @ |v|: the kernel and the oracle differ in f32 summation order
(scores by at most e_s, see `score_err`) and in which running maximum the spec's `p.astype(bf16)` rounds
against (the kernel rescales per 64-key block, the spec per block of its own), which moves each weight by
at most 2^-8 relative. f32 q, k, v run on the vector ALUs in f32: within 1e-4 of float64 (the reference's
own tolerance, tests/test_examples.py:97-101).
"""

import pytest
import torch

from examples.causal_attention import AttentionBlocks, causal_attention
from oracle import kernels
from tests.tolerance import SOFTMAX_BAR, check_bf16, score_err, softmax_floor

pytestmark = pytest.mark.gpu


def _inputs(b, h, s, d, seed=0):
    gens = [torch.Generator().manual_seed(seed + i) for i in range(3)]
    q, k, v = (torch.randn(b, h, s, d, generator=g).to(torch.bfloat16) for g in gens)
    return (q.float() * d**-0.5).to(torch.bfloat16), k, v


def _floor(q, k, v):
    """The softmax floor: softmax(q k^T) @ |v| in float64 on the CPU (the float64 oracle is linear in v)."""
    weighted = torch.as_tensor(kernels.attention_float64(q, k, v.float().abs()))
    return softmax_floor(weighted, q.shape[2], score_err(q, k))


def _close(what, got, want, floor):
    check_bf16(what, got.cpu(), torch.as_tensor(want).cpu(), floor)


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
    floor = _floor(q, k, v)
    _close(f"attention {shape} {blocks} vs oracle", got, kernels.causal_attention(q, k, v, blocks.block_q,
                                                                                 blocks.block_kv), floor)
    _close(f"attention {shape} {blocks} vs float64", got, kernels.attention_float64(q, k, v), floor)


def _reference_f32(q, k, v):
    """Causal softmax(q k^T) v in float32 on the GPU, 8 heads at a time (bmm on contiguous operands)."""
    B, H, S, D = q.shape
    qf, vf = q.float().reshape(B * H, S, D), v.float().reshape(B * H, S, D)
    kt = k.float().reshape(B * H, S, D).transpose(-1, -2).contiguous()
    mask = torch.ones(S, S, dtype=torch.bool, device=q.device).tril()
    out = torch.empty(B * H, S, D, device=q.device)
    for i in range(0, B * H, 8):
        s = (qf[i:i + 8] @ kt[i:i + 8]).masked_fill(~mask, float("-inf"))
        out[i:i + 8] = torch.softmax(s, -1) @ vf[i:i + 8]
    return out.reshape(B, H, S, D)


@pytest.mark.parametrize("shape,block", [((4, 16, 2048, 128), 512), ((1, 16, 4096, 128), 512),
                                         ((4, 16, 2048, 128), 256), ((4, 16, 2048, 128), 1024),
                                         ((1, 16, 4096, 128), 256), ((1, 16, 4096, 128), 1024)])
def test_causal_attention_baseline_shapes(shape, block):
    """both shapes at every block shape it lists (256^2, 512^2, 1024^2), every output
    against the CPU oracle at the same blocks (the spec's loop nest, which rounds p to bf16 as the spec does),
    to the softmax bar (tests/tolerance.py: SOFTMAX_BAR), and against a float32 softmax on the GPU with p
    unrounded, to the floor."""
    q, k, v = _inputs(*shape, seed=7)
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    blocks = AttentionBlocks(block, block)
    print(f"attention {shape} {blocks}", flush=True)
    got = causal_attention(qd, kd, vd, blocks)
    want = _reference_f32(qd, kd, vd)
    floor = softmax_floor(_reference_f32(qd, kd, vd.abs()), shape[2], score_err(q, k))
    torch.cuda.synchronize()
    check_bf16(f"attention {shape} {blocks} vs f32", got, want, floor)
    oracle = kernels.causal_attention(q, k, v, block, block)
    check_bf16(f"attention {shape} {blocks} vs oracle", got.cpu(), oracle, floor.cpu(), **SOFTMAX_BAR)


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
    qc, kc, vc = q.cpu(), k.cpu(), v.cpu()
    _close("attention (1, 2, 1024, 128) split", outs[0], kernels.causal_attention(qc, kc, vc, 256, 256),
           _floor(qc, kc, vc))
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])


@pytest.mark.parametrize("hardware,buffers", [
    ((("bkv", 64), ("waves", 8)), 2),
    ((("bkv", 32), ("waves", 4)), 2),
    ((("bkv", 32), ("waves", 8)), 2),
    ((), 3),  # K and V two blocks ahead through three LDS stages
    ((), 4),
    ((("bkv", 64), ("split", 0), ("waves", 4)), 2),  # no split-KV
    ((("bkv", 64), ("split", 10), ("waves", 4)), 2),  # split above one share
])
def test_kernel_shapes_the_tuner_tries(hardware, buffers):
    """Each gfx950 kernel shape the tuner may pick (waves per workgroup, keys per block, ring depth, split-KV
    share) against the oracle, at a shape where every block class (full, partial, skipped) occurs."""
    from tilejax_amd import Pipeline
    from tilejax_amd.tune import Config

    shape, blocks = (2, 4, 1024, 128), AttentionBlocks(256, 256)
    q, k, v = _inputs(*shape, seed=3)
    sig = causal_attention.signature(q, k, v)
    lowered = causal_attention.lowered(sig, Config(blocks, Pipeline(buffers, 2), False, hardware))
    print(f"attention {shape} {blocks} hardware={hardware} buffers={buffers}", flush=True)
    got = lowered.run(q.cuda(), k.cuda(), v.cuda())
    torch.cuda.synchronize()
    _close(f"attention {hardware} {buffers}", got, kernels.causal_attention(q, k, v, 256, 256), _floor(q, k, v))


def test_sixty_four_query_rows_a_wave():
    """The knob `rows` 64: a wave's rows as two 32-row halves that share every K and V fragment it reads from
    LDS. Each row's products and softmax are the same, so without split tiles the output is the default
    kernel's bit for bit; with them (their chunks cut elsewhere) it is within the attention tolerance of the
    oracle."""
    from tilejax_amd import Pipeline
    from tilejax_amd.tune import Config

    shape, blocks = (2, 4, 1024, 128), AttentionBlocks(256, 256)
    q, k, v = _inputs(*shape, seed=5)
    sig = causal_attention.signature(q, k, v)
    whole = [causal_attention.lowered(sig, Config(blocks, Pipeline(2, 2), False, (("split", 0),) + hw))
             for hw in ((), (("rows", 64),))]
    split64 = causal_attention.lowered(sig, Config(blocks, Pipeline(2, 2), False, (("rows", 64),)))
    assert whole[1].program.notes["block_q"] == 256 and split64.program.notes["split_items"] > 0
    print(f"attention {shape} with 64 query rows a wave", flush=True)
    dev = (q.cuda(), k.cuda(), v.cuda())
    want, got, chunked = whole[0].run(*dev), whole[1].run(*dev), split64.run(*dev)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    _close("attention 64 rows a wave, split", chunked, kernels.causal_attention(q, k, v, 256, 256), _floor(q, k, v))


@pytest.mark.parametrize("shape,blocks", [((2, 4, 1024, 128), (256, 256)), ((1, 2, 1024, 128), (256, 256))])
def test_k_fragments_in_registers_are_bit_equal(shape, blocks):
    """The knob `kreg` loads each block's K fragments from memory straight into registers (LDS holds V only).
    The S products read the same K values in the same order, so the output is the default kernel's, bit for
    bit, split tiles included (both shapes split their longest items)."""
    from tilejax_amd.tune import Config

    q, k, v = _inputs(*shape, seed=4)
    sig = causal_attention.signature(q, k, v)
    base = causal_attention.default_config(sig)
    tiles = AttentionBlocks(*blocks)
    plain = causal_attention.lowered(sig, Config(tiles, base.pipeline, False, ()))
    kreg = causal_attention.lowered(sig, Config(tiles, base.pipeline, False, (("kreg", 1),)))
    assert kreg.program.lds_bytes * 2 == plain.program.lds_bytes
    print(f"attention {shape} {blocks} with K in registers", flush=True)
    dev = (q.cuda(), k.cuda(), v.cuda())
    want, got = plain.run(*dev), kreg.run(*dev)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
