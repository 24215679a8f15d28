"""Parity of the generic gfx950 kernel (the lowering of nests no kernel family takes) with the oracle and
with closed forms: two masked phases with values carried across them, row sums, phases back to back, and
the reference's attention_block (attention, RMSNorm and the feed-forward in one nest).

Tolerance: f32 results within rtol 1e-4 plus 1e-4 of float64 (the reference's f32 tolerance,
tests/test_codegen.py:626-634). bf16 results (attention_block) within 2 bf16 ulp of the oracle plus a floor
for the spec's three roundings to bf16 (p, the normalized rows, the hidden activations): the kernel and
the oracle run the same operations in the same blocks and differ only in f32 summation order, so a value
can round to the other side of a bf16 boundary, moving it by 2^-8 of itself; the floor allows two such
moves of every hidden activation and normalized row element, carried through the products after them
(|normed| @ |w_up| times 1.13, GELU's largest slope, plus |hidden|, then @ |w_down|). Against float64, the
reference's own bound: 3e-2 of the largest |want| (tests/test_examples.py:180-188).
"""

import numpy as np
import pytest
import torch

from examples.attention_block import BlockTiles, attention_block
from oracle import kernels
from tests.helpers import make_kernel
from tests.test_generic import MASKED_PHASES, _block_inputs, masked_phases_float64
from tests.tolerance import P_ROUND, check_bf16

pytestmark = pytest.mark.gpu


def _close_f32(what, got, want):
    got, want = got.double().cpu(), torch.as_tensor(want).double().cpu()
    bad = (got - want).abs() > 1e-4 * want.abs() + 1e-4
    assert not bad.any(), f"{what}: {int(bad.sum())} of {want.numel()} differ; max {(got - want).abs().max().item()}"
    print(f"{what}: max |diff| {(got - want).abs().max().item():.3g}", flush=True)


def test_masked_phases():
    k = make_kernel(MASKED_PHASES)
    g = torch.Generator().manual_seed(1)
    x, w = torch.randn(256, 384, generator=g), torch.randn(128, 128, generator=g) / 8
    lowered = k.lower(x, w)
    assert lowered.program.notes["family"] == "generic"
    print("generic: masked phases", flush=True)
    got = lowered.run(x.cuda(), w.cuda())
    torch.cuda.synchronize()
    _close_f32("masked phases", got, masked_phases_float64(x, w))


def test_row_sums_and_phases_back_to_back():
    rows = make_kernel("""
    def row_sums(x):
        M, N = x.shape
        out = jnp.zeros((M, 128), jnp.float32)
        for i in range(0, M, 128):
            acc = jnp.zeros((128, 128), jnp.float32)
            for j in range(0, N, 128):
                acc += x[i : i + 128, j : j + 128]
            out = out.at[i : i + 128, :].set(acc)
        return out
    """)
    twice = make_kernel("""
    def twice(x):
        out = jnp.zeros((128, 128))
        for i in range(0, 128, 128):
            a = jnp.zeros((128, 128))
            for k in range(0, 256, 128):
                a += x[i : i + 128, k : k + 128]
            for k2 in range(0, 256, 128):
                a = jnp.maximum(a, x[i : i + 128, k2 : k2 + 128])
            out = out.at[i : i + 128, :].set(a)
        return out
    """)
    g = torch.Generator().manual_seed(2)
    x = torch.randn(256, 512, generator=g)
    print("generic: row sums", flush=True)
    got = rows(x.cuda())
    want = sum(x.double()[:, j:j + 128] for j in range(0, 512, 128))
    _close_f32("row sums", got, want)
    x2 = torch.randn(128, 256, generator=g)
    print("generic: phases back to back", flush=True)
    got = twice(x2.cuda())
    a = x2.double()[:, :128] + x2.double()[:, 128:]
    want = torch.maximum(torch.maximum(a, x2.double()[:, :128]), x2.double()[:, 128:])
    _close_f32("phases back to back", got, want)


def _block_floor(ins):
    q, k, v, gamma, w_up, w_down = ins
    a = torch.as_tensor(kernels.attention_float64(q, k, v))
    B, H, S, Dh = a.shape
    a = a.permute(0, 2, 1, 3).reshape(B, S, H * Dh)
    normed = a / torch.sqrt((a * a).mean(dim=-1, keepdim=True) + 1e-6) * gamma.double()
    up = normed @ w_up.double()
    hidden = kernels._gelu_tanh(up)
    moved = 1.13 * (normed.abs() @ w_up.double().abs()) + hidden.abs()
    return 2 * P_ROUND * (moved @ w_down.double().abs())


@pytest.mark.parametrize("block_q, block_kv", [(128, 128), (256, 128)])
def test_attention_block(block_q, block_kv):
    """The reference's tests/test_examples.py:180-188 case: (1, 2, 512, 128) heads, F = 512, bf16."""
    ins = _block_inputs()
    tiles = BlockTiles(block_q=block_q, block_kv=block_kv)
    print(f"generic: attention_block {tiles}", flush=True)
    got = attention_block(*(t.cuda() for t in ins), tiles)
    torch.cuda.synchronize()
    want = kernels.attention_block(*ins, bq=block_q, bk=block_kv, bf=512)
    check_bf16(f"attention_block {tiles} vs oracle", got.cpu(), want, _block_floor(ins))
    exact = torch.as_tensor(kernels.attention_block_float64(*ins))
    assert (got.cpu().double() - exact).abs().max().item() < 3e-2 * exact.abs().max().item()
    attention_block.verify(*(t.cuda() for t in ins), tiles)


def test_attention_block_streams_the_feed_forward():
    """block_f below F: the feed-forward is a second phase that streams w_up and w_down (two phases, values
    carried from the first into the second)."""
    ins = _block_inputs(S=256, F=1024, seed=5)
    tiles = BlockTiles(block_q=128, block_kv=128, block_f=256)
    lowered = attention_block.lower(*ins, tiles)
    assert [p.range.var for p in lowered.plan.phases] == ["j", "f"]
    print(f"generic: attention_block {tiles}", flush=True)
    got = lowered.run(*(t.cuda() for t in ins))
    torch.cuda.synchronize()
    want = kernels.attention_block(*ins, bq=128, bk=128, bf=256)
    check_bf16(f"attention_block {tiles} vs oracle", got.cpu(), want, _block_floor(ins))


def test_attention_block_f32():
    """f32 inputs: nothing rounds to bf16, so within rtol 1e-3 plus 1e-3 of the largest |want| of float64."""
    ins = _block_inputs(S=256, F=256, seed=7, dtype=torch.float32)
    tiles = BlockTiles(block_q=128, block_kv=128, block_f=256)
    print(f"generic: attention_block f32 {tiles}", flush=True)
    got = attention_block(*(t.cuda() for t in ins), tiles)
    want = torch.as_tensor(kernels.attention_block_float64(*ins))
    diff = (got.cpu().double() - want).abs()
    assert not (diff > 1e-3 * want.abs() + 1e-3 * want.abs().max()).any(), diff.max().item()
