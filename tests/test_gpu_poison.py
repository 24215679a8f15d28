"""Poisoned runs of every kernel family on the GPU (tilejax_amd/codegen/poison.py): the LDS arrays, outputs and
workspaces start as NaN bytes, and the result must be the plain run's, bit for bit, with no NaN.

This stands in for the reference running its kernels with `uninitialized_memory="nan"` (its
tests/helpers.py:26-35): a kernel that reads LDS before its loads land, reads a workspace element no launch
wrote (split-K partials, split-KV partials, step tables, the generic kernel's tile memory), or leaves an output
element unwritten (the zero rows of an unused expert, the filled tiles above a causal diagonal) gives NaN or
other bits here.
"""

import pytest
import torch

from tilejax_amd import Pipeline
from tilejax_amd.tune import Config

pytestmark = pytest.mark.gpu


def _both(kernel, args, tunable=None, cursor=False):
    """The plain and the poisoned program's outputs for `args` (GPU tensors), default config unless `tunable`."""
    sig = kernel.signature(*args)
    base = kernel.lowered(sig, kernel.default_config(sig))
    tunable = base.config.tunable if tunable is None else tunable
    plain = kernel.lowered(sig, Config(tunable, base.config.pipeline, cursor))
    poisoned = kernel.lowered(sig, Config(tunable, base.config.pipeline, cursor, (("poison", 1),)))
    assert poisoned.program.notes.get("poison") and not plain.program.notes.get("poison")
    want = plain.run(*args)
    got = poisoned.run(*args)
    torch.cuda.synchronize()
    return want, got, poisoned.program.notes


def _same(what, want, got):
    print(f"poisoned {what}: compared {want.numel()} outputs", flush=True)
    assert not torch.isnan(want.float()).any(), f"{what}: the plain run has NaN"
    assert not torch.isnan(got.float()).any(), f"{what}: the poisoned run has NaN (an unwritten output or a poisoned read)"
    assert torch.equal(want, got), f"{what}: the poisoned run differs from the plain one"


def _randn(*shape, seed=0, scale=1.0, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype).cuda()


def test_causal_matmul_with_split_chunks_and_fills():
    """8192^3 causal: the last round's tiles cut along K write partials the fixup kernel adds; the tiles above the
    diagonal are filled, not computed."""
    from examples.causal_matmul import causal_matmul
    from examples.matmul import MatmulTiles

    x, y = _randn(8192, 8192, seed=1), _randn(8192, 8192, seed=2)
    want, got, notes = _both(causal_matmul, (x, y), MatmulTiles(512, 512, 512))
    assert notes["split"] is not None
    _same("causal matmul 8192^3", want, got)


def test_dense_and_f32_operand_matmuls():
    from examples.matmul import MatmulTiles, matmul

    x, y = _randn(1024, 768, seed=3), _randn(768, 1280, seed=4)
    _same("matmul 1024x768x1280", *_both(matmul, (x, y), MatmulTiles(256, 256, 256))[:2])
    xf, yf = _randn(256, 384, seed=5, dtype=torch.float32), _randn(384, 256, seed=6, dtype=torch.float32)
    want, got, notes = _both(matmul, (xf, yf), MatmulTiles(128, 128, 128))
    assert notes["f32_operands"]  # the operands' bf16 parts go through a workspace
    _same("matmul f32 operands", want, got)


def test_grouped_matmul_with_an_unused_expert():
    """Runtime step tables (a workspace the builder writes) and a group whose expert is -1: its rows are stored as
    zeros by the kernel, never computed."""
    from examples.moe import GroupTiles, grouped_matmul

    xs, w = _randn(1024, 512, seed=7), _randn(4, 512, 1024, seed=8, scale=0.05)
    ge = torch.tensor([0, -1, 3, 1], dtype=torch.int32).cuda()
    want, got, _ = _both(grouped_matmul, (xs, w, ge), GroupTiles(512, 256))
    assert (want[256:512] == 0).all()
    _same("grouped matmul", want, got)


def test_rmsnorm_matmul_row_pass():
    from examples.rmsnorm_matmul import NormMatmulTiles, rmsnorm_matmul

    x, w = _randn(512, 768, seed=9), _randn(768, 256, seed=10)
    gamma = (1 + 0.1 * _randn(1, 768, seed=11).float()).to(torch.bfloat16)
    _same("rmsnorm matmul", *_both(rmsnorm_matmul, (x, gamma, w), NormMatmulTiles(256, 256, 256))[:2])


def test_attention_with_split_kv_chunks():
    """(1, 2, 1024, 128) at 256^2 blocks cuts its longest items into chunks merged by a second kernel."""
    from examples.causal_attention import AttentionBlocks, causal_attention

    q = (_randn(1, 2, 1024, 128, seed=12).float() * 128 ** -0.5).to(torch.bfloat16)
    k, v = _randn(1, 2, 1024, 128, seed=13), _randn(1, 2, 1024, 128, seed=14)
    want, got, notes = _both(causal_attention, (q, k, v), AttentionBlocks(256, 256))
    assert notes["split_items"] > 0
    _same("attention (1, 2, 1024, 128) 256^2", want, got)
    q2 = (_randn(2, 4, 1024, 128, seed=15).float() * 128 ** -0.5).to(torch.bfloat16)
    k2, v2 = _randn(2, 4, 1024, 128, seed=16), _randn(2, 4, 1024, 128, seed=17)
    _same("attention (2, 4, 1024, 128) 512^2", *_both(causal_attention, (q2, k2, v2), AttentionBlocks(512, 512))[:2])


@pytest.mark.parametrize("cursor", [False, True])
def test_paged_decode(cursor):
    """Step tables (or the cursor's scan in LDS), split partials and the merge, ragged lengths (one empty)."""
    from examples.decode import paged_gqa_decode

    B, H, Hkv, D, P, pages = 6, 32, 8, 128, 16, 40
    q = (_randn(B, 1, H, D, seed=18).float() * D ** -0.5).to(torch.bfloat16)
    g = torch.Generator().manual_seed(19)
    table = torch.randperm(B * pages, generator=g).reshape(B, pages).to(torch.int32).cuda()
    kp, vp = _randn(B * pages, P, Hkv * D, seed=20), _randn(B * pages, P, Hkv * D, seed=21)
    lengths = torch.tensor([0, 1, 17, 300, 640, 511], dtype=torch.int32).cuda()
    want, got, _ = _both(paged_gqa_decode, (q, kp, vp, table, lengths), cursor=cursor)
    _same(f"paged decode cursor={cursor}", want, got)


def test_expert_ffn_chain():
    """The chain of two matmul-family kernels: the hidden activations are a workspace the gate kernel writes
    and the down kernel reads (poisoned, a row the gate kernel left unwritten would reach the output), and
    both kernels' step tables are workspaces too."""
    from examples.moe import ExpertTiles, expert_ffn

    xs = _randn(512, 256, seed=22)
    wg, wu = _randn(4, 256, 512, seed=23, scale=1 / 16), _randn(4, 256, 512, seed=24, scale=1 / 16)
    wd = _randn(4, 512, 256, seed=25, scale=1 / 16)
    te = torch.tensor([0, 2, -1, 1], dtype=torch.int32).cuda()
    want, got, notes = _both(expert_ffn, (xs, wg, wu, wd, te), ExpertTiles(block_f=128))
    assert notes["family"] == "gemm" and notes["chain"]
    _same("expert_ffn", want, got)


def test_a_nest_on_the_generic_kernel():
    """The generic kernel: its tile memory is a workspace (global memory). A nest of no family's form (an
    elementwise map and a row sum in one tile)."""
    from tests.helpers import make_kernel

    kernel = make_kernel("""
    def rowmix(x):
        M, N = x.shape
        dtype = x.dtype
        out = jnp.zeros((M, N), dtype)
        for i in range(0, M, 64):
            t = x[i : i + 64, :].astype(jnp.float32)
            s = jnp.sum(t * t, axis=1, keepdims=True)
            out = out.at[i : i + 64, :].set((jnp.tanh(t) * s).astype(dtype))
        return out
    """)
    x = _randn(256, 384, seed=26)
    want, got, notes = _both(kernel, (x,))
    assert notes["family"] == "generic"
    _same("generic rowmix", want, got)
