"""Trace-region profiles and the autotuner on the MI355X (the reference's tests/test_tpu.py:44-96)."""

import pytest
import torch

import tilejax_amd as autokernel
from examples.matmul import MatmulTiles, matmul
from tilejax_amd.codegen.program import TRACE_FIELDS
from tilejax_amd.jaxlite import jnp

pytestmark = pytest.mark.gpu


def _inputs(n, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n, n, generator=g).to(torch.bfloat16).cuda()
    y = torch.randn(n, n, generator=g).to(torch.bfloat16).cuda()
    return x, y


def test_profile_has_trace_regions():
    x, y = _inputs(2048)
    tiles = MatmulTiles(512, 512, 512)
    print("profile matmul 2048^3 512^3", flush=True)
    p = autokernel.profile(matmul, x, y, tiles, runs=3)
    print(p, flush=True)
    assert p.calls == 3 and p.regions
    assert p.steps == pytest.approx(matmul.lower(x, y, tiles).steps)
    assert 0 < p.compute_s < p.device_s and p.wait_s >= p.fill_s > 0
    assert p.bottleneck in ("dma", "overhead", "compute")
    assert 0.5e9 < p.clock_hz <= 2.45e9, p.clock_hz  # measured in the kernel; the chip's peak is 2.4 GHz


@autokernel.tunable
class Small:
    tm: int = autokernel.choice(128, 256, 512, 1024)
    tn: int = autokernel.choice(128, 256, 512, 1024)
    tk: int = autokernel.choice(128, 256, 512, 1024)


@autokernel.kernel
def small_matmul(x, y, tiles=Small()):
    M, K = x.shape
    N = y.shape[1]
    dtype = x.dtype
    out = jnp.zeros((M, N), dtype)
    for i in range(0, M, tiles.tm):
        for j in range(0, N, tiles.tn):
            acc = jnp.zeros((tiles.tm, tiles.tn), jnp.float32)
            for k in range(0, K, tiles.tk):
                acc += x[i : i + tiles.tm, k : k + tiles.tk] @ y[k : k + tiles.tk, j : j + tiles.tn]
            out = out.at[i : i + tiles.tm, j : j + tiles.tn].set(acc.astype(dtype))
    return out


def test_tuning_beats_small_default_tiles():
    x, y = _inputs(4096, seed=1)
    print("tuning small_matmul 4096^3 from 128^3 tiles", flush=True)
    tuning = small_matmul.tuning(x, y)
    print(tuning, flush=True)
    first = tuning.trials[0]
    assert first.config.tunable == Small() and first.profile is not None and first.profile.regions
    assert tuning.best.seconds < 0.7 * first.seconds  # 128x128 workgroup tiles re-read LDS twice as often
    assert small_matmul.lower(x, y).config == tuning.config
    scale = small_matmul(x, y).float().abs().max().item()
    assert small_matmul.verify(x, y) <= 1e-2 * scale  # (verify asserts the dtype tolerances itself)


def _attention_inputs(shape, seed=0):
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(*shape, generator=g).to(torch.bfloat16) for _ in range(3))
    q = (q.float() * shape[-1] ** -0.5).to(torch.bfloat16)
    return q.cuda(), k.cuda(), v.cuda()


@pytest.mark.parametrize("shape, blocks", [((2, 4, 1024, 128), (256, 256)), ((1, 16, 4096, 128), (512, 512))])
def test_attention_profile_has_trace_regions(shape, blocks):
    """The flash family's regions: the first block's wait is the fill, later waits and compute per block;
    a traced build computes what the untraced one does."""
    from examples.causal_attention import AttentionBlocks, causal_attention

    q, k, v = _attention_inputs(shape)
    tiles = AttentionBlocks(*blocks)
    print(f"profile causal_attention {shape} {blocks}", flush=True)
    p = autokernel.profile(causal_attention, q, k, v, tiles, runs=3)
    print(p, flush=True)
    assert p.calls == 3 and p.regions
    assert 0 < p.compute_s < p.device_s and p.wait_s >= p.fill_s > 0
    assert p.bottleneck in ("dma", "overhead", "compute")
    plain = causal_attention.lower(q, k, v, tiles)
    traced = causal_attention.lowered(causal_attention.signature(q, k, v), plain.config, trace=True)
    out, trace = traced.program.run_traced(q, k, v)
    assert trace is not None and torch.equal(out, plain.run(q, k, v))
    # a workgroup's slices are the key blocks of its work item (the item table's block count column)
    items = traced.program.tables["fa_items"].reshape(-1, 5 + 2 * traced.program.notes["waves"])
    assert trace.view(-1, TRACE_FIELDS)[:, 4].sum().item() == int(items[:, 3].sum())
    # the shader clock the workgroups ran at, measured in the kernel: within the chip's range (2.4 GHz peak)
    assert 0.5e9 < p.clock_hz <= 2.45e9, p.clock_hz


def test_decode_profile_has_trace_regions():
    """The decode family's regions over its attention kernel; slices are the step table's steps."""
    from examples.decode import paged_gqa_decode

    g = torch.Generator().manual_seed(5)
    B, pages, P, W = 8, 64, 16, 1024
    q = (torch.randn(B, 1, 32, 128, generator=g) * 128**-0.5).to(torch.bfloat16).cuda()
    kp = torch.randn(B * pages, P, W, generator=g).to(torch.bfloat16).cuda()
    vp = torch.randn(B * pages, P, W, generator=g).to(torch.bfloat16).cuda()
    table = torch.randperm(B * pages, generator=g).reshape(B, pages).to(torch.int32).cuda()
    lengths = torch.tensor([0, 1, 17, 300, 512, 777, 1000, 1024], dtype=torch.int32).cuda()
    print("profile paged_gqa_decode 8 sequences", flush=True)
    p = autokernel.profile(paged_gqa_decode, q, kp, vp, table, lengths, runs=3)
    print(p, flush=True)
    assert p.calls == 3 and p.regions
    assert 0 < p.compute_s < p.device_s and p.wait_s >= p.fill_s > 0
    # one step per page in use, one empty step per empty sequence (the reference's table)
    want = sum(-(-int(n) // P) for n in lengths.tolist()) + sum(1 for n in lengths.tolist() if n == 0)
    assert p.steps == want
    plain = paged_gqa_decode.lower(q, kp, vp, table, lengths)
    traced = paged_gqa_decode.lowered(paged_gqa_decode.signature(q, kp, vp, table, lengths), plain.config, trace=True)
    out, trace = traced.program.run_traced(q, kp, vp, table, lengths)
    assert trace is not None and torch.equal(out, plain.run(q, kp, vp, table, lengths))


def test_tuning_decode_tries_both_ways_of_finding_steps():
    """A kernel with runtime masks may find its steps from device tables or with a cursor; tuning tries
    both (the reference's tune.py:186-187) and keeps the faster."""
    from examples.decode import paged_gqa_decode

    g = torch.Generator().manual_seed(8)
    B, pages, P, W = 16, 64, 16, 1024
    q = (torch.randn(B, 1, 32, 128, generator=g) * 128**-0.5).to(torch.bfloat16).cuda()
    kp = torch.randn(B * pages, P, W, generator=g).to(torch.bfloat16).cuda()
    vp = torch.randn(B * pages, P, W, generator=g).to(torch.bfloat16).cuda()
    table = torch.randperm(B * pages, generator=g).reshape(B, pages).to(torch.int32).cuda()
    lengths = torch.randint(0, pages * P + 1, (B,), generator=g, dtype=torch.int32).cuda()
    print("tuning paged_gqa_decode 16 sequences", flush=True)
    tuning = paged_gqa_decode.tuning(q, kp, vp, table, lengths)
    print(tuning, flush=True)
    assert {t.config.cursor for t in tuning.trials if t.profile is not None} == {False, True}


def test_tuning_at_the_dense_baseline_tries_workgroup_tiles():
    """BASELINE config 2 (dense 8192^3 bf16 at 512^3 tiles): tuning tries the matmul family's other workgroup
    tiles, each a different kernel that is checked against the reference, and picks one at least as fast
    as the default."""
    from tilejax_amd.tune import tune

    x, y = _inputs(8192, seed=2)
    print("tuning matmul 8192^3 from its default tiles", flush=True)
    tuning = tune(matmul, matmul.signature(x, y), [x, y], budget=6)
    print(tuning, flush=True)
    shapes = {t.config.hardware for t in tuning.trials if t.profile is not None}
    assert len(shapes) >= 3, shapes  # the default 256 x 256 and at least two others ran
    first = tuning.trials[0]
    assert first.config == matmul.default_config(matmul.signature(x, y)) and first.profile is not None
    assert tuning.best.seconds <= first.seconds
