"""Trace-region profiles and the autotuner on the MI355X (the reference's tests/test_tpu.py:44-96)."""

import pytest
import torch

import tilejax_amd as autokernel
from examples.matmul import MatmulTiles, matmul
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
