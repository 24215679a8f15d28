"""Parity of the generated gfx950 matmul kernels with the CPU oracle (same seeded inputs).

Tolerance (tests/tolerance.py): bf16 outputs within 2 bf16 ulp of the oracle plus the f32 summation floor
2 * K * 2^-24 * (|x| @ |y|), as the north star asks; the two differ only in f32 summation order. f32
operands (`@` at full precision) are multiplied as six bf16 products of their three bf16 parts, within a
few 2^-24 of the exact product: the outputs are checked against float64 within rtol 1e-4 of |want| plus
1e-4 (the reference's f32 tolerance, tests/test_examples.py:27-32, with a tighter absolute floor).
"""

import pytest
import torch

from examples.causal_matmul import causal_matmul
from examples.matmul import MatmulTiles, matmul
from oracle import kernels
from tests.tolerance import MATMUL_BAR, check_bf16, matmul_floor

pytestmark = pytest.mark.gpu


def _inputs(m, k, n, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    g = torch.Generator().manual_seed(seed + 1)
    y = torch.randn(k, n, generator=g).to(torch.bfloat16)
    return x, y


def _close(got, want, x, y, what="matmul", bar=None):
    """2 bf16 ulp of the oracle plus the f32 summation floor of x @ y; with `bar` (the BASELINE sizes), also
    the 2-ulp bar the floor leaves open (tests/tolerance.py: MATMUL_BAR)."""
    check_bf16(what, got.cpu(), want.cpu(), matmul_floor(x.cpu(), y.cpu()), **(bar or {}))


@pytest.mark.parametrize("m,k,n,tiles", [
    (1024, 1024, 1024, MatmulTiles(512, 512, 512)),
    (512, 256, 512, MatmulTiles(256, 256, 128)),
    (1024, 1024, 1024, MatmulTiles(256, 256, 256)),
    (512, 512, 512, MatmulTiles(128, 128, 128)),
])
def test_matmul_matches_oracle(m, k, n, tiles):
    x, y = _inputs(m, k, n)
    print(f"matmul {m}x{k}x{n} {tiles}", flush=True)
    got = matmul(x.cuda(), y.cuda(), tiles)
    torch.cuda.synchronize()
    _close(got, kernels.matmul(x, y, tiles.tm, tiles.tn, tiles.tk), x, y)


@pytest.mark.parametrize("n,tiles", [(1024, MatmulTiles(256, 256, 256)), (512, MatmulTiles(128, 128, 128)),
                                     (1024, MatmulTiles(512, 512, 512))])
def test_causal_matmul_matches_oracle(n, tiles):
    x, y = _inputs(n, n, n, seed=3)
    print(f"causal {n} {tiles}", flush=True)
    got = causal_matmul(x.cuda(), y.cuda(), tiles)
    torch.cuda.synchronize()
    want = kernels.causal_matmul(x, y, tiles.tm, tiles.tn, tiles.tk)
    _close(got, want, x, y, "causal")
    assert not got.cpu().float().triu(1).any()  # above the diagonal: exactly the fill


def test_matmul_verify_against_reference():
    x, y = _inputs(512, 256, 512, seed=5)
    err = matmul.verify(x.cuda(), y.cuda(), MatmulTiles(256, 256, 128))
    assert err < 1.0


def test_causal_matmul_full_size_balanced_split():
    """The 8192^3 causal matmul at 512^3 tiles: 528 computed 256x256 tiles on 256 workgroups, so 16 of them are
    cut along K into 8 chunks of 16 slices whose partials a fixup kernel adds. Checked against the oracle
    everywhere."""
    n, tiles = 8192, MatmulTiles(512, 512, 512)
    x, y = _inputs(n, n, n, seed=7)
    lowered = causal_matmul.lower(x, y, tiles)
    assert lowered.program.notes["split"] == (16, 8, 16)
    print(f"causal {n} {tiles} split {lowered.program.notes['split']}", flush=True)
    got = lowered.run(x.cuda(), y.cuda())
    torch.cuda.synchronize()
    want = kernels.causal_matmul(x, y, tiles.tm, tiles.tn, tiles.tk)
    _close(got, want, x, y, "causal", MATMUL_BAR)
    assert not got.cpu().float().triu(1).any()


def _f32_product_on_gpu(x, y):
    """x @ y in float32 on the GPU (no reduced-precision f32 modes), and its f32 summation floor."""
    allow = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    try:
        want = x.float() @ y.float()
        floor = matmul_floor(x, y)
    finally:
        torch.backends.cuda.matmul.allow_tf32 = allow
    return want, floor


@pytest.mark.parametrize("tiles", [MatmulTiles(512, 512, 512), MatmulTiles(1024, 2048, 1024)])
def test_dense_headline_full_output(tiles):
    """BASELINE.json config 2, the benchmark's headline: dense x @ y at 8192^3 (seeds 0 and 1, as bench.py
    draws them). Every output against a float32 product on the GPU rounded to bf16, within 2 bf16 ulp plus
    the f32 summation floor, and with every typical output within 2 ulp and 99.99 % of all within 2 ulp with no
    floor; then a band of 512 rows against the CPU oracle's own loop nest, to the same bar."""
    n = 8192
    x, y = _inputs(n, n, n, seed=0)
    xd, yd = x.cuda(), y.cuda()
    lowered = matmul.lower(xd, yd, tiles)
    print(f"dense {n}^3 {tiles} {lowered.program.notes.get('hw_tile')}", flush=True)
    got = lowered.run(xd, yd)
    want, floor = _f32_product_on_gpu(xd, yd)
    torch.cuda.synchronize()
    check_bf16(f"dense {n}^3 {tiles} vs f32 product", got, want.to(torch.bfloat16), floor, **MATMUL_BAR)
    del want, floor
    band = kernels.matmul(x[:512], y, 512, 512, 512)
    _close(got[:512], band, x[:512], y, f"dense {n}^3 {tiles} rows 0..511 vs oracle", MATMUL_BAR)


def test_causal_headline_1024x2048x1024():
    """BASELINE.json config 2's causal variant at its second reported tile shape, 1024 x 2048 x 1024: every
    output against the CPU oracle (the spec's loop nest at the same tiles), above the diagonal exactly the
    fill."""
    n, tiles = 8192, MatmulTiles(1024, 2048, 1024)
    x, y = _inputs(n, n, n, seed=8)
    lowered = causal_matmul.lower(x, y, tiles)
    print(f"causal {n} {tiles} split {lowered.program.notes.get('split')}", flush=True)
    got = lowered.run(x.cuda(), y.cuda())
    torch.cuda.synchronize()
    want = kernels.causal_matmul(x, y, tiles.tm, tiles.tn, tiles.tk)
    _close(got, want, x, y, "causal 1024x2048x1024", MATMUL_BAR)
    assert not got.cpu().float().triu(1).any()


def test_split_chunks_start_from_the_initial_value_once():
    """A matmul nest whose accumulator starts at 1 and whose epilogue reads the tile's loop values: with 16
    tiles on 256 workgroups each tile is cut into 4 chunks, and the fixup must add the start value once and
    place every tile."""
    from tests.helpers import make_kernel

    k = make_kernel('''
        def offset_matmul(x, y):
            M, K = x.shape
            N = y.shape[1]
            out = jnp.zeros((M, N), jnp.float32)
            for i in range(0, M, 256):
                for j in range(0, N, 256):
                    acc = jnp.full((256, 256), 1.0, jnp.float32)
                    for kk in range(0, K, 512):
                        acc += x[i : i + 256, kk : kk + 512] @ y[kk : kk + 512, j : j + 256]
                    out = out.at[i : i + 256, j : j + 256].set(acc * 0.5 + (i + 2 * j))
            return out
    ''')
    x, y = _inputs(1024, 2048, 1024, seed=11)
    lowered = k.lower(x, y)
    assert lowered.program.notes["split"] is not None
    got = lowered.run(x.cuda(), y.cuda())
    torch.cuda.synchronize()
    want = k.reference(x, y)
    assert torch.allclose(got.cpu(), want, rtol=1e-4, atol=1e-3), (got.cpu() - want).abs().max()


def test_four_input_buffers_take_half_depth_slices():
    """Four input buffers don't fit as 64-deep slices of a 256 x 256 tile; the kernel then streams 32-deep
    slices through four LDS stages, and computes the same."""
    from tilejax_amd.pipeline import Pipeline
    from tilejax_amd.tune import Config

    x, y = _inputs(1024, 1024, 1024, seed=5)
    tiles = MatmulTiles(512, 512, 512)
    lowered = matmul.lowered(matmul.signature(x, y), Config(tiles, Pipeline(4, 2)))
    assert lowered.program.notes["hw_tile"][2] == 32 and lowered.program.notes["stages"] == 4
    print("matmul 1024^3, four 32-deep stages", flush=True)
    got = lowered.run(x.cuda(), y.cuda())
    _close(got, kernels.matmul(x, y, 512, 512, 512), x, y)
    plain = matmul.lowered(matmul.signature(x, y), Config(tiles, Pipeline(2, 2))).run(x.cuda(), y.cuda())
    assert torch.equal(got, plain)  # the same K order, so the same bits


def _inputs_f32(m, k, n, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(m, k, generator=g), torch.randn(k, n, generator=torch.Generator().manual_seed(seed + 1))


def _close_f32(got, want):
    got, want = got.double().cpu(), torch.as_tensor(want).double().cpu()
    scale = want.abs().max().item()
    bad = (got - want).abs() > 1e-4 * want.abs() + 1e-4
    assert not bad.any(), f"{int(bad.sum())} of {want.numel()} differ; max |diff| {(got - want).abs().max().item()}"


@pytest.mark.parametrize("m,k,n,tiles", [
    (256, 384, 256, MatmulTiles(128, 128, 128)),  # three reduction steps
    (256, 384, 256, MatmulTiles(256, 128, 512)),  # one reduction step: no accumulator
    (256, 384, 256, MatmulTiles(256, 256, 128)),
    (1024, 1024, 1024, MatmulTiles(512, 512, 512)),
])
def test_matmul_f32_operands(m, k, n, tiles):
    """The reference's f32 cases (tests/test_examples.py:18-32): `@` of f32 operands against float64."""
    x, y = _inputs_f32(m, k, n)
    print(f"matmul f32 {m}x{k}x{n} {tiles}", flush=True)
    lowered = matmul.lower(x, y, tiles)
    assert lowered.program.notes["f32_operands"]
    got = lowered.run(x.cuda(), y.cuda())
    torch.cuda.synchronize()
    assert got.dtype == torch.float32
    _close_f32(got, x.double() @ y.double())


def test_matmul_one_reduction_step_bf16():
    """tk covering the whole reduction: the loop of one step joins the tile code, and no value is carried."""
    x, y = _inputs(256, 384, 256, seed=4)
    tiles = MatmulTiles(256, 128, 512)
    assert not matmul.lower(x, y, tiles).plan.carried
    print(f"matmul bf16 one step {tiles}", flush=True)
    got = matmul(x.cuda(), y.cuda(), tiles)
    torch.cuda.synchronize()
    _close(got, kernels.matmul(x, y, tiles.tm, tiles.tn, tiles.tk), x, y)


def test_causal_matmul_f32_operands():
    """tests/test_examples.py:55-63 of the reference in f32: tril(x @ y) against float64, above the diagonal
    exactly the fill."""
    x, y = _inputs_f32(512, 256, 512, seed=2)
    tiles = MatmulTiles(128, 128, 128)
    print(f"causal f32 {tiles}", flush=True)
    got = causal_matmul(x.cuda(), y.cuda(), tiles)
    torch.cuda.synchronize()
    _close_f32(got, torch.tril(x.double() @ y.double()))
    assert not got.cpu().triu(1).any()


@pytest.mark.parametrize("hardware,buffers", [
    ((("bm", 256), ("bn", 128)), 2),
    ((("bm", 128), ("bn", 256)), 2),
    ((("bm", 128), ("bn", 128)), 3),
    ((), 4),
    ((("bm", 256), ("bn", 256), ("waves", 8)), 2),  # the default, spelled out
    ((("bm", 256), ("bn", 256), ("waves", 4)), 2),
    ((("bm", 256), ("bn", 256), ("waves", 4)), 4),
    ((("bm", 256), ("bn", 128), ("waves", 8)), 3),
    ((("bm", 128), ("bn", 128), ("waves", 8)), 2),
])
def test_workgroup_tiles_the_tuner_tries(hardware, buffers):
    """Each gfx950 workgroup tile, wave count and LDS ring depth the tuner may pick, dense and causal, against
    the oracle."""
    from tilejax_amd import Pipeline
    from tilejax_amd.tune import Config

    tiles = MatmulTiles(512, 512, 512)
    x, y = _inputs(1024, 1024, 1024, seed=7)
    for kernel, oracle in ((matmul, kernels.matmul), (causal_matmul, kernels.causal_matmul)):
        lowered = kernel.lowered(kernel.signature(x, y), Config(tiles, Pipeline(buffers, 2), False, hardware))
        print(f"{kernel.nest.name} 1024^3 {tiles} hardware={hardware} buffers={buffers} "
              f"-> {lowered.program.notes['hw_tile']} x{lowered.program.notes['stages']} in {lowered.program.notes['waves']} waves",
              flush=True)
        got = lowered.run(x.cuda(), y.cuda())
        torch.cuda.synchronize()
        _close(got, oracle(x, y, 512, 512, 512), x, y, f"{kernel.nest.name} {hardware}")
