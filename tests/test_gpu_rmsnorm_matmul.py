"""Parity of RMSNorm fused with the projection after it (the reference's examples/rmsnorm_matmul.py) with
the CPU oracle on the same seeded inputs, and at a larger size with a float32 GPU reference.

The kernel runs a row pass (each row's sum of squares, and bf16(x * gamma), the matmul's left operand)
and then the matmul, whose epilogue scales each row by rsqrt(sum_sq / D + eps).

Tolerance (tests/tolerance.py): bf16 outputs within 2 bf16 ulp of the spec's oracle plus the f32 summation
floor of the product: the sum of squares is added in another order than the spec's tk-deep blocks, and the
products in MFMA order. Against float64 (no rounding of x * gamma), the floor adds 2^-8 * (|x gamma| @ |w|)
times the row scale: the spec rounds its left operand bf16(x * gamma), each element within 2^-9.
f32 inputs (the left operand's prologue then stays f32, and the products take its three bf16 parts):
within rtol 1e-4 plus 1e-4 of float64, the reference's f32 tolerance
(tests/test_examples.py:136-152).
"""

import pytest
import torch

from examples.rmsnorm_matmul import NormMatmulTiles, rmsnorm_matmul
from oracle import kernels
from tests.tolerance import P_ROUND, U32, check_bf16

pytestmark = pytest.mark.gpu


def _inputs(m, d, n, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, d, generator=g).to(torch.bfloat16)
    gamma = (1 + 0.1 * torch.randn(1, d, generator=g)).to(torch.bfloat16)
    w = (torch.randn(d, n, generator=g) / d**0.5).to(torch.bfloat16)
    return x, gamma, w


def _floors(x, gamma, w):
    """(the f32 summation floor, the floor against float64): both scale |x gamma| @ |w| by each row's
    rsqrt(mean(x^2) + eps); rmsnorm_matmul_float64 of |x|, |gamma|, |w| is exactly that magnitude."""
    mag = torch.as_tensor(kernels.rmsnorm_matmul_float64(x.float().abs(), gamma.float().abs(), w.float().abs()))
    f32 = 2.0 * x.shape[1] * U32 * mag
    return f32, f32 + P_ROUND * mag


def _close(what, got, want, floor):
    check_bf16(what, got.cpu(), torch.as_tensor(want).cpu(), floor)


@pytest.mark.parametrize("m,d,n,tiles", [
    (1024, 1024, 512, NormMatmulTiles(512, 512, 512)),
    (512, 768, 256, NormMatmulTiles(256, 256, 256)),
    (256, 512, 512, NormMatmulTiles(128, 128, 128)),
])
def test_rmsnorm_matmul_matches_oracle(m, d, n, tiles):
    x, gamma, w = _inputs(m, d, n)
    print(f"rmsnorm_matmul {m}x{d}x{n} {tiles}", flush=True)
    got = rmsnorm_matmul(x.cuda(), gamma.cuda(), w.cuda(), tiles)
    torch.cuda.synchronize()
    f32, f64 = _floors(x, gamma, w)
    what = f"rmsnorm_matmul {m}x{d}x{n} {tiles}"
    _close(what, got, kernels.rmsnorm_matmul(x, gamma, w, tiles.tm, tiles.tn, tiles.tk), f32)
    _close(what + " vs float64", got, kernels.rmsnorm_matmul_float64(x, gamma, w), f64)


def test_rmsnorm_matmul_whole_model_dim_in_one_step():
    """tk = D (tests/test_examples.py:141 of the reference): no carried values; each row's sum of squares is
    a sum over the whole row in the tile's epilogue, which the row pass computes."""
    x, gamma, w = _inputs(256, 512, 512, seed=6)
    tiles = NormMatmulTiles(128, 256, 512)
    lowered = rmsnorm_matmul.lower(x, gamma, w, tiles)
    assert not lowered.plan.carried
    print(f"rmsnorm_matmul one step {tiles}", flush=True)
    got = lowered.run(x.cuda(), gamma.cuda(), w.cuda())
    torch.cuda.synchronize()
    f32, f64 = _floors(x, gamma, w)
    _close("rmsnorm_matmul one step", got, kernels.rmsnorm_matmul(x, gamma, w, tiles.tm, tiles.tn, tiles.tk), f32)
    _close("rmsnorm_matmul one step vs float64", got, kernels.rmsnorm_matmul_float64(x, gamma, w), f64)


@pytest.mark.parametrize("tiles", [NormMatmulTiles(128, 128, 128), NormMatmulTiles(256, 128, 512)])
def test_rmsnorm_matmul_f32(tiles):
    g = torch.Generator().manual_seed(8)
    x = torch.randn(256, 512, generator=g)
    gamma = 1 + 0.1 * torch.randn(1, 512, generator=g)
    w = torch.randn(512, 512, generator=g) / 512**0.5
    print(f"rmsnorm_matmul f32 {tiles}", flush=True)
    got = rmsnorm_matmul(x.cuda(), gamma.cuda(), w.cuda(), tiles)
    torch.cuda.synchronize()
    assert got.dtype == torch.float32
    want = torch.as_tensor(kernels.rmsnorm_matmul_float64(x, gamma, w))
    scale = want.abs().max().item()
    diff = (got.double().cpu() - want).abs()
    assert not (diff > 1e-4 * want.abs() + 1e-4).any(), diff.max().item()


def test_rmsnorm_matmul_verify_against_the_spec():
    x, gamma, w = _inputs(512, 512, 512, seed=2)
    tiles = NormMatmulTiles(256, 256, 256)
    print("rmsnorm_matmul verify", flush=True)
    err = rmsnorm_matmul.verify(x.cuda(), gamma.cuda(), w.cuda(), tiles)
    assert err <= 1e-2 * 4  # the outputs are O(1): within a few bf16 ulp of the spec's own evaluation


def test_rmsnorm_matmul_large():
    """4096 x 4096 x 4096 at the default tiles against float32 on the GPU."""
    x, gamma, w = _inputs(4096, 4096, 4096, seed=1)
    x, gamma, w = x.cuda(), gamma.cuda(), w.cuda()
    print("rmsnorm_matmul 4096^3", flush=True)
    got = rmsnorm_matmul(x, gamma, w, NormMatmulTiles())
    xf = x.float()
    scale = torch.rsqrt((xf * xf).mean(dim=1, keepdim=True) + 1e-6)
    want = (xf * scale * gamma.float()) @ w.float()
    mag = ((xf.abs() * gamma.float().abs()) @ w.float().abs()) * scale
    _close("rmsnorm_matmul 4096^3 vs f32", got, want, (P_ROUND + 4.0 * 4096 * U32) * mag)


TWO_PASS = """
def two_pass(x, w):
    M, D = x.shape
    out = jnp.zeros((M, 256))
    for i in range(0, M, 128):
        sum_sq = jnp.zeros((128, 128))
        for k in range(0, D, 128):
            xk = x[i : i + 128, k : k + 128]
            sum_sq += xk * xk
        scale = jax.lax.rsqrt(jnp.sum(sum_sq, axis=1, keepdims=True) / D + 1e-6)
        acc = jnp.zeros((128, 256))
        for k2 in range(0, D, 128):
            acc += (x[i : i + 128, k2 : k2 + 128] * scale) @ w[k2 : k2 + 128, :]
        out = out.at[i : i + 128, :].set(acc)
    return out
"""


def test_two_reduction_loops_per_tile():
    """The reference's tests/test_codegen.py:580-611: a first loop sums each row's squares (a tile summed
    elementwise), the code between the loops turns them into a row scale, and the second loop multiplies the
    scaled rows. The row pass computes the sums and the scale, then writes the operand's parts (f32)."""
    from tests.helpers import make_kernel

    kernel = make_kernel(TWO_PASS)
    g = torch.Generator().manual_seed(12)
    x, w = torch.randn(256, 384, generator=g), torch.randn(384, 256, generator=g)
    lowered = kernel.lower(x, w)
    assert [p.range.var for p in lowered.plan.phases] == ["k", "k2"] and lowered.steps == 2 * 6
    print("two_pass f32 256x384x256", flush=True)
    got = lowered.run(x.cuda(), w.cuda())
    torch.cuda.synchronize()
    xd = x.double()
    want = xd / torch.sqrt((xd * xd).mean(dim=1, keepdim=True) + 1e-6) @ w.double()
    diff = (got.double().cpu() - want).abs()
    assert not (diff > 1e-4 * want.abs() + 1e-4).any(), diff.max().item()  # test_codegen.py:604
