"""Parity of the grouped matmul with runtime expert windows (BASELINE.json config 4's spec, examples/moe.py)
with the CPU oracle, and of the device step-table builder with the reference's table semantics restated in
oracle/schedule.py: bit-exact tables, counts and codes.

Tolerance for the matmul (tests/tolerance.py): bf16 outputs within 2 bf16 ulp of the expected value plus the
f32 summation floor 2 * K * 2^-24 * (|xs| @ |w_e|) of each group's product; f32
operands (six bf16 products of their parts) within rtol 1e-4 plus 1e-4 of float64,
the reference's f32 tolerance for its grouped kernels (tests/test_moe.py:252-275).
"""

import numpy as np
import pytest
import torch

from examples.moe import GroupTiles, grouped_matmul
from oracle import kernels
from oracle import schedule as oracle_schedule
from tests.tolerance import MATMUL_BAR, check_bf16, matmul_floor

pytestmark = pytest.mark.gpu


def _inputs(M, K, N, E, experts, seed=0):
    g = torch.Generator().manual_seed(seed)
    xs = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w = (torch.randn(E, K, N, generator=g) * 0.02).to(torch.bfloat16)
    return xs, w, torch.tensor(experts, dtype=torch.int32)


def _floor(xs, w, experts):
    """Each group's f32 summation floor through its (clamped) expert; zero for unused groups."""
    G = xs.shape[0] // len(experts)
    floor = torch.zeros(xs.shape[0], w.shape[2], dtype=torch.float32, device=xs.device)
    for g, e in enumerate(experts):
        if e >= 0:
            rows = slice(g * G, (g + 1) * G)
            floor[rows] = matmul_floor(xs[rows], w[min(e, w.shape[0] - 1)])
    return floor


@pytest.mark.parametrize("experts,tiles", [
    ([0, 1, 2, 3], GroupTiles(512, 256)),
    ([0, 0, 2, -1], GroupTiles(256, 512)),  # an unused group keeps its zeros
    ([3, 9, -1, 1], GroupTiles(512, 512)),  # 9 is past the 4 experts: clamped to the last, as JAX clamps
    ([-1, -1, -1, -1], GroupTiles(512, 256)),  # every group unused: every tile one empty step
])
def test_grouped_matmul_matches_oracle(experts, tiles):
    xs, w, ge = _inputs(1024, 512, 1024, 4, experts)
    print(f"grouped matmul experts={experts} {tiles}", flush=True)
    got = grouped_matmul(xs.cuda(), w.cuda(), ge.cuda(), tiles)
    torch.cuda.synchronize()
    check_bf16(f"grouped matmul experts={experts}", got.cpu(), kernels.grouped_matmul(xs, w, ge, tiles.tn, tiles.tk),
               _floor(xs, w, experts))
    for g, e in enumerate(experts):
        if e < 0:
            assert not got[g * 256:(g + 1) * 256].float().any()


def test_grouped_matmul_f32_operands():
    experts = [2, -1, 0, 9]
    g = torch.Generator().manual_seed(4)
    xs, w = torch.randn(1024, 512, generator=g), torch.randn(4, 512, 1024, generator=g) * 0.02
    ge = torch.tensor(experts, dtype=torch.int32)
    tiles = GroupTiles(512, 256)
    print(f"grouped matmul f32 experts={experts} {tiles}", flush=True)
    got = grouped_matmul(xs.cuda(), w.cuda(), ge.cuda(), tiles)
    torch.cuda.synchronize()
    want = torch.zeros(1024, 1024, dtype=torch.float64)
    for grp, e in enumerate(experts):
        if e >= 0:
            rows = slice(grp * 256, (grp + 1) * 256)
            want[rows] = xs[rows].double() @ w[min(e, 3)].double()
    diff = (got.double().cpu() - want).abs()
    assert not (diff > 1e-4 * want.abs() + 1e-4).any(), diff.max().item()


def test_device_step_tables_are_bit_exact():
    experts = [2, -1, 0, -1, 1, 1, -1, 3]
    xs, w, ge = _inputs(2048, 1024, 512, 4, experts)
    tiles = GroupTiles(512, 256)
    lowered = grouped_matmul.lower(xs, w, ge, tiles)
    got = lowered.program.step_tables(xs.cuda(), w.cuda(), ge.cuda())
    tiles_i = [{"i": 256 * g} for g in range(8)]
    step_tile, step_code, count = oracle_schedule.runtime_tables(
        tiles_i, [("k", 0, 256, 4, lambda v: experts[v["i"] // 256] < 0)])
    assert int(got["count"][0]) == count == 5 * 4 + 3
    np.testing.assert_array_equal(got["step_tile"].cpu().numpy(), step_tile)
    np.testing.assert_array_equal(got["step_code"].cpu().numpy(), step_code)
    starts = got["tile_steps"].cpu().numpy()
    assert starts[-1] == count and (np.diff(starts) >= 1).all()


def test_baseline_config_against_torch():
    """16384 tokens x 4096 -> 14336, 8 experts, groups of 256 with seeded multinomial
    counts, sorted by expert; every group checked against a float32 product on the GPU, to the 2-ulp bar
    (tests/tolerance.py: MATMUL_BAR)."""
    g = torch.Generator().manual_seed(0)
    counts = torch.multinomial(torch.full((8,), 1 / 8), 64, replacement=True, generator=g).bincount(minlength=8)
    ge = torch.repeat_interleave(torch.arange(8), counts).to(torch.int32)
    xs = torch.randn(16384, 4096, generator=g).to(torch.bfloat16).cuda()
    w = (torch.randn(8, 4096, 14336, generator=g) * 0.02).to(torch.bfloat16).cuda()
    print("grouped matmul 16384x4096x14336, 8 experts", flush=True)
    got = grouped_matmul(xs, w, ge.cuda(), GroupTiles(512, 512))
    torch.backends.cuda.matmul.allow_tf32 = False
    worst = 0.0
    for grp in range(64):
        e = int(ge[grp])
        rows = slice(grp * 256, (grp + 1) * 256)
        want = xs[rows].float() @ w[e].float()
        report = check_bf16(f"MoE group {grp} (expert {e})", got[rows], want.to(torch.bfloat16),
                            matmul_floor(xs[rows], w[e]), **MATMUL_BAR)
        worst = max(worst, report["bound_use"])
    print(f"MoE config 4: largest bound use over all 64 groups {worst:.3f}", flush=True)


def _ffn_floor(xs, wg, wu, wd, experts):
    """The expert layer's bound beyond 2 bf16 ulp, per output: the gate and up products' f32 summation floors
    carried through silu(g) * u (|silu'| <= 1.1), the rounding of the hidden activations to bf16 moving each by
    up to 2^-8 of itself (the kernel and the reference can round to either side), both through |w_down|, plus
    the down product's own f32 floor. Zero for unused tiles. All tensors on one device."""
    from tests.tolerance import P_ROUND

    M, D = xs.shape
    E = wg.shape[0]
    G = M // len(experts)
    floor = torch.zeros(M, D, device=xs.device)
    for t, e in enumerate(experts):
        if e < 0:
            continue
        e = min(e, E - 1)
        rows = xs[t * G:(t + 1) * G].float()
        gate, up = rows @ wg[e].float(), rows @ wu[e].float()
        hidden = (gate * torch.sigmoid(gate) * up).abs()
        moved = 1.1 * matmul_floor(rows, wg[e]) * up.abs() + gate.abs() * matmul_floor(rows, wu[e])
        floor[t * G:(t + 1) * G] = ((moved + 2 * P_ROUND * hidden) @ wd[e].float().abs()
                                    + matmul_floor(hidden.to(torch.bfloat16), wd[e]))
    return floor


def _ffn_inputs(M, D, F, E, seed, scale=1 / 16):
    g = torch.Generator().manual_seed(seed)
    xs = torch.randn(M, D, generator=g).to(torch.bfloat16)
    wg, wu = ((torch.randn(E, D, F, generator=g) * scale).to(torch.bfloat16) for _ in range(2))
    wd = (torch.randn(E, F, D, generator=g) * scale).to(torch.bfloat16)
    return xs, wg, wu, wd


@pytest.mark.parametrize("experts,block_f", [([0, 2, -1, 9], 128), ([1, 1, 0, -1], 512)])
def test_expert_ffn_matches_oracle(experts, block_f):
    """The reference's SwiGLU layer with runtime expert windows (examples/moe.py:167-187), lowered as a chain
    of two matmul-family kernels (codegen/chain.py): the gate kernel (gate and up products of one xs slice,
    silu(g) * u in registers, stored as bf16 hidden activations) and the down kernel (the grouped product
    with w_down under the original mask). Bar: 2 bf16 ulp of the oracle plus `_ffn_floor`, within 3e-2 of the
    float64 layer's largest output, and zeros for unused tiles."""
    from examples.moe import ExpertTiles, expert_ffn

    M, D, F, E = 512, 256, 512, 4
    xs, wg, wu, wd = _ffn_inputs(M, D, F, E, 11)
    te = torch.tensor(experts, dtype=torch.int32)
    tiles = ExpertTiles(block_f=block_f)
    lowered = expert_ffn.lower(xs, wg, wu, wd, te, tiles)
    notes = lowered.program.notes
    assert notes["family"] == "gemm" and notes["chain"] and notes["products"] == 2
    print(f"expert_ffn experts={experts} {tiles}", flush=True)
    got = lowered.run(xs.cuda(), wg.cuda(), wu.cuda(), wd.cuda(), te.cuda())
    torch.cuda.synchronize()
    want = kernels.expert_ffn(xs, wg, wu, wd, te, block_f)
    check_bf16(f"expert_ffn experts={experts}", got.cpu(), want, _ffn_floor(xs, wg, wu, wd, experts))
    exact = torch.as_tensor(kernels.expert_ffn_float64(xs, wg, wu, wd, te))
    assert (got.cpu().double() - exact).abs().max().item() < 3e-2 * exact.abs().max().item()
    G = M // len(experts)
    for t, e in enumerate(experts):
        if e < 0:
            assert not got[t * G:(t + 1) * G].float().any()


def test_expert_ffn_step_tables_pin_the_steps():
    """The program's step tables are the down kernel's, which are the original nest's (the reference's
    tests/test_moe.py:277-283): one step per hidden block of each tile whose expert is used, and one empty
    step per unused tile, bit-exact against the reference's table semantics (oracle/schedule.py)."""
    from examples.moe import ExpertTiles, expert_ffn

    experts = [2, -1, 0, -1, 1, 1, -1, 3]
    M, D, F, E, bf = 1024, 256, 512, 4, 128
    xs, wg, wu, wd = _ffn_inputs(M, D, F, E, 12)
    te = torch.tensor(experts, dtype=torch.int32)
    lowered = expert_ffn.lower(xs, wg, wu, wd, te, ExpertTiles(block_f=bf))
    print("expert_ffn step tables, 8 tiles", flush=True)
    got = lowered.program.step_tables(xs.cuda(), wg.cuda(), wu.cuda(), wd.cuda(), te.cuda())
    G, nf = M // len(experts), F // bf
    step_tile, step_code, count = oracle_schedule.runtime_tables(
        [{"i": G * t} for t in range(len(experts))], [("f", 0, bf, nf, lambda v: experts[v["i"] // G] < 0)])
    used = sum(1 for e in experts if e >= 0)
    assert int(got["count"][0]) == count == nf * used + (len(experts) - used)
    np.testing.assert_array_equal(got["step_tile"].cpu().numpy(), step_tile)
    np.testing.assert_array_equal(got["step_code"].cpu().numpy(), step_code)
    full = (got["step_code"].cpu().numpy()[:count] & 4) == 0  # the steps that compute
    assert int(full.sum()) == nf * used
    assert {experts[int(t)] for t in got["step_tile"].cpu().numpy()[:count][full]} == {e for e in experts if e >= 0}


def test_expert_ffn_mixtral_width():
    """The expert layer at Mixtral 8x7B's width (the bench's expert_ffn leg): 16384 routed rows in 64 tiles of
    256, D = 4096, F = 14336, 8 experts, each tile's expert drawn at random and two tiles unused. Eight tiles
    (the unused ones among them) are checked against a float32 GPU reference of the spec (h rounded to bf16
    as the spec rounds it), with the same bar as the small cases."""
    from examples.moe import ExpertTiles, expert_ffn

    M, D, F, E, G = 16384, 4096, 14336, 8, 256
    g = torch.Generator().manual_seed(13)
    experts = torch.randint(0, E, (M // G,), generator=g)
    experts[[5, 40]] = -1
    xs = torch.randn(M, D, generator=g).to(torch.bfloat16).cuda()
    wg, wu = ((torch.randn(E, D, F, generator=g) * 0.02).to(torch.bfloat16).cuda() for _ in range(2))
    wd = (torch.randn(E, F, D, generator=g) * 0.02).to(torch.bfloat16).cuda()
    te = experts.to(torch.int32).cuda()
    print("expert_ffn 16384 x 4096 x 14336, 8 experts", flush=True)
    got = expert_ffn(xs, wg, wu, wd, te, ExpertTiles(block_f=256))
    torch.cuda.synchronize()
    torch.backends.cuda.matmul.allow_tf32 = False
    for t in (0, 5, 17, 31, 40, 41, 62, 63):
        rows = slice(t * G, (t + 1) * G)
        e = int(experts[t])
        if e < 0:
            assert not got[rows].float().any(), t
            continue
        x = xs[rows].float()
        gate, up = x @ wg[e].float(), x @ wu[e].float()
        h = (gate * torch.sigmoid(gate) * up).to(torch.bfloat16)
        want = (h.float() @ wd[e].float()).to(torch.bfloat16)
        floor = _ffn_floor(xs[rows], wg[e:e + 1], wu[e:e + 1], wd[e:e + 1], [0])
        check_bf16(f"expert_ffn Mixtral width, tile {t} (expert {e})", got[rows].cpu(), want.cpu(), floor.cpu())
