"""What the gfx950 lowering builds for a loop nest, checked on the CPU (no kernel runs): the passes and
workspaces f32 operands and one-step reductions take, and the error for what isn't lowered."""

import pytest

from examples.causal_attention import AttentionBlocks, causal_attention
from examples.matmul import MatmulTiles, matmul
from examples.rmsnorm_matmul import NormMatmulTiles, rmsnorm_matmul
from tilejax_amd import jaxlite
from tilejax_amd.errors import KernelError

F32, BF16 = jaxlite.float32, jaxlite.bfloat16


def _symbols(lowered):
    return [launch.symbol for launch in lowered.program.launches]


def test_f32_operands_take_their_bf16_parts():
    lowered = matmul.lower(((256, 384), F32), ((384, 256), F32), MatmulTiles(128, 128, 128))
    prog = lowered.program
    assert prog.notes["f32_operands"]
    assert _symbols(lowered)[:3] == ["tj_matmul_parts_b", "tj_matmul_parts_a", "tj_matmul"]
    # six bf16 slices for each of the operand's: 2 bytes x 6 per element
    assert prog.workspace["x3_a"] == 12 * 256 * 384 and prog.workspace["x3_b"] == 12 * 384 * 256
    # three reduction steps of 128: 2 slices of 64 each, so 12 slices of the parts per step
    assert prog.notes["slices_per_step"] == 12


def test_bf16_operands_read_the_arrays_themselves():
    lowered = matmul.lower(((256, 384), BF16), ((384, 256), BF16), MatmulTiles(128, 128, 128))
    assert not lowered.program.notes["f32_operands"]
    assert _symbols(lowered) == ["tj_matmul"] and not lowered.program.workspace


def test_one_reduction_step_is_lowered():
    """tk = K: the loop of one step joins the tile code (its variable bound to its start), nothing is
    carried, and the lowering reads the k window at that value."""
    lowered = matmul.lower(((256, 384), BF16), ((384, 256), BF16), MatmulTiles(256, 128, 512))
    assert not lowered.plan.carried and not lowered.plan.phases
    assert _symbols(lowered) == ["tj_matmul"]


def test_one_step_rmsnorm_sums_rows_in_the_row_pass():
    lowered = rmsnorm_matmul.lower(((256, 512), BF16), ((1, 512), BF16), ((512, 512), BF16),
                                   NormMatmulTiles(128, 256, 512))
    assert not lowered.plan.carried
    assert _symbols(lowered)[:2] == ["tj_rmsnorm_matmul_rows", "tj_rmsnorm_matmul"]
    sums = [k for k in lowered.program.workspace if k.startswith("rn__sum")]
    assert len(sums) == 1 and lowered.program.workspace[sums[0]] == 4 * 256


def test_f32_rmsnorm_writes_the_left_operands_parts_in_its_row_pass():
    lowered = rmsnorm_matmul.lower(((256, 512), F32), ((1, 512), F32), ((512, 512), F32),
                                   NormMatmulTiles(128, 128, 128))
    assert _symbols(lowered)[:3] == ["tj_rmsnorm_matmul_rows", "tj_rmsnorm_matmul_parts_b", "tj_rmsnorm_matmul"]
    assert lowered.program.workspace["rn_a"] == 12 * 256 * 512 and "x3_a" not in lowered.program.workspace


def test_f32_attention_runs_on_the_vector_alus():
    spec = ((1, 1, 256, 128), F32)
    lowered = causal_attention.lower(spec, spec, spec, AttentionBlocks(128, 128))
    assert lowered.program.notes["f32_operands"] and "mfma" not in lowered.source
    assert _symbols(lowered) == ["tj_causal_attention"]


def test_what_no_family_takes_lowers_to_the_generic_kernel():
    from tests.helpers import make_kernel

    k = make_kernel('''
        def row_sums(x):
            M, N = x.shape
            out = jnp.zeros((M, 128), jnp.float32)
            for i in range(0, M, 128):
                acc = jnp.zeros((128, 128), jnp.float32)
                for j in range(0, N, 128):
                    acc += x[i : i + 128, j : j + 128]
                out = out.at[i : i + 128, :].set(acc)
            return out
    ''')
    lowered = k.lower(((256, 512), F32))  # no family takes it: the generic kernel does
    assert lowered.program.notes["family"] == "generic"


def test_two_reduction_loops_lower_to_a_row_pass_and_the_matmul():
    from tests.test_gpu_rmsnorm_matmul import TWO_PASS
    from tests.helpers import make_kernel

    k = make_kernel(TWO_PASS)
    lowered = k.lower(((256, 384), F32), ((384, 256), F32))
    assert _symbols(lowered)[:3] == ["tj_two_pass_rows", "tj_two_pass_parts_b", "tj_two_pass"]
    assert "ps_0 = ak_wave_sum(ps_0)" in lowered.source and "st_0" in lowered.source


def test_a_first_loop_over_another_array_lowers_to_the_generic_kernel():
    from tests.helpers import make_kernel
    from tests.test_gpu_rmsnorm_matmul import TWO_PASS

    other = TWO_PASS.replace("def two_pass(x, w):", "def two_pass(x, z, w):").replace(
        "xk = x[i : i + 128, k : k + 128]", "xk = z[i : i + 128, k : k + 128]")
    k = make_kernel(other)
    lowered = k.lower(((256, 384), F32), ((256, 384), F32), ((384, 256), F32))  # the generic kernel takes it
    assert lowered.program.notes["family"] == "generic"


def test_the_f32_part_pairs_give_products_to_f32_accuracy():
    """The slices F32_PARTS lays out, multiplied pairwise as the kernel's MFMAs do, give each product of
    f32 operands to within a few 2^-24 (three bf16 parts each, split as ak_split3 does: each part the bf16
    rounding of what the earlier parts leave). A table that dropped a pair or doubled one would be off by
    2^-16 or more."""
    import torch

    from tilejax_amd.codegen.gemm import F32_PARTS

    def split3(x):
        p1 = x.bfloat16().float()
        p2 = (x - p1).bfloat16().float()
        p3 = (x - p1 - p2).bfloat16().float()
        return {1: p1, 2: p2, 3: p3}

    g = torch.Generator().manual_seed(0)
    a = torch.randn(100000, generator=g) * torch.exp(torch.randn(100000, generator=g) * 4)
    b = torch.randn(100000, generator=g) * torch.exp(torch.randn(100000, generator=g) * 4)
    pa, pb = split3(a), split3(b)
    assert len(F32_PARTS["a"]) == len(F32_PARTS["b"]) == 6
    got = sum(pa[i].double() * pb[j].double() for i, j in zip(F32_PARTS["a"], F32_PARTS["b"]))
    exact = a.double() * b.double()
    rel = ((got - exact).abs() / exact.abs()).max().item()
    assert rel < 8 * 2.0**-24, rel
