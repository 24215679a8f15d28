"""The feed-forward chain on the CPU (tilejax_amd/codegen/chain.py): which nests it takes, the two nests it
writes (their references, run eagerly, compose to the original's), the matmul family's form of both kernels
(two right operands for the gate kernel), their LDS ring protocols, and a gfx950 build."""

import pytest
import torch

import tilejax_amd
from examples.moe import ExpertTiles, expert_ffn
from tests.helpers import make_kernel, rand
from tilejax_amd import runtime
from tilejax_amd.codegen import chain, gemm
from tilejax_amd.codegen.protocol import check


def _ffn_args(M=512, D=256, F=512, E=4, experts=(0, 2, -1, 1), seed=0):
    xs = rand((M, D), seed, torch.bfloat16)
    wg, wu = (rand((E, D, F), seed + k, torch.bfloat16) / 16 for k in (1, 2))
    wd = rand((E, F, D), seed + 3, torch.bfloat16) / 16
    return xs, wg, wu, wd, torch.tensor(experts, dtype=torch.int32)


def _plan(kernel, *args, tunable=None):
    sig = kernel.signature(*args)
    return kernel.build(sig, tunable if tunable is not None else kernel.default_config(sig).tunable)


def test_expert_ffn_is_a_chain_of_two_matmul_kernels():
    args = _ffn_args()
    lowered = expert_ffn.lower(*args, ExpertTiles(128))
    prog = lowered.program
    notes = prog.notes
    assert notes["family"] == "gemm" and notes["chain"] and notes["products"] == 2
    gate, down = prog.parts
    # the gate kernel holds both weights' slices in LDS: its workgroup tile is BN columns of each
    assert gate.notes["hw_tile"][1] == 128 and "ak_h" in prog.workspace
    assert [l.symbol for l in prog.launches] == ["tj_expert_ffn_gate_steps", "tj_expert_ffn_gate",
                                                 "tj_expert_ffn_down_steps", "tj_expert_ffn_down"]
    assert prog.workspace["ak_h"] == 512 * 512 * 2  # (rows, F) bf16
    # the gate kernel writes h (its output is the workspace), the down kernel reads it as its first input
    gate_args = {a.name: a for a in prog.launches[1].args}
    down_args = {a.name: a for a in prog.launches[3].args}
    assert gate_args["ak_h_out"].kind == "workspace" and gate_args["ak_h_out"].key == "ak_h"
    assert down_args["ak_h"].kind == "workspace" and down_args["ak_h"].key == "ak_h"
    assert down_args["out_out"].kind == "output"
    # the program's step tables are the down kernel's (the original nest's), the gate's prefixed
    assert notes["step_builder"] == "tj_expert_ffn_down_steps" and "g_step_code" in prog.workspace
    runtime.compile_source(prog.source, f"{prog.name}.hip")


@pytest.mark.parametrize("block_f", [128, 512])
def test_the_two_nests_compose_to_the_original(block_f):
    """The gate nest's reference then the down nest's (run eagerly on the CPU, as the spec runs) give the
    original nest's reference: the same arithmetic, only the f32 sums of the gate and up products taken in
    slices of the feature dim (so h may round to the other side of a bf16 value now and then)."""
    args = _ffn_args(experts=(0, 2, -1, 9))
    tiles = ExpertTiles(block_f)
    plan, _ = _plan(expert_ffn, *args, tunable=tiles)
    c = chain.match(plan)
    assert c is not None and c.products == 2 and c.h_shape == (512, 512)
    gate = tilejax_amd.kernel(chain._function(c.gate_source, c.gate_name, plan))
    down = tilejax_amd.kernel(chain._function(c.down_source, c.down_name, plan))
    h = gate.reference(*args, tiles)
    got = down.reference(h, *args, tiles).float()
    want = expert_ffn.reference(*args, tiles).float()
    scale = want.abs().max().item()
    assert (got - want).abs().max().item() <= 1e-2 * scale
    assert torch.equal(got[256:384], torch.zeros_like(got[256:384]))  # the unused tile stays zero


def test_the_gate_nest_matches_with_two_right_operands():
    args = _ffn_args()
    plan, _ = _plan(expert_ffn, *args, tunable=ExpertTiles(256))
    c = chain.match(plan)
    gplan, _ = chain._plan(c.gate_source, c.gate_name, plan, list(plan.inputs))
    m = gemm.match(gplan)
    assert m is not None and m.b2 is not None and m.acc2 is not None
    assert (m.b.tile.array, m.b2.tile.array) == ("w_gate", "w_up")  # in the carried values' name order
    hw = gemm.hardware_tile(m, tilejax_amd.Pipeline(2, 2))
    assert hw.dual and hw.bn_lds == 2 * hw.bn and hw.lds == hw.stages * (hw.bm + 2 * hw.bn) * hw.bk * 2


def test_the_chain_source_is_the_same_every_time():
    args = _ffn_args()
    a = expert_ffn.lower(*args, ExpertTiles(256)).program.source
    plan, _ = _plan(expert_ffn, *args, tunable=ExpertTiles(256))
    b = chain.lower(plan, _plan(expert_ffn, *args, tunable=ExpertTiles(256))[1], tilejax_amd.Pipeline(2, 2),
                    chain.match(plan), "tj_expert_ffn").source
    assert a == b


@pytest.mark.parametrize("rounds", [1, 2, 3])
def test_both_kernels_keep_the_lds_ring_protocol(rounds):
    prog = expert_ffn.lower(*_ffn_args(), ExpertTiles(256)).program
    for part in prog.parts:
        T = rounds * part.notes["stages"]
        for counts in ([T], [T, 0, 2 * T], [0, T, T]):
            check(part.protocol.replay(counts), f"{part.name}, items of {counts} slices")


DENSE_SWIGLU = """
def swiglu(x, w1, w2, w3):
    M, D = x.shape
    F = w1.shape[1]
    dtype = x.dtype
    out = jnp.zeros((M, D), dtype)
    for i in range(0, M, 256):
        acc = jnp.zeros((256, D), jnp.float32)
        for f in range(0, F, 256):
            h = jax.nn.silu(x[i : i + 256, :] @ w1[:, f : f + 256]) * (x[i : i + 256, :] @ w2[:, f : f + 256])
            acc += h.astype(dtype) @ w3[f : f + 256, :]
        out = out.at[i : i + 256, :].set(acc.astype(dtype))
    return out
"""

GELU_FFN = """
def gelu_ffn(x, w1, w2):
    M, D = x.shape
    F = w1.shape[1]
    dtype = x.dtype
    out = jnp.zeros((M, D), dtype)
    for i in range(0, M, 128):
        acc = jnp.zeros((128, D), jnp.float32)
        for f in range(0, F, 256):
            xt = x[i : i + 128, :]
            acc += jax.nn.gelu(xt @ w1[:, f : f + 256]).astype(dtype) @ w2[f : f + 256, :]
        out = out.at[i : i + 128, :].set(acc.astype(dtype))
    return out
"""


def test_a_dense_swiglu_written_inline_is_a_chain():
    kernel = make_kernel(DENSE_SWIGLU)
    x = rand((512, 256), 1, torch.bfloat16)
    w1, w2 = rand((256, 512), 2, torch.bfloat16) / 16, rand((256, 512), 3, torch.bfloat16) / 16
    w3 = rand((512, 256), 4, torch.bfloat16) / 16
    prog = kernel.lower(x, w1, w2, w3).program
    assert prog.notes["chain"] and prog.notes["products"] == 2
    assert "ak_step" not in prog.source  # no masks: no step tables
    runtime.compile_source(prog.source, f"{prog.name}.hip")


def test_one_product_is_a_chain_with_one_right_operand():
    kernel = make_kernel(GELU_FFN)
    x = rand((256, 256), 1, torch.bfloat16)
    w1, w2 = rand((256, 512), 2, torch.bfloat16) / 16, rand((512, 256), 3, torch.bfloat16) / 16
    prog = kernel.lower(x, w1, w2).program
    assert prog.notes["chain"] and prog.notes["products"] == 1
    gate, _ = prog.parts
    assert not gate.notes["dual"] and "rsb2" not in gate.source
    runtime.compile_source(prog.source, f"{prog.name}.hip")


@pytest.mark.parametrize("body", [
    # the activation reads the left window pointwise too: not a chain
    "xt = x[i : i + 128, :]\n            acc += ((xt @ w1[:, f : f + 256]) * jnp.sum(xt, axis=1, keepdims=True))"
    ".astype(dtype) @ w2[f : f + 256, :]",
    # the products' hidden block isn't the down weights' block
    "acc += (x[i : i + 128, :] @ w1[:, 0 : 256]).astype(dtype) @ w2[f : f + 256, :]",
])
def test_nests_the_chain_does_not_take(body):
    source = GELU_FFN.replace(
        "xt = x[i : i + 128, :]\n            acc += jax.nn.gelu(xt @ w1[:, f : f + 256]).astype(dtype) @ w2[f : f + 256, :]",
        body)
    assert source != GELU_FFN
    kernel = make_kernel(source)
    x = rand((256, 256), 1, torch.bfloat16)
    w1, w2 = rand((256, 512), 2, torch.bfloat16), rand((512, 256), 3, torch.bfloat16)
    plan, _ = _plan(kernel, x, w1, w2)
    assert chain.match(plan) is None
