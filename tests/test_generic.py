"""Nests no kernel family takes, on the CPU: they lower to the generic kernel (one persistent kernel that
evaluates the traced tile code per tile), the plan facts the reference pins for them hold, the
reference interpreter agrees with the oracle, and the oracle's attention_block with float64."""

import numpy as np
import pytest
import torch

from examples.attention_block import BlockTiles, attention_block
from oracle import kernels
from tests.helpers import make_kernel, spec
from tilejax_amd import jaxlite

BF = jaxlite.bfloat16


def _block_inputs(B=1, H=2, S=512, Dh=128, F=512, seed=0, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    D = H * Dh
    q = (torch.randn(B, H, S, Dh, generator=g) * Dh ** -0.5).to(dtype)
    k, v = torch.randn(B, H, S, Dh, generator=g).to(dtype), torch.randn(B, H, S, Dh, generator=g).to(dtype)
    gamma = (1 + 0.1 * torch.randn(1, D, generator=g)).to(dtype)
    w_up = (torch.randn(D, F, generator=g) / D ** 0.5).to(dtype)
    w_down = (torch.randn(F, D, generator=g) / F ** 0.5).to(dtype)
    return q, k, v, gamma, w_up, w_down


@pytest.mark.parametrize("block_q, block_kv", [(128, 128), (256, 128)])
def test_attention_block_plan_facts(block_q, block_kv):
    """The reference's tests/test_examples.py:180-198: operand kinds and the step count, the one-step
    feed-forward loop joining the tile code (block_f covers F)."""
    specs = (spec(1, 2, 512, 128, dtype=BF),) * 3 + (spec(1, 256, dtype=BF), spec(256, 512, dtype=BF),
                                                    spec(512, 256, dtype=BF))
    lowered = attention_block.lower(*specs, BlockTiles(block_q=block_q, block_kv=block_kv))
    assert {op.name: op.kind.value for op in lowered.plan.operands} == {
        "q": "tile", "k": "stream", "v": "stream", "gamma": "once", "w_up": "once", "w_down": "once"}
    assert lowered.steps == sum(i // block_kv + 1 for i in range(block_q - 1, 512, block_q))
    assert lowered.program.notes["family"] == "generic"


def test_oracle_attention_block_against_float64():
    """The oracle's restatement (p and the normalized rows rounded to bf16 as the spec rounds them) against
    the float64 block within the reference's own bound, atol 3e-2 of the largest |want|; the same block
    with the causal mask left out is far outside it."""
    ins = _block_inputs()
    got = kernels.attention_block(*ins, bq=128, bk=128, bf=512).double()
    want = torch.as_tensor(kernels.attention_block_float64(*ins))
    scale = want.abs().max().item()
    assert (got - want).abs().max().item() < 3e-2 * scale
    q, k, v = ins[:3]
    s = q.double() @ k.double().transpose(-1, -2)
    leaky = (torch.softmax(s, -1) @ v.double()).permute(0, 2, 1, 3).reshape(1, 512, 256)  # no mask
    a = torch.as_tensor(kernels.attention_float64(*ins[:3])).permute(0, 2, 1, 3).reshape(1, 512, 256)
    assert (leaky - a).abs().max().item() > 0.1  # the planted mistake moves the attention output itself


def test_reference_interpreter_on_attention_block():
    ins = _block_inputs(S=256, F=256, seed=3)
    tiles = BlockTiles(block_q=128, block_kv=64, block_f=128)
    got = attention_block.reference(*ins, tiles)
    want = kernels.attention_block(*ins, bq=128, bk=64, bf=128)
    assert (got.float() - want.float()).abs().max().item() <= 2.0 ** -6 * want.float().abs().max().item()


MASKED_PHASES = """
def masked_phases(x, w):
    out = jnp.zeros((256, 128))
    for i in range(0, 256, 128):
        a = jnp.zeros((128, 128))
        for k in range(0, 384, 128):
            if k > i:
                continue
            y = x[i : i + 128, k : k + 128]
            a += y
        y = y * 2
        a = a + y
        t = a * 0
        for c in range(0, 128, 128):
            t = t + w[c : c + 128, :]
        b = jnp.zeros((128, 128))
        for k2 in range(0, 256, 128):
            if k2 > i:
                continue
            b += x[i : i + 128, k2 : k2 + 128] @ w[0:128, :]
        b = b * 3
        out = out.at[i : i + 128, :].set(a + b + t)
    return out
"""


def masked_phases_float64(x, w):
    """The reference's tests/test_codegen.py:626-634 closed form of MASKED_PHASES."""
    xf, wf = x.double(), w.double()
    out = torch.zeros(256, 128, dtype=torch.float64)
    for i in (0, 1):
        rows = xf[i * 128:(i + 1) * 128]
        a = sum(rows[:, k * 128:(k + 1) * 128] for k in range(i + 1))
        a = a + 2 * rows[:, i * 128:(i + 1) * 128]
        b = 3 * sum(rows[:, k * 128:(k + 1) * 128] @ wf for k in range(i + 1))
        out[i * 128:(i + 1) * 128] = a + b + (a * 0 + wf)
    return out


def test_masked_phases_schedule():
    """The reference's tests/test_codegen.py:636-649: two masked phases, a loop of one iteration inline, and
    the exact step list."""
    k = make_kernel(MASKED_PHASES)
    x, w = spec(256, 384), spec(128, 128)
    lowered = k.lower(x, w)
    sch = lowered.schedule
    assert [p.range.var for p in lowered.plan.phases] == ["k", "k2"] and sch.step_tables
    assert sch.steps == 2 + 4 and sch.phase_steps == (3, 3)
    assert [sch.step_at(s) for s in range(sch.steps)] == [(0, 0, 0), (0, 1, 0), (1, 0, 0), (1, 0, 1), (1, 1, 0),
                                                          (1, 1, 1)]
    assert lowered.program.notes["family"] == "generic"


def test_masked_phases_reference_against_closed_form():
    k = make_kernel(MASKED_PHASES)
    g = torch.Generator().manual_seed(1)
    x, w = torch.randn(256, 384, generator=g), torch.randn(128, 128, generator=g) / 8
    got = k.reference(x, w)
    np.testing.assert_allclose(got.double().numpy(), masked_phases_float64(x, w).numpy(), rtol=1e-4, atol=1e-4)
