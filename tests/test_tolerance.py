"""The parity bar itself (tests/tolerance.py), on the CPU: bf16 ulps are what the format says, a correct
evaluation in another summation order passes, and plausible mistakes fail."""

import pytest
import torch

from oracle import kernels
from tests.tolerance import MATMUL_BAR, SOFTMAX_BAR, bf16_ulp, check_bf16, matmul_floor, score_err, softmax_floor


def test_bf16_ulp_is_the_spacing_of_bf16_values():
    w = torch.tensor([1.0, 1.5, 255.0, 256.0, -3.0, 2.0 ** -20])
    want = torch.tensor([2.0 ** -7, 2.0 ** -7, 1.0, 2.0, 2.0 ** -6, 2.0 ** -27], dtype=torch.float64)
    assert torch.equal(bf16_ulp(w), want)
    # the next bf16 value above w is w + ulp
    for v in (1.0, 3.0, 100.0, 0.0078125):
        t = torch.tensor([v], dtype=torch.bfloat16)
        nxt = (t.view(torch.int16) + 1).view(torch.bfloat16)  # the next bf16 value up (one more in the bits)
        assert float(nxt) - v == float(bf16_ulp(t.float()))


def _mm(m, k, n, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(m, k, generator=g).to(torch.bfloat16), torch.randn(k, n, generator=g).to(torch.bfloat16)


def test_matmul_in_another_order_passes():
    x, y = _mm(256, 1024, 256, 0)
    want = kernels.matmul(x, y, 256, 256, 256)
    other = (x.double() @ y.double()).to(torch.bfloat16)  # exact sum, then rounded
    report = check_bf16("matmul vs float64", other, want, matmul_floor(x, y))
    assert report["ulp_max_typical"] <= 1.0 and report["within_2ulp"] == 1.0


def test_matmul_dropped_step_fails():
    x, y = _mm(256, 1024, 256, 1)
    want = kernels.matmul(x, y, 256, 256, 256)
    dropped = (x[:, 256:].float() @ y[256:].float()).to(torch.bfloat16)  # the first k block left out
    with pytest.raises(AssertionError):
        check_bf16("dropped step", dropped, want, matmul_floor(x, y))


def test_matmul_transposed_operand_fails():
    x, y = _mm(256, 256, 256, 2)
    want = kernels.matmul(x, y, 128, 128, 128)
    with pytest.raises(AssertionError):
        check_bf16("transposed", (x.float() @ y.float().T).to(torch.bfloat16), want, matmul_floor(x, y))


def test_matmul_floor_is_not_loose_enough_to_hide_a_1_percent_error():
    x, y = _mm(256, 512, 256, 3)
    want = kernels.matmul(x, y, 256, 256, 256)
    with pytest.raises(AssertionError):
        check_bf16("scaled", (want.float() * 1.01).to(torch.bfloat16), want, matmul_floor(x, y))


def test_strict_bar_catches_a_1_percent_error_at_k_8192():
    """At K = 8192 (BASELINE config 2's depth) the worst-case floor alone admits a 1 % scale error on every
    output; the 2-ulp bar on typical outputs and the 99.99 % share within 2 ulp do not. A correct evaluation
    in another summation order passes all three."""
    x, y = _mm(64, 8192, 128, 5)
    want = kernels.matmul(x, y, 64, 128, 512)
    floor = matmul_floor(x, y)
    scaled = (want.float() * 1.01).to(torch.bfloat16)
    check_bf16("1 % scaled, floor only", scaled, want, floor)  # the floor by itself is this loose
    with pytest.raises(AssertionError, match="typical size"):
        check_bf16("1 % scaled", scaled, want, floor, **MATMUL_BAR)
    with pytest.raises(AssertionError, match="within 2 bf16 ulp"):
        check_bf16("1 % scaled", scaled, want, floor, min_within=MATMUL_BAR["min_within"])
    other = (x.double() @ y.double()).to(torch.bfloat16)
    report = check_bf16("K 8192 vs float64", other, want, floor, **MATMUL_BAR)
    assert report["ulp_max_typical"] <= 1.0


def _attn(seed, S=256):
    gens = [torch.Generator().manual_seed(seed + i) for i in range(3)]
    q, k, v = (torch.randn(1, 2, S, 128, generator=g).to(torch.bfloat16) for g in gens)
    return (q.float() * 128 ** -0.5).to(torch.bfloat16), k, v


def test_attention_other_blocking_passes():
    """The spec at two block shapes rounds p against different running maxima: within the softmax floor."""
    q, k, v = _attn(0)
    a = kernels.causal_attention(q, k, v, 128, 128)
    b = kernels.causal_attention(q, k, v, 64, 32)
    weighted = torch.as_tensor(kernels.attention_float64(q, k, v.float().abs()))
    check_bf16("attention blockings", a, b, softmax_floor(weighted, 256, score_err(q, k)))
    check_bf16("attention vs float64", a, kernels.attention_float64(q, k, v),
               softmax_floor(weighted, 256, score_err(q, k)))
    check_bf16("attention blockings, 2-ulp bar", a, b, softmax_floor(weighted, 256, score_err(q, k)),
               **SOFTMAX_BAR)


def test_softmax_bar_catches_a_1_percent_error():
    """The softmax bar (typical outputs within 2 ulp) fails a 1 % scale error the floor alone admits."""
    q, k, v = _attn(2, S=512)
    want = kernels.causal_attention(q, k, v, 128, 128)
    weighted = torch.as_tensor(kernels.attention_float64(q, k, v.float().abs()))
    floor = softmax_floor(weighted, 512, score_err(q, k))
    scaled = (want.float() * 1.01).to(torch.bfloat16)
    with pytest.raises(AssertionError):
        check_bf16("attention 1 % scaled", scaled, want, floor, **SOFTMAX_BAR)


def test_attention_off_by_one_mask_fails():
    """Letting each row see one key in its future moves the output far beyond the floor."""
    q, k, v = _attn(4)
    S = q.shape[2]
    s = q.double() @ k.double().transpose(-1, -2)
    mask = torch.ones(S, S, dtype=torch.bool).tril(1)
    wrong = torch.softmax(s.masked_fill(~mask, float("-inf")), -1) @ v.double()
    weighted = torch.as_tensor(kernels.attention_float64(q, k, v.float().abs()))
    with pytest.raises(AssertionError):
        check_bf16("future key", wrong.to(torch.bfloat16), kernels.attention_float64(q, k, v),
                   softmax_floor(weighted, S, score_err(q, k)))
