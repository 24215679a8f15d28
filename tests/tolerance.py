"""The parity bar for bf16 outputs: within 2 bf16 ulp of the expected value, plus a floor that bounds
what the two computations may legitimately differ by before their final rounding to bf16.

Why a floor at all: the kernel and its oracle are two evaluations of one loop nest that differ in f32
summation order (and, for softmax kernels, in which running maximum each p is rounded to bf16 against).
Each rounds its own f32 result to bf16, so two outputs can be 1 ulp apart from rounding alone, and
where the f32 results themselves differ by d, the bf16 outputs differ by at most d + 1 ulp. The floor
is a bound on d, derived per kind of computation:

- a dot product of K terms summed in f32 in any order is within K * 2^-24 * sum|x_i y_i| of the exact
  value (the standard worst-case bound of recursive summation, gamma_K ~ K u); two such evaluations are
  within twice that of each other: `matmul_floor`.
- a softmax-weighted sum whose weights p_j are rounded to bf16 (the spec's `p.astype(bf16) @ v`) moves by
  at most 2^-9 * sum_j p_j |v_j| / sum_j p_j per evaluation (each p_j within 2^-9 relative of exact);
  two evaluations that round against different running maxima are within 2^-8 of that weighted |v|
  average of each other: `softmax_floor`.

Every check also reports how close it came: the largest error in bf16 ulps over outputs of at least
typical size (|want| >= rms(want)), the share of all outputs within 2 ulp with no floor at all, and the
largest |got - want| / bound (<= 1 passes).

The floor is a worst-case bound, and at large K it is loose: at K = 8192 with N(0, 1) operands it is about
5 against 2 ulp of about 1 for a typical output of 90, so a scale error of a few percent would pass it.
The checks of the BASELINE configurations therefore
also assert the 2-ulp bar directly, on what the floor leaves open:
- matmul family (`MATMUL_BAR`): every output of typical size within 2 ulp (`typical_ulps`), and at least
  99.99 % of all outputs within 2 ulp with no floor at all (`min_within`);
- softmax kernels (`SOFTMAX_BAR`), against the oracle that rounds p as the spec does: at least 99.95 % of the
  outputs of typical size within 2 ulp (`typical_within`), none beyond 4, and at least 85 % of all outputs
  within 2 ulp with no floor. The kernel rounds each p to bf16 against its own running maximum (attention
  rescales per 64-key block and lazily; decode splits a sequence over workgroups, each starting its own
  maximum), the spec against its block's, so the two round each p independently: an output's two
  evaluations then differ by a sum of independent roundings, about 2^-9 * sqrt(2/3) of the output's own
  spread in standard deviation, plus each side's final rounding. Over the 8.4 million outputs of an
  attention config (0.99998 of the typical ones within 2 ulp, the largest 3) and the 262 thousand of the
  decode config (0.99983, the largest 4) the tail of that sum passes 2 ulp for a few; outputs much smaller
  than the weighted |v| average (cancellation) differ by more than 2 of their own ulps, which is what the
  floor admits.

Two bf16 ulp is about 1 % (2^-7 to 2^-8 relative), so a 1 % scale error still leaves most outputs within 2
ulp once both sides are rounded to bf16: what tells it apart is the share within 2 ulp (about 98 % of the
outputs of typical size for a 1 % error, against at least 99.98 % for the kernels), which the bars assert.
"""

from __future__ import annotations

from typing import Any, Dict, Optional

import torch

U32 = 2.0 ** -24  # f32 unit roundoff
P_ROUND = 2.0 ** -8  # two bf16 roundings of one value (each within 2^-9 relative) are within this of each other
ULPS = 2.0
MATMUL_BAR = {"typical_ulps": 2.0, "min_within": 0.9999}
SOFTMAX_BAR = {"typical_ulps": 4.0, "typical_within": 0.9995, "min_within": 0.85}


def bf16_ulp(w: torch.Tensor) -> torch.Tensor:
    """The spacing of bf16 values at |w| (8 significant bits): 2^(floor(log2|w|) - 7); subnormals and zero take
    the smallest normal's."""
    a = w.abs().double().clamp(min=2.0 ** -126)
    return torch.exp2(torch.floor(torch.log2(a)) - 7)


def check_bf16(what: str, got: Any, want: Any, floor: Any = 0.0, ulps: float = ULPS,
               chunk_rows: int = 1024, typical_ulps: Optional[float] = None,
               min_within: Optional[float] = None, typical_within: Optional[float] = None) -> Dict[str, float]:
    """Assert |got - want| <= ulps * ulp_bf16(want) + floor elementwise (floor: a tensor broadcastable to want,
    or a number); return the report (see the module docstring). With `typical_ulps`, also assert that every
    output of typical size (|want| >= rms(want)) is within that many ulps with no floor; with `typical_within`,
    that at least that share of the outputs of typical size is within 2 ulp with no floor; with `min_within`,
    that at least that share of all outputs is within 2 ulp with no floor. Works on the tensors' own device,
    a block of rows at a time."""
    want = torch.as_tensor(want)
    got = torch.as_tensor(got).to(want.device)
    if got.shape != want.shape:
        raise AssertionError(f"{what}: shape {tuple(got.shape)}, expected {tuple(want.shape)}")
    floor_t = torch.as_tensor(floor, dtype=torch.float64).to(want.device)
    if floor_t.dim():
        floor_t = floor_t.expand(want.shape) if floor_t.shape != want.shape else floor_t
    g2 = got.reshape(want.shape[0] if want.dim() > 1 else 1, -1)
    w2 = want.reshape(g2.shape)
    f2 = floor_t.reshape(g2.shape) if floor_t.dim() else floor_t
    sq = sum(float((w2[i:i + chunk_rows].double() ** 2).sum()) for i in range(0, w2.shape[0], chunk_rows))
    rms = (sq / max(w2.numel(), 1)) ** 0.5
    bad, within, ulp_max, ratio_max, err_max = 0, 0, 0.0, 0.0, 0.0
    n_typical, n_typical_within = 0, 0
    first_bad: Optional[str] = None
    for i in range(0, w2.shape[0], chunk_rows):
        g = g2[i:i + chunk_rows].double()
        w = w2[i:i + chunk_rows].double()
        f = f2[i:i + chunk_rows].double() if f2.dim() else f2.double()
        ulp = bf16_ulp(w)
        err = (g - w).abs()
        err = torch.where(torch.isnan(g) & torch.isnan(w), torch.zeros_like(err), err)
        err = torch.nan_to_num(err, nan=float("inf"))
        bound = ulps * ulp + f
        over = err > bound
        n_over = int(over.sum())
        if n_over and first_bad is None:
            at = int(torch.nonzero(over.reshape(-1))[0])
            first_bad = (f"e.g. flat index {i * w2.shape[1] + at}: got {float(g.reshape(-1)[at]):.6g}, "
                         f"want {float(w.reshape(-1)[at]):.6g}, bound {float(bound.reshape(-1)[at]):.3g}")
        bad += n_over
        within += int((err <= ULPS * ulp).sum())
        typical = w.abs() >= rms
        if typical.any():
            ulp_max = max(ulp_max, float((err / ulp)[typical].max()))
            n_typical += int(typical.sum())
            n_typical_within += int(((err <= ULPS * ulp) & typical).sum())
        ratio_max = max(ratio_max, float((err / bound).max()))
        err_max = max(err_max, float(err.max()))
    report = {"ulp_max_typical": round(ulp_max, 3), "within_2ulp": round(within / max(w2.numel(), 1), 6),
              "typical_within_2ulp": round(n_typical_within / max(n_typical, 1), 7),
              "bound_use": round(ratio_max, 4), "max_abs_err": err_max}
    print(f"{what}: {report}", flush=True)
    if bad:
        raise AssertionError(f"{what}: {bad} of {w2.numel()} outputs beyond {ulps} bf16 ulp + floor; "
                             f"largest |diff| {err_max:.4g}; {first_bad}")
    if typical_ulps is not None and ulp_max > typical_ulps:
        raise AssertionError(f"{what}: an output of typical size is {ulp_max:.3g} bf16 ulp off (bar {typical_ulps})")
    if typical_within is not None and report["typical_within_2ulp"] < typical_within:
        raise AssertionError(f"{what}: {report['typical_within_2ulp']:.7f} of the outputs of typical size within "
                             f"2 bf16 ulp (bar {typical_within})")
    if min_within is not None and report["within_2ulp"] < min_within:
        raise AssertionError(f"{what}: {report['within_2ulp']:.6f} of the outputs within 2 bf16 ulp "
                             f"(bar {min_within})")
    return report


def matmul_floor(x: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
    """Twice the f32 summation bound of x @ y: 2 * K * 2^-24 * (|x| @ |y|), computed in f32 on x's device
    (a bound: its own rounding changes it by a negligible fraction)."""
    K = x.shape[-1]
    return 2.0 * K * U32 * (x.float().abs() @ y.float().abs())


def softmax_floor(weighted_abs_v: torch.Tensor, terms: int, score_err: float = 0.0) -> torch.Tensor:
    """The floor for a softmax-weighted sum of v whose weights are rounded to bf16: 2^-8 times the same
    softmax applied to |v| (`weighted_abs_v`), plus the f32 summation bound over `terms` terms, plus twice
    the largest difference of a score between the two evaluations (`score_err`, see `score_err`): a score
    moved by d moves its weight by a factor within e^±d, so the weighted sum by at most 2d of the weighted
    |v| average."""
    w = torch.as_tensor(weighted_abs_v).double()
    return (P_ROUND + 2.0 * terms * U32 + 2.0 * score_err) * w


def score_err(q: torch.Tensor, k: torch.Tensor) -> float:
    """A bound on how far two f32 evaluations of a score q . k (head dim D, in any summation order) differ:
    2 * D * 2^-24 * max_i ||q_i||_1 * max|k| (each within D u sum_d |q_d k_d| of exact)."""
    D = q.shape[-1]
    return 2.0 * D * U32 * float(q.float().abs().sum(-1).max()) * float(k.float().abs().max())
