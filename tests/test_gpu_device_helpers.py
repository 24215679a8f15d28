"""The device prelude's lane helpers on known inputs: the attention kernels combine a query row's two halves
(lanes l and l ^ 32) with them, so their lane layout is pinned here against numpy."""

import struct

import numpy as np
import pytest
import torch

from tilejax_amd import runtime
from tilejax_amd.codegen.device import PRELUDE

pytestmark = pytest.mark.gpu

SOURCE = PRELUDE + r"""
struct helper_args { const float* x; float* out; };
extern "C" __global__ void __launch_bounds__(64) lane_helpers(const helper_args args) {
  const int l = threadIdx.x;
  const float x = args.x[l];
  args.out[l] = ak_xor32(x);
  args.out[64 + l] = ak_xor32_max(x);
  args.out[128 + l] = ak_xor32_sum(x);
}
"""


def test_xor32_helpers_match_numpy():
    x = torch.tensor(np.random.default_rng(0).standard_normal(64), dtype=torch.float32, device="cuda")
    out = torch.full((192,), float("nan"), device="cuda")
    module = runtime.load(SOURCE, "lane_helpers.hip")
    module.kernel("lane_helpers").launch((1, 1, 1), (64, 1, 1), 0, struct.pack("<QQ", x.data_ptr(), out.data_ptr()),
                                         runtime.current_stream())
    torch.cuda.synchronize()
    xs, got = x.cpu().numpy(), out.cpu().numpy()
    partner = xs[np.arange(64) ^ 32]
    np.testing.assert_array_equal(got[:64], partner)
    np.testing.assert_array_equal(got[64:128], np.maximum(xs, partner))
    np.testing.assert_array_equal(got[128:], (xs + partner).astype(np.float32))
