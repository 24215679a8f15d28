"""The per-element emitter (codegen/expr.py ElementEmitter) against concrete evaluation: the decode spec's
per-tile query rows (`block_diagonal(query_rows(q[b]))`: reshape, jnp.tile, where, concatenate, astype)
and its epilogue (`finish(own_blocks(acc))`: slices, where, reshape), generated as C, compiled with the
host compiler and compared element by element with the same code run by jaxlite on the CPU."""

import os
import shutil
import subprocess
import tempfile

import numpy as np
import pytest
import torch

from examples.decode import block_diagonal, finish, own_blocks, query_rows, row_index
from tilejax_amd import jaxlite
from tilejax_amd.codegen.expr import ElementEmitter

HOST_PRELUDE = r"""
#include <cstdio>
#include <cstring>
#include <cmath>
static unsigned ak_bf16_bits(float x) { unsigned u; std::memcpy(&u, &x, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u; u += 0x7fffu + ((u >> 16) & 1u); return u >> 16; }
static float ak_round_bf16(float x) { unsigned u = ak_bf16_bits(x) << 16; float f; std::memcpy(&f, &u, 4); return f; }
static float ak_maximum(float a, float b) { return (a != a || b != b) ? a + b : (a > b ? a : b); }
static float bits(unsigned u) { float f; std::memcpy(&f, &u, 4); return f; }
#define __builtin_bit_cast(T, v) bits(v)
"""


def _run_c(body: str) -> np.ndarray:
    if shutil.which("g++") is None:
        pytest.skip("no host C++ compiler")
    with tempfile.TemporaryDirectory() as d:
        src, exe = os.path.join(d, "t.cpp"), os.path.join(d, "t")
        open(src, "w").write(HOST_PRELUDE + body)
        subprocess.run(["g++", "-O1", "-o", exe, src], check=True, capture_output=True)
        out = subprocess.run([exe], check=True, capture_output=True, text=True).stdout
    return np.array([float.fromhex(v) for v in out.split()], np.float64)


def _trace(fn, *args_shapes):
    """Trace fn on symbolic inputs (leaves named in0, in1, ...); the root Node."""
    with jaxlite.trace():
        syms = [jaxlite.leaf("load", shape, dt, operand=f"in{k}") for k, (shape, dt) in enumerate(args_shapes)]
        return fn(*syms).node


@pytest.mark.parametrize("T,H,Hkv,D", [(1, 8, 2, 128), (1, 32, 8, 128), (2, 8, 4, 128)])
def test_block_diagonal_query_rows(T, H, Hkv, D):
    R = T * H
    root = _trace(lambda q: block_diagonal(query_rows(q), row_index(R, H, Hkv)[1], Hkv, jaxlite.bfloat16),
                  ((T, H, D), jaxlite.bfloat16))
    em = ElementEmitter(lambda n, idx: f"Q[({idx[0]}) * {H * D} + ({idx[1]}) * {D} + ({idx[2]})]" if n.op == "load" else None)
    expr = em.at(root, ("r", "c"))
    q = torch.randn(T, H, D).to(torch.bfloat16)
    vals = ", ".join(repr(float(v)) for v in q.float().reshape(-1))
    got = _run_c(f"static const float Q[] = {{{vals}}};\nint main() {{ for (int r = 0; r < {R}; ++r) "
                 f"for (int c = 0; c < {Hkv * D}; ++c) std::printf(\"%a\\n\", (double)({expr})); }}\n")
    with jaxlite.default_device("cpu"):
        want = block_diagonal(query_rows(jaxlite.Array(q)), row_index(R, H, Hkv)[1], Hkv, jaxlite.bfloat16)
    np.testing.assert_array_equal(got, want.t.float().reshape(-1).numpy())


@pytest.mark.parametrize("T,H,Hkv,D", [(1, 8, 2, 128), (1, 32, 8, 128)])
def test_finish_own_blocks(T, H, Hkv, D):
    R, W = T * H, Hkv * D

    def epilogue(acc, row_sum):
        return finish(own_blocks(acc, row_index(R, H, Hkv)[1], Hkv), row_sum, (T, H, D), jaxlite.bfloat16)

    root = _trace(epilogue, ((R, W), jaxlite.float32), ((R, 128), jaxlite.float32))

    def leaves(n, idx):
        if n.op == "load" and n.kwargs["operand"] == "in0":
            return f"ACC[({idx[0]}) * {W} + ({idx[1]})]"
        if n.op == "load":
            return f"L[{idx[0]}]"
        return None

    expr = ElementEmitter(leaves).at(root, ("t", "h", "d"))
    acc = torch.randn(R, W)
    rs = torch.rand(R) + 0.5
    rs[0] = 0.0  # a row that saw no key: 0, not inf
    acc_s = ", ".join(repr(float(v)) for v in acc.reshape(-1))
    l_s = ", ".join(repr(float(v)) for v in rs)
    got = _run_c(f"static const float ACC[] = {{{acc_s}}};\nstatic const float L[] = {{{l_s}}};\n"
                 f"int main() {{ for (int t = 0; t < {T}; ++t) for (int h = 0; h < {H}; ++h) for (int d = 0; d < {D}; ++d) "
                 f"std::printf(\"%a\\n\", (double)({expr})); }}\n")
    with jaxlite.default_device("cpu"):
        want = epilogue(jaxlite.Array(acc), jaxlite.Array(rs[:, None].expand(R, 128).contiguous()))
    np.testing.assert_array_equal(got, want.t.float().reshape(-1).numpy())
