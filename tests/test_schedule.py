"""Step order and tables, bit-exact with the reference's schedule semantics.

The pinned numbers are the reference's own test expectations (tests/test_schedule.py:35-51,
tests/test_api.py:20-30, tests/test_examples.py:57-63 and 91-95, tests/test_index_arrays.py:128-140 of
the reference), and every table is also checked against a brute-force enumeration of the loop nest
(oracle/schedule.py).
"""

import itertools

import numpy as np
import pytest

from examples.causal_attention import AttentionBlocks, causal_attention
from examples.causal_matmul import causal_matmul
from examples.matmul import MatmulTiles, matmul
from helpers import make_kernel, schedule_of, spec
from oracle import schedule as oracle_schedule
from tilejax_amd import KernelError, jaxlite
from tilejax_amd.schedule import STEP_CODE, STEP_TILE

BANDED = """
def f(x):
    out = jnp.zeros((B, 512, 512))
    for b in range(B):
        for i in range(0, 512, 128):
            for j in range(0, 512, 128):
                if j > i:
                    continue
                acc = jnp.zeros((128, 128))
                for k in range(0, 512, 128):
                    if k < i - 128:
                        continue
                    acc += x[b, i : i + 128, k : k + 128]
                out = out.at[b, i : i + 128, j : j + 128].set(acc)
    return out
"""


def test_tables_walk_exactly_the_nests_steps():
    sch = schedule_of(make_kernel(BANDED, B=3), spec(3, 512, 512))
    want = [((b, i, j), k) for b, i, j in itertools.product(range(3), range(4), range(4)) if j <= i
            for k in range(4) if k >= i - 1]
    got = []
    for step in range(sch.steps):
        tile, phase, k = sch.step_at(step)
        assert phase == 0
        got.append((sch.blocks_at(tile), k))
    assert got == want
    assert sch.tiles == 30 and sch.total_tiles == 48 and sch.fills == 18 and sch.repeats == 3
    assert [r.var for r in sch.outer] == ["b"] and [r.var for r in sch.inner] == ["i", "j"]


def test_banded_tables_match_brute_force():
    sch = schedule_of(make_kernel(BANDED, B=3), spec(3, 512, 512))
    inner = [("i", 0, 128, 4), ("j", 0, 128, 4)]
    active, skipped, step_tile, step_code = oracle_schedule.static_tables(
        inner, lambda v: v["j"] > v["i"], [("k", 0, 128, 4, lambda v: v["k"] < v["i"] - 128)])
    np.testing.assert_array_equal(sch.tables[STEP_TILE], step_tile)
    np.testing.assert_array_equal(sch.tables[STEP_CODE], step_code)
    np.testing.assert_array_equal(sch.tables["tile_i"], [a[0] for a in active])
    np.testing.assert_array_equal(sch.tables["fill_j"], [s[1] for s in skipped])


def test_without_masks_steps_are_arithmetic():
    sch = schedule_of(make_kernel(BANDED.replace("if j > i:", "if False:").replace("if k < i - 128:", "if False:"), B=2),
                      spec(2, 512, 512))
    assert sch.tables == {} and sch.steps_per_tile == 4
    sch = schedule_of(make_kernel("""
        def f(x):
            out = jnp.zeros((256, 256))
            for i in range(0, 256, 128):
                for j in range(0, 256, 128):
                    out = out.at[i : i + 128, j : j + 128].set(x[i : i + 128, j : j + 128])
            return out
        """), spec(256, 256))
    assert (sch.steps, sch.steps_per_tile, sch.tables) == (4, 1, {})
    assert [sch.blocks_at(t) for t in range(4)] == [(0, 0), (0, 1), (1, 0), (1, 1)]


@pytest.mark.parametrize(("tile_mask", "step_mask", "message"), [
    ("True", "False", "the masks skip every output tile"),
    ("False", "undefined", "can't evaluate `undefined`"),
])
def test_mask_errors(tile_mask, step_mask, message):
    source = BANDED.replace("if j > i:", f"if {tile_mask}:").replace("if k < i - 128:", f"if {step_mask}:")
    with pytest.raises(KernelError, match=message):
        schedule_of(make_kernel(source, B=1), spec(1, 512, 512))


def test_matmul_counts():
    bf = jaxlite.bfloat16
    tiles = MatmulTiles(tm=128, tn=128, tk=128)
    sch = schedule_of(matmul, spec(256, 384, dtype=bf), spec(384, 256, dtype=bf), tunable=tiles)
    assert (sch.steps, sch.tiles, sch.total_tiles) == (12, 4, 4)
    assert sch.steps_per_tile == 3 and sch.tables == {}


def test_causal_matmul_counts():
    bf = jaxlite.bfloat16
    sch = schedule_of(causal_matmul, spec(512, 256, dtype=bf), spec(256, 512, dtype=bf),
                      tunable=MatmulTiles(tm=128, tn=128, tk=128))
    assert (sch.tiles, sch.total_tiles, sch.steps) == (10, 16, 20)
    # The BASELINE.json config: 8192^3 at 512^3 tiles runs 136 of 256 tiles, 2176 steps, 120 fills.
    sch = schedule_of(causal_matmul, spec(8192, 8192, dtype=bf), spec(8192, 8192, dtype=bf),
                      tunable=MatmulTiles(512, 512, 512))
    assert (sch.tiles, sch.total_tiles, sch.steps, sch.fills) == (136, 256, 2176, 120)


def test_causal_attention_skips_future_blocks():
    bf = jaxlite.bfloat16
    sch = schedule_of(causal_attention, *[spec(2, 4, 512, 128, dtype=bf)] * 3,
                      tunable=AttentionBlocks(block_q=128, block_kv=128))
    assert sch.steps == 2 * 4 * (1 + 2 + 3 + 4)
    assert sch.repeats == 8 and len(sch.tables[STEP_TILE]) == 10
    inner = [("i", 0, 128, 4)]
    _, _, step_tile, step_code = oracle_schedule.static_tables(
        inner, lambda v: False, [("j", 0, 128, 4, lambda v: v["j"] > v["i"] + 128 - 1)])
    np.testing.assert_array_equal(sch.tables[STEP_TILE], step_tile)
    np.testing.assert_array_equal(sch.tables[STEP_CODE], step_code)
    # BASELINE.json config 3 at 512^2 blocks: a 10-step pattern repeated over the 64 (b, h) pairs.
    sch = schedule_of(causal_attention, *[spec(4, 16, 2048, 128, dtype=bf)] * 3, tunable=AttentionBlocks(512, 512))
    assert (sch.steps, sch.repeats, len(sch.tables[STEP_TILE])) == (640, 64, 10)


GMM = """
def gmm(x, w, starts, ends):
    M, K = x.shape
    E, _, N = w.shape
    out = jnp.zeros((M, N), jnp.float32)
    for j in range(0, N, 128):
        for i in range(0, M, 128):
            acc = jnp.zeros((128, 128), jnp.float32)
            for e in range(E):
                if ends[e] <= i or starts[e] >= i + 128:
                    continue
                rows = i + jax.lax.broadcasted_iota(jnp.int32, (128, K), 0)
                mine = (rows >= starts[e]) & (rows < ends[e])
                acc += jnp.where(mine, x[i : i + 128, :], 0.0) @ w[e, :, j : j + 128]
            out = out.at[i : i + 128, j : j + 128].set(acc)
    return out
"""


def test_grouped_matmul_runtime_capacity():
    kernel = make_kernel(GMM)
    sch = schedule_of(kernel, spec(512, 256), spec(4, 256, 256), spec(4, dtype=jaxlite.int32),
                      spec(4, dtype=jaxlite.int32))
    assert sch.runtime and sch.repeats == 2 and sch.steps == 2 * 4 * 4


DECODE = """
def f(cache, lengths):
    B, S, D = cache.shape
    out = jnp.zeros((B, 8, D))
    for b in range(B):
        acc = jnp.zeros((8, D))
        for j in range(0, S, 128):
            if j >= lengths[b]:
                continue
            acc += jnp.sum(cache[b, j : j + 128, :].reshape(16, 8, D), axis=0)
        out = out.at[b, :, :].set(acc)
    return out
"""


def test_runtime_mask_tables_count_the_steps_that_run():
    """For lengths (0, 1, 300, 512) at blocks of 128 the device tables keep 1 + 1 + 3 + 4 steps, the empty
    sequence taking one empty step (the reference's tests/test_index_arrays.py:57-72)."""
    kernel = make_kernel(DECODE)
    sch = schedule_of(kernel, spec(4, 512, 128), spec(4, dtype=jaxlite.int32))
    assert sch.runtime and sch.empty and sch.steps == 16
    lengths = [0, 1, 300, 512]
    tiles = [{"b": b} for b in range(4)]
    step_tile, step_code, count = oracle_schedule.runtime_tables(
        tiles, [("j", 0, 128, 4, lambda v: v["j"] >= lengths[v["b"]])])
    assert count == 1 + 1 + 3 + 4
    assert step_code[0] & 4 and step_code[0] & 3 == 3  # the empty sequence's one step: empty, first, last
    assert list(step_tile[:count]) == [0, 1, 2, 2, 2, 3, 3, 3, 3]


@pytest.mark.parametrize("skip,empty", [("True", True), ("i == 0", True), ("i == 128 and k == 0", False)])
def test_a_tile_whose_mask_skips_every_step_takes_one_empty_step(skip, empty):
    """The reference's tests/test_schedule.py:100-130: a tile all of whose blocks the mask skips still takes
    one step, marked empty (its body doesn't run); the others take exactly their blocks."""
    from tests.codegen_cases import EMPTY_SOURCE

    kernel = make_kernel(EMPTY_SOURCE.replace("SKIP", skip))
    sch = schedule_of(kernel, spec(256, 256))
    assert sch.empty == empty
    steps = [(sch.step_at(s), sch.empty_at(s)) for s in range(sch.steps)]
    runs = {(i, k) for i in (0, 128) for k in (0, 128) if not eval(skip, {"i": i, "k": k})}
    for i in (0, 128):
        mine = [k for (tile, _, k), is_empty in steps if tile == i // 128 and not is_empty]
        assert mine == [k // 128 for ii, k in sorted(runs) if ii == i]
        assert any(tile == i // 128 for (tile, _, _), _e in steps)  # every tile takes a step


def test_values_a_masked_loop_makes_for_the_code_after_it_are_carried():
    from tests.codegen_cases import MASKED_CARRIED

    kernel = make_kernel(MASKED_CARRIED.source)
    assert set(kernel.lower(spec(256, 256)).plan.carried) == {"acc", "twice"}


def test_step_arithmetic_stays_in_int32():
    kernel = make_kernel("""
    def f(x):
        out = jnp.zeros((2**20, 256, 128))
        for b in range(2**20):
            for i in range(0, 256, 128):
                if i:
                    continue
                out = out.at[b, i : i + 128, :].set(1.0)
        return out
    """)
    with pytest.raises(KernelError, match="int32 step arithmetic"):
        schedule_of(kernel, spec(8, 128))


def test_a_causal_matmul_of_one_tile_needs_no_tables():
    from examples.causal_matmul import causal_matmul
    from examples.matmul import MatmulTiles

    lowered = causal_matmul.lower(spec(256, 256), spec(256, 256), MatmulTiles(256, 256, 128))
    assert lowered.schedule.tables == {}
