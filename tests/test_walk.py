"""Plans of the tile as written (tilejax_amd/walk.py), on the CPU: repeat loops, runtime loop bounds and a
runtime count of tiles, ragged rows, windows gathered through index-array slices, outputs updated in place and
scattered, outputs stored per step, and index arrays the tile code computes.

The cases restate the reference's tests of these forms (tests/test_repeat_loops.py, test_runtime_ranges.py,
test_in_place.py, test_step_outputs.py, test_computed_indices.py), each with a float64 closed form written
from the loop nest's meaning (not from the kernel's code). Here `kernel.reference` (the nest run eagerly over
jaxlite) is checked against those closed forms, the plans against the reference's own plan facts where they
carry over (which values a tile keeps, step counts), and every generated kernel is compiled for gfx950 (no
GPU needed); tests/test_gpu_walk.py runs the kernels.
"""

import numpy as np
import pytest
import torch

import tilejax_amd
from tests.helpers import make_kernel, rand
from tilejax_amd import KernelError, jaxlite, runtime
from tilejax_amd.jaxlite import jax, jnp


def f64(a):
    return np.asarray(torch.as_tensor(np.asarray(a)).double() if not isinstance(a, torch.Tensor) else a.double())


def i32(*values):
    return torch.tensor(values, dtype=torch.int32)


def close(got, want, rtol=1e-4, atol=1e-3):
    np.testing.assert_allclose(f64(got), want, rtol=rtol, atol=atol)


def compiles(lowered):
    """The generated kernel (the generic one) compiles for gfx950."""
    assert lowered.program.notes["family"] == "generic", lowered.program.notes
    runtime.compile_source(lowered.source, f"{lowered.program.name}.hip")


# ------------------------------------------------------------------------------------- repeat loops

FFN_STACK = """
def ffn_stack(x, gamma, w_up, w_down):
    M, D = x.shape
    L, _, F = w_up.shape
    out = jnp.zeros((M, D), jnp.float32)
    for i in range(0, M, 128):
        h = x[i : i + 128, :]
        for l in range(L):  # a layer per iteration
            n = h * gamma[l, 0:1, :]
            y = jnp.zeros((128, D))
            for f in range(0, F, 128):
                y += jnp.maximum(n @ w_up[l, :, f : f + 128], 0.0) @ w_down[l, f : f + 128, :]
            h = h + y * (l + 1)
        out = out.at[i : i + 128, :].set(h)
    return out
"""


def ffn_stack_float64(x, gamma, w_up, w_down):
    h = f64(x)
    for layer in range(w_up.shape[0]):
        n = h * f64(gamma[layer])
        h = h + (layer + 1) * np.maximum(n @ f64(w_up[layer]), 0) @ f64(w_down[layer])
    return h


def ffn_inputs(layers=3):
    return (rand((256, 128)), 1 + 0.1 * rand((layers, 1, 128), 1), rand((layers, 128, 256), 2) / 12,
            rand((layers, 256, 128), 3) / 16)


LAYERED = """
def layered(x, w, limits):
    M, K = x.shape
    L = w.shape[0]
    out = jnp.zeros((M, 128), jnp.float32)
    for i in range(0, M, 128):
        a = jnp.zeros((128, 128))
        for k in range(0, K, 128):  # a reduction loop before the repeat loop
            a += x[i : i + 128, k : k + 128]
        h = a * 0.5
        for l in range(L):
            y = jnp.zeros((128, 128))
            for f in range(0, 384, 128):  # layer l runs l + 1 blocks: a mask reading the repeat loop
                if f > l * 128:
                    continue
                y += h @ w[l, f : f + 128, :]
            h = h + y * 0.1
            z = h * 0
            for g in range(0, 256, 128):  # a mask read when the kernel runs
                if g >= limits[l]:
                    continue
                z += x[i : i + 128, g : g + 128] * (l + 1)
            h = h + z
        t = h * 2
        for c in range(0, 256, 128):  # one after it
            t = t + x[i : i + 128, c : c + 128]
        out = out.at[i : i + 128, :].set(t)
    return out
"""


def layered_float64(x, w, limits):
    x, w = f64(x), f64(w)
    out = []
    for i in range(0, x.shape[0], 128):
        blocks = [x[i : i + 128, k : k + 128] for k in range(0, x.shape[1], 128)]
        h = sum(blocks) * 0.5
        for layer in range(w.shape[0]):
            y = sum(h @ w[layer, f : f + 128] for f in range(0, 128 * (layer + 1), 128) if f < 384)
            h = h + y * 0.1
            h = h + sum((layer + 1) * blocks[g // 128] for g in range(0, 256, 128) if g < limits[layer])
        out.append(2 * h + blocks[0] + blocks[1])
    return np.concatenate(out)


TWO_REPEATS = """
def two_repeats(x, w):
    out = jnp.zeros((128, 128), jnp.float32)
    for i in range(0, 128, 128):
        h = x[i : i + 128, :]
        for l in range(2):
            for f in range(0, 256, 128):
                if f > l * 128:
                    continue
                h = h + w[l, f : f + 128, :]
        u = h * 1
        for m in range(2):
            v = u * 2
            for g in range(0, 256, 128):
                v = v + w[m, g : g + 128, :] * (m + 1)
            u = v
        out = out.at[i : i + 128, :].set(u)
    return out
"""


def two_repeats_float64(x, w):
    xf, wf = f64(x), f64(w)
    h = xf + wf[0, :128] + wf[1, :128] + wf[1, 128:]
    for m in range(2):
        h = 2 * h + (m + 1) * (wf[m, :128] + wf[m, 128:])
    return h


def test_repeat_loop_carries_layers():
    kernel = make_kernel(FFN_STACK)
    inputs = ffn_inputs()
    close(kernel.reference(*inputs), ffn_stack_float64(*inputs))
    lowered = kernel.lower(*inputs)
    plan = lowered.plan
    assert plan.walk and set(plan.kept) == {"h", "n", "y"}
    assert [b.kind for b in plan.tree] == ["code", "repeat", "code"]
    assert lowered.steps == 2 * 3 * 2  # (tiles, layers, blocks of hidden units)
    compiles(lowered)


@pytest.mark.parametrize("limits", [(256, 0, 100), (0, 0, 0)])
def test_reductions_around_and_in_a_repeat_loop_with_masks(limits):
    kernel = make_kernel(LAYERED)
    x, w = rand((256, 256)), rand((3, 384, 128), 1) / 20
    lim = i32(*limits)
    close(kernel.reference(x, w, lim), layered_float64(x, w, limits))
    lowered = kernel.lower(x, w, lim)
    assert lowered.plan.walk and [b.kind for b in lowered.plan.tree] == ["code", "loop", "code", "repeat", "code",
                                                                         "loop", "code"]
    compiles(lowered)


def test_two_repeat_loops():
    kernel = make_kernel(TWO_REPEATS)
    x, w = rand((128, 128)), rand((2, 256, 128), 1)
    close(kernel.reference(x, w), two_repeats_float64(x, w))
    lowered = kernel.lower(x, w)
    assert lowered.steps == 1 + 2 + 2 * 2  # (the masked step of the first loop's first iteration skipped)
    compiles(lowered)


def test_repeat_loop_errors():
    nested = """
    def f(x):
        out = jnp.zeros((128, 128))
        for i in range(0, 128, 128):
            h = x[i : i + 128, :]
            for l in range(2):
                for m in range(2):
                    for f in range(0, 128, 128):
                        h = h + x[f : f + 128, :]
            out = out.at[i : i + 128, :].set(h)
        return out
    """
    with pytest.raises(KernelError, match="repeat loops don't nest"):
        make_kernel(nested)
    changes_shape = """
    def f(x):
        out = jnp.zeros((128, 128))
        for i in range(0, 128, 128):
            h = x[i : i + 128, :]
            for l in range(2):
                for f in range(0, 128, 128):
                    h = jnp.concatenate([h, h], axis=0)
            out = out.at[i : i + 128, :].set(h[0:128, :])
        return out
    """
    with pytest.raises(KernelError, match="changes shape"):
        make_kernel(changes_shape).lower(rand((128, 128)))


# ------------------------------------------------------------------------------------- runtime ranges

SUMS = """
def sums(cache, lengths):
    B, S, D = cache.shape
    out = jnp.zeros((B, 8, D))
    for b in range(B):
        acc = jnp.zeros((8, D))
        for j in range(0, lengths[b], 128):  # the cache's blocks up to its length
            rows = j + jax.lax.broadcasted_iota(jnp.int32, (128, D), 0)
            acc += jnp.sum(jnp.where(rows < lengths[b], cache[b, j : j + 128, :], 0.0).reshape(16, 8, D), axis=0)
        out = out.at[b, :, :].set(acc)
    return out
"""


def sums_float64(cache, lengths):
    out = np.zeros((cache.shape[0], 8, cache.shape[2]))
    for b, n in enumerate(np.asarray(lengths)):
        rows = np.concatenate([f64(cache[b, :n]), np.zeros((-n % 8, cache.shape[2]))])
        out[b] = rows.reshape(-1, 8, cache.shape[2]).sum(0)
    return out


SPANS = """
def spans(x, w, lo, hi):
    B, S, D = x.shape
    out = jnp.zeros((B, 8, D))
    for b in range(B):
        acc = jnp.zeros((8, D))
        for j in range(lo[b], hi[b], 8):  # from lo[b] to hi[b]
            acc += x[b, j : j + 8, :]
        for k in range(0, 256, 128):  # a static loop after it
            acc += jnp.sum(w[k : k + 128, :].reshape(16, 8, D), axis=0)
        out = out.at[b, :, :].set(acc)
    return out
"""


def spans_float64(x, w, lo, hi):
    want = np.stack([f64(x[b, int(a):int(z)]).reshape(-1, 8, x.shape[2]).sum(0) for b, (a, z) in enumerate(zip(lo, hi))])
    return want + f64(w).reshape(-1, 8, w.shape[1]).sum(0)


COUNTED = """
def counted(x, n):
    B, S, _, D = x.shape
    out = jnp.zeros((B, 8, D))
    for b in range(B):
        if b == 1:
            continue
        acc = jnp.zeros((8, D))
        for j in range(n[b]):
            acc += x[b, j, :, :]
        out = out.at[b, :, :].set(acc)
    return out
"""


def counted_float64(x, n):
    want = np.stack([f64(x[b, : min(int(c), x.shape[1])]).sum(0) for b, c in enumerate(n)])
    want[1] = 0
    for b, c in enumerate(n):  # steps past the dim read its last block (the index is clamped, as JAX clamps)
        if b != 1 and int(c) > x.shape[1]:
            want[b] += (int(c) - x.shape[1]) * f64(x[b, -1])
    return want


def test_runtime_range_steps_through_each_tiles_blocks():
    kernel = make_kernel(SUMS)
    cache, lengths = rand((4, 512, 128)), i32(0, 1, 300, 512)  # (an empty range)
    close(kernel.reference(cache, lengths), sums_float64(cache, lengths), 1e-5, 1e-4)
    lowered = kernel.lower(cache, lengths)
    assert lowered.plan.walk and not lowered.plan.bounds["j"].static
    compiles(lowered)


def test_runtime_ranges_with_a_start_and_a_static_loop():
    kernel = make_kernel(SPANS)
    x, w = rand((3, 64, 128)), rand((256, 128), 1)
    lo, hi = i32(0, 8, 16), i32(16, 8, 64)
    close(kernel.reference(x, w, lo, hi), spans_float64(x, w, lo, hi), 1e-5, 1e-4)
    compiles(kernel.lower(x, w, lo, hi))


def test_runtime_range_indexes_with_its_value_under_a_tile_mask():
    kernel = make_kernel(COUNTED)
    x, n = rand((3, 4, 8, 128)), i32(2, 4, 9)  # (9: past the dim, clamped)
    close(kernel.reference(x, n), counted_float64(x, n), 1e-5, 1e-4)
    compiles(kernel.lower(x, n))


# ------------------------------------------------------------------------------------- ragged rows, gathers

RAGGED = """
def ragged(q, rows, n):
    T, D, dtype = q.shape[0], q.shape[2], q.dtype
    out = q
    for k in range(n[0]):  # the tiles, counted as the kernel runs
        x = q[tilejax_amd.rows(rows[k], rows[k + 1], 16), :, :]
        acc = jnp.zeros((16, 8, D))
        for j in range(0, 2 * D, D):
            acc += x.astype(jnp.float32) * 2
        out = out.at[tilejax_amd.rows(rows[k], rows[k + 1], 16), :, :].set(acc.astype(dtype))
    return out
"""


def ragged_float64(q, rows, n):
    want = f64(q).copy()
    want[: int(rows[int(n[0])])] *= 4
    return want


STATIC_RAGGED = """
def static_ragged(q, rows):
    out = q
    for k in range(3):
        acc = jnp.zeros((16, 8, 128))
        for j in range(0, rows[k + 1] - rows[k], 16):
            acc += q[tilejax_amd.rows(rows[k], rows[k + 1], 16), :, :] * 3
        out = out.at[tilejax_amd.rows(rows[k], rows[k + 1], 16), :, :].set(acc)
    return out
"""

GATHER = """
def gather(pages, table, w):
    B = table.shape[0] // 4
    out = jnp.zeros((B, 8, 128))
    for b in range(B):
        acc = jnp.sum(w[table[b * 4 : b * 4 + 2], :, :], axis=0) * 0  # (a tile's own gathered window)
        for p in range(0, 4, 2):  # two pages a step, gathered through the table
            acc += jnp.sum(pages[table[b * 4 + p : b * 4 + p + 2], :, :], axis=0) * w[table[0 : 0 + 2], :, :][0]
        out = out.at[b, :, :].set(acc)
    return out
"""


def gather_float64(pages, table, w):
    t = np.asarray(table).reshape(-1, 4)
    return np.stack([f64(pages)[t[b]].sum(0) * f64(w)[int(table[0])] for b in range(t.shape[0])])


NESTED = """
def nested(pages, table, first, n):
    out = jnp.zeros((2, 8, 128))
    for b in range(2):
        acc = jnp.zeros((8, 128))
        for p in range(n[b]):
            acc += pages[table[first[b] + p], :, :]
        out = out.at[b, :, :].set(acc)
    return out
"""


def test_ragged_rows_and_a_runtime_count_of_tiles():
    kernel = make_kernel(RAGGED, tilejax_amd=tilejax_amd)
    q = rand((64, 8, 128), dtype=torch.bfloat16)
    rows, n = i32(0, 5, 21, 37, 40, 40, 40), i32(4)  # tiles of 5, 16, 16 and 3 rows; rows 40.. untouched
    close(kernel.reference(q, rows, n), ragged_float64(q, rows, n), 1e-2, 0)
    np.testing.assert_array_equal(f64(kernel.reference(q, rows, i32(0))), f64(q))  # no tiles at all
    lowered = kernel.lower(q, rows, n)
    assert lowered.schedule.runtime_tiles and lowered.plan.aliases == {"out": 0}
    compiles(lowered)


def test_ragged_stores_of_static_tiles():
    kernel = make_kernel(STATIC_RAGGED, tilejax_amd=tilejax_amd)
    q, rows = rand((48, 8, 128)), i32(0, 16, 20, 36)
    want = f64(q).copy()
    want[:36] *= 3
    close(kernel.reference(q, rows), want, 1e-5, 1e-5)
    compiles(kernel.lower(q, rows))


def test_windows_gathered_through_index_array_slices():
    kernel = make_kernel(GATHER)
    pages, w = rand((10, 8, 128)), rand((10, 8, 128), 1)
    table = i32(3, 1, 4, 1, 5, 9, 2, 6)
    close(kernel.reference(pages, table, w), gather_float64(pages, table, w), 1e-5, 1e-4)
    lowered = kernel.lower(pages, table, w)
    assert [ix.name for ix in lowered.plan.indices] == ["table"]
    assert lowered.plan.accesses["pages"].dims[0].gather is not None
    compiles(lowered)


def test_nested_elements_in_windows_are_clamped():
    kernel = make_kernel(NESTED)
    pages, table, first, n = rand((6, 8, 128)), i32(5, 4, 3, 2), i32(0, 3), i32(2, 2)  # 3 + 1: past the table
    want = np.stack([f64(pages[5]) + f64(pages[4]), f64(pages[2]) + f64(pages[2])])
    close(kernel.reference(pages, table, first, n), want, 1e-5, 1e-4)
    compiles(kernel.lower(pages, table, first, n))


# ------------------------------------------------------------------------------------- in place, per step

SCATTER = """
def scatter(x, pool, slots):
    B, H, D = x.shape
    new = pool
    out = jnp.zeros((B, H, D))
    for b in range(B):
        for h in range(0, H, 8):
            old = pool[slots[b], h : h + 8, :]
            out = out.at[b, h : h + 8, :].set(old * 2)
            new = new.at[slots[b], h : h + 8, :].set(old + x[b, h : h + 8, :])
    return out, new
"""


def scatter_float64(x, pool, slots):
    pool, x = f64(pool), f64(x)
    out, new = np.zeros(x.shape), pool.copy()
    for b, s in enumerate(np.asarray(slots)):
        out[b], new[s] = 2 * pool[s], pool[s] + x[b]
    return out, new


WRAPPED = """
def wrapped(x, pool, slots, shift):
    B, H, D = x.shape
    new = pool
    for b in range(B):
        for h in range(0, H, 8):
            new = new.at[slots[b], h : h + 8, :].set(x[b, h : h + 8, :] * 2 + pool[shift[b - 1], h : h + 8, :])
    return new
"""


def wrapped_float64(x, pool, slots, shift):
    """JAX's integer indices: a negative one counts from the end (a read at shift[-1] takes the last element,
    a row index -2 the second to last), and an update at a row still outside the pool is dropped."""
    pool, x = f64(pool), f64(x)
    new = pool.copy()
    slots, shift = np.asarray(slots), np.asarray(shift)
    n = pool.shape[0]
    for b in range(x.shape[0]):
        row = int(shift[b - 1])  # numpy counts b - 1 = -1 from the end too
        row = min(max(row + n if row < 0 else row, 0), n - 1)
        s = int(slots[b])
        s = s + n if s < 0 else s
        if 0 <= s < n:
            new[s] = 2 * x[b] + pool[row]
    return new


def test_negative_indices_count_from_the_end_and_stores_outside_are_dropped():
    """The reference's `kernel.fn` semantics for integer indices the tile reads at run time: slots (-1, 7, 2)
    store into the pool's last row, nowhere (7 is past the 7 rows), and row 2; shift[b - 1] at b = 0 reads
    shift's last element, and the row index -2 read from it takes the pool's second to last row."""
    kernel = make_kernel(WRAPPED)
    x, pool, slots, shift = rand((3, 16, 128)), rand((7, 16, 128), 1), i32(-1, 7, 2), i32(4, -2, 5)
    got = kernel.reference(x, pool, slots, shift)
    want = wrapped_float64(x, pool, slots, shift)
    close(got, want, 1e-6, 0)
    assert np.array_equal(want[[0, 1, 3, 4, 5]], f64(pool)[[0, 1, 3, 4, 5]])
    compiles(kernel.lower(x, pool, slots, shift))


MASKED_IN_PLACE = """
def masked_in_place(x):
    out = jnp.zeros((256, 256))
    new = x
    for i in range(0, 256, 128):
        for j in range(0, 256, 128):
            if j > i:
                continue
            out = out.at[i : i + 128, j : j + 128].set(x[i : i + 128, j : j + 128] + 1)
            new = new.at[i : i + 128, j : j + 128].set(x[i : i + 128, j : j + 128] * 3)
    return out, new
"""

SCAN = """
def scan(x, w):
    S, D = x.shape
    out = jnp.zeros((S, D), jnp.float32)
    last = jnp.zeros((8, D), jnp.float32)
    for j in range(0, D, 128):
        state = jnp.zeros((128, 128), jnp.float32)
        for i in range(0, S, 128):  # a chunk per step: its outputs stored by the step
            state = state * 0.5 + x[i : i + 128, j : j + 128] @ w[:, :]
            out = out.at[i : i + 128, j : j + 128].set(state)
        last = last.at[:, j : j + 128].set(state[0:8, :])
    return out, last
"""


def scan_float64(x, w):
    x, w = f64(x), f64(w)
    out = np.zeros_like(x)
    for j in range(0, x.shape[1], 128):
        state = np.zeros((128, 128))
        for i in range(0, x.shape[0], 128):
            state = state * 0.5 + x[i : i + 128, j : j + 128] @ w
            out[i : i + 128, j : j + 128] = state
    last = np.concatenate([out[-128:-120, j : j + 128] for j in range(0, x.shape[1], 128)], 1)
    return out, last


def test_random_index_arrays_that_place_stores_hold_distinct_values():
    """The reference's tests/test_in_place.py:163-172: tuning draws an index array that places stores from 0
    to the last slot of the dim it places (6 here, where the loops go to 16), without repeats, so no two
    tiles store into one window; an array too long for that many distinct values still stays in bounds."""
    from tilejax_amd.tune import _index_bounds, random_inputs

    kernel = make_kernel(SCATTER)
    signature = kernel.signature(rand((3, 16, 128)), rand((7, 16, 128), 1), i32(0, 1, 2))
    bounds, distinct = _index_bounds(kernel, signature, kernel.default_config(signature))
    assert bounds == {2: 6} and distinct == {2}
    for seed in range(5):
        slots = random_inputs(signature, bounds, seed, distinct, device="cpu")[2]
        assert slots.dtype == torch.int32 and len(set(slots.tolist())) == 3
        assert int(slots.min()) >= 0 and int(slots.max()) <= 6
    many = random_inputs((((8,), jaxlite.int32),), {0: 3}, distinct=frozenset({0}), device="cpu")[0]
    assert many.shape == (8,) and int(many.min()) >= 0 and int(many.max()) <= 3


def test_scatter_into_an_input_updated_in_place():
    kernel = make_kernel(SCATTER)
    x, pool, slots = rand((3, 16, 128)), rand((7, 16, 128), 1), i32(5, 0, 2)
    got_out, got_new = kernel.reference(x, pool, slots)
    want_out, want_new = scatter_float64(x, pool, slots)
    close(got_out, want_out, 1e-6, 0)
    close(got_new, want_new, 1e-6, 0)  # slots 1, 3, 4, 6 as they were
    assert torch.equal(pool, rand((7, 16, 128), 1))  # the input itself is unchanged
    lowered = kernel.lower(x, pool, slots)
    assert lowered.plan.aliases == {"new": 1} and lowered.plan.outputs[1].fill is None
    compiles(lowered)


def test_masked_tiles_of_an_input_updated_in_place_keep_its_values():
    kernel = make_kernel(MASKED_IN_PLACE)
    x = rand((256, 256))
    out, new = kernel.reference(x)
    keep = np.kron(np.tril(np.ones((2, 2))), np.ones((128, 128))).astype(bool)
    close(out, np.where(keep, f64(x) + 1, 0.0), 1e-6, 0)
    close(new, np.where(keep, f64(x) * 3, f64(x)), 1e-6, 0)
    compiles(kernel.lower(x))


def test_a_scan_stores_a_tile_per_step():
    kernel = make_kernel(SCAN)
    x, w = rand((512, 256)), rand((128, 128), 1) / 16
    got = kernel.reference(x, w)
    for g, want in zip(got, scan_float64(x, w)):
        close(g, want, 1e-4, 1e-4)
    lowered = kernel.lower(x, w)
    assert lowered.plan.walk and lowered.steps == 2 * 4
    compiles(lowered)


@pytest.mark.parametrize(("code", "message"), [
    ("out = jnp.zeros((7, 8, 128))\n    for b in range(3):\n        out = out.at[slots[b], :, :].set(x[b, :, :])",
     "an index array places this tile, so no tile might store the rest of `out`: allocate it as an input updated in "
     "place"),
    ("out = slots\n    for b in range(3):\n        out = out.at[b].set(slots[b])",
     "output `out` updates `slots` in place, but `slots` is an index array"),
    ("out = wrong\n    for b in range(3):\n        out = out.at[b, :, :].set(x[b, :, :])",
     r"allocate output `out` with jnp.zeros\(shape, dtype\) or jnp.full\(shape, value, dtype\), or as an input "
     r"updated in place \(`out = x`\)"),
])
def test_in_place_errors(code, message):
    kernel = make_kernel(f"def f(x, slots):\n    {code}\n    return out\n", wrong=3)
    with pytest.raises(KernelError, match=message):
        kernel.lower(rand((3, 8, 128)), i32(0, 1, 2))


def test_an_input_updated_in_place_whole():
    kernel = make_kernel("def f(x, slots):\n    out = x\n    for b in range(3):\n"
                         "        out = out.at[b, :, :].set(x[b, :, :])\n    return out\n")
    x = rand((3, 8, 128))
    close(kernel.reference(x, i32(0, 1, 2)), f64(x), 0, 0)
    compiles(kernel.lower(x, i32(0, 1, 2)))


# ------------------------------------------------------------------------------------- computed index arrays

E, K = 8, 2


def route(logits):
    """The K experts with the highest summed logits over the tokens, how many to use (the second only if its
    score is positive), and each token's weight for each, (K, T, 1)."""
    lanes = jax.lax.broadcasted_iota(jnp.int32, (1, logits.shape[1]), 1)
    score = jnp.where(lanes < E, jnp.sum(logits, axis=0, keepdims=True), -jnp.inf)
    chosen, weights, scores = [], [], []
    for _ in range(K):
        best = jnp.max(score, axis=1, keepdims=True)
        pick = jnp.min(jnp.where(score == best, lanes, logits.shape[1]), axis=1, keepdims=True)
        chosen.append(pick)
        scores.append(best)
        weights.append(jax.nn.sigmoid(jnp.sum(jnp.where(lanes == pick, logits, 0.0), axis=1, keepdims=True)))
        score = jnp.where(lanes == pick, -jnp.inf, score)
    ids = jnp.concatenate(chosen, axis=1).reshape(K).astype(jnp.int32)
    n = (1 + (scores[1] > 0).astype(jnp.int32)).reshape(1)
    return ids, n, jnp.stack(weights)


MOE = """
def routed(x, router, w):
    T, D = x.shape
    L = w.shape[0]
    out = jnp.zeros((T, D))
    for i in range(0, T, T):
        h = x[i : i + T, :]
        for layer in range(L):
            blocks = jnp.stack([h[:, 0:128], h[:, 128:256]])
            logits = jnp.zeros((T, 128))
            for d in range(0, D, 128):  # the router, a block of rows a step
                logits += blocks[d // 128] @ router[layer, d : d + 128, :]
            chosen, n, weights = route(logits)
            acc = jnp.zeros((T, D))
            for c in range(0, n[0] * D, D):  # the chosen experts: as many as the routing says
                acc += weights[c // D] * (h @ w[layer, chosen[c // D], :, :])
            h = h + acc
        out = out.at[i : i + T, :].set(h)
    return out
"""


def routed_float64(x, router, w):
    """The routing decided in f32 as the kernel decides it (from float64 logits rounded to f32), the rest in
    float64."""
    h = f64(x)
    for layer in range(w.shape[0]):
        logits = h @ f64(router[layer])
        ids, n, weights = (np.asarray(a) for a in route(jaxlite.Array(torch.tensor(logits, dtype=torch.float32))))
        h = h + sum(f64(weights[k]) * (h @ f64(w[layer, ids[k]])) for k in range(int(n[0])))
    return h


def moe_inputs(seed=0):
    return rand((8, 256), seed), rand((3, 256, 128), seed + 1) * 0.1, rand((3, E, 256, 256), seed + 2) * 0.05


def test_routing_inside_the_kernel_places_and_counts_later_steps():
    kernel = make_kernel(MOE, route=route)
    x, router, w = moe_inputs()
    np.testing.assert_allclose(f64(kernel.reference(x, router, w)), routed_float64(x, router, w), rtol=2e-4,
                               atol=2e-4)
    lowered = kernel.lower(x, router, w)
    kept = lowered.plan.kept
    assert kept["chosen"].shape == (K,) and kept["n"].shape == (1,) and kept["chosen"].dtype == jaxlite.int32
    compiles(lowered)


OFFSETS = (0, 2)

ONCE_PER_TILE = """
def once_per_tile(x):
    out = jnp.zeros((16, 128))
    for i in range(0, 16, 8):
        acc = jnp.zeros((8, 128))
        for d in range(0, 256, 128):
            acc += x[0, i : i + 8, d : d + 128]
        n = (jnp.sum(acc > 0) % 3).astype(jnp.int32).reshape(1)  # made once per tile
        for c in range(1, n[0] + OFFSETS[1] + 1):
            acc += x[c, i : i + 8, 0:128]
        out = out.at[i : i + 8, :].set(acc)
    return out
"""


def once_per_tile_float64(x):
    x = f64(x)
    out = []
    for i in range(0, 16, 8):
        acc = x[0, i : i + 8, :128] + x[0, i : i + 8, 128:]
        n = int((acc > 0).sum()) % 3
        for c in range(1, n + OFFSETS[1] + 1):
            acc = acc + x[min(c, x.shape[0] - 1), i : i + 8, :128]
        out.append(acc)
    return np.concatenate(out)


def test_indices_made_once_per_tile_and_constants_in_bounds():
    kernel = make_kernel(ONCE_PER_TILE, OFFSETS=OFFSETS)
    x = rand((5, 16, 256))
    close(kernel.reference(x), once_per_tile_float64(x), 1e-5, 1e-4)
    compiles(kernel.lower(x))


PICKED = """
def picked(x, ids):
    out = jnp.zeros((512, 128))
    for i in range(0, 512, 128):
        b = jnp.minimum(ids[i // 128], 3)
        out = out.at[i : i + 128, :].set(x[i : i + 128, :] * ids[b])
    return out
"""


def picked_float64(x, ids):
    ids = np.asarray(ids)
    scale = np.repeat([ids[min(int(ids[t]), 3)] for t in range(4)], 128)[:, None]
    return np.asarray(x.double()) * scale


def test_an_element_index_the_tile_code_computes():
    """`ids[b]` with `b` computed by the tile: the reference's planner rejects naming an element first
    (tests/test_index_arrays.py:299-311); here the walk planner reads the element as the tile runs."""
    kernel = make_kernel(PICKED)
    x, ids = rand((512, 128)), i32(2, 0, 7, 1)
    lowered = kernel.lower(x, ids)
    assert lowered.plan.walk
    close(kernel.reference(x, ids), picked_float64(x, ids), 1e-6, 0)
    compiles(lowered)


EARLY = """
def early(x):
    out = jnp.zeros((8, 128))
    for i in range(0, 8, 8):
        ids = 1 - jnp.arange(2, dtype=jnp.int32)  # made before the first loop, then again
        ids = ids + 0
        acc = jnp.zeros((8, 128))
        for c in range(2):
            acc += x[ids[c], i : i + 8, :] * (c + 1)
        out = out.at[i : i + 8, :].set(acc)
    return out
"""


def early_float64(x):
    x = f64(x)
    return x[1, 0:8] + 2 * x[0, 0:8]


def test_windows_placed_by_an_array_made_before_the_loop():
    """The reference's planner rejects an index array made before the first reduction loop, or assigned
    twice (tests/test_computed_indices.py:205-232); the walk planner keeps it and places the windows."""
    kernel = make_kernel(EARLY)
    x = rand((2, 8, 128))
    assert kernel.lower(x).plan.walk
    close(kernel.reference(x), early_float64(x), 1e-6, 1e-6)
    compiles(kernel.lower(x))


def test_a_window_placed_by_what_the_same_part_computes_is_an_error():
    source = EARLY.replace("        for c in range(2):\n            acc += x[ids[c], i : i + 8, :] * (c + 1)\n",
                           "        acc += x[ids[0], i : i + 8, :]\n")
    assert source != EARLY
    with pytest.raises(KernelError, match="a window is placed by `ids`, which the same part of the tile computes"):
        make_kernel(source).lower(rand((2, 8, 128)))


CHOSEN = """
def chosen(x, w, ids, n):
    M, K = x.shape
    C = ids.shape[0]
    out = jnp.zeros((M, K), jnp.float32)
    for i in range(0, M, 128):
        h = x[i : i + 128, :]
        acc = jnp.zeros((128, K))
        for c in range(C):  # the chosen experts, then padding
            for f in range(0, K, K):
                if c >= n[0]:  # padding: an empty step, its expert's weights never read
                    continue
                acc += h @ w[ids[c], :, :] * (c + 1)
        out = out.at[i : i + 128, :].set(acc)
    return out
"""


def chosen_inputs():
    return rand((256, 128)), rand((6, 128, 128), 1) / 10, i32(4, 1, 0, 0), i32(2)


def chosen_float64(x, w, ids, n):
    x, w = f64(x), f64(w)
    return sum(x @ w[int(ids[c])] * (c + 1) for c in range(int(n[0])))


def test_an_empty_iteration_skips_what_only_its_steps_read():
    """The reference's tests/test_repeat_loops.py:214-227: padding iterations take no work."""
    kernel = make_kernel(CHOSEN)
    ins = chosen_inputs()
    close(kernel.reference(*ins), chosen_float64(*ins), 1e-4, 1e-3)
    compiles(kernel.lower(*ins))


ONE_LAYER_STEPS = FFN_STACK.replace("range(0, F, 128)", "range(0, F, F)").replace("f + 128", "f + F")


def test_repeat_loops_of_one_iteration_and_of_whole_layer_steps():
    """The reference's tests/test_repeat_loops.py:230-247: a repeat loop whose reduction is one step a
    layer, and a repeat loop of one iteration."""
    for source, layers in ((ONE_LAYER_STEPS, 3), (FFN_STACK, 1)):
        kernel = make_kernel(source)
        ins = ffn_inputs(layers)
        close(kernel.reference(*ins), ffn_stack_float64(*ins))
        compiles(kernel.lower(*ins))


RUNTIME_IN_REPEAT = """
def runtime_in_repeat(x, n):
    out = jnp.zeros((8, 128))
    for i in range(0, 8, 8):
        acc = jnp.zeros((8, 128))
        for j in range(n[0]):
            acc += x[i : i + 8, 0:128]
        for l in range(3):
            for k in range(0, n[1 + l], 128):
                acc += x[i : i + 8, k : k + 128] * (l + 1)
        out = out.at[i : i + 8, :].set(acc)
    return out
"""


def runtime_in_repeat_float64(x, n):
    x = f64(x)
    want = int(n[0]) * x[:, :128]
    for layer in range(3):
        for k in range(0, int(n[1 + layer]), 128):
            want = want + x[:, k:k + 128] * (layer + 1)
    return want


MIXED_MASKS = """
def mixed_masks(x, n, lengths):
    out = jnp.zeros((24, 128))
    for i in range(0, 24, 8):
        acc = jnp.zeros((8, 128))
        for j in range(0, n[0], 128):  # a runtime range
            acc += x[i : i + 8, j : j + 128]
        for j2 in range(0, 512, 128):
            if j2 >= lengths[i // 8] or j2 == 128:  # a runtime mask
                continue
            acc += x[i : i + 8, j2 : j2 + 128] * 2
        for j3 in range(0, 256, 128):
            if j3 > 0:  # a static mask
                continue
            acc += x[i : i + 8, j3 : j3 + 128] * 3
        out = out.at[i : i + 8, :].set(acc)
    return out
"""


def mixed_masks_float64(x, n, lengths):
    x = f64(x)
    out = np.zeros((24, 128))
    for t, length in enumerate(lengths.tolist()):
        rows = x[8 * t:8 * t + 8]
        want = sum(rows[:, j:j + 128] for j in range(0, int(n[0]), 128)) + 3 * rows[:, :128]
        want = want + 2 * sum(rows[:, j:j + 128] for j in range(0, 512, 128) if j < length and j != 128)
        out[8 * t:8 * t + 8] = want
    return out


def test_runtime_ranges_in_repeat_loops_and_mixed_masks():
    """The reference's tests/test_computed_indices.py:140-193: a runtime range inside a repeat loop, and a
    runtime range, a runtime mask and a static mask in one tile."""
    kernel = make_kernel(RUNTIME_IN_REPEAT)
    x, n = rand((8, 384)), i32(2, 384, 0, 256)
    close(kernel.reference(x, n), runtime_in_repeat_float64(x, n), 1e-5, 1e-5)
    compiles(kernel.lower(x, n))
    kernel = make_kernel(MIXED_MASKS)
    x, n, lengths = rand((24, 512)), i32(256), i32(512, 0, 200)
    close(kernel.reference(x, n, lengths), mixed_masks_float64(x, n, lengths), 1e-5, 1e-5)
    compiles(kernel.lower(x, n, lengths))


ONLY_IN_PLACE = """
def only_in_place(x):
    new = x
    for i in range(0, 256, 128):
        if i > 0:
            continue
        new = new.at[i : i + 128, :].set(x[i : i + 128, :] * 3)
    return new
"""


def only_in_place_float64(x):
    x = f64(x)
    return np.concatenate([3 * x[:128], x[128:]])


RAGGED_BOTH = """
def ragged_both(x, y, n):
    out = jnp.zeros((8, 256))
    for i in range(0, 8, 8):
        a = x[tilejax_amd.rows(n[0], n[1], 8), :]
        b = y[0:8, tilejax_amd.rows(n[2], n[3], 256)]
        rows = jax.lax.broadcasted_iota(jnp.int32, (8, 256), 0)
        cols = jax.lax.broadcasted_iota(jnp.int32, (8, 256), 1)
        ok = (rows < n[1] - n[0]) & (cols < n[3] - n[2])  # (past the stops: unspecified)
        out = out.at[i : i + 8, :].set(jnp.where(ok, a + b, 0.0))
    return out
"""


def ragged_both_float64(x, y, n):
    want = np.zeros((8, 256))
    want[:5, :172] = f64(x)[4:9, :172] + f64(y)[:5, 128:300]
    return want


PAIRS_PER_ITERATION = """
def pairs_per_iteration(kv, x):
    out = jnp.zeros((16, 128))
    for i in range(0, 16, 16):
        acc = jnp.zeros((16, 128))
        for l in range(2):
            for k in range(0, 32, 16):
                keys = jax.lax.bitcast_convert_type(tilejax_amd.pairs(kv[l, :, :, :]) << 16, jnp.float32)
                acc += keys + x[l, k : k + 16, :]
        out = out.at[i : i + 16, :].set(acc)
    return out
"""


def pairs_per_iteration_float64(kv, x):
    return sum(2 * f64(kv)[n, :, 0, :] + f64(x)[n, :16] + f64(x)[n, 16:] for n in range(2))


def test_in_place_ragged_and_pairs_forms():
    """The reference's tests/test_in_place.py:98-113 (an output updated in place fills nothing),
    tests/test_runtime_ranges.py:170-204 (ragged reads along both dims of a tile) and :278-298 (pairs of a
    window read once per repeat iteration)."""
    x = rand((256, 128))
    kernel = make_kernel(ONLY_IN_PLACE)
    close(kernel.reference(x), only_in_place_float64(x), 1e-6, 0)
    compiles(kernel.lower(x))
    kernel = make_kernel(RAGGED_BOTH, tilejax_amd=tilejax_amd)
    x, y, n = rand((20, 256)), rand((8, 512)), i32(4, 9, 128, 300)
    close(kernel.reference(x, y, n), ragged_both_float64(x, y, n), 1e-6, 0)
    compiles(kernel.lower(x, y, n))
    kernel = make_kernel(PAIRS_PER_ITERATION, tilejax_amd=tilejax_amd)
    kv, x = rand((2, 16, 2, 128), dtype=torch.bfloat16), rand((2, 32, 128))
    close(kernel.reference(kv, x), pairs_per_iteration_float64(kv, x), 1e-5, 1e-5)
    compiles(kernel.lower(kv, x))


def test_the_step_planner_still_takes_the_phases_of_steps_form():
    """A nest of the phases-of-steps form keeps its step plan (the kernel families read it)."""
    kernel = make_kernel("""
    def mm(x, y):
        out = jnp.zeros((256, 256), jnp.float32)
        for i in range(0, 256, 128):
            for j in range(0, 256, 128):
                acc = jnp.zeros((128, 128), jnp.float32)
                for k in range(0, 256, 128):
                    acc += x[i : i + 128, k : k + 128] @ y[k : k + 128, j : j + 128]
                out = out.at[i : i + 128, j : j + 128].set(acc)
        return out
    """)
    assert not kernel.lower(rand((256, 256)), rand((256, 256))).plan.walk


# ------------------------------------------------------------------------------------- row pairs as words

PAIRS = """
def pairs_kernel(kv, table):
    out = jnp.zeros((2, 16, 128), jnp.float32)
    for b in range(2):
        acc = jnp.zeros((16, 128), jnp.float32)
        for p in range(2):
            words = tilejax_amd.pairs(kv[table[b * 2 + p], :, :, :, :])  # (16, 4, 128)
            lows = jnp.stack([words[:, g, :] for g in range(4)])
            whole = tilejax_amd.pairs(kv[table[b * 2 + p], :, :, :, :])[0]
            k = jax.lax.bitcast_convert_type(lows << 16, jnp.float32)
            high = tilejax_amd.pairs(kv[table[b * 2 + p], :, :, :, :])[:, 1, :] & jnp.uint32(0xFFFF0000)
            v = jax.lax.bitcast_convert_type(high, jnp.float32)
            acc += jnp.sum(k, axis=0) + v + jnp.sum(jax.lax.bitcast_convert_type(whole << 16, jnp.float32)) * 0
        out = out.at[b, :, :].set(acc)
    return out
"""


def pairs_float64(kv, table):
    """Row 0 of each pair summed over the 4 heads, plus head 1's row 1, over each batch's 2 pages."""
    x = kv.double()
    t = table.reshape(2, 2).tolist()
    return np.stack([sum((x[t[b][p], :, :, 0, :].sum(1) + x[t[b][p], :, 1, 1, :]).numpy() for p in range(2))
                     for b in range(2)])


WRITE = """
def write(cache, keys, values, table, page, first, stop, src, n):
    ps, dtype = cache.shape[1], cache.dtype
    out = cache
    for w in range(n[0]):  # a step per run of rows, counted as the kernel runs
        k = keys[tilejax_amd.rows(src[w], src[w] + stop[w] - first[w], ps), :, :]
        v = values[tilejax_amd.rows(src[w], src[w] + stop[w] - first[w], ps), :, :]
        bits = jax.lax.bitcast_convert_type(k.astype(jnp.float32), jnp.uint32) >> 16
        words = bits | (jax.lax.bitcast_convert_type(v.astype(jnp.float32), jnp.uint32) & jnp.uint32(0xFFFF0000))
        out = out.at[table[page[w]], tilejax_amd.rows(first[w], stop[w], ps), :, :, :].set(
            tilejax_amd.unpairs(words, dtype)
        )
    return out
"""


def write_inputs():
    cache = rand((6, 16, 4, 2, 128), dtype=torch.bfloat16)
    keys, values = rand((32, 4, 128), 1, torch.bfloat16), rand((32, 4, 128), 2, torch.bfloat16)
    return (cache, keys, values, i32(5, 2, 0, 4), i32(1, 3, 0, 0), i32(3, 0, 10, 0), i32(16, 7, 11, 0),
            i32(0, 13, 20, 0))


def write_expected(cache, keys, values, n):
    """Runs (page, first, stop, source row): tokens src.. go to page table[page] positions first..stop."""
    want = cache.clone()
    for page, a, b, r in [(2, 3, 16, 0), (4, 0, 7, 13), (5, 10, 11, 20)][:n]:
        want[page, a:b, :, 0, :], want[page, a:b, :, 1, :] = keys[r:r + b - a], values[r:r + b - a]
    return want


def test_pairs_read_a_tiles_row_pairs_as_words():
    kernel = make_kernel(PAIRS, tilejax_amd=tilejax_amd)
    kv, table = rand((5, 16, 4, 2, 128), dtype=torch.bfloat16), i32(4, 0, 2, 3)
    close(kernel.reference(kv, table), pairs_float64(kv, table), 1e-5, 1e-4)
    compiles(kernel.lower(kv, table))


@pytest.mark.parametrize("n", [3, 0])
def test_runs_counted_as_the_kernel_runs_store_words(n):
    kernel = make_kernel(WRITE, tilejax_amd=tilejax_amd)
    ins = write_inputs()
    got = kernel.reference(*ins, i32(n))
    assert torch.equal(got, write_expected(*ins[:3], n))
    compiles(kernel.lower(*ins, i32(n)))


@pytest.mark.parametrize(("code", "message"), [
    ("a = tilejax_amd.pairs(x[i : i + 16, :])", r"takes a 16-bit tile of pairs of rows \(\.\.\., 2, d\), not float32"),
])
def test_pairs_errors(code, message):
    kernel = make_kernel(f"""
    def f(x):
        out = jnp.zeros((32, 128))
        for i in range(0, 32, 16):
            {code}
            out = out.at[i : i + 16, :].set(x[i : i + 16, :])
        return out
    """, tilejax_amd=tilejax_amd)
    with pytest.raises(KernelError, match=message):
        kernel.lower(rand((32, 128)))


# ------------------------------------------------------------------------------------- ragged paged attention

def rpa_inputs(kv_lens=(20, 64, 5, 0), decodes=2, H=32, Hkv=8, D=128, ps=16, pps=4, seed=0):
    """A paged cache (pages, ps, Hkv, 2, D) bf16 with each sequence's pages distinct random pages of the
    pool, q (T, H, D) with one row per sequence, and the distribution (sequences below `decodes` decode)."""
    g = torch.Generator().manual_seed(seed)
    S = len(kv_lens)
    pages = S * pps + 1
    cache = torch.randn(pages, ps, Hkv, 2, D, generator=g).to(torch.bfloat16)
    table = torch.randperm(pages - 1, generator=g)[:S * pps].to(torch.int32) + 1
    q = (torch.randn(S, H, D, generator=g) * D**-0.5).to(torch.bfloat16)
    return q, cache, torch.tensor(kv_lens, dtype=torch.int32), table, torch.tensor([decodes, S, S], dtype=torch.int32)


def rpa_decode_float64(q, cache, kv_lens, table, distribution, sm_scale):
    """Each decode sequence's heads attending their kv head (h // (H / Hkv)) over positions below kv_len,
    in float64; the other rows are their queries."""
    S, H, D = q.shape
    ps, Hkv = cache.shape[1], cache.shape[2]
    pps = table.shape[0] // S
    out = q.double().clone()
    for s in range(S):
        n = int(kv_lens[s])
        if s >= int(distribution[0]) or n == 0:
            if s >= int(distribution[0]):
                continue
            out[s] = 0.0  # no positions: acc 0 over a clamped sum
            continue
        pos = torch.arange(n)
        pages = table[s * pps + pos // ps].long()
        k = cache[pages, pos % ps, :, 0, :].double()  # (n, Hkv, D)
        v = cache[pages, pos % ps, :, 1, :].double()
        for h in range(H):
            g = h // (H // Hkv)
            w = torch.softmax(sm_scale * (k[:, g, :] @ q[s, h].double()), 0)
            out[s, h] = w @ v[:, g, :]
    return out.numpy()


def test_rpa_write_and_decode():
    from examples.ragged_paged_attention import make_decode, rpa_write

    ins = write_inputs()
    cache, keys, values, table, page, first, stop, src = ins
    got = rpa_write.reference(cache, keys, values, table, page, src, first, stop, i32(3))
    assert torch.equal(got, write_expected(cache, keys, values, 3))
    compiles(rpa_write.lower(cache, keys, values, table, page, src, first, stop, i32(3)))
    decode = make_decode(0.5)
    q, cache, kv_lens, table, dist = rpa_inputs()
    want = rpa_decode_float64(q, cache, kv_lens, table, dist, 0.5)
    close(decode.reference(q, cache, kv_lens, table, dist), want, 2e-2, 2e-2)
    lowered = decode.lower(q, cache, kv_lens, table, dist)
    assert lowered.plan.walk and lowered.plan.aliases == {"out": 0}
    compiles(lowered)


def prefill_inputs(q_lens=(40, 25), kv_lens=(70, 25), H=8, Hkv=2, D=128, ps=64, pps=2, block_q=32, seed=1):
    """Prefill sequences' new queries (T, H, D), a paged cache holding them, and the prefill tiles: a tile per
    block of block_q queries of a sequence (first query at position kv_len - q_len)."""
    g = torch.Generator().manual_seed(seed)
    S, T = len(q_lens), sum(q_lens)
    pages = S * pps + 1
    cache = torch.randn(pages, ps, Hkv, 2, D, generator=g).to(torch.bfloat16)
    table = (torch.randperm(pages - 1, generator=g)[:S * pps] + 1).to(torch.int32)
    q = (torch.randn(T, H, D, generator=g) * D**-0.5).to(torch.bfloat16)
    tile_page, rows, pos, stop = [], [0], [], []
    start = 0
    for s, (ql, kl) in enumerate(zip(q_lens, kv_lens)):
        for b in range(0, ql, block_q):
            n = min(block_q, ql - b)
            tile_page.append(s * pps)
            rows.append(start + b + n)
            pos.append(kl - ql + b)
            stop.append(kl - ql + b + n)
        start += ql
    t = lambda v: torch.tensor(v, dtype=torch.int32)  # noqa: E731
    return q, cache, table, t(tile_page), t(rows), t(pos), t(stop), t([len(pos)])


def rpa_prefill_float64(q, cache, table, tile_page, tile_rows, tile_pos, tile_stop, n_tiles, sm_scale):
    """Each tile's queries attending causally (positions up to their own, below the stop) over their
    sequence's pages, head h to kv head h // (H / Hkv), in float64; rows of no tile keep their queries."""
    T, H, D = q.shape
    ps, Hkv = cache.shape[1], cache.shape[2]
    out = q.double().clone()
    for k in range(int(n_tiles[0])):
        for r in range(int(tile_rows[k]), int(tile_rows[k + 1])):
            own = int(tile_pos[k]) + r - int(tile_rows[k])
            n = min(own + 1, int(tile_stop[k]))
            pos = torch.arange(n)
            pages = table[int(tile_page[k]) + pos // ps].long()
            keys = cache[pages, pos % ps, :, 0, :].double()
            vals = cache[pages, pos % ps, :, 1, :].double()
            for h in range(H):
                gk = h // (H // Hkv)
                w = torch.softmax(sm_scale * (keys[:, gk, :] @ q[r, h].double()), 0)
                out[r, h] = w @ vals[:, gk, :]
    return out.numpy()


def test_rpa_prefill():
    from examples.ragged_paged_attention import PrefillTiles, make_prefill

    prefill = make_prefill(0.5, block_q=32)
    ins = prefill_inputs()
    want = rpa_prefill_float64(*ins, 0.5)
    close(prefill.reference(*ins, PrefillTiles(2)), want, 2e-2, 2e-2)
    lowered = prefill.lower(*ins, PrefillTiles(2))
    assert lowered.plan.walk and lowered.schedule.runtime_tiles
    compiles(lowered)
