"""The generic gfx950 kernel walking plans of the tile as written (tilejax_amd/walk.py), against float64
closed forms: repeat loops, runtime loop bounds and a runtime count of tiles, ragged rows, windows gathered
through index-array slices, outputs updated in place and scattered, outputs stored per step, and index
arrays the tile code computes (routing inside a kernel). The cases and closed forms are tests/test_walk.py's.

Tolerance: f32 results within the reference's own f32 bounds for these tests (rtol 1e-4 plus 1e-3, or 1e-5
plus 1e-4 for sums of a few terms; tests/test_repeat_loops.py, test_runtime_ranges.py of the reference);
integer-placed results (scatters, copies, in-place outputs) exactly where no arithmetic happens. The bf16
ragged case within rtol 1e-2 (2 bf16 ulp) of float64.
"""

import numpy as np
import pytest
import torch

import tilejax_amd
from tests.helpers import make_kernel, rand
from tests.test_walk import (FFN_STACK, GATHER, LAYERED, MASKED_IN_PLACE, MOE, NESTED, OFFSETS, ONCE_PER_TILE,
                             RAGGED, SCAN, SCATTER, SPANS, WRAPPED, wrapped_float64, STATIC_RAGGED, SUMS, TWO_REPEATS, COUNTED, PICKED, EARLY, CHOSEN,
                             MIXED_MASKS, ONE_LAYER_STEPS, RUNTIME_IN_REPEAT, chosen_float64, chosen_inputs,
                             ONLY_IN_PLACE, RAGGED_BOTH, PAIRS_PER_ITERATION, only_in_place_float64,
                             ragged_both_float64, pairs_per_iteration_float64,
                             counted_float64, mixed_masks_float64, runtime_in_repeat_float64,
                             ffn_inputs, ffn_stack_float64, gather_float64, i32, layered_float64, moe_inputs,
                             picked_float64, early_float64,
                             once_per_tile_float64, ragged_float64, route, routed_float64, scan_float64,
                             scatter_float64, spans_float64, sums_float64, two_repeats_float64)

pytestmark = pytest.mark.gpu


def run(kernel, *inputs, what):
    print(f"walk: {what} {[tuple(t.shape) for t in inputs if isinstance(t, torch.Tensor)]}", flush=True)
    lowered = kernel.lower(*inputs)
    assert lowered.plan.walk and lowered.program.notes["family"] == "generic"
    got = lowered.run(*(t.cuda() for t in inputs if isinstance(t, torch.Tensor)))
    torch.cuda.synchronize()
    return tuple(g.cpu() for g in got) if isinstance(got, tuple) else got.cpu()


def close(got, want, rtol=1e-4, atol=1e-3):
    got = np.asarray(got.double())
    err = np.abs(got - want)
    bad = err > atol + rtol * np.abs(want)
    assert not bad.any(), f"{int(bad.sum())} of {bad.size} differ; max |diff| {err.max():.3g}"
    print(f"  max |diff| {err.max():.3g}", flush=True)


def test_repeat_loop_carries_layers():
    inputs = ffn_inputs()
    close(run(make_kernel(FFN_STACK), *inputs, what="ffn_stack"), ffn_stack_float64(*inputs))


@pytest.mark.parametrize("limits", [(256, 0, 100), (0, 0, 0)])
def test_reductions_around_and_in_a_repeat_loop_with_masks(limits):
    x, w = rand((256, 256)), rand((3, 384, 128), 1) / 20
    got = run(make_kernel(LAYERED), x, w, i32(*limits), what=f"layered {limits}")
    close(got, layered_float64(x, w, limits))


def test_two_repeat_loops():
    x, w = rand((128, 128)), rand((2, 256, 128), 1)
    close(run(make_kernel(TWO_REPEATS), x, w, what="two repeats"), two_repeats_float64(x, w))


def test_runtime_ranges():
    cache, lengths = rand((4, 512, 128)), i32(0, 1, 300, 512)
    close(run(make_kernel(SUMS), cache, lengths, what="sums"), sums_float64(cache, lengths), 1e-5, 1e-4)
    x, w = rand((3, 64, 128)), rand((256, 128), 1)
    lo, hi = i32(0, 8, 16), i32(16, 8, 64)
    close(run(make_kernel(SPANS), x, w, lo, hi, what="spans"), spans_float64(x, w, lo, hi), 1e-5, 1e-4)
    x, n = rand((3, 4, 8, 128)), i32(2, 4, 9)
    close(run(make_kernel(COUNTED), x, n, what="counted"), counted_float64(x, n), 1e-5, 1e-4)


def test_ragged_rows_and_a_runtime_count_of_tiles():
    kernel = make_kernel(RAGGED, tilejax_amd=tilejax_amd)
    q = rand((64, 8, 128), dtype=torch.bfloat16)
    rows = i32(0, 5, 21, 37, 40, 40, 40)
    for n in (4, 6, 0):  # (6: two empty tiles; 0: no tiles, the input as it was)
        got = run(kernel, q, rows, i32(n), what=f"ragged n={n}")
        close(got, ragged_float64(q, rows, i32(n)), 1e-2, 0)
    got = run(make_kernel(STATIC_RAGGED, tilejax_amd=tilejax_amd), rand((48, 8, 128)), i32(0, 16, 20, 36),
              what="static ragged")
    want = np.asarray(rand((48, 8, 128)).double())
    want[:36] *= 3
    close(got, want, 1e-5, 1e-5)


def test_gathered_and_nested_windows():
    pages, w, table = rand((10, 8, 128)), rand((10, 8, 128), 1), i32(3, 1, 4, 1, 5, 9, 2, 6)
    close(run(make_kernel(GATHER), pages, table, w, what="gather"), gather_float64(pages, table, w), 1e-5, 1e-4)
    pages, table, first, n = rand((6, 8, 128)), i32(5, 4, 3, 2), i32(0, 3), i32(2, 2)
    want = np.stack([np.asarray(pages[5].double() + pages[4].double()), np.asarray(2 * pages[2].double())])
    close(run(make_kernel(NESTED), pages, table, first, n, what="nested"), want, 1e-5, 1e-4)


def test_scatter_into_an_input_updated_in_place():
    x, pool, slots = rand((3, 16, 128)), rand((7, 16, 128), 1), i32(5, 0, 2)
    out, new = run(make_kernel(SCATTER), x, pool, slots, what="scatter")
    want_out, want_new = scatter_float64(x, pool, slots)
    close(out, want_out, 0, 0)  # (x2: exact)
    close(new, want_new, 1e-6, 0)
    assert torch.equal(new[[1, 3, 4, 6]], pool[[1, 3, 4, 6]])  # the slots no tile stores, as they were


def test_negative_indices_and_stores_outside_the_array():
    """Slots (-1, 7, 2): the pool's last row, a dropped update (past the 7 rows), row 2; shift[b - 1] at b = 0
    reads shift's last element; the row index -2 counts from the end. Exact (x2 plus one value)."""
    x, pool, slots, shift = rand((3, 16, 128)), rand((7, 16, 128), 1), i32(-1, 7, 2), i32(4, -2, 5)
    new = run(make_kernel(WRAPPED), x, pool, slots, shift, what="negative indices")
    close(new, wrapped_float64(x, pool, slots, shift), 1e-6, 0)
    assert torch.equal(new[[0, 1, 3, 4, 5]], pool[[0, 1, 3, 4, 5]])


def test_masked_tiles_of_an_input_updated_in_place_keep_its_values():
    x = rand((256, 256))
    out, new = run(make_kernel(MASKED_IN_PLACE), x, what="masked in place")
    keep = np.kron(np.tril(np.ones((2, 2))), np.ones((128, 128))).astype(bool)
    close(out, np.where(keep, np.asarray(x.double()) + 1, 0.0), 1e-6, 0)
    close(new, np.where(keep, np.asarray(x.double()) * 3, np.asarray(x.double())), 1e-6, 0)


def test_a_scan_stores_a_tile_per_step():
    x, w = rand((512, 256)), rand((128, 128), 1) / 16
    got = run(make_kernel(SCAN), x, w, what="scan")
    for g, want in zip(got, scan_float64(x, w)):
        close(g, want, 1e-4, 1e-4)


def test_routing_inside_the_kernel():
    kernel = make_kernel(MOE, route=route)
    for seed in (0, 3):
        x, router, w = moe_inputs(seed)
        close(run(kernel, x, router, w, what=f"routed seed {seed}"), routed_float64(x, router, w), 2e-4, 2e-4)


def test_an_element_index_the_tile_code_computes():
    x = rand((512, 128))
    for ids in (i32(2, 0, 7, 1), i32(3, 3, 0, 9)):
        close(run(make_kernel(PICKED), x, ids, what=f"picked {ids.tolist()}"), picked_float64(x, ids), 1e-6, 0)


def test_windows_placed_by_an_array_made_before_the_loop():
    x = rand((2, 8, 128))
    close(run(make_kernel(EARLY), x, what="early"), early_float64(x), 1e-6, 1e-6)


def test_padding_iterations_and_layers_of_one_step():
    ins = chosen_inputs()
    close(run(make_kernel(CHOSEN), *ins, what="chosen"), chosen_float64(*ins), 1e-4, 1e-3)
    for source, layers in ((ONE_LAYER_STEPS, 3), (FFN_STACK, 1)):
        ins = ffn_inputs(layers)
        close(run(make_kernel(source), *ins, what=f"ffn layers={layers}"), ffn_stack_float64(*ins))


def test_runtime_ranges_in_repeat_loops_and_mixed_masks():
    x, n = rand((8, 384)), i32(2, 384, 0, 256)
    close(run(make_kernel(RUNTIME_IN_REPEAT), x, n, what="runtime in repeat"), runtime_in_repeat_float64(x, n),
          1e-5, 1e-5)
    x, n, lengths = rand((24, 512)), i32(256), i32(512, 0, 200)
    close(run(make_kernel(MIXED_MASKS), x, n, lengths, what="mixed masks"), mixed_masks_float64(x, n, lengths),
          1e-5, 1e-5)


def test_in_place_ragged_and_pairs_forms():
    x = rand((256, 128))
    close(run(make_kernel(ONLY_IN_PLACE), x, what="only in place"), only_in_place_float64(x), 1e-6, 0)
    x, y, n = rand((20, 256)), rand((8, 512)), i32(4, 9, 128, 300)
    got = run(make_kernel(RAGGED_BOTH, tilejax_amd=tilejax_amd), x, y, n, what="ragged both dims")
    close(got, ragged_both_float64(x, y, n), 1e-6, 0)
    kv, x = rand((2, 16, 2, 128), dtype=torch.bfloat16), rand((2, 32, 128))
    got = run(make_kernel(PAIRS_PER_ITERATION, tilejax_amd=tilejax_amd), kv, x, what="pairs per iteration")
    close(got, pairs_per_iteration_float64(kv, x), 1e-5, 1e-5)


def test_indices_made_once_per_tile():
    x = rand((5, 16, 256))
    got = run(make_kernel(ONCE_PER_TILE, OFFSETS=OFFSETS), x, what="once per tile")
    close(got, once_per_tile_float64(x), 1e-5, 1e-4)


def test_pairs_and_word_stores():
    from tests.test_walk import PAIRS, WRITE, pairs_float64, write_expected, write_inputs

    kv, table = rand((5, 16, 4, 2, 128), dtype=torch.bfloat16), i32(4, 0, 2, 3)
    print("generic: pairs", flush=True)
    got = make_kernel(PAIRS, tilejax_amd=tilejax_amd).lower(kv, table).run(kv.cuda(), table.cuda())
    torch.cuda.synchronize()
    close(got.cpu(), pairs_float64(kv, table), 1e-5, 1e-4)
    ins = write_inputs()
    for n in (3, 0):  # (0: no runs, the cache as it was)
        got = run(make_kernel(WRITE, tilejax_amd=tilejax_amd), *ins, i32(n), what=f"word stores n={n}")
        assert torch.equal(got, write_expected(*ins[:3], n))  # bits moved, nothing computed: exact


def test_ragged_paged_attention_write_and_decode():
    """The reference's RPA cache write and decode kernels (examples/ragged_paged_attention.py): the write
    exact, the decode within 2e-2 of float64 (bf16 p and outputs; the reference's attention tolerance)."""
    from examples.ragged_paged_attention import make_decode, rpa_write
    from tests.test_walk import rpa_decode_float64, rpa_inputs, write_expected, write_inputs

    cache, keys, values, table, page, first, stop, src = write_inputs()
    got = run(rpa_write, cache, keys, values, table, page, src, first, stop, i32(3), what="rpa_write")
    assert torch.equal(got, write_expected(cache, keys, values, 3))
    decode = make_decode(0.5)
    for lens, decodes in (((20, 64, 5, 0), 2), ((33, 1, 64, 17), 4)):
        ins = rpa_inputs(lens, decodes)
        got = run(decode, *ins, what=f"rpa_decode kv_lens={lens} decodes={decodes}")
        close(got, rpa_decode_float64(*ins, 0.5), 2e-2, 2e-2)
        rows = torch.arange(len(lens)) >= decodes
        assert torch.equal(got[rows], ins[0][rows])  # the other rows keep their queries


def test_ragged_paged_attention_prefill():
    """RPA's prefill kernel (the reference's examples/ragged_paged_attention.py make_prefill): tiles of a
    sequence's queries counted as the kernel runs, ragged rows, pages gathered two a step through the page
    table, causal GQA attention; within 2e-2 of float64, rows of no tile exactly their queries."""
    from examples.ragged_paged_attention import PrefillTiles, make_prefill
    from tests.test_walk import prefill_inputs, rpa_prefill_float64

    prefill = make_prefill(0.5, block_q=32)
    for q_lens, kv_lens in (((40, 25), (70, 25)), ((33, 7), (100, 7))):
        ins = prefill_inputs(q_lens, kv_lens)
        got = run(prefill, *ins, PrefillTiles(2), what=f"rpa_prefill q_lens={q_lens} kv_lens={kv_lens}")
        close(got, rpa_prefill_float64(*ins, 0.5), 2e-2, 2e-2)
