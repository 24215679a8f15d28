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


def test_attention_splits_only_the_longest_items():
    """Split-KV: an item (128 query rows) is cut along the keys only above 1.5 shares of the work over the
    512 resident workgroups. At (1, 16, 4096, 128) the 96 items of 54..64 key blocks are split in two (a
    share is 35 blocks: 16896 blocks plus 2 per item, over 512); at (4, 16, 2048, 128) no item (at most 32
    blocks) reaches 1.5 shares of 38. The tuner's knob moves the threshold: never, or above one share."""
    from tilejax_amd.tune import Config
    from tilejax_amd import Pipeline

    blocks = AttentionBlocks(512, 512)
    for shape, split, chunks in (((1, 16, 4096, 128), 96, 192), ((4, 16, 2048, 128), 0, 0)):
        notes = causal_attention.lower(*(((shape), BF16) for _ in range(3)), blocks).program.notes
        assert (notes["split_items"], notes["chunks"]) == (split, chunks), shape
    sig = causal_attention.signature(*(((1, 16, 4096, 128), BF16) for _ in range(3)))
    never = causal_attention.lowered(sig, Config(blocks, Pipeline(2, 2), False, (("split", 0),))).program
    assert never.notes["split_items"] == 0 and "fa_merge" not in never.tables
    one = causal_attention.lowered(sig, Config(blocks, Pipeline(2, 2), False, (("split", 10),))).program
    # above one share: every item of 36 blocks or more, each cut into chunks of at most 35
    assert one.notes["split_items"] == 16 * 15
    items = one.tables["fa_items"].reshape(-1, 5 + 2 * one.notes["waves"])
    assert items[:, 3].max() <= 35


def test_causal_remainder_chunks_go_to_xcds_by_k_range():
    """Causal 8192^3 at 512^3 tiles: 528 computed 256^2 tiles on 256 workgroups, so the last 16 are cut into
    8 chunks of 16 K-slices. The chunks are handed out by K range, an XCD's 32 workgroups at a time
    (workgroup w runs on XCD w % 8): XCD x takes chunks 2x and 2x + 1 of all 16 tiles, so it reads those
    tiles' panels over two K ranges into its L2 once."""
    from examples.causal_matmul import causal_matmul

    prog = causal_matmul.lower(((8192, 8192), BF16), ((8192, 8192), BF16), MatmulTiles(512, 512, 512)).program
    assert prog.notes["split"] == (16, 8, 16)
    offsets, items = prog.tables["wg_items"], prog.tables["items"].reshape(-1, 3)
    seen = {}
    for w in range(len(offsets) - 1):
        for t, code, slot in items[offsets[w]:offsets[w + 1]]:
            if code >> 16 == 3:
                seen.setdefault(w % 8, set()).add(int(slot) % 8)
    assert seen == {x: {2 * x, 2 * x + 1} for x in range(4)}
    assert sum(1 for _, code, _ in items if code >> 16 == 3) == 128


def test_dense_rounds_give_each_xcd_a_patch_8_tiles_wide_and_4_high():
    """Dense 8192^3 at 512^3 tiles: 1024 256^2 tiles, four rounds of 256 workgroups. In every round, the 32
    tiles an XCD runs together (workgroup w runs on XCD w % 8) form one patch of 8 tile columns by 4 tile
    rows, so the XCD's L2 serves 12 operand panels for them, and the 8 XCDs' patches tile the output."""
    prog = matmul.lower(((8192, 8192), BF16), ((8192, 8192), BF16), MatmulTiles(512, 512, 512)).program
    offsets, items = prog.tables["wg_items"], prog.tables["items"].reshape(-1, 3)
    assert all(offsets[w + 1] - offsets[w] == 4 for w in range(256))
    sub_n = 2  # 256^2 sub-tiles of a 512^2 spec tile, 2 x 2
    for rnd in range(4):
        covered = set()
        for x in range(8):
            cells = set()
            for w in range(x, 256, 8):
                t, code, _ = (int(v) for v in items[offsets[w] + rnd])
                sm, sn = divmod(code & 0xFFFF, sub_n)
                cells.add(((t // 16) * 2 + sm, (t % 16) * 2 + sn))  # (tile row, tile column) of the output
            rows, cols = {r for r, _ in cells}, {c for _, c in cells}
            assert (len(cells), len(rows), len(cols)) == (32, 4, 8), (rnd, x)
            assert max(rows) - min(rows) == 3 and max(cols) - min(cols) == 7, (rnd, x)
            covered |= cells
        assert len(covered) == 256, rnd


def test_attention_stages_past_lds_are_refused_before_compiling():
    """Three LDS stages of 128-key blocks at head dim 128 would take 192 KiB (gfx950 has 160 KiB per CU):
    a KernelError on the host, so the tuner skips the shape, rather than a compiler error."""
    from tilejax_amd import Pipeline
    from tilejax_amd.tune import Config

    sig = causal_attention.signature(*(((1, 2, 1024, 128), BF16) for _ in range(3)))
    with pytest.raises(KernelError, match="LDS stages of 128 keys"):
        causal_attention.lowered(sig, Config(AttentionBlocks(512, 512), Pipeline(3, 2), False,
                                             (("bkv", 128), ("waves", 8)))).program


def test_decode_sets_up_query_rows_in_the_builders_launch():
    """Decode with step tables takes three launches: the step-table builder, whose launch carries the
    workgroups that set up each sequence's query rows, the attention kernel and the merge. With a cursor the
    attention kernel computes its waves' own query rows itself (knob "qrows", on with a cursor), so the call
    is two launches; without it a setup launch takes the builder's place. With the knob "fold", the
    attention kernel merges each sequence's partials itself (the last workgroup to finish it; a device
    counter per sequence)."""
    from examples.decode import paged_gqa_decode
    from tilejax_amd.codegen.steps import builder_groups
    from tilejax_amd.tune import Config

    I32 = jaxlite.int32
    sig = paged_gqa_decode.signature(((4, 1, 32, 128), BF16), ((256, 16, 1024), BF16), ((256, 16, 1024), BF16),
                                     ((4, 64), I32), ((4,), I32))
    tables = paged_gqa_decode.lowered(sig, paged_gqa_decode.default_config(sig)).program
    symbols = [ln.symbol for ln in tables.launches]
    assert symbols == ["tj_paged_gqa_decode_steps", "tj_paged_gqa_decode", "tj_paged_gqa_decode_merge"]
    assert not tables.notes["merge_folded"] and not tables.state
    words = 4 * 1  # 4 sequences x one 64-block word of their 64 pages
    assert tables.launches[0].grid[0] > builder_groups(words)  # the setup workgroups come after the builder's
    assert "xb_" in tables.source and "_setup(" not in tables.source
    assert not tables.notes["query_rows_in_kernel"] and "dc_q" in tables.workspace
    base = paged_gqa_decode.default_config(sig)
    cursor = paged_gqa_decode.lowered(sig, Config(base.tunable, base.pipeline, True)).program
    assert [ln.symbol for ln in cursor.launches] == ["tj_paged_gqa_decode", "tj_paged_gqa_decode_merge"]
    assert cursor.notes["query_rows_in_kernel"] and "dc_q" not in cursor.workspace and "dc_rows" in cursor.source
    staged = paged_gqa_decode.lowered(sig, Config(base.tunable, base.pipeline, True, (("qrows", 0),))).program
    assert [ln.symbol for ln in staged.launches] == ["tj_paged_gqa_decode_setup", "tj_paged_gqa_decode",
                                                      "tj_paged_gqa_decode_merge"]
    own_q = paged_gqa_decode.lowered(sig, Config(base.tunable, base.pipeline, False, (("qrows", 1),))).program
    assert own_q.launches[0].grid[0] == builder_groups(words) and "xb_" not in own_q.source
    assert "dc_q" not in own_q.workspace
    for use_cursor, first in ((False, ["tj_paged_gqa_decode_steps"]), (True, [])):
        folded = paged_gqa_decode.lowered(sig, Config(base.tunable, base.pipeline, use_cursor, (("fold", 1),))).program
        assert [ln.symbol for ln in folded.launches] == first + ["tj_paged_gqa_decode"]
        assert folded.notes["merge_folded"] and folded.state == {"dc_arrive": 4}
        assert "_merge(" not in folded.source and "__ATOMIC_RELEASE" in folded.source


def _decode_signature(kernel, B, T, H, Hkv, pages=64, P=16, D=128):
    I32 = jaxlite.int32
    return kernel.signature(((B, T, H, D), BF16), ((B * pages, P, Hkv * D), BF16), ((B * pages, P, Hkv * D), BF16),
                            ((B, pages), I32), ((B,), I32))


@pytest.mark.parametrize("T,H,Hkv,owners", [
    (1, 32, 8, [h // 4 for h in range(32)]),  # GQA: four query heads a kv head, a kv head a wave
    (1, 8, 8, list(range(8))),  # MHA: a head a wave
    (2, 16, 4, None),  # four kv heads: a head's 128 columns are two waves' spans of 64
])
def test_decode_waves_own_their_query_rows(T, H, Hkv, owners):
    """Where each query row's values sit in one wave's span of columns (found by running the spec's setup and
    epilogue eagerly), each wave scores its own rows and loads its own columns of V, and the kernel step has no
    workgroup barrier; elsewhere the waves share the scores through LDS."""
    from examples.decode import paged_gqa_decode
    from tilejax_amd.codegen import decode
    from tilejax_amd.tune import Config

    sig = _decode_signature(paged_gqa_decode, 4, T, H, Hkv)
    base = paged_gqa_decode.default_config(sig)
    lowered = paged_gqa_decode.lowered(sig, base)
    m = decode.match(lowered.plan)
    assert decode.row_owners(lowered.plan, m, m.width // decode.WAVES) == owners
    prog = lowered.program
    assert prog.notes["own_rows"] == (owners is not None)
    shared = paged_gqa_decode.lowered(sig, Config(base.tunable, base.pipeline, False, (("own", 0),))).program
    assert not shared.notes["own_rows"]
    if owners is None:
        assert prog.source == shared.source
        return
    assert "dc_owner" in prog.source and "dc_owner" not in shared.source
    # the shared kernel synchronises the workgroup every step; the own-rows kernel every SYNC_DEFAULT steps
    every = decode.SYNC_DEFAULT
    own2, own10, shared2, shared10 = [sum(ev[0] == "barrier" for ev in p.protocol.replay(n))
                                      for p in (prog, shared) for n in (2, 10)]
    assert own10 - own2 == -(-10 // every) - -(-2 // every) and shared10 - shared2 >= 8


@pytest.mark.parametrize("was,now", [
    # every query row dense across the width: no row has one wave's span
    ("block_diagonal(query_rows(q[b, :, :, :]), group, Hkv, dtype)",
     "jnp.tile(query_rows(q[b, :, :, :]), (1, Hkv)).astype(dtype)"),
    # the epilogue reads every row's first block, outside most rows' spans
    ("own_blocks(acc, group, Hkv)", "acc[:, :Dh]"),
    # the setup reads an index array, whose values the probe cannot know
    ("block_diagonal(query_rows(q[b, :, :, :]), group, Hkv, dtype)",
     "block_diagonal(query_rows(q[b, :, :, :]) * (lengths[b] > 0).astype(jnp.float32), group, Hkv, dtype)"),
])
def test_decode_rows_the_probe_does_not_give_to_one_wave(was, now):
    import inspect

    import examples.decode as ed
    from tests.helpers import make_kernel, spec

    source = inspect.getsource(ed.gqa_decode.fn.__wrapped__).split("\n", 1)[1]  # without the decorator
    assert was in source
    names = ("LANES", "MASK_VALUE", "row_index", "block_diagonal", "query_rows", "visible", "online_softmax",
             "finish", "own_blocks", "widen", "DecodeTiles")
    args = (spec(4, 1, 32, 128, dtype=BF16), spec(4, 2048, 1024, dtype=BF16), spec(4, 2048, 1024, dtype=BF16),
            spec(4, dtype=jaxlite.int32))
    assert make_kernel(source, **{n: getattr(ed, n) for n in names}).lower(*args).program.notes["own_rows"]
    prog = make_kernel(source.replace(was, now), **{n: getattr(ed, n) for n in names}).lower(*args).program
    assert prog.notes["family"] == "decode" and not prog.notes["own_rows"]


def test_tile_values_in_arithmetic_sequence_are_computed():
    """A runtime schedule's per-tile loop values are computed where they form an arithmetic sequence (no load
    then waits for them) and read from their table otherwise; the expression gives the table's values."""
    from types import SimpleNamespace

    import numpy as np

    from tilejax_amd.codegen.common import tile_value

    sch = SimpleNamespace(tile_values={"b": np.arange(64, dtype=np.int32), "g": np.array([256, 768, 1280], np.int32),
                                       "p": np.array([0, 1, 3], np.int32), "one": np.array([7], np.int32)})
    assert tile_value(sch, "b", "t") == "(0 + (t) * 1)"
    assert tile_value(sch, "one", "t") == "(7 + (t) * 0)"
    assert tile_value(sch, "p", "t") == "ak_ldc(args.tv_p, t)"
    expr = tile_value(sch, "g", "t")
    assert [eval(expr, {"t": t}) for t in range(3)] == [256, 768, 1280]
