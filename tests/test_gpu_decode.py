"""Parity of paged GQA decode (BASELINE.json config 5's spec, examples/decode.py) with the CPU oracle on the
same seeded inputs, of its device step tables with the reference's table semantics (bit-exact), and at
the size of BASELINE.json config 5 with a float32 GPU reference on sampled sequences.

Tolerance (tests/tolerance.py): bf16 outputs within 2 bf16 ulp of the expected value plus the softmax floor
(2^-8 + 2 n 2^-24 + 2 e_s) * softmax(s) @ |v|: the kernel merges per-workgroup partial softmaxes (the online
softmax's own rescaling rule) where the spec runs one pass per page, so the two differ in f32 summation
order and in which running maximum p is rounded to bf16 against.
"""

import numpy as np
import pytest
import torch

from examples.decode import paged_gqa_decode
from oracle import kernels
from oracle import schedule as oracle_schedule
from tests.tolerance import SOFTMAX_BAR, check_bf16, score_err, softmax_floor

pytestmark = pytest.mark.gpu


def _inputs(B, H, Hkv, D, P, pages, lengths, seed=0):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(B, 1, H, D, generator=g) * D**-0.5).to(torch.bfloat16)
    n_pages = B * pages
    k_pages = torch.randn(n_pages, P, Hkv * D, generator=g).to(torch.bfloat16)
    v_pages = torch.randn(n_pages, P, Hkv * D, generator=g).to(torch.bfloat16)
    table = torch.randperm(n_pages, generator=g).reshape(B, pages).to(torch.int32)
    return q, k_pages, v_pages, table, torch.tensor(lengths, dtype=torch.int32)


def _with_tables(kernel, ins):
    """The kernel as built from device step tables (its default; called on GPU tensors without a schedule,
    it is tuned, and tuning may choose a cursor)."""
    signature = kernel.signature(*ins)
    return kernel.lowered(signature, kernel.default_config(signature))


def _close(what, got, want, ins):
    """2 bf16 ulp plus the softmax floor of these inputs (q, k_pages, v_pages, table, lengths)."""
    q, kp, vp, table, lengths = ins
    weighted = torch.as_tensor(kernels.gqa_float64(q, kp, vp.float().abs(), table, lengths))
    floor = softmax_floor(weighted, int(lengths.max()), score_err(q, kp))
    check_bf16(what, got.cpu(), torch.as_tensor(want).cpu(), floor)


@pytest.mark.parametrize("lengths", [(0, 1, 300, 1024), (16, 17, 512, 999), (1024, 1024, 1024, 1024)])
def test_paged_decode_matches_oracle(lengths):
    ins = _inputs(4, 32, 8, 128, 16, 64, lengths)
    print(f"paged decode lengths={lengths}", flush=True)
    got = paged_gqa_decode(*(t.cuda() for t in ins))
    torch.cuda.synchronize()
    want = kernels.paged_gqa_decode(*ins)
    _close(f"paged decode lengths={lengths}", got, want, ins)
    for b, n in enumerate(lengths):
        if n == 0:
            assert not got[b].float().any()  # an empty sequence gives zeros


def test_paged_decode_against_float64():
    ins = _inputs(4, 32, 8, 128, 16, 64, (5, 100, 640, 1000), seed=3)
    got = paged_gqa_decode(*(t.cuda() for t in ins))
    _close("paged decode vs float64", got, kernels.gqa_float64(*ins), ins)


def test_decode_step_tables_are_bit_exact():
    lengths = (0, 1, 300, 1024)
    ins = _inputs(4, 32, 8, 128, 16, 64, lengths)
    lowered = _with_tables(paged_gqa_decode, ins)
    got = lowered.program.step_tables(*(t.cuda() for t in ins))
    step_tile, step_code, count = oracle_schedule.runtime_tables(
        [{"b": b} for b in range(4)], [("p", 0, 1, 64, lambda v: v["p"] * 16 >= lengths[v["b"]])])
    assert int(got["count"][0]) == count == 1 + 1 + 19 + 64
    np.testing.assert_array_equal(got["step_tile"].cpu().numpy(), step_tile)
    np.testing.assert_array_equal(got["step_code"].cpu().numpy(), step_code)


def test_decode_step_tables_ragged_words():
    """100 pages per sequence: two mask words per tile, the second partial; an empty sequence, a full one,
    and lengths either side of a word boundary (64 pages = 1024 positions)."""
    lengths = (0, 5, 1600, 1023, 1025)
    ins = _inputs(5, 32, 8, 128, 16, 100, lengths, seed=4)
    print(f"decode step tables lengths={lengths}", flush=True)
    lowered = _with_tables(paged_gqa_decode, ins)
    got = lowered.program.step_tables(*(t.cuda() for t in ins))
    step_tile, step_code, count = oracle_schedule.runtime_tables(
        [{"b": b} for b in range(5)], [("p", 0, 1, 100, lambda v: v["p"] * 16 >= lengths[v["b"]])])
    assert int(got["count"][0]) == count == 1 + 1 + 100 + 64 + 65
    np.testing.assert_array_equal(got["step_tile"].cpu().numpy(), step_tile)
    np.testing.assert_array_equal(got["step_code"].cpu().numpy(), step_code)
    tile_steps = got["tile_steps"].cpu().numpy()
    np.testing.assert_array_equal(tile_steps, np.cumsum([0, 1, 1, 100, 64, 65]))
    out = paged_gqa_decode(*(t.cuda() for t in ins))
    _close("paged decode, ragged words", out, kernels.paged_gqa_decode(*ins), ins)


def test_baseline_config_every_sequence():
    """64 sequences, 32 q heads / 8 kv heads, head dim 128, 16-token pages, a seeded
    random page table over 32768 pages, lengths uniform in [128, 8192]; every sequence checked against the
    CPU oracle (the spec's loop nest, p rounded to bf16 per page) to the softmax bar (tests/tolerance.py:
    SOFTMAX_BAR), with the floor from a float32 GPU computation of the same softmax applied to |v|."""
    B, H, Hkv, D, P, pages = 64, 32, 8, 128, 16, 512
    g = torch.Generator().manual_seed(0)
    lengths = torch.randint(128, 8193, (B,), generator=g, dtype=torch.int32)
    q_c = (torch.randn(B, 1, H, D, generator=g) * D**-0.5).to(torch.bfloat16)
    table_c = torch.randperm(B * pages, generator=g).reshape(B, pages).to(torch.int32)
    k_c = torch.randn(B * pages, P, Hkv * D, generator=g).to(torch.bfloat16)
    v_c = torch.randn(B * pages, P, Hkv * D, generator=g).to(torch.bfloat16)
    q, table, k_pages, v_pages = q_c.cuda(), table_c.cuda(), k_c.cuda(), v_c.cuda()
    print("paged decode 64 x 32/8 heads, lengths in [128, 8192]", flush=True)
    got = paged_gqa_decode(q, k_pages, v_pages, table, lengths.cuda()).cpu()
    print("paged decode config 5: the CPU oracle", flush=True)
    oracle = kernels.paged_gqa_decode(q_c, k_c, v_c, table_c, lengths)
    e_s = score_err(q, k_pages)
    want, floor = torch.empty(B, H, D), torch.empty(B, H, D, dtype=torch.float64)
    for b in range(B):
        n = int(lengths[b])
        idx = table[b, : -(-n // P)].long()
        kk = k_pages[idx].reshape(-1, Hkv, D)[:n].float().permute(1, 2, 0).contiguous()  # (g, d, n)
        vv = v_pages[idx].reshape(-1, Hkv, D)[:n].float().permute(1, 0, 2).contiguous()  # (g, n, d)
        qq = q[b, 0].float().reshape(Hkv, H // Hkv, D)
        p = torch.softmax(torch.bmm(qq, kk), -1)
        want[b] = torch.bmm(p, vv).reshape(H, D).cpu()
        floor[b] = softmax_floor(torch.bmm(p, vv.abs()).reshape(H, D), n, e_s).cpu()
    check_bf16("decode config 5, all 64 sequences, vs f32", got[:, 0], want, floor)
    check_bf16("decode config 5, all 64 sequences, vs oracle", got[:, 0], oracle[:, 0], floor, **SOFTMAX_BAR)


def test_decode_step_tables_bit_exact_at_baseline_size():
    """The builder at BASELINE.json config 5's size (64 sequences x 512 pages: 512 mask words, written by 16
    workgroups, each repeating the masks and the scan and writing its own words) against the reference's
    table semantics."""
    B, pages = 64, 512
    g = torch.Generator().manual_seed(0)
    lengths = torch.randint(128, 8193, (B,), generator=g, dtype=torch.int32)
    lengths[5], lengths[9] = 0, 8192  # an empty sequence and a full one
    ins = _inputs(B, 32, 8, 128, 16, pages, tuple(int(n) for n in lengths))
    lowered = _with_tables(paged_gqa_decode, ins)
    assert lowered.program.launches[0].grid[0] > 1
    got = lowered.program.step_tables(*(t.cuda() for t in ins))
    lens = [int(n) for n in lengths]
    step_tile, step_code, count = oracle_schedule.runtime_tables(
        [{"b": b} for b in range(B)], [("p", 0, 1, pages, lambda v: v["p"] * 16 >= lens[v["b"]])])
    assert int(got["count"][0]) == count == sum(max(1, -(-n // 16)) for n in lens)
    np.testing.assert_array_equal(got["step_tile"].cpu().numpy(), step_tile)
    np.testing.assert_array_equal(got["step_code"].cpu().numpy(), step_code)
    np.testing.assert_array_equal(got["tile_steps"].cpu().numpy(), np.cumsum([0] + [max(1, -(-n // 16)) for n in lens]))


def _cursor_run(kernel, ins):
    """The kernel built with a cursor (its attention kernel finds its steps itself) and with tables."""
    from tilejax_amd.tune import Config

    plain = _with_tables(kernel, ins)
    cursor = kernel.lowered(kernel.signature(*ins), Config(plain.config.tunable, plain.config.pipeline, True))
    # with tables, the builder's launch also sets up the query rows; with a cursor, the attention kernel
    # computes its waves' own rows (or, where the waves own none, a setup launch does)
    builders = [[ln.symbol.endswith("_steps") for ln in lt.program.launches] for lt in (plain, cursor)]
    assert cursor.program.notes["cursor"] and any(builders[0]) and not any(builders[1])
    in_kernel = cursor.program.notes["query_rows_in_kernel"]
    assert len(plain.program.launches) == 3 and len(cursor.program.launches) == (2 if in_kernel else 3)
    dev = [t.cuda() for t in ins]
    return plain.run(*dev), cursor.run(*dev)


@pytest.mark.parametrize("lengths, pages", [((0, 1, 300, 1024), 64), ((0, 5, 1600, 1023, 1025), 100)])
def test_cursor_equals_step_tables(lengths, pages):
    """With a cursor each workgroup evaluates the mask and finds its own steps; it takes the same steps in
    the same order as the device tables give, so the outputs agree bit for bit."""
    ins = _inputs(len(lengths), 32, 8, 128, 16, pages, lengths, seed=6)
    print(f"decode cursor vs tables lengths={lengths}", flush=True)
    tables, cursor = _cursor_run(paged_gqa_decode, ins)
    assert torch.equal(tables, cursor)
    _close(f"decode cursor lengths={lengths}", cursor, kernels.paged_gqa_decode(*ins), ins)


def test_cursor_at_baseline_size():
    B, pages = 64, 512
    g = torch.Generator().manual_seed(0)
    lengths = torch.randint(128, 8193, (B,), generator=g, dtype=torch.int32)
    lengths[5], lengths[9] = 0, 8192
    ins = _inputs(B, 32, 8, 128, 16, pages, tuple(int(n) for n in lengths))
    print("decode cursor vs tables at 64 x 512 pages", flush=True)
    tables, cursor = _cursor_run(paged_gqa_decode, ins)
    assert torch.equal(tables, cursor)


@pytest.mark.parametrize("cursor", [False, True])
def test_paged_decode_with_new_tokens(cursor):
    """Two new tokens per sequence (32 query rows: 2 tokens x 16 heads, 4 kv heads): token t sits at
    lengths[b] - 2 + t and sees the positions up to it (the reference's tests/test_decode.py:215-221)."""
    from tilejax_amd.tune import Config

    g = torch.Generator().manual_seed(11)
    B, T, H, Hkv, D, P, pages = 4, 2, 16, 4, 128, 16, 32
    q = (torch.randn(B, T, H, D, generator=g) * D**-0.5).to(torch.bfloat16)
    kp = torch.randn(B * pages, P, Hkv * D, generator=g).to(torch.bfloat16)
    vp = torch.randn(B * pages, P, Hkv * D, generator=g).to(torch.bfloat16)
    table = torch.randperm(B * pages, generator=g).reshape(B, pages).to(torch.int32)
    lengths = torch.tensor([2, 17, 300, 512], dtype=torch.int32)
    ins = (q, kp, vp, table, lengths)
    print(f"paged decode, two new tokens, cursor={cursor}", flush=True)
    plain = _with_tables(paged_gqa_decode, ins)
    lowered = paged_gqa_decode.lowered(paged_gqa_decode.signature(*ins),
                                       Config(plain.config.tunable, plain.config.pipeline, cursor))
    got = lowered.run(*(t.cuda() for t in ins))
    _close(f"decode two tokens cursor={cursor}", got, kernels.paged_gqa_decode(*ins), ins)
    _close(f"decode two tokens cursor={cursor} vs float64", got, kernels.gqa_float64(*ins), ins)


@pytest.mark.parametrize("buffers,cursor", [(2, False), (4, False), (2, True), (4, True)])
def test_depths_the_tuner_tries(buffers, cursor):
    """Decode with 2 and 4 steps fetched ahead (the pipeline's input buffers; the default is 3), from tables
    and with a cursor, against the oracle."""
    from tilejax_amd import Pipeline
    from tilejax_amd.tune import Config

    lengths = (0, 5, 1600, 1023, 1025)
    ins = _inputs(5, 32, 8, 128, 16, 100, lengths, seed=9)
    lowered = paged_gqa_decode.lowered(paged_gqa_decode.signature(*ins), Config(None, Pipeline(buffers, 2), cursor))
    print(f"paged decode depth {buffers} cursor={cursor}", flush=True)
    got = lowered.run(*(t.cuda() for t in ins))
    torch.cuda.synchronize()
    _close(f"paged decode depth {buffers} cursor={cursor}", got, kernels.paged_gqa_decode(*ins), ins)


@pytest.mark.parametrize("cursor", [False, True])
def test_waves_with_their_own_rows_are_bit_equal(cursor):
    """Each wave scores its own query rows against its own kv head's columns and loads its own columns of V
    (the default where the spec's rows are block-diagonal): every other column contributed exact zeros to
    those scores, so the output is bit-equal to the kernel whose waves share the scores through LDS."""
    from tilejax_amd.tune import Config

    g = torch.Generator().manual_seed(23)
    B, pages, P, W = 8, 128, 16, 1024
    q = (torch.randn(B, 1, 32, 128, generator=g) * 128 ** -0.5).to(torch.bfloat16).cuda()
    kp = torch.randn(B * pages, P, W, generator=g).to(torch.bfloat16).cuda()
    vp = torch.randn(B * pages, P, W, generator=g).to(torch.bfloat16).cuda()
    table = torch.randperm(B * pages, generator=g).reshape(B, pages).to(torch.int32).cuda()
    lengths = torch.tensor([0, 1, 17, 300, 2048, 777, 1500, 2000], dtype=torch.int32).cuda()
    ins = (q, kp, vp, table, lengths)
    sig = paged_gqa_decode.signature(*ins)
    base = paged_gqa_decode.default_config(sig)
    own = paged_gqa_decode.lowered(sig, Config(base.tunable, base.pipeline, cursor))
    shared = paged_gqa_decode.lowered(sig, Config(base.tunable, base.pipeline, cursor, (("own", 0),)))
    # without the barrier every few steps that keeps the waves together
    drifting = paged_gqa_decode.lowered(sig, Config(base.tunable, base.pipeline, cursor, (("sync", 0),)))
    # the query rows the other way: computed by the attention kernel (tables), or by a setup launch (cursor)
    other_q = paged_gqa_decode.lowered(sig, Config(base.tunable, base.pipeline, cursor, (("qrows", int(not cursor)),)))
    assert own.program.notes["own_rows"] and not shared.program.notes["own_rows"]
    assert own.program.notes["query_rows_in_kernel"] == cursor != other_q.program.notes["query_rows_in_kernel"]
    print(f"decode own rows vs shared scores, cursor={cursor}", flush=True)
    want = shared.run(*ins)
    got = own.run(*ins)
    unsynced = drifting.run(*ins)
    rows_other_way = other_q.run(*ins)
    torch.cuda.synchronize()
    assert torch.equal(got, want) and torch.equal(unsynced, want) and torch.equal(rows_other_way, want)


@pytest.mark.parametrize("cursor", [False, True])
def test_multi_head_decode_gives_each_wave_one_head(cursor):
    """MHA (8 query heads, 8 kv heads): 8 query rows, a row a wave, the kernel's other 24 rows owned by none;
    with a cursor the attention kernel computes each wave's one row itself."""
    from tilejax_amd.tune import Config

    ins = _inputs(4, 8, 8, 128, 16, 64, (0, 33, 700, 1024), seed=5)
    plain = _with_tables(paged_gqa_decode, ins)
    lowered = paged_gqa_decode.lowered(paged_gqa_decode.signature(*ins),
                                       Config(plain.config.tunable, plain.config.pipeline, cursor))
    assert lowered.program.notes["own_rows"] and lowered.program.notes["query_rows_in_kernel"] == cursor
    print(f"paged decode MHA 8 heads, cursor={cursor}", flush=True)
    got = lowered.run(*(t.cuda() for t in ins))
    torch.cuda.synchronize()
    _close(f"paged decode MHA cursor={cursor}", got, kernels.paged_gqa_decode(*ins), ins)


@pytest.mark.parametrize("cursor", [False, True])
def test_merge_in_the_attention_kernel_is_bit_equal(cursor):
    """The knob "fold" merges each sequence's partials in the attention kernel: the last workgroup to finish a
    sequence (a device counter per sequence, left at zero for the next call) merges it after an agent-scope
    acquire, each workgroup's partials released by one fence at its exit. The same partials summed in the
    same order: bit-equal to the merge launch's output, on two calls in a row (the counters reset)."""
    from tilejax_amd.tune import Config

    g = torch.Generator().manual_seed(21)
    B, pages, P, W = 8, 128, 16, 1024
    q = (torch.randn(B, 1, 32, 128, generator=g) * 128 ** -0.5).to(torch.bfloat16).cuda()
    kp = torch.randn(B * pages, P, W, generator=g).to(torch.bfloat16).cuda()
    vp = torch.randn(B * pages, P, W, generator=g).to(torch.bfloat16).cuda()
    table = torch.randperm(B * pages, generator=g).reshape(B, pages).to(torch.int32).cuda()
    lengths = torch.tensor([0, 1, 17, 300, 2048, 777, 1500, 2000], dtype=torch.int32).cuda()
    ins = (q, kp, vp, table, lengths)
    sig = paged_gqa_decode.signature(*ins)
    base = paged_gqa_decode.default_config(sig)
    plain = paged_gqa_decode.lowered(sig, Config(base.tunable, base.pipeline, cursor))
    folded = paged_gqa_decode.lowered(sig, Config(base.tunable, base.pipeline, cursor, (("fold", 1),)))
    assert folded.program.notes["merge_folded"] and not plain.program.notes["merge_folded"]
    print(f"decode merge folded, cursor={cursor}", flush=True)
    want = plain.run(*ins)
    for call in range(2):
        got = folded.run(*ins)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"call {call}"
    assert not folded.program.device_tables(q.device)["dc_arrive"].any()  # every counter back at zero
