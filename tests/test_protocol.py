"""The LDS ring protocol of the generated kernels, checked on the CPU (tilejax_amd/codegen/protocol.py).

Each kernel family records, as it emits the kernel's text, the waits, barriers, loads and reads of its loop;
the checker replays them for many block counts (matmul items back to back, as the persistent kernel runs
them) and requires every read to follow a wait and barrier that landed its block, and every load into a
stage to follow a wait and barrier after the reads of the block it replaces. This stands in for the
reference's interpreter race detector (tests/helpers.py:26-35 of the reference), which has no gfx950
counterpart. A planted mistake in each family's events (a barrier dropped, a wait loosened) must fail.
"""

import pytest

from examples.causal_attention import AttentionBlocks, causal_attention
from examples.causal_matmul import causal_matmul
from examples.decode import paged_gqa_decode
from examples.matmul import MatmulTiles, matmul
from examples.moe import GroupTiles, grouped_matmul
from tests.helpers import spec
from tilejax_amd import Pipeline, jaxlite
from tilejax_amd.codegen.protocol import ItemRecorder, ProtocolError, check, loads_reads
from tilejax_amd.tune import Config

BF, F32, I32 = jaxlite.bfloat16, jaxlite.float32, jaxlite.int32


def _lowered(kernel, args, tunable, buffers=2, hardware=(), cursor=False):
    return kernel.lowered(kernel.signature(*args), Config(tunable, Pipeline(buffers, 2), cursor, hardware))


def _matmul_cases():
    sq = (spec(1024, 1024, dtype=BF), spec(1024, 1024, dtype=BF))
    for buffers in (2, 3, 4):
        for hw in ((), (("bm", 256), ("bn", 128)), (("bm", 128), ("bn", 128))):
            yield f"matmul b{buffers} {hw}", _lowered(matmul, sq, MatmulTiles(512, 512, 512), buffers, hw)
    yield "causal", _lowered(causal_matmul, sq, MatmulTiles(512, 512, 512))
    yield "matmul tk 32", _lowered(matmul, sq, MatmulTiles(256, 256, 32))
    yield "matmul f32", _lowered(matmul, (spec(256, 384, dtype=F32), spec(384, 256, dtype=F32)), MatmulTiles(128, 128, 128))
    yield "grouped", _lowered(grouped_matmul, (spec(1024, 512, dtype=BF), spec(4, 512, 1024, dtype=BF), spec(4, dtype=I32)),
                              GroupTiles(512, 256))


@pytest.mark.parametrize("name,lowered", list(_matmul_cases()), ids=lambda x: x if isinstance(x, str) else "")
def test_matmul_ring(name, lowered):
    """A workgroup's items back to back: the next loading item's first slices go into the stages during the
    current item's last ones; items without slices (a tile without steps) load nothing in between."""
    prog = lowered.program
    rec, stages = prog.protocol, prog.notes["stages"]
    assert isinstance(rec, ItemRecorder)
    covered = set()
    for rounds in (1, 2, 3, 5):
        T = rounds * stages  # slices per item: the kernel's loop takes whole rounds of its stages
        for counts in ([T], [T, T, 2 * T], [T, 0, T], [0, T, 0, 0, 3 * T], [2 * T, T, 0]):
            events = rec.replay(counts)
            check(events, f"{name}, items of {counts} slices")
            covered |= loads_reads(events)
            assert events[-1] == ("wait_vm", 0)  # nothing in flight when the workgroup ends
    assert covered == {(k, s) for k in ("load", "read") for s in range(stages)}


def test_matmul_items_prefetch_the_next():
    """The second item's first slices are loaded during the first item (no load at its start), and a
    dropped barrier at an item's start, or a dropped refill barrier, fails the check."""
    sq = (spec(1024, 1024, dtype=BF), spec(1024, 1024, dtype=BF))
    rec = _lowered(matmul, sq, MatmulTiles(512, 512, 512)).program.protocol
    events = rec.replay([4, 4])
    loads = [i for i, ev in enumerate(events) if ev[0] == "load"]
    second_first = [i for i, ev in enumerate(events) if ev[0] == "load" and ev[2] == 4]
    first_read_of_second = next(i for i, ev in enumerate(events) if ev[0] == "read" and ev[2] == 4)
    assert second_first and second_first[0] < first_read_of_second
    assert len(loads) == 2 + 4 + 4  # the first item's fill, then one refill per slice, no second fill
    check(events, "two items")
    barriers = [i for i, ev in enumerate(events) if ev[0] == "barrier"]
    # the first item's fill barrier guards its first read; each refill barrier (followed by a load into the
    # stage just read) guards that load, the next item's included
    needed = [1] + [k + 1 for k, i in enumerate(barriers) if events[i + 1][0] == "load"]
    assert len(needed) == 1 + 8
    for k in needed:
        with pytest.raises(ProtocolError):
            check(_drop(events, "barrier", k), f"without barrier {k}")


def _flash_cases():
    args = tuple(spec(2, 4, 1024, 128, dtype=BF) for _ in range(3))
    for buffers in (2, 3, 4):
        for hw in ((), (("bkv", 32), ("waves", 8))):
            yield f"attention b{buffers} {hw}", _lowered(causal_attention, args, AttentionBlocks(256, 256), buffers, hw)


@pytest.mark.parametrize("name,lowered", list(_flash_cases()), ids=lambda x: x if isinstance(x, str) else "")
def test_attention_ring(name, lowered):
    rec = lowered.program.protocol
    for nblk in range(0, 14):
        check(rec.replay(nblk), f"{name}, {nblk} blocks")


@pytest.mark.parametrize("buffers,cursor", [(2, False), (3, False), (4, False), (3, True)])
def test_decode_rings(buffers, cursor):
    args = (spec(5, 1, 32, 128, dtype=BF), spec(500, 16, 1024, dtype=BF), spec(500, 16, 1024, dtype=BF),
            spec(5, 100, dtype=I32), spec(5, dtype=I32))
    rec = _lowered(paged_gqa_decode, args, None, buffers, cursor=cursor).program.protocol
    for steps in range(1, 14):
        check(rec.replay(steps), f"decode depth {buffers}, {steps} steps")


def _drop(events, kind, which=1):
    """The events with the `which`-th event of `kind` removed."""
    seen = 0
    for i, ev in enumerate(events):
        if ev[0] == kind:
            seen += 1
            if seen == which:
                return events[:i] + events[i + 1:]
    raise AssertionError(f"no {which}th {kind}")


def _loosen(events, which=2):
    """The `which`-th wait for loads allowed one more instruction in flight."""
    seen = 0
    out = list(events)
    for i, ev in enumerate(out):
        if ev[0] == "wait_vm":
            seen += 1
            if seen == which:
                out[i] = ("wait_vm", ev[1] + 1)
                return out
    raise AssertionError("no such wait")


def test_planted_mistakes_fail():
    sq = (spec(1024, 1024, dtype=BF), spec(1024, 1024, dtype=BF))
    mm = _lowered(matmul, sq, MatmulTiles(512, 512, 512)).program.protocol.replay([8, 8])
    fa = _lowered(causal_attention, tuple(spec(2, 4, 1024, 128, dtype=BF) for _ in range(3)),
                  AttentionBlocks(256, 256)).program.protocol.replay(6)
    args = (spec(5, 1, 32, 128, dtype=BF), spec(500, 16, 1024, dtype=BF), spec(500, 16, 1024, dtype=BF),
            spec(5, 100, dtype=I32), spec(5, dtype=I32))
    dc = _lowered(paged_gqa_decode, args, None, 3, (("own", 0),)).program.protocol.replay(8)
    for name, events in (("matmul", mm), ("attention", fa), ("decode", dc)):
        check(events, name)
        with pytest.raises(ProtocolError):  # (the first block's barriers can be redundant)
            check(_drop(events, "barrier", 3), f"{name} without its third barrier")
        with pytest.raises(ProtocolError):
            check(_loosen(events, 2), f"{name} with a loose wait")
    with pytest.raises(ProtocolError, match="still read"):  # the matmul's wait for its LDS reads dropped
        check(_drop(mm, "wait_lgkm", 1), "matmul without a read wait")


@pytest.mark.parametrize("cursor,sync", [(False, None), (True, None), (False, 0), (False, 3)])
def test_decode_waves_with_their_own_rows(cursor, sync):
    """Decode whose waves own their query rows: each wave loads its own columns of V into a region of the stage
    only it reads ("read_mine"), so its own waits order its loads and reads, and the only barrier is the one
    every `sync` steps that keeps the waves together. A wait loosened, or the wait for the reads before the
    region's next load dropped, must fail."""
    from tilejax_amd.codegen.decode import SYNC_DEFAULT

    args = (spec(5, 1, 32, 128, dtype=BF), spec(500, 16, 1024, dtype=BF), spec(500, 16, 1024, dtype=BF),
            spec(5, 100, dtype=I32), spec(5, dtype=I32))
    hw = () if sync is None else (("sync", sync),)
    every = SYNC_DEFAULT if sync is None else sync
    prog = _lowered(paged_gqa_decode, args, None, 3, hw, cursor=cursor).program
    assert prog.notes["own_rows"]
    for steps in range(1, 20):
        events = prog.protocol.replay(steps)
        check(events, f"decode with own rows, {steps} steps")
        assert sum(ev[0] == "barrier" for ev in events) == (-(-steps // every) if every else 0)
        assert {ev[0] for ev in events} >= {"read_mine", "read_own"} and not any(ev[0] == "read" for ev in events)
    events = prog.protocol.replay(8)
    with pytest.raises(ProtocolError, match="before its loads landed"):
        check(_loosen(events, 2), "own rows with a loose wait")
    with pytest.raises(ProtocolError, match="still read"):
        check(_drop(events, "wait_lgkm", 1), "own rows without a read wait")
