"""A check of the LDS ring protocol of a generated kernel, on the CPU.

The matmul, attention and decode kernels stream operand blocks through LDS stages: a block's loads
(`buffer_load ... lds`, counted by vmcnt) go into a stage while the waves compute on others; a wave waits
for its own loads (`s_waitcnt vmcnt(n)`: all but its last n load instructions have landed) and its LDS reads
(`s_waitcnt lgkmcnt(0)`), and `s_barrier` makes every wave's progress visible to the others. The reference
checks its kernels' copies and semaphores by running them in an interpreter with a race detector and
NaN-filled buffers; here each family's generator records, as it emits the kernel's text, the events of its
loop (the same calls that write the waits, barriers, loads and reads), and `check` replays them for a number
of blocks, as every wave runs them, and enforces:

- read after load: a read of (stage, block) comes after a barrier that every wave reaches after a wait that
  completed its own loads of that block into that stage (and no other block was loaded into the stage
  since);
- load after read: a load into a stage comes after a barrier that every wave reaches after a wait that
  completed its own reads of the block the stage held.

Events are tuples: ("load", stage, block, instructions), ("read", stage, block), ("wait_vm", n),
("wait_lgkm",), ("barrier",); a "stage" may also be a set of registers a wave loads for itself, used with
("read_own", stage, block), which needs only that wave's wait, or an LDS region only its own wave loads and
reads, used with ("read_mine", stage, block): a read needs that wave's wait for the loads, and a later load
into the region needs its wait for the reads (wait_lgkm), no barrier. A loop is recorded once per position of its unrolled body, with the block as an
offset from the loop's block variable and a condition on it; `Recorder.replay` instantiates it.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Callable, Dict, List, Optional, Sequence, Set, Tuple

__all__ = ["ProtocolError", "Recorder", "ItemRecorder", "check"]


class ProtocolError(AssertionError):
    """The kernel's waits and barriers don't order its LDS loads and reads."""


Event = Tuple


@dataclass
class _Stage:
    block: Optional[int] = None  # the block whose loads went into the stage last
    loaded: bool = False  # those loads completed (this wave) ...
    visible: bool = False  # ... and a barrier since: every wave's loads of it completed
    reads: List[str] = field(default_factory=list)  # this block's reads: "issued", "done" (this wave), "all"


def check(events: Sequence[Event], what: str = "kernel") -> None:
    """Replay one wave's events (every wave runs the same ones); ProtocolError at the first violation."""
    stages: Dict[int, _Stage] = {}
    outstanding: List[Tuple[int, int, int]] = []  # (stage, block, instructions) of loads not yet waited for
    for at, ev in enumerate(events):
        kind = ev[0]
        if kind == "load":
            _, s, b, n = ev
            st = stages.setdefault(s, _Stage())
            if st.block is not None and any(r not in ("all", "mine_done") for r in st.reads):
                raise ProtocolError(f"{what}: event {at}: block {b} is loaded into stage {s} while a wave may still "
                                    f"read block {st.block} there (no wait and barrier after its reads)")
            if any(o[0] == s for o in outstanding):
                raise ProtocolError(f"{what}: event {at}: block {b} is loaded into stage {s} while block "
                                    f"{st.block}'s loads into it are still in flight")
            stages[s] = _Stage(block=b)
            outstanding.append((s, b, n))
        elif kind == "wait_vm":
            # all but the most recent `keep` load instructions have landed (they land in order): a block's
            # loads are done when at least `keep` instructions were issued after its last one
            keep, after = ev[1], 0
            remaining: List[Tuple[int, int, int]] = []
            for o in reversed(outstanding):
                if after >= keep:
                    if stages[o[0]].block == o[1]:
                        stages[o[0]].loaded = True
                else:
                    remaining.append(o)
                after += o[2]
            outstanding = remaining[::-1]
        elif kind == "wait_lgkm":
            for st in stages.values():
                st.reads = ["done" if r == "issued" else "mine_done" if r == "mine_issued" else r for r in st.reads]
        elif kind == "barrier":
            for st in stages.values():
                if st.loaded:
                    st.visible = True
                st.reads = ["all" if r == "done" else r for r in st.reads]
        elif kind in ("read", "read_own", "read_mine"):
            _, s, b = ev
            st = stages.get(s)
            if st is None or st.block != b:
                held = None if st is None else st.block
                raise ProtocolError(f"{what}: event {at}: block {b} is read from stage {s}, which holds block {held}")
            if kind == "read_own":  # registers the wave loaded itself: its own wait suffices
                if not st.loaded:
                    raise ProtocolError(f"{what}: event {at}: block {b} is used from {s} before its loads landed")
                st.reads.append("all")
                continue
            if kind == "read_mine":  # an LDS region only this wave loads: its own waits order loads and reads
                if not st.loaded:
                    raise ProtocolError(f"{what}: event {at}: block {b} is read from {s} before its loads landed")
                st.reads.append("mine_issued")
                continue
            if not st.visible:
                raise ProtocolError(f"{what}: event {at}: block {b} is read from stage {s} before every wave's loads "
                                    "of it are known to have landed (a wait, then a barrier)")
            st.reads.append("issued")
        else:
            raise ValueError(f"unknown protocol event {ev!r}")


@dataclass
class Recorder:
    """Events as a generator emits them: straight-line events (`add`) and the events of an unrolled loop's
    positions (`at(position, ...)`), each with a condition on the block index. `replay(nblocks)` gives the
    event sequence for a kernel that takes `nblocks` blocks."""

    prologue: List[Tuple[Event, Callable[[int], bool]]] = field(default_factory=list)
    body: Dict[int, List[Tuple[Callable[[int, int], Event], Callable[[int, int], bool]]]] = field(default_factory=dict)
    epilogue: List[Tuple[Event, Callable[[int], bool]]] = field(default_factory=list)
    unroll: int = 1
    after: bool = False  # `end_loop` ran: straight-line events go after the loop

    def add(self, event: Event, when: Callable[[int], bool] = lambda n: True) -> None:
        """A straight-line event (before the loop, or after it once `end_loop` ran); `when(nblocks)`."""
        (self.epilogue if self.after else self.prologue).append((event, when))

    def loop(self, unroll: int) -> None:
        self.unroll = unroll

    def at(self, position: int, event: Callable[[int, int], Event],
           when: Callable[[int, int], bool] = lambda b, n: True) -> None:
        """An event of the loop body at unrolled position `position`, made from the block index and the
        block count; it happens when `when(block, nblocks)` (the code's own condition)."""
        self.body.setdefault(position, []).append((event, when))

    def end_loop(self) -> None:
        self.after = True

    def replay(self, nblocks: int) -> List[Event]:
        out = [ev for ev, when in self.prologue if when(nblocks)]
        for b in range(nblocks):
            for make, when in self.body.get(b % self.unroll, []):
                if when(b, nblocks):
                    out.append(make(b, nblocks))
        out += [ev for ev, when in self.epilogue if when(nblocks)]
        return out


@dataclass
class ItemRecorder:
    """Events of a persistent kernel whose work items each walk their own blocks through the same LDS stages,
    the next item's first blocks loaded during the current item's last ones. An event maker takes the
    item's block count `n`, whether a next item that loads follows (`nxt`), the block index `b` (the loop's
    positions; for straight-line events 0) and the global id `gid(k)` of the item's k-th block: its own blocks
    for k < n, then the next item's (k - n), or, with no next item, the item's last block again (a reload that
    keeps the in-flight counts uniform). `replay([n0, n1, ...])` gives the events of those items back to back,
    with block ids unique across items."""

    head: List[Tuple[Callable, Callable]] = field(default_factory=list)  # at an item's start
    body: Dict[int, List[Tuple[Callable, Callable]]] = field(default_factory=dict)
    tail: List[Tuple[Callable, Callable]] = field(default_factory=list)  # at an item's end
    end: List[Event] = field(default_factory=list)  # once, after the last item
    unroll: int = 1
    where: str = "head"

    def add(self, make: Callable, when: Callable = lambda n, nxt, pre: True) -> None:
        """A straight-line event at the item's start (before `loop`) or end (after `end_loop`); `when(n, nxt,
        prefetched)`, where `prefetched` says the previous item already loaded this one's first blocks."""
        (self.head if self.where == "head" else self.tail).append((make, when))

    def loop(self, unroll: int) -> None:
        self.unroll, self.where = unroll, "body"

    def at(self, position: int, make: Callable, when: Callable = lambda b, n, nxt: True) -> None:
        self.body.setdefault(position, []).append((make, when))

    def end_loop(self) -> None:
        self.where = "tail"

    def replay(self, counts: Sequence[int]) -> List[Event]:
        out: List[Event] = []
        base, prefetched = 0, False
        for i, n in enumerate(counts):
            # items without blocks load nothing: the next item that loads is the first later one with blocks
            nxt = n > 0 and any(c > 0 for c in counts[i + 1:])
            nbase = base + n

            def gid(k: int, base=base, n=n, nxt=nxt, nbase=nbase) -> int:
                return base + k if k < n else (nbase + k - n if nxt else base + n - 1)

            for make, when in self.head:
                if when(n, nxt, prefetched):
                    out.append(make(0, n, nxt, gid))
            for b in range(n):
                for make, when in self.body.get(b % self.unroll, []):
                    if when(b, n, nxt):
                        out.append(make(b, n, nxt, gid))
            for make, when in self.tail:
                if when(n, nxt, prefetched):
                    out.append(make(0, n, nxt, gid))
            if n > 0:
                prefetched = nxt
            base = nbase
        return out + list(self.end)


def loads_reads(events: Sequence[Event]) -> Set[Tuple[str, int]]:
    """(kind, stage) of every load and read: what a test checks the replay covers."""
    return {(ev[0], ev[1]) for ev in events if ev[0] in ("load", "read")}
