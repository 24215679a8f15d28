"""TEST INFRASTRUCTURE ONLY. Step and tile tables by brute-force enumeration of a loop nest.

Restates, as plain nested loops over Python values, what the reference's schedule computes
(src/autokernel/schedule.py:138-342) and what its device step-table builder computes for runtime masks
(src/autokernel/codegen.py:376-451): the kernel's tiles in row-major order of the parallel loops, each
tile's phases' blocks that run (a phase none of whose blocks run takes one empty step at block 0), and each
step's code `((block * phases + phase) * iterations + iteration) << 3 | empty << 2 | first << 1 | last`.
For runtime masks, every step that could run is listed and the kept ones are moved to the front in order
(a stable partition), followed by the others in order; the count is how many were kept.
"""

from __future__ import annotations

import itertools
from typing import Callable, Dict, List, Sequence, Tuple

import numpy as np

CODE_SHIFT = 3


def code(block: int, phase: int, phases: int, iteration: int, iterations: int, empty: bool, first: bool,
         last: bool) -> int:
    return ((((block * phases + phase) * iterations + iteration) << CODE_SHIFT) | (int(empty) << 2)
            | (int(first) << 1) | int(last))


def pow2(n: int) -> int:
    p = 1
    while p < n:
        p *= 2
    return p


def static_tables(inner: Sequence[Tuple[str, int, int, int]], tile_mask: Callable[[Dict[str, int]], bool],
                  phases: Sequence[Tuple[str, int, int, int, Callable[[Dict[str, int]], bool]]]):
    """inner: (var, start, step, count) of the parallel loops the tables cover; phases: (var, start, step,
    count, mask). Returns (tile blocks, fill blocks, step_tile, step_code)."""
    radix = pow2(len(phases))
    active, skipped, step_tile, step_code = [], [], [], []
    for blocks in itertools.product(*(range(c) for _, _, _, c in inner)):
        values = {v: s + b * st for (v, s, st, _), b in zip(inner, blocks)}
        if tile_mask(values):
            skipped.append(blocks)
            continue
        t = len(active)
        active.append(blocks)
        for p, (var, start, step, count, mask) in enumerate(phases):
            run = [kb for kb in range(count) if not mask({**values, var: start + kb * step})]
            empty = not run
            run = run or [0]
            for n, kb in enumerate(run):
                step_tile.append(t)
                step_code.append(code(kb, p, radix, 0, 1, empty, n == 0, n == len(run) - 1))
    return active, skipped, np.array(step_tile, np.int32), np.array(step_code, np.int32)


def runtime_tables(tiles: Sequence[Dict[str, int]],
                   phases: Sequence[Tuple[str, int, int, int, Callable[[Dict[str, int]], bool]]]):
    """The device step tables of runtime masks: (step_tile, step_code, count) over every step that could
    run, kept ones first (in order), then the rest (in order)."""
    radix = pow2(len(phases))
    entries: List[Tuple[bool, int, int]] = []
    for t, values in enumerate(tiles):
        for p, (var, start, step, count, mask) in enumerate(phases):
            run = [not mask({**values, var: start + kb * step}) for kb in range(count)]
            empty = not any(run)
            keep = [r or (empty and kb == 0) for kb, r in enumerate(run)]
            kept = [kb for kb in range(count) if keep[kb]]
            first, last = kept[0], kept[-1]
            for kb in range(count):
                entries.append((keep[kb], t, code(kb, p, radix, 0, 1, empty and kb == 0, kb == first, kb == last)))
    front = [(t, c) for k, t, c in entries if k]
    back = [(t, c) for k, t, c in entries if not k]
    both = front + back
    return (np.array([t for t, _ in both], np.int32), np.array([c for _, c in both], np.int32), len(front))
