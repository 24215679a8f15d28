"""`rows`: a window of rows a kernel finds as it runs, as many as are valid (ragged batches).

The reference's `autokernel.rows` (src/autokernel/ragged.py:23-28) has this meaning: as a tile read's index,
`q[rows(start, stop, n), :]` is the n rows from `start` (rows at or past `stop` are whatever the array holds
there: reads clamp into the array, as JAX clamps); as an output store's index,
`out = out.at[rows(start, stop, n), :].set(v)` writes v's first `stop - start` rows from `start` and nothing
past `stop` (JAX drops updates out of the array, and every index past `stop` is out of it).

The gfx950 lowering reads such a window element by element from `start` and masks the store's rows past
`stop`; run eagerly (kernel.fn, kernel.reference) it is this index array.
"""

from __future__ import annotations

from typing import Any

from . import jaxlite

__all__ = ["PAST", "rows"]

PAST = 2**31 - 1  # an index out of every array: a store there is dropped, a read is clamped


def rows(start: Any, stop: Any, size: int) -> Any:
    """start, start + 1, ..., start + size - 1 as an int32 index array, every entry at or past `stop` moved
    out of bounds (PAST). `size` is an int when the kernel is built."""
    index = jaxlite.arange(size, dtype=jaxlite.int32) + start
    return jaxlite.where(index < stop, index, PAST)
