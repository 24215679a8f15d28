"""`pairs` and `unpairs`: a 16-bit tile's pairs of rows as 32-bit words, and back.

The reference's `autokernel.pairs` / `unpairs` (src/autokernel/packing.py:22-34) read a tile (..., 2, d) of a
16-bit dtype (a cache page holding each head's key and value side by side) as uint32 words (..., d), row 0
in each word's low half and row 1 in its high half, and store words back as such a tile. On gfx950 the
generic kernel evaluates them per element (a word is its two halves' bits); run eagerly (kernel.fn,
kernel.reference) they are the same bit moves on torch tensors.
"""

from __future__ import annotations

from .jaxlite import pairs, unpairs

__all__ = ["pairs", "unpairs"]
