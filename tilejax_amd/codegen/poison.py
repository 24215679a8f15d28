"""A poisoned build of a generated program: every buffer a kernel could read before writing starts as NaN.

The reference runs its kernels in an interpreter with uninitialised memory filled with NaN and a race
detector (its tests/helpers.py:26-35), so a kernel that reads a VMEM buffer before copying into it, or leaves
an output element unwritten, produces NaN. The gfx950 counterpart is a build option (`hardware` knob
`poison`, see `codegen.generate`) that changes two things and nothing else:

- each kernel's first statements set every byte of the LDS arrays it uses to 0xFF (a NaN in bf16 and in
  f32, -1 in an int), then synchronise the workgroup, before any load into LDS is issued or anything is read;
- the program allocates its outputs filled with NaN (integer outputs with -1) and its workspace buffers
  (split-K partials, decode partials, device step tables) with 0xFF bytes.

A correct kernel reads LDS only where its own loads landed, every workspace element only after a kernel wrote
it, and writes every output element, so its poisoned run gives the same bits as the plain one. The GPU tests
require exactly that of every kernel family (tests/test_gpu_poison.py).
"""

from __future__ import annotations

import re
from typing import Dict, List

from .program import Program

__all__ = ["poison_source", "poison_program"]

# `__shared__ [attributes] type name[size];` at file scope, as every family declares its LDS arrays
_SHARED = re.compile(r"^__shared__[^;\[\n]*?(\w+)\s*(?:\[[^\]]+\])+\s*;", re.M)
# a kernel's signature line, ending with the brace that opens its body
_KERNEL = re.compile(r'^extern "C" __global__ void[^{\n]*\b(\w+)\(const \w+ args\) \{\s*$', re.M)
# a `__shared__` declaration inside a kernel body (indented: the cursor scan, the step builder, the merges)
_LOCAL_SHARED = re.compile(r"^([ \t]+)__shared__ ([^;]*);", re.M)


def _fill(name: str) -> str:
    """Every byte of LDS object `name` (an array or a scalar) to 0xFF, 16 bytes a thread at a time where its size
    and alignment allow, else a byte at a time."""
    return (f"{{ unsigned char* p_ = (unsigned char*)&({name}); const unsigned n_ = sizeof({name}); "
            f"if (n_ % 16 == 0 && ((unsigned long long)p_ & 15) == 0) {{ for (unsigned i_ = 16 * threadIdx.x; i_ < n_; i_ += 16 * blockDim.x) "
            f"*(uint4*)(p_ + i_) = make_uint4(~0u, ~0u, ~0u, ~0u); }} "
            f"else {{ for (unsigned i_ = threadIdx.x; i_ < n_; i_ += blockDim.x) p_[i_] = 0xFF; }} }}")


def _declared(decl: str) -> List[str]:
    """The names a declaration (without `__shared__` and `;`) declares: `int a[4], b[8]` -> [a, b]."""
    parts, depth, cur = [], 0, ""
    for ch in decl:
        depth += ch == "["
        depth -= ch == "]"
        if ch == "," and depth == 0:
            parts.append(cur)
            cur = ""
        else:
            cur += ch
    parts.append(cur)
    names = []
    for k, part in enumerate(parts):
        head = part.split("[", 1)[0]
        words = re.findall(r"\w+", head)
        names.append(words[-1] if k == 0 else words[0])
    return names


def _body_end(source: str, brace: int) -> int:
    """The index just past the brace that closes the one at `brace` (braces counted over the text: the
    generated kernels have none in strings or comments)."""
    depth = 0
    for i in range(brace, len(source)):
        depth += source[i] == "{"
        depth -= source[i] == "}"
        if depth == 0:
            return i + 1
    return len(source)


def poison_source(source: str) -> str:
    """`source` with each kernel starting by filling the file-scope LDS arrays it uses with 0xFF bytes (then a
    barrier), and each LDS object a kernel declares in its body filled right after its declaration."""
    arrays: List[str] = _SHARED.findall(source)
    kernels = list(_KERNEL.finditer(source))
    out, at = [], 0
    for match in kernels:
        body = source[match.end():_body_end(source, match.end() - 1)]
        used = [a for a in arrays if re.search(rf"\b{a}\b", body)]
        out.append(source[at:match.end()])
        if used:
            fills = " ".join(_fill(a) for a in used)
            out.append(f"\n  // poisoned build: LDS starts as 0xFF bytes\n  {fills}\n  __syncthreads();")
        at = match.end()
    out.append(source[at:])
    text = "".join(out)
    # body-scope declarations sit at the kernels' top level (after at most a workgroup-uniform return), so the
    # whole workgroup reaches the barrier after their fill
    return _LOCAL_SHARED.sub(lambda m: f"{m.group(0)}\n{m.group(1)}{' '.join(_fill(n) for n in _declared(m.group(2)))} "
                                       "__syncthreads();", text)


def poison_program(program: Program) -> Program:
    """Turn `program` into its poisoned build (in place): LDS-filling kernels, NaN-filled outputs and
    workspaces (`Program._run` reads `notes["poison"]`)."""
    program.source = poison_source(program.source)
    notes: Dict = program.notes
    notes["poison"] = True
    return program
