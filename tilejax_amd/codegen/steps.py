"""The device step-table builder: runtime masks evaluated on the GPU just before the kernel.

The reference emits this as plain-JAX ops ahead of its `pallas_call` (src/autokernel/codegen.py:376-451,
`_steps_definitions`): for every pattern tile t and block kb of the reduction loop, `run = not mask`; a tile
none of whose blocks run keeps one empty step at block 0; each step gets its code
`((kb * phases + phase) * iterations + iteration) << 3 | empty << 2 | first << 1 | last`; the kept steps are
moved to the front in (t, kb) order and the rest follow in order (a stable partition); the count of kept
steps is the third output.

Here it is a few workgroups of 1024 threads, generated from the mask expression. Every workgroup evaluates
all the masks, 64 blocks per ballot, into words kept in LDS, and a block-wide scan turns the tiles' kept
counts into offsets; this part is cheap and repeated, so no workgroup waits for another. Each workgroup then
writes its own range of words' entries, a wave per word, at ballot-prefix positions. Besides the reference's three outputs it writes `tile_steps`,
each pattern tile's first kept step (and the total at the end), which the kernels use to find a tile's steps
without a search.
"""

from __future__ import annotations

from typing import List, Sequence

import numpy as np

from ..errors import KernelError
from ..plan import Plan
from ..schedule import CODE_SHIFT, Schedule
from .common import Index, tile_value
from .expr import int_expr
from .program import Arg, Launch, Program, c_struct

THREADS = 1024
MAX_TILES = 4096
MAX_WORDS = 4096  # 64-block mask words kept in LDS (32 KiB)


def builder_source(plan: Plan, sch: Schedule, name: str, args: List[Arg], extra: str = "") -> str:
    """The builder kernel; `extra` is the owner kernel's code for the workgroups past the builder's own
    (`xb_` numbers them from 0), which run beside it in the same launch."""
    if len(plan.phases) != 1:
        raise KernelError("runtime masks over more than one reduction loop are not lowered by the gfx950 backend yet")
    phase = plan.phases[0].range
    if phase.mask is None:
        raise KernelError("internal: a runtime schedule without a mask")
    pt, count = sch.pattern_tiles, phase.count
    if pt > MAX_TILES:
        raise KernelError(f"runtime step tables for {pt} tiles: the builder takes at most {MAX_TILES}")
    index = Index(plan, lambda v: f"lv_{v}")
    mask = index.expr(phase.mask)
    radix = sch.phase_radix * sch.iterations
    decode = " ".join(f"const int lv_{r.var} = {tile_value(sch, r.var, 't')};" for r in sch.inner)
    struct = c_struct(f"{name}_args", args)
    per = (pt + THREADS - 1) // THREADS
    nb = -(-count // 64)  # 64-block words per tile
    words = pt * nb
    if words > MAX_WORDS:
        raise KernelError(f"runtime step tables for {pt} tiles x {count} blocks: the builder takes at most "
                          f"{MAX_WORDS * 64} (tile, block) pairs")
    waves = THREADS // 64
    rounds = -(-pt // waves)
    groups = builder_groups(words)
    wpg = -(-words // groups)  # words each workgroup writes
    return f"""
{struct}
// Step tables for `{plan.nest.name}`: {pt} pattern tiles x {count} blocks of `{phase.var}`, as {words} words of
// 64 blocks. Pass 1: each wave evaluates one tile's words per round (a ballot each; the tile's loads are
// made once), two rounds' loads in flight together. Then per-tile kept counts, a block-wide scan of them,
// and pass 2: each wave writes one word's entries at ballot-prefix positions, from the words alone.
extern "C" __global__ void __launch_bounds__({THREADS}) {name}(const {name}_args args) {{
{extra_blocks(extra, groups)}  __shared__ unsigned long long run_w[{words}];
  __shared__ int before_w[{words}], keep_n[{pt}], first_t[{pt}], last_t[{pt}], scan_k[{THREADS}];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
#pragma unroll 2
  for (int i = 0; i < {rounds}; ++i) {{
    const int t = wave + {waves} * i;
    if (t < {pt}) {{
      {decode}
      for (int wi = 0; wi < {nb}; ++wi) {{
        const int kb = wi * 64 + lane;
        bool run = false;
        if (kb < {count}) {{
          const int lv_{phase.var} = {phase.start} + kb * {phase.step};
          run = !({mask});
        }}
        const unsigned long long m = __ballot(run);
        if (lane == 0) run_w[t * {nb} + wi] = m;
      }}
    }}
  }}
  __syncthreads();
  // per tile: running blocks before each word, the first and last running block, the kept count
  for (int t = tid; t < {pt}; t += {THREADS}) {{
    int kept = 0, first = -1, last = -1;
    for (int i = 0; i < {nb}; ++i) {{
      const unsigned long long m = run_w[t * {nb} + i];
      before_w[t * {nb} + i] = kept;
      if (m) {{
        if (first < 0) first = i * 64 + __ffsll((long long)m) - 1;
        last = i * 64 + 63 - __clzll((long long)m);
      }}
      kept += __popcll(m);
    }}
    keep_n[t] = kept ? kept : 1;  // a tile with no block running takes one empty step
    first_t[t] = first;
    last_t[t] = last;
  }}
  __syncthreads();
  // each thread sums a run of tiles; a block-wide inclusive scan of those sums
  const int t0 = tid * {per}, t1 = ak_imin(t0 + {per}, {pt});
  int my_k = 0;
  for (int t = t0; t < t1; ++t) my_k += keep_n[t];
  scan_k[tid] = my_k;
  __syncthreads();
  for (int s = 1; s < {THREADS}; s <<= 1) {{
    const int a = tid >= s ? scan_k[tid - s] : 0;
    __syncthreads();
    scan_k[tid] += a;
    __syncthreads();
  }}
  const int total = scan_k[{THREADS - 1}];
  // exclusive per-tile offsets of kept steps, in place over keep_n; tile t's dropped steps start t*count - that
  {{
    int ok = scan_k[tid] - my_k;
    for (int t = t0; t < t1; ++t) {{ const int n = keep_n[t]; keep_n[t] = ok; ok += n; }}
  }}
  __syncthreads();
  const unsigned long long below = lane ? (~0ull >> (64 - lane)) : 0ull;
  const int w_end = ak_imin((int)(blockIdx.x + 1) * {wpg}, {words});
#pragma unroll 4
  for (int i = 0; i < {-(-wpg // waves)}; ++i) {{
    const int w = blockIdx.x * {wpg} + wave + {waves} * i;
    if (w >= w_end) break;
    const int t = w / {nb}, wi = w % {nb}, k0 = wi * 64, kb = k0 + lane;
    int first = first_t[t], last = last_t[t], before = before_w[w];
    const int empty = first < 0;
    unsigned long long mk = run_w[w];
    if (empty) {{ first = 0; last = 0; mk = wi == 0 ? 1ull : 0ull; before = k0 > 0; }}
    const unsigned long long valid = {count} - k0 >= 64 ? ~0ull : ((1ull << ({count} - k0)) - 1);
    const unsigned long long md = valid & ~mk;
    const int ok = keep_n[t] + before, od = t * {count} - keep_n[t] + (k0 - before);
    if (wi == 0 && lane == 0) args.rt_tile_steps[t] = keep_n[t];
    if (kb < {count}) {{
      const bool keep = (mk >> lane) & 1;
      const int code = ((kb * {radix}) << {CODE_SHIFT}) | ((empty && kb == 0) << 2) | ((kb == first) << 1) | (kb == last);
      const int at = keep ? ok + __popcll(mk & below) : total + od + __popcll(md & below);
      args.rt_step_tile[at] = t;
      args.rt_step_code[at] = code;
    }}
  }}
  if (blockIdx.x == 0 && tid == 0) {{
    args.rt_count[0] = total;
    args.rt_tile_steps[{pt}] = total;
  }}
}}
"""


def extra_blocks(extra: str, groups: int) -> str:
    if not extra:
        return ""
    return (f"  if (blockIdx.x >= {groups}) {{  // the owner kernel's workgroups, beside the builder's\n"
            f"    const int xb_ = blockIdx.x - {groups};\n{extra}\n    return;\n  }}\n")


def builder_groups(words: int) -> int:
    """Workgroups of the builder: about 32 mask words (2048 table entries) each, at most 64."""
    return max(1, min(64, -(-words // 32)))


def attach_step_builder(prog: Program, plan: Plan, sch: Schedule, kernel_name: str,
                        extra: str = "", extra_args: Sequence[Arg] = (), extra_groups: int = 0) -> None:
    """Add the builder's launch (first, on the same stream), its tables and its workspace to `prog`; with
    `extra`, `extra_groups` more workgroups of the launch run that code (the owner kernel's own work that
    needs no step table, so it needs no launch of its own), reading `extra_args` too."""
    name = f"{kernel_name}_steps"
    args: List[Arg] = []
    for ix in plan.indices:
        args.append(Arg("input", ix.param, "const int* __restrict__", ix.name))
    for r in sch.inner:
        table = f"tv_{r.var}"
        prog.tables[table] = np.asarray(sch.tile_values[r.var], np.int32)
        args.append(Arg("table", table, "const int* __restrict__", table))
    capacity = sch.pattern_steps
    for ws, n in (("step_tile", capacity), ("step_code", capacity), ("count", 1), ("tile_steps", sch.pattern_tiles + 1)):
        prog.workspace[ws] = 4 * n
        args.append(Arg("workspace", ws, "int* __restrict__", f"rt_{ws}"))
    names = {a.name for a in args}
    args += [a for a in extra_args if a.name not in names]
    prog.source += builder_source(plan, sch, name, args, extra)
    words = sch.pattern_tiles * -(-plan.phases[0].range.count // 64)
    groups = builder_groups(words) + (extra_groups if extra else 0)
    prog.launches.insert(0, Launch(name, args, (groups, 1, 1), (THREADS, 1, 1), 0))
    prog.notes["step_builder"] = name
