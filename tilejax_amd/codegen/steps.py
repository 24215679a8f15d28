"""The device step-table builder: runtime masks evaluated on the GPU just before the kernel.

The reference emits this as plain-JAX ops ahead of its `pallas_call` (src/autokernel/codegen.py:376-451,
`_steps_definitions`): for every pattern tile t and block kb of the reduction loop, `run = not mask`; a tile
none of whose blocks run keeps one empty step at block 0; each step gets its code
`((kb * phases + phase) * iterations + iteration) << 3 | empty << 2 | first << 1 | last`; the kept steps are
moved to the front in (t, kb) order and the rest follow in order (a stable partition); the count of kept
steps is the third output.

Here it is one workgroup of 1024 threads, generated from the mask expression: each thread evaluates the
masks of a run of tiles, a block-wide scan turns kept/dropped counts into offsets, and every tile writes its
entries. Besides the reference's three outputs it writes `tile_steps`, each pattern tile's first kept
step (and the total at the end), which the matmul kernel uses to find a tile's steps without a search.
"""

from __future__ import annotations

from typing import List

import numpy as np

from ..errors import KernelError
from ..plan import Plan
from ..schedule import CODE_SHIFT, Schedule
from .common import Index
from .expr import int_expr
from .program import Arg, Launch, Program, c_struct

THREADS = 1024
MAX_TILES = 8192


def builder_source(plan: Plan, sch: Schedule, name: str, args: List[Arg]) -> str:
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
    decode = "\n      ".join(f"const int lv_{r.var} = args.tv_{r.var}[t];" for r in sch.inner)
    struct = c_struct(f"{name}_args", args)
    per = (pt + THREADS - 1) // THREADS
    return f"""
{struct}
// Step tables for `{plan.nest.name}`: {pt} pattern tiles x {count} blocks of `{phase.var}`.
extern "C" __global__ void __launch_bounds__({THREADS}) {name}(const {name}_args args) {{
  __shared__ int keep_n[{pt}], drop_n[{pt}], scan_k[{THREADS}], scan_d[{THREADS}];
  const int tid = threadIdx.x;
  const int t0 = tid * {per}, t1 = ak_imin(t0 + {per}, {pt});
  int my_k = 0, my_d = 0;
  for (int t = t0; t < t1; ++t) {{
      {decode}
      int kept = 0;
      for (int kb = 0; kb < {count}; ++kb) {{
        const int lv_{phase.var} = {phase.start} + kb * {phase.step};
        kept += !({mask});
      }}
      const int k = kept ? kept : 1;  // a tile with no block running takes one empty step
      keep_n[t] = k;
      drop_n[t] = {count} - k;
      my_k += k;
      my_d += {count} - k;
  }}
  scan_k[tid] = my_k;
  scan_d[tid] = my_d;
  __syncthreads();
  for (int s = 1; s < {THREADS}; s <<= 1) {{  // inclusive scan of the threads' totals
    const int a = tid >= s ? scan_k[tid - s] : 0, b = tid >= s ? scan_d[tid - s] : 0;
    __syncthreads();
    scan_k[tid] += a;
    scan_d[tid] += b;
    __syncthreads();
  }}
  const int total = scan_k[{THREADS - 1}];
  int ok = scan_k[tid] - my_k, od = scan_d[tid] - my_d;
  for (int t = t0; t < t1; ++t) {{
      {decode}
      args.rt_tile_steps[t] = ok;
      int first = -1, last = -1;
      for (int kb = 0; kb < {count}; ++kb) {{
        const int lv_{phase.var} = {phase.start} + kb * {phase.step};
        if (!({mask})) {{ if (first < 0) first = kb; last = kb; }}
      }}
      const int empty = first < 0;
      if (empty) {{ first = 0; last = 0; }}
      int nk = 0, nd = 0;
      for (int kb = 0; kb < {count}; ++kb) {{
        const int lv_{phase.var} = {phase.start} + kb * {phase.step};
        const int keep = empty ? (kb == 0) : !({mask});
        const int code = ((kb * {radix}) << {CODE_SHIFT}) | ((empty && kb == 0) << 2) | ((kb == first) << 1) | (kb == last);
        const int at = keep ? ok + nk++ : total + od + nd++;
        args.rt_step_tile[at] = t;
        args.rt_step_code[at] = code;
      }}
      ok += keep_n[t];
      od += drop_n[t];
  }}
  if (tid == 0) {{
    args.rt_count[0] = total;
    args.rt_tile_steps[{pt}] = total;
  }}
}}
"""


def attach_step_builder(prog: Program, plan: Plan, sch: Schedule, kernel_name: str) -> None:
    """Add the builder's launch (first, on the same stream), its tables and its workspace to `prog`."""
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
    prog.source += builder_source(plan, sch, name, args)
    prog.launches.insert(0, Launch(name, args, (1, 1, 1), (THREADS, 1, 1), 0))
    prog.notes["step_builder"] = name
