"""TEST INFRASTRUCTURE ONLY — the CPU oracle the GPU kernels are checked against.

Only `tests/`, `__graft_entry__.smoke()` and `bench.py`'s CPU-baseline leg may import this package, and
only as the checker (or the timed CPU baseline): the product path (`tilejax_amd`) never imports, calls
or links it, and fails loudly without its HIP library instead of falling back to anything here.

- `kernels`: the five spec loop nests restated as plain loops over tiles on CPU tensors, with the
  reference's `@` semantics (bf16 products accumulated in f32: src/autokernel/mxu.py:21-43 of the
  reference), each citing the example it follows;
- `schedule`: the step and tile tables restated by brute-force enumeration of the loop nest
  (src/autokernel/schedule.py:138-342 and the device table builder, src/autokernel/codegen.py:376-451).
"""
