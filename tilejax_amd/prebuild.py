"""Compile, ahead of time, the kernels the benchmark and GPU tests use, into the code-object cache.

A kernel is compiled by hiprtc the first time it is lowered for a signature and schedule; the cache keeps
the code object by a hash of its source, so compiling here (no GPU needed) saves the GPU run the
compile. This is a build-speed measure only: nothing here is a tuning result.
"""

from __future__ import annotations

import os
import sys
from typing import Iterator, List, Tuple

from . import jaxlite
from .errors import KernelError

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bf16(*shape: int) -> Tuple[Tuple[int, ...], jaxlite.DType]:
    return (tuple(shape), jaxlite.bfloat16)


def _f32(*shape: int) -> Tuple[Tuple[int, ...], jaxlite.DType]:
    return (tuple(shape), jaxlite.float32)


def _i32(*shape: int) -> Tuple[Tuple[int, ...], jaxlite.DType]:
    return (tuple(shape), jaxlite.int32)


def standard() -> Iterator[Tuple[object, tuple]]:
    """(kernel, lower() arguments) of the kernels the benchmark and the GPU tests build."""
    if ROOT not in sys.path:
        sys.path.insert(0, ROOT)
    from examples import causal_matmul as cm
    from examples import matmul as mm

    T = mm.MatmulTiles
    for n, tiles in ((8192, T(512, 512, 512)), (1024, T(512, 512, 512)), (8192, T(1024, 2048, 1024)),
                     (512, T(256, 256, 128)), (1024, T(256, 256, 256))):
        yield mm.matmul, (_bf16(n, n), _bf16(n, n), tiles)
    for n, tiles in ((8192, T(512, 512, 512)), (1024, T(256, 256, 256)), (512, T(128, 128, 128)),
                     (8192, T(1024, 2048, 1024)), (2048, T(256, 256, 256))):
        yield cm.causal_matmul, (_bf16(n, n), _bf16(n, n), tiles)
    yield mm.matmul, (_bf16(512, 256), _bf16(256, 512), T(256, 256, 128))
    yield mm.matmul, (_bf16(256, 384), _bf16(384, 256), T(256, 128, 512))
    for tiles in (T(128, 128, 128), T(256, 128, 512), T(256, 256, 128)):  # f32 operands
        yield mm.matmul, (_f32(256, 384), _f32(384, 256), tiles)
    yield mm.matmul, (_f32(1024, 1024), _f32(1024, 1024), T(512, 512, 512))
    yield cm.causal_matmul, (_f32(512, 256), _f32(256, 512), T(128, 128, 128))
    from examples import moe

    GT = moe.GroupTiles
    for (m, k, n, e, g), tiles in (((1024, 512, 1024, 4, 4), GT(512, 256)), ((1024, 512, 1024, 4, 4), GT(256, 512)),
                                   ((1024, 512, 1024, 4, 4), GT(512, 512)), ((2048, 1024, 512, 4, 8), GT(512, 256)),
                                   ((16384, 4096, 14336, 8, 64), GT(512, 512))):
        yield moe.grouped_matmul, (_bf16(m, k), _bf16(e, k, n), _i32(g), tiles)
    yield moe.grouped_matmul, (_f32(1024, 512), _f32(4, 512, 1024), _i32(4), GT(512, 256))
    ET = moe.ExpertTiles
    for (m, d, f, e, t), tiles in (((512, 256, 512, 4, 4), ET(128)), ((512, 256, 512, 4, 4), ET(512)),
                                   ((1024, 256, 512, 4, 8), ET(128)), ((16384, 4096, 14336, 8, 64), ET(256))):
        yield moe.expert_ffn, (_bf16(m, d), _bf16(e, d, f), _bf16(e, d, f), _bf16(e, f, d), _i32(t), tiles)
    from examples import rmsnorm_matmul as rm

    R = rm.NormMatmulTiles
    for (m, d, n), tiles in (((1024, 1024, 512), R(512, 512, 512)), ((512, 768, 256), R(256, 256, 256)),
                             ((256, 512, 512), R(128, 128, 128)), ((512, 512, 512), R(256, 256, 256)),
                             ((4096, 4096, 4096), R()), ((8192, 8192, 8192), R())):
        yield rm.rmsnorm_matmul, (_bf16(m, d), _bf16(1, d), _bf16(d, n), tiles)
    yield rm.rmsnorm_matmul, (_bf16(256, 512), _bf16(1, 512), _bf16(512, 512), R(128, 256, 512))
    for tiles in (R(128, 128, 128), R(256, 128, 512)):
        yield rm.rmsnorm_matmul, (_f32(256, 512), _f32(1, 512), _f32(512, 512), tiles)
    from examples import decode

    for b, pages, n_pages in ((4, 64, 256), (5, 100, 500), (64, 512, 32768), (8, 128, 1024), (4, 32, 128)):
        yield decode.paged_gqa_decode, (_bf16(b, 1, 32, 128), _bf16(n_pages, 16, 1024), _bf16(n_pages, 16, 1024),
                                        _i32(b, pages), _i32(b))
    yield decode.paged_gqa_decode, (_bf16(4, 1, 32, 128), _bf16(16, 128, 1024), _bf16(16, 128, 1024), _i32(4, 4),
                                    _i32(4))
    yield decode.paged_gqa_decode, (_bf16(4, 1, 8, 128), _bf16(256, 16, 1024), _bf16(256, 16, 1024), _i32(4, 64),
                                    _i32(4))
    for b, s, block in ((4, 512, 128), (4, 512, 256), (4, 512, 512), (64, 8192, 512)):
        yield decode.gqa_decode, (_bf16(b, 1, 32, 128), _bf16(b, s, 1024), _bf16(b, s, 1024), _i32(b),
                                  decode.DecodeTiles(block))
    for t, h, kv, block in ((1, 8, 2, 128), (1, 4, 4, 256), (3, 8, 2, 128)):
        yield decode.gqa_decode, (_bf16(4, t, h, 128), _bf16(4, 512, kv * 128), _bf16(4, 512, kv * 128), _i32(4),
                                  decode.DecodeTiles(block))
    from examples import attention_block as ab

    BT = ab.BlockTiles
    for (s_, f_, dt), tiles in ((((512, 512, _bf16)), BT(128, 128)), (((512, 512, _bf16)), BT(256, 128)),
                                (((256, 1024, _bf16)), BT(128, 128, 256)), (((256, 256, _f32)), BT(128, 128, 256))):
        yield ab.attention_block, (dt(1, 2, s_, 128), dt(1, 2, s_, 128), dt(1, 2, s_, 128), dt(1, 256),
                                   dt(256, f_), dt(f_, 256), tiles)
    try:
        from examples import causal_attention as ca

        A = ca.AttentionBlocks
        for shape, blocks in (((4, 16, 2048, 128), A(512, 512)), ((1, 16, 4096, 128), A(512, 512)),
                              ((4, 16, 2048, 128), A(256, 256)), ((1, 16, 4096, 128), A(256, 256)),
                              ((4, 16, 2048, 128), A(1024, 1024)), ((1, 16, 4096, 128), A(1024, 1024)),
                              ((2, 4, 512, 128), A(128, 128)), ((1, 2, 1024, 128), A(256, 256)),
                              ((1, 2, 512, 128), A(128, 128)), ((2, 2, 512, 128), A(256, 128)),
                              ((2, 2, 512, 128), A(128, 128)), ((2, 2, 512, 128), A(128, 256)),
                              ((1, 1, 1024, 128), A(512, 512))):
            yield ca.causal_attention, (_bf16(*shape), _bf16(*shape), _bf16(*shape), blocks)
        for shape, blocks in (((1, 1, 256, 128), A(128, 128)), ((2, 2, 512, 128), A(256, 128)),
                              ((1, 2, 512, 128), A(128, 256))):
            yield ca.causal_attention, (_f32(*shape), _f32(*shape), _f32(*shape), blocks)
    except ImportError:
        pass


def shapes() -> Iterator[Tuple[object, tuple, object, bool]]:
    """(kernel, signature arguments, Config, trace) of the kernel shapes the GPU tests pin and the tuning test
    at the dense BASELINE config tries (the tuner builds with trace regions)."""
    if ROOT not in sys.path:
        sys.path.insert(0, ROOT)
    from examples import causal_attention as ca
    from examples import causal_matmul as cm
    from examples import decode
    from examples import matmul as mm

    from .codegen import hardware_choices
    from .pipeline import Pipeline
    from .tune import Config

    tiles = mm.MatmulTiles(512, 512, 512)
    for kernel in (mm.matmul, cm.causal_matmul):
        for hw, n in (((("bm", 256), ("bn", 128)), 2), ((("bm", 128), ("bn", 256)), 2), ((("bm", 128), ("bn", 128)), 3),
                      ((), 4), ((("bm", 256), ("bn", 256), ("waves", 4)), 2), ((("bm", 256), ("bn", 256), ("waves", 4)), 4),
                      ((("bm", 256), ("bn", 256), ("waves", 8)), 2), ((("bm", 256), ("bn", 128), ("waves", 8)), 3),
                      ((("bm", 128), ("bn", 128), ("waves", 8)), 2)):
            yield kernel, (_bf16(1024, 1024), _bf16(1024, 1024)), Config(tiles, Pipeline(n, 2), False, hw), False
    args = (_bf16(8192, 8192), _bf16(8192, 8192))
    plan, schedule = mm.matmul.build(mm.matmul.signature(*args), mm.matmul.default_tunable)
    for hw in hardware_choices(plan, schedule):
        for n in (2, 3):
            yield mm.matmul, args, Config(mm.matmul.default_tunable, Pipeline(n, 2), False, hw), True
    blocks = ca.AttentionBlocks(256, 256)
    for hw, n in (((("bkv", 64), ("waves", 8)), 2), ((("bkv", 32), ("waves", 4)), 2),
                  ((("bkv", 32), ("waves", 8)), 2), ((), 3), ((), 4),
                  ((("bkv", 64), ("split", 0), ("waves", 4)), 2)):
        yield ca.causal_attention, tuple(_bf16(2, 4, 1024, 128) for _ in range(3)), Config(blocks, Pipeline(n, 2), False, hw), False
    for hw in ((("split", 0),), (("split", 0), ("rows", 64)), (("rows", 64),)):
        yield ca.causal_attention, tuple(_bf16(2, 4, 1024, 128) for _ in range(3)), Config(blocks, Pipeline(2, 2), False, hw), False
    ins = (_bf16(5, 1, 32, 128), _bf16(500, 16, 1024), _bf16(500, 16, 1024), _i32(5, 100), _i32(5))
    for n in (2, 4):
        for cursor in (False, True):
            yield decode.paged_gqa_decode, ins, Config(None, Pipeline(n, 2), cursor), False
    ins = (_bf16(8, 1, 32, 128), _bf16(1024, 16, 1024), _bf16(1024, 16, 1024), _i32(8, 128), _i32(8))
    sig = decode.paged_gqa_decode.signature(*ins)
    base = decode.paged_gqa_decode.default_config(sig)
    for hw in ((("own", 0),), (("fold", 1),), (("sync", 0),)):
        for cursor in (False, True):
            yield decode.paged_gqa_decode, ins, Config(base.tunable, base.pipeline, cursor, hw), False
    for cursor in (False, True):
        yield decode.paged_gqa_decode, ins, Config(base.tunable, base.pipeline, cursor, (("qrows", int(not cursor)),)), False
    ins = (_bf16(4, 1, 8, 128), _bf16(256, 16, 1024), _bf16(256, 16, 1024), _i32(4, 64), _i32(4))  # MHA
    base = decode.paged_gqa_decode.default_config(decode.paged_gqa_decode.signature(*ins))
    yield decode.paged_gqa_decode, ins, Config(base.tunable, base.pipeline, True), False


def compile_all(verbose: bool = True) -> List[str]:
    """Lower and compile every standard kernel and tested kernel shape; the names of those the backend can't
    lower yet."""
    from . import runtime

    skipped = []
    for kernel, args, config, trace in shapes():
        lowered = kernel.lowered(kernel.signature(*args), config, trace=trace)
        runtime.compile_source(lowered.source, f"{kernel.nest.name}.hip")
        if verbose:
            print(f"compiled {kernel.nest.name} {[a[0] for a in args]} {config}{' traced' if trace else ''}", flush=True)
    for kernel, args in standard():
        try:
            lowered = kernel.lower(*args)
        except KernelError as e:
            skipped.append(f"{kernel.nest.name}: {str(e).splitlines()[0]}")
            continue
        from . import runtime

        runtime.compile_source(lowered.source, f"{kernel.nest.name}.hip")
        if verbose:
            print(f"compiled {kernel.nest.name} {[a[0] for a in args[:-1]]} {args[-1]}", flush=True)
    for s in skipped:
        print("not lowered yet:", s, flush=True)
    return skipped
