"""The poisoned build (tilejax_amd/codegen/poison.py), on the CPU: every LDS object a kernel uses is filled with
0xFF bytes before the kernel touches it, and the poisoned source still compiles for gfx950. The GPU side (the
poisoned run gives the plain run's bits) is tests/test_gpu_poison.py."""

import re

import pytest

from examples.causal_attention import AttentionBlocks, causal_attention
from examples.decode import paged_gqa_decode
from examples.matmul import MatmulTiles, matmul
from examples.moe import GroupTiles, grouped_matmul
from tests.helpers import spec
from tilejax_amd import Pipeline, jaxlite, runtime
from tilejax_amd.codegen.poison import _KERNEL, _SHARED, _body_end, poison_source
from tilejax_amd.tune import Config

BF, I32 = jaxlite.bfloat16, jaxlite.int32


def _program(kernel, args, tunable, cursor=False, poison=True):
    sig = kernel.signature(*args)
    base = kernel.lowered(sig, kernel.default_config(sig)) if tunable is None else None
    pipeline = base.config.pipeline if base is not None else Pipeline(2, 2)
    tunable = base.config.tunable if base is not None else tunable
    hardware = (("poison", 1),) if poison else ()
    return kernel.lowered(sig, Config(tunable, pipeline, cursor, hardware)).program


def _cases():
    sq = (spec(8192, 8192, dtype=BF), spec(8192, 8192, dtype=BF))
    yield "matmul", matmul, sq, MatmulTiles(512, 512, 512), False
    yield "grouped", grouped_matmul, (spec(1024, 512, dtype=BF), spec(4, 512, 1024, dtype=BF), spec(4, dtype=I32)), \
        GroupTiles(512, 256), False
    yield "attention", causal_attention, tuple(spec(1, 2, 1024, 128, dtype=BF) for _ in range(3)), \
        AttentionBlocks(256, 256), False
    dec = (spec(5, 1, 32, 128, dtype=BF), spec(500, 16, 1024, dtype=BF), spec(500, 16, 1024, dtype=BF),
           spec(5, 100, dtype=I32), spec(5, dtype=I32))
    yield "decode", paged_gqa_decode, dec, None, False
    yield "decode cursor", paged_gqa_decode, dec, None, True


@pytest.mark.parametrize("name,kernel,args,tunable,cursor", list(_cases()), ids=lambda x: x if isinstance(x, str) else "")
def test_every_lds_object_is_filled_first(name, kernel, args, tunable, cursor):
    plain = _program(kernel, args, tunable, cursor, poison=False)
    prog = _program(kernel, args, tunable, cursor)
    assert prog.notes["poison"] and not plain.notes.get("poison")
    src = prog.source
    assert poison_source(plain.source) == src
    kernels = [src[m.end():_body_end(src, m.end() - 1)] for m in _KERNEL.finditer(src)]
    assert kernels
    file_scope = _SHARED.findall(src)
    assert file_scope or "__shared__" in src
    for body in kernels:
        # each file-scope array the kernel uses is filled before its first other use
        for a in file_scope:
            uses = [m.start() for m in re.finditer(rf"\b{a}\b", body)]
            if uses:
                fill = body.find(f"(unsigned char*)&({a})")
                assert 0 <= fill <= uses[0] + len(f"(unsigned char*)&(") and body.count(f"&({a})") == 1, a
        # each body-scope declaration is followed by its fill and a barrier
        for m in re.finditer(r"(?m)^[ \t]+__shared__ ([^;]*);\n([^\n]*)", body):
            assert "0xFF" in m.group(2) and "__syncthreads();" in m.group(2), m.group(0)
    if name == "matmul":  # compiles for gfx950 (hiprtc; no GPU needed)
        runtime.compile_source(src, prog.name)


def test_poisoned_outputs_and_workspaces_start_as_nan():
    import torch

    from tilejax_amd.codegen.program import _poisoned

    assert torch.isnan(_poisoned((4, 4), torch.bfloat16, "cpu")).all()
    assert (_poisoned((3,), torch.int32, "cpu") == -1).all()
