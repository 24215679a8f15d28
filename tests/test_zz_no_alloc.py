"""The entry point that allocates nothing (include/ak.h, ak_launch_scratch): every launch of a program with
workspace buffers, run through the C-ABI with those buffers placed in the library's own scratch array,
gives the same bits as the ordinary call (the same kernels in the same order), on two calls in a row, the
second with a smaller input."""

import pytest
import torch

from examples.causal_matmul import causal_matmul
from examples.decode import paged_gqa_decode
from examples.matmul import MatmulTiles
from tilejax_amd import KernelError, runtime
from tilejax_amd.tune import Config

pytestmark = pytest.mark.gpu


def _allocator_counts():
    """torch's caching allocator's counters for the current device: allocations made so far, and bytes
    reserved from the device."""
    stats = torch.cuda.memory_stats()
    return stats.get("allocation.all.allocated", 0), stats.get("reserved_bytes.all.current", 0)


def _run_without_allocating(program, ins, out):
    """program.run_no_alloc, asserting that torch's allocator saw no allocation and reserved nothing more
    during the call (the kernel's tables were uploaded by the ordinary call before)."""
    torch.cuda.synchronize()
    before = _allocator_counts()
    program.run_no_alloc(*ins, outputs=[out])
    torch.cuda.synchronize()
    assert _allocator_counts() == before, (before, _allocator_counts())


def _decode_inputs(B, pages, lengths, seed):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(B, 1, 32, 128, generator=g) * 128 ** -0.5).to(torch.bfloat16)
    kp = torch.randn(B * pages, 16, 1024, generator=g).to(torch.bfloat16)
    vp = torch.randn(B * pages, 16, 1024, generator=g).to(torch.bfloat16)
    table = torch.randperm(B * pages, generator=g).reshape(B, pages).to(torch.int32)
    return [t.cuda() for t in (q, kp, vp, table, torch.tensor(lengths, dtype=torch.int32))]


@pytest.mark.parametrize("cursor", [False, True])
def test_decode_without_allocating(cursor):
    cases = [(8, 128, (0, 17, 300, 2048, 1, 999, 1024, 1600)), (4, 32, (5, 512, 0, 100))]
    for B, pages, lengths in cases:  # the second call is smaller: a smaller workspace in the same array
        ins = _decode_inputs(B, pages, lengths, seed=B)
        sig = paged_gqa_decode.signature(*ins)
        base = paged_gqa_decode.default_config(sig)
        lowered = paged_gqa_decode.lowered(sig, Config(base.tunable, base.pipeline, cursor))
        program = lowered.program
        assert program.workspace, "decode keeps its partial softmaxes in a workspace"
        print(f"no-alloc decode B={B} cursor={cursor} workspace {sum(program.workspace.values())} bytes", flush=True)
        want = lowered.run(*ins)
        out = torch.full_like(want, float("nan"))
        _run_without_allocating(program, ins, out)
        assert torch.equal(out, want)


def test_causal_split_without_allocating():
    """The 8192^3 causal matmul's split tiles keep their f32 partials (32 MiB, half the scratch array) in the
    workspace; then a 2048^3 call at 256^3 tiles reuses the front of it."""
    for n, tiles in ((8192, MatmulTiles(512, 512, 512)), (2048, MatmulTiles(256, 256, 256))):
        g = torch.Generator().manual_seed(n)
        x = torch.randn(n, n, generator=g).to(torch.bfloat16).cuda()
        y = torch.randn(n, n, generator=g).to(torch.bfloat16).cuda()
        lowered = causal_matmul.lower(x, y, tiles)
        print(f"no-alloc causal {n} {tiles} workspace {lowered.program.workspace}", flush=True)
        want = lowered.run(x, y)
        out = torch.full_like(want, float("nan"))
        _run_without_allocating(lowered.program, (x, y), out)
        assert torch.equal(out, want)


def test_rejects_a_workspace_past_the_scratch_array():
    """Offsets beyond AK_SCRATCH_BYTES are refused before anything launches (and so are outputs of the wrong
    shape, on the host)."""
    ins = _decode_inputs(4, 32, (5, 512, 0, 100), seed=1)
    sig = paged_gqa_decode.signature(*ins)
    program = paged_gqa_decode.lowered(sig, paged_gqa_decode.default_config(sig)).program
    launch = next(ln for ln in program.launches if any(a.kind == "workspace" for a in ln.args))
    kernel = program.module(0).kernel(launch.symbol)
    args = bytes(8 * len(launch.args) + 64)
    with pytest.raises(KernelError, match="exceeds the scratch array"):
        kernel.launch_scratch(launch.grid, launch.block, launch.lds, args, runtime.current_stream(),
                              [(0, runtime.SCRATCH_BYTES - 256, 512)])
    with pytest.raises(KernelError, match="must be a contiguous"):
        program.run_no_alloc(*ins, outputs=[torch.empty(1, device="cuda")])
