"""The autotuner on the CPU: the search, and the proposals each bottleneck leads to, on synthetic profiles
(the reference's tests/test_tune.py:51-120). Timing and testing candidates on the GPU is in test_gpu_tune.py."""

import pytest
import torch
from helpers import make_kernel, spec

import tilejax_amd as autokernel
from tilejax_amd import Config, KernelError, KernelProfile, Pipeline, Trial, jaxlite
from tilejax_amd.tune import proposals, search


def profile(config, seconds=10e-6, steps=4, wait=0.0, out_wait=0.0, compute=None, regions=True):
    """A KernelProfile with these times (`compute` defaults to all of the time not waiting)."""
    compute = seconds - wait - out_wait if compute is None else compute
    return KernelProfile("f", config, 1, seconds, regions, steps, wait, 0.0, out_wait, compute)


# ------------------------------------------------------------------------------------------- search


def test_search_climbs_to_the_fastest_and_stops():
    times = {1: 9.0, 2: 7.0, 3: 8.0, 4: 6.0}

    def measure(config):
        return Trial(config, profile(config, seconds=times[config]))

    tuning = search(1, measure, lambda trial: [trial.config + 1, trial.config + 2] if trial.config < 4 else [], 10)
    assert tuning.config == 4 and [t.config for t in tuning.trials] == [1, 2, 3, 4]
    assert "chose 4" in str(tuning) and str(tuning).count("*") == 1


def test_search_skips_what_it_tried_ignores_failures_and_keeps_to_its_budget():
    def measure(config):
        if config == "broken":
            return Trial(config, error="doesn't build")
        return Trial(config, profile(config, seconds={"a": 5.0, "b": 4.0, "c": 3.0}[config]))

    proposals_ = {"a": ["broken", "a", "b"], "b": ["a", "c"], "c": []}
    tuning = search("a", measure, lambda t: proposals_[t.config], 3)
    assert [t.config for t in tuning.trials] == ["a", "broken", "b"] and tuning.config == "b"
    assert "doesn't build" in str(tuning)


def test_search_needs_a_schedule_that_runs():
    with pytest.raises(KernelError, match="no schedule tried ran: start: no"):
        search("start", lambda c: Trial(c, error="no"), lambda t: [], 5)


def test_a_failing_start_is_replaced_by_the_first_proposal_that_runs():
    def measure(config):
        return Trial(config, error="out of LDS") if config == "big" else Trial(config, profile(config, seconds=2.0))

    tuning = search("big", measure, lambda t: ["small"] if t.config == "big" else [], 5)
    assert tuning.config == "small" and [t.config for t in tuning.trials] == ["big", "small"]


def test_a_small_gain_isnt_a_gain():
    def measure(config):
        return Trial(config, profile(config, seconds=1.0 if config == "a" else 0.995))

    assert search("a", measure, lambda t: ["b"], 5).config == "a"


# ------------------------------------------------------------------------------------------ proposals


@autokernel.tunable
class Tiles:
    tm: int = autokernel.choice(64, 128, 256, 512, default=128)
    tk: int = autokernel.choice(128, 256, 512, default=128)


SOURCE = """
def f(x, y, t=Tiles()):
    M, K = x.shape
    out = jnp.zeros((M, 128), jnp.float32)
    for i in range(0, M, t.tm):
        acc = jnp.zeros((t.tm, 128), jnp.float32)
        for k in range(0, K, t.tk):
            acc += x[i : i + t.tm, k : k + t.tk] @ y[k : k + t.tk, :]
        out = out.at[i : i + t.tm, :].set(acc)
    return out
"""


def test_proposals_follow_the_bottleneck():
    k = make_kernel(SOURCE, Tiles=Tiles)
    bf = jaxlite.bfloat16
    sig = k.signature(spec(256, 256, dtype=bf), spec(256, 128, dtype=bf))
    start = Config(Tiles(), Pipeline(2, 2))

    def tiles(found):  # the tunable moves (the family's other kernel shapes keep the tunable)
        return [c.tunable for c in found if not c.hardware]

    # Per-step overhead: bigger tiles only, fewest steps first (tm=512 doesn't divide the 256 rows).
    overhead = Trial(start, profile(start, seconds=10.0, compute=1.0))
    assert tiles(proposals(k, sig, overhead)) == [Tiles(tm=256), Tiles(tk=256)]
    # ... after the other kernel shapes at these tiles: the 128 x 128 workgroup tile in eight waves
    assert [c.hardware for c in proposals(k, sig, overhead) if c.hardware] == [(("bm", 256), ("bn", 256), ("waves", 8))]
    # Exposed input waits: one more LDS stage first, then the schedules that move fewer bytes.
    dma = Trial(start, profile(start, seconds=10.0, wait=5.0))
    assert proposals(k, sig, dma)[0] == Config(Tiles(), Pipeline(3, 2))
    assert tiles(proposals(k, sig, dma)[1:]) == [Tiles(tm=256), Tiles(tk=256)]
    # Exposed output waits: no more output buffers (gfx950 kernels store from registers: nothing to queue).
    outs = Trial(start, profile(start, seconds=10.0, out_wait=5.0))
    assert all(c.pipeline.output_buffers == 2 for c in proposals(k, sig, outs))
    # Compute-bound: every neighbour, fewest steps first; without regions the same plus one more stage.
    compute = Trial(start, profile(start, seconds=10.0))
    assert tiles(proposals(k, sig, compute)) == [Tiles(tm=256), Tiles(tk=256), Tiles(tm=64)]
    blind = Trial(start, profile(start, seconds=10.0, wait=5.0, regions=False))
    assert proposals(k, sig, blind)[1:] == proposals(k, sig, compute)
    # After a failure: two buffers, then the neighbours that build.
    failed = Trial(Config(Tiles(), Pipeline(3, 2)), error="out of LDS")
    assert proposals(k, sig, failed)[0] == Config(Tiles(), Pipeline(2, 2))


# --------------------------------------------------------------------------------- testing candidates


def test_the_reference_runs_the_fewest_iterations():
    """The reference's tests/test_tune.py:159-164: the tuner evaluates the reference at the defaults or the
    largest choices, whichever plans with fewer loop iterations."""
    from tilejax_amd.tune import _reference_config

    k = make_kernel(SOURCE, Tiles=Tiles)
    sig = k.signature(spec(256, 256), spec(256, 128))
    assert _reference_config(k, sig, k.default_config(sig)) == Tiles()  # tm=512 doesn't divide 256 rows
    sig = k.signature(spec(1024, 512), spec(512, 128))
    assert _reference_config(k, sig, k.default_config(sig)) == Tiles(tm=512, tk=512)
    plain = make_kernel(SOURCE.replace("t=Tiles()", "").replace("t.tm", "128").replace("t.tk", "128"))
    sig = plain.signature(spec(256, 256), spec(256, 128))
    assert _reference_config(plain, sig, plain.default_config(sig)) is None


def test_random_inputs():
    from tilejax_amd.tune import random_inputs

    a, b, c = random_inputs((((8, 128), jaxlite.bfloat16), ((4,), jaxlite.int32), ((64,), jaxlite.int32)),
                            bounds={2: 5}, device="cpu")
    assert a.dtype == torch.bfloat16 and b.dtype == torch.int32 and c.dtype == torch.int32
    assert int(b.abs().max()) <= 8 and float(a.float().std()) > 0.5
    assert int(c.min()) >= 0 and int(c.max()) <= 5  # an index array: from 0 to the furthest loop value


def test_a_kernel_without_a_tunable_tunes_its_buffering():
    """The reference's tests/test_tune.py:146-156: with nothing to choose in the tiles, exposed input waits
    propose one more input buffer."""
    k = make_kernel(SOURCE.replace("t=Tiles()", "").replace("t.tm", "128").replace("t.tk", "128"))
    bf = jaxlite.bfloat16
    sig = k.signature(spec(256, 256, dtype=bf), spec(256, 128, dtype=bf))
    start = k.default_config(sig)
    assert start.tunable is None and str(start) == f"{start.pipeline}"
    dma = Trial(start, profile(start, seconds=10.0, wait=5.0))
    bigger = Pipeline(start.pipeline.input_buffers + 1, start.pipeline.output_buffers)
    assert proposals(k, sig, dma)[0] == Config(None, bigger)


# --------------------------------------------------------------------------------- the gfx950 vocabulary


def test_hardware_choices_are_distinct_kernels():
    """The tuner's gfx950 vocabulary: the matmul's workgroup tiles (in four or eight waves) and attention's
    waves, key blocks and split-KV share each build a different kernel (or, for the share, different work
    items), and each compiles."""
    from examples.causal_attention import AttentionBlocks, causal_attention
    from examples.matmul import MatmulTiles, matmul
    from tilejax_amd import runtime
    from tilejax_amd.codegen import hardware_choices
    from tilejax_amd.tune import _built

    bf = jaxlite.bfloat16
    cases = [(matmul, (spec(1024, 1024, dtype=bf), spec(1024, 1024, dtype=bf)), MatmulTiles(512, 512, 512), 8),
             (causal_attention, tuple(spec(2, 4, 512, 128, dtype=bf) for _ in range(3)), AttentionBlocks(256, 256), 6)]
    for kernel, args, tiles, count in cases:
        sig = kernel.signature(*args)
        plan, schedule = kernel.build(sig, tiles)
        shapes = hardware_choices(plan, schedule)
        assert len(shapes) == count and shapes[0] == ()
        built = set()
        for hw in shapes:
            lowered = kernel.lowered(sig, Config(tiles, Pipeline(2, 2), False, hw))
            runtime.compile_source(lowered.source, f"{kernel.nest.name}.hip")
            built.add(_built(lowered))
        assert len(built) == count
    plan, schedule = matmul.build(matmul.signature(spec(1024, 1024, dtype=bf), spec(1024, 1024, dtype=bf)),
                                  MatmulTiles(512, 512, 512))
    tiles = [{"bm": 256, "bn": 128}, {"bm": 128, "bn": 256}, {"bm": 128, "bn": 128}]
    # 256 x 256 runs eight waves by default, the smaller tiles four: each is also offered with the other count
    assert [dict(h) for h in hardware_choices(plan, schedule)][1:] == (
        tiles + [{"bm": 256, "bn": 256, "waves": 4}] + [{**t, "waves": 8} for t in tiles])


# ------------------------------------------------------------------------------------- tuning a kernel


def test_off_the_gpu_tuning_uses_the_defaults():
    """The reference's tests/test_tune.py:190-197: without a device to time on, the defaults, once per
    signature."""
    k = make_kernel(SOURCE, Tiles=Tiles)
    x, y = spec(256, 256), spec(256, 128)
    tuning = k.tuning(x, y)
    assert tuning.config == k.default_config(k.signature(x, y)) and tuning.trials == []
    assert k.tuning(x, y) is tuning


def test_tuning_climbs_to_bigger_tiles_when_steps_are_overhead(monkeypatch):
    """The reference's tests/test_tune.py:200-215, with the measurement simulated (device time in proportion
    to the steps, most of it overhead): the search follows the proposals to the one-step tiles."""
    from tilejax_amd import tune

    def measure(kernel, signature, config, inputs, want):
        steps = kernel.lowered(signature, config).steps
        return Trial(config, profile(config, seconds=steps * 10e-6, steps=steps, compute=steps * 1e-6))

    monkeypatch.setattr(tune, "_can_time", lambda: True)
    monkeypatch.setattr(tune, "_measure", measure)
    monkeypatch.setattr(tune, "random_inputs", lambda signature, bounds=None, seed=0, distinct=(): [
        torch.zeros(s, dtype=dt.torch) for s, dt in signature])
    k = make_kernel(SOURCE, Tiles=Tiles)
    x, y = spec(256, 256), spec(256, 128)
    tuning = k.tuning(x, y)
    assert tuning.config.tunable == Tiles(tm=256, tk=256)  # one step a tile, one tile: the least overhead
    tiles = [t.config.tunable for t in tuning.trials if not t.config.hardware]  # (beside the other kernel shapes)
    assert tiles[:3] == [Tiles(), Tiles(tm=256), Tiles(tm=256, tk=256)]
    assert "Tiles(tm=256, tk=256)" in str(tuning)


def test_neighbours_that_build_the_same_kernel_arent_proposed():
    """The reference's tests/test_tune.py:254-262: at tiles as large as the arrays, only smaller ones change
    the kernel."""
    from examples.matmul import MatmulTiles, matmul

    sig = matmul.signature(spec(512, 512, dtype=jaxlite.bfloat16), spec(512, 512, dtype=jaxlite.bfloat16))
    start = matmul.default_config(sig)
    proposed = proposals(matmul, sig, Trial(start, profile(start, seconds=10.0)))
    assert [c.tunable for c in proposed if not c.hardware] == [MatmulTiles(tm=256), MatmulTiles(tn=256),
                                                               MatmulTiles(tk=256)]


def test_the_default_schedule_is_the_nearest_that_builds():
    @autokernel.tunable
    class Rows:
        tm: int = autokernel.choice(128, 256, 512, 1024, default=1024)

    k = make_kernel("""
    def f(x, t=Rows()):
        out = jnp.zeros((512, 128))
        for i in range(0, 512, t.tm):
            out = out.at[i : i + t.tm, :].set(x[i : i + t.tm, :])
        return out
    """, Rows=Rows)
    assert k.default_config(k.signature(spec(512, 128))).tunable == Rows(tm=512)  # 1024 doesn't divide 512


def test_a_kernel_and_its_tunable_can_be_local():
    from helpers import rand
    from tilejax_amd.jaxlite import jnp

    @autokernel.tunable
    class Local:
        tm: int = autokernel.choice(8, 16)

    @autokernel.kernel
    def double(x, tiles=Local()):
        out = jnp.zeros(x.shape)
        for i in range(0, x.shape[0], tiles.tm):
            out = out.at[i : i + tiles.tm, :].set(x[i : i + tiles.tm, :] * 2)
        return out

    x = rand((32, 128))
    assert torch.equal(double.reference(x), 2 * x) and torch.equal(double.reference(x, Local(tm=16)), 2 * x)
    assert double.lower(x).schedule.tiles == 4 and double.lower(x, Local(tm=16)).schedule.tiles == 2
