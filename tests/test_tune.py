"""The autotuner on the CPU: the search, and the proposals each bottleneck leads to, on synthetic profiles
(the reference's tests/test_tune.py:51-120). Timing and testing candidates on the GPU is in test_gpu_tune.py."""

import pytest
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
    # Per-step overhead: bigger tiles only, fewest steps first (tm=512 doesn't divide the 256 rows).
    overhead = Trial(start, profile(start, seconds=10.0, compute=1.0))
    assert [c.tunable for c in proposals(k, sig, overhead)] == [Tiles(tm=256), Tiles(tk=256)]
    # Exposed input waits: one more LDS stage first, then the schedules that move fewer bytes.
    dma = Trial(start, profile(start, seconds=10.0, wait=5.0))
    assert proposals(k, sig, dma)[0] == Config(Tiles(), Pipeline(3, 2))
    assert [c.tunable for c in proposals(k, sig, dma)[1:]] == [Tiles(tm=256), Tiles(tk=256)]
    # Exposed output waits: one more output buffer.
    outs = Trial(start, profile(start, seconds=10.0, out_wait=5.0))
    assert proposals(k, sig, outs)[0] == Config(Tiles(), Pipeline(2, 3))
    # Compute-bound: every neighbour, fewest steps first; without regions the same plus one more stage.
    compute = Trial(start, profile(start, seconds=10.0))
    assert [c.tunable for c in proposals(k, sig, compute)] == [Tiles(tm=256), Tiles(tk=256), Tiles(tm=64)]
    blind = Trial(start, profile(start, seconds=10.0, wait=5.0, regions=False))
    assert proposals(k, sig, blind)[1:] == proposals(k, sig, compute)
    # After a failure: two buffers, then the neighbours that build.
    failed = Trial(Config(Tiles(), Pipeline(3, 2)), error="out of LDS")
    assert proposals(k, sig, failed)[0] == Config(Tiles(), Pipeline(2, 2))
