"""Trace-region profiles on the CPU: summing per-workgroup region totals and classifying the bottleneck
(the reference's profiling.py:95-220 and tests/test_profiling.py)."""

import numpy as np

from tilejax_amd.profiling import CLOCK_HZ, DMA_BOUND_SHARE, OVERHEAD_BOUND_SHARE, KernelProfile, summarize


def test_summarize_averages_workgroups_and_calls():
    # two workgroups, two calls summed: [wait, fill, out_wait, compute, steps] in 100 MHz ticks
    stamps = np.array([[400, 100, 40, 1200, 8], [600, 100, 60, 1000, 8]])
    p = summarize(stamps, "k", None, calls=2, device_s=20e-6, workgroups=2)
    tick = 1 / CLOCK_HZ
    assert p.regions and p.calls == 2 and p.steps == 8
    assert np.isclose(p.wait_s, 250 * tick) and np.isclose(p.fill_s, 50 * tick)
    assert np.isclose(p.out_wait_s, 25 * tick) and np.isclose(p.compute_s, 550 * tick)
    assert np.isclose(p.exposed_wait_s, 200 * tick)
    assert np.isclose(p.other_s, 20e-6 - (250 + 25 + 550) * tick)


def test_summarize_divides_by_the_workgroups_that_run_side_by_side():
    # four workgroups on two slots (each slot runs two in turn): a slot's time is the sum of its two
    stamps = np.array([[100, 50, 10, 300, 2]] * 4)
    p = summarize(stamps, "k", None, calls=1, device_s=10e-6, workgroups=4, slots=2)
    tick = 1 / CLOCK_HZ
    assert np.isclose(p.compute_s, 600 * tick) and np.isclose(p.wait_s, 200 * tick) and p.steps == 8
    # no more slots than workgroups
    assert np.isclose(summarize(stamps, "k", None, 1, 10e-6, 4, slots=16).compute_s, 300 * tick)


def test_bottleneck_thresholds():
    def prof(wait=0.0, out=0.0, compute=10.0, fill=0.0, regions=True):
        return KernelProfile("k", None, 1, 10.0, regions, 4, wait, fill, out, compute)

    assert prof(regions=False).bottleneck is None
    assert prof(wait=DMA_BOUND_SHARE * 10 + 0.1, compute=7.0).bottleneck == "dma"
    # waits that only fill the pipeline aren't exposed
    assert prof(wait=3.0, fill=3.0, compute=7.0).bottleneck == "compute"
    assert prof(out=2.5, compute=7.0).bottleneck == "dma"
    assert prof(compute=10 - OVERHEAD_BOUND_SHARE * 10 - 0.5).bottleneck == "overhead"
    assert prof().bottleneck == "compute"
    assert "bottleneck: compute" in str(prof())


def test_summarize_reads_the_shader_clock_weighted_by_run_time():
    # [wait, fill, out_wait, compute, steps, shader cycles, 100 MHz ticks]: one workgroup at 2.0 GHz for
    # 1000 ticks, one at 1.5 GHz for 3000 ticks; the clock is total cycles over total ticks (1.625 GHz)
    stamps = np.array([[0, 0, 0, 1000, 4, 20000, 1000], [0, 0, 0, 3000, 4, 45000, 3000]])
    p = summarize(stamps, "k", None, calls=1, device_s=40e-6, workgroups=2)
    assert np.isclose(p.clock_hz, 65000 / 4000 * CLOCK_HZ)
    assert "1.625 GHz" in str(p)
    # rows without the clock fields (or no ticks) report none
    assert summarize(stamps[:, :5], "k", None, 1, 40e-6, 2).clock_hz == 0.0
