"""The headline benchmark: bf16 TFLOP/s and % of MFMA peak on one MI355X.

`python bench.py [--gpus 1] [--steps K] [--warmup W]` prints ONE JSON line. A step is one call of the
generated kernel for the workload of BASELINE.json's metric: the dense 8192^3 bf16 matmul `x @ y`
(examples/matmul.py of the reference, f32 accumulate, bf16 out), inputs ~N(0,1) from seeds 0 and 1,
already resident in HBM. `value` is its TFLOP/s (2*M*N*K / time) at MatmulTiles(512, 512, 512). The same line
carries the other BASELINE.json configurations in `legs`, each timed the same way:
- dense at MatmulTiles(1024, 2048, 1024);
- causal `tril(x @ y)` at the same size, with its time over the dense time;
- RMSNorm fused with the same matmul (`rmsnorm_matmul`, the reference's examples/rmsnorm_matmul.py);
- causal MHA at (4, 16, 2048, 128) and (1, 16, 4096, 128), each beside torch's scaled_dot_product_attention
  (its flash backend) on the same inputs;
- the MoE grouped GEMM (16384 x 4096 x 14336, 8 experts);
- paged GQA decode (64 sequences, HBM GB/s), with step tables and with a cursor, and the same sequences
  over a contiguous cache (the reference's gqa_decode).

It also carries:

- `roofline`: the dense kernel's achieved TFLOP/s (algorithmic 2*8192^3 FLOP per launch over its mean
  launch time, from HIP events recorded on the stream the kernel runs on) against the 2.5 PFLOP/s bf16
  dense MFMA peak; `traffic` is HBM bytes per launch from rocprofv3 FETCH_SIZE/WRITE_SIZE runs
  (profiles/traffic.json, used only when its recorded source hash is this run's dense kernel's; null
  otherwise), or `--traffic`;
- `cpu_baseline`: the CPU oracle's restatement of `kernel.fn` (oracle/kernels.py: the same loop nest,
  bf16 products accumulated in f32) timed on this host's cores on a bounded band of the same workload.

Only one GPU: `--gpus N` with N > 1 exits with a message.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
N_DENSE = 8192
# BASELINE.json config 2's sweep over {128..2048}^3: every cube, the two reported shapes, and shapes long along one
# dimension each
SWEEP_TILES = [(128, 128, 128), (256, 256, 256), (512, 512, 512), (1024, 1024, 1024), (2048, 2048, 2048),
               (1024, 2048, 1024), (2048, 1024, 512), (512, 2048, 256), (2048, 512, 2048), (256, 1024, 2048),
               (128, 2048, 512), (2048, 128, 1024)]


def _log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


WARM_S = [1.0]  # seconds of untimed calls before each leg's warm-up steps (--warm-seconds)


def time_kernel(run, steps: int, warmup: int):
    """(mean ms per call, per-call ms list): HIP events around each call on torch's current stream, which
    is the stream the generated kernels are launched on.

    Before the `warmup` untimed steps, the leg is run back to back for WARM_S seconds: after host work leaves
    the GPU idle its clock takes 50-100 calls of an 8192^3 matmul (tens of ms) to return to its sustained
    level, so a few warm-up steps alone would time the ramp, not the kernel."""
    import torch

    from tilejax_amd import runtime

    stream = runtime.current_stream()
    events = [runtime.Event() for _ in range(steps + 1)]
    # The spin kernel's module is loaded (on its first use in the process) before the warm-up: loaded between
    # the warm-up and the timed calls, it left the GPU idle long enough for the clock to drop, and the first
    # leg of a run measured about 10 % slower than the same kernel later (920 against 830-845 us).
    runtime.spin(0.0, stream)
    start = time.perf_counter()
    while time.perf_counter() - start < WARM_S[0]:
        for _ in range(8):
            run()
        torch.cuda.synchronize()
    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    # A short spin kernel ahead of the start event: the host queues the first calls while it runs, so the
    # first timed call doesn't wait for its own launch (the timed region is still exactly the K calls).
    runtime.spin(2e-3, stream)
    events[0].record(stream)
    for s in range(steps):
        run()
        events[s + 1].record(stream)
    torch.cuda.synchronize()
    per = [events[s].elapsed_ms(events[s + 1]) for s in range(steps)]
    return events[0].elapsed_ms(events[-1]) / steps, per


def check_dense(got, x, y) -> dict:
    """The timed kernel's output against a float32 product on the GPU: every element within 2 bf16 ulp of
    it plus twice the f32 summation bound K * 2^-24 * (|x| @ |y|). Raises if not; returns the largest error
    in ulps and the largest share of the bound used."""
    import torch

    allow = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    worst_ulp, worst_use = 0.0, 0.0
    try:
        for r in range(0, x.shape[0], 2048):
            xs = x[r:r + 2048]
            want = (xs.float() @ y.float()).to(torch.bfloat16).float()
            floor = 2.0 * x.shape[1] * 2.0 ** -24 * (xs.float().abs() @ y.float().abs())
            ulp = torch.exp2(torch.floor(torch.log2(want.abs().clamp(min=2.0 ** -126))) - 7)
            err = (got[r:r + 2048].float() - want).abs()
            use = float((err / (2 * ulp + floor)).max())
            if not use <= 1.0:
                raise AssertionError(f"dense {x.shape[0]}^3: rows {r}.. differ from a float32 product beyond 2 bf16 ulp "
                                     f"plus the f32 summation floor (bound use {use:.3g})")
            worst_use = max(worst_use, use)
            worst_ulp = max(worst_ulp, float((err / ulp)[want.abs() >= want.abs().mean()].max()))
    finally:
        torch.backends.cuda.matmul.allow_tf32 = allow
    return {"ulp_max_typical": round(worst_ulp, 3), "bound_use": round(worst_use, 4)}


def time_cpu(call, calls: int, repeats: int = 5) -> float:
    """Seconds per call on the CPU, as the reference's benchmarks/timing.py:12-22 times: one warm-up call,
    then the median over `repeats` of the mean over `calls` back-to-back calls."""
    call()
    means = []
    for _ in range(repeats):
        t0 = time.perf_counter()
        for _ in range(calls):
            call()
        means.append((time.perf_counter() - t0) / calls)
    return statistics.median(means)


def cpu_leg(what: str, call, work: float, unit: str, calls: int = 1) -> dict:
    """A leg's CPU baseline: `call` runs the spec's own reference path (kernel.reference: the loop nest
    through jaxlite on torch CPU tensors, `@` accumulating in f32) on a bounded sample of the leg's workload
    that does `work` FLOP (or bytes); its rate in `unit` (TFLOP/s or GB/s)."""
    import torch

    t = time_cpu(call, calls)
    scale = 1e12 if unit == "TFLOP/s" else 1e9
    return {"value": round(work / t / scale, 4), "unit": unit, "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"{what}; median of 5 means of {calls} call(s), {t * 1e3:.1f} ms per call"}


def cpu_baseline(budget_s: float = 12.0):
    """The oracle (oracle/kernels.matmul: the loop nest over 512^3 tiles, f32 accumulation) on a band of
    512 rows of the 8192^3 workload (x[:512] @ y, 1/16 of the FLOPs), repeated until `budget_s`."""
    import torch

    from oracle import kernels

    g = torch.Generator().manual_seed(0)
    x = torch.randn(512, N_DENSE, generator=g).to(torch.bfloat16)
    g = torch.Generator().manual_seed(1)
    y = torch.randn(N_DENSE, N_DENSE, generator=g).to(torch.bfloat16)
    flop = 2.0 * 512 * N_DENSE * N_DENSE
    kernels.matmul(x, y, 512, 512, 512)  # warm-up
    times = []
    start = time.perf_counter()
    while time.perf_counter() - start < budget_s or len(times) < 3:
        t0 = time.perf_counter()
        kernels.matmul(x, y, 512, 512, 512)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    return {"value": round(flop / t / 1e12, 4), "unit": "TFLOP/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"oracle.kernels.matmul (torch CPU, f32 accumulate) on x[:512] @ y of the 8192^3 workload, "
                      f"512^3 tiles, median of {len(times)} calls ({t * 1e3:.1f} ms each)"}


def library_attention(q, k, v, ours, args):
    """torch's scaled_dot_product_attention on the same inputs (causal, scale 1: q is pre-scaled), for
    comparison: its flash backend, else its memory-efficient one. Never its math path, whose bf16 batched
    products of transposed views this build avoids. None if neither backend runs here."""
    import torch
    from torch.nn.attention import SDPBackend, sdpa_kernel

    for backend in (SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION):
        def run():
            with sdpa_kernel([backend]):
                return torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=True, scale=1.0)
        try:
            got = run()
        except RuntimeError:
            continue
        diff = (got.float() - ours.float()).abs().max().item()
        ms, _ = time_kernel(run, args.steps, args.warmup)
        return {"what": f"torch scaled_dot_product_attention, {backend.name} backend", "us": round(ms * 1e3, 2),
                "tflops": round(2.0 * q.shape[0] * q.shape[1] * q.shape[2] ** 2 * q.shape[3] / (ms * 1e-3) / 1e12, 2),
                "max_abs_diff_to_kernel": diff}
    return None


def source_hash(source: str) -> str:
    import hashlib

    return hashlib.sha256(source.encode()).hexdigest()[:16]


def _measured_traffic(tiles, source: str):
    """HBM bytes per launch of the dense kernel at these tiles, from the committed rocprofv3 FETCH_SIZE and
    WRITE_SIZE runs (profiles/traffic.json, scaled by a known-size copy), or None: also when the kernel
    measured there (its source's hash) is not the kernel this run generated."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            data = json.load(f)
    except (OSError, ValueError):
        return None
    entry = data.get("dense_8192_" + "x".join(str(t) for t in tiles))
    if not entry or entry.get("source_sha256") != source_hash(source):
        _log("roofline.traffic: profiles/traffic.json measured another dense kernel; null until it is re-measured")
        return None
    return float(entry["bytes_per_launch"])


def leg_regions(kernel, lowered, arrays) -> dict:
    """The leg's kernel rebuilt with trace regions (the same kernel, stamping s_memrealtime around its waits,
    compute and stores) and profiled: per call, its region totals and the shader clock its workgroups ran at,
    measured in the kernel as s_memtime cycles over s_memrealtime ticks."""
    from tilejax_amd import profiling

    traced = kernel.lowered(kernel.signature(*arrays), lowered.config, trace=True)
    p = profiling.measure(traced, list(arrays), runs=5)
    _log("  " + str(p).replace("\n", "\n  "))
    us = lambda s: round(s * 1e6, 1)  # noqa: E731
    return {"device_us": us(p.device_s), "compute_us": us(p.compute_s), "input_wait_us": us(p.exposed_wait_s),
            "fill_us": us(p.fill_s), "output_us": us(p.out_wait_s), "clock_ghz": round(p.clock_hz / 1e9, 3),
            "bottleneck": p.bottleneck}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    # Each leg starts after host work (lowering, input set-up) that leaves the GPU idle, and the clock then
    # takes tens of milliseconds of load to return to its sustained level: `--warm-seconds` of untimed calls
    # (time_kernel) cover that for every leg, whatever the warm-up step count.
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--tiles", default="512,512,512", help="dense matmul spec tiles tm,tn,tk")
    ap.add_argument("--causal-tiles", default="512,512,512")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--only", default="",
                    help="comma list of legs to run: dense,library,dense2,config1,causal,rmsnorm,attention,moe,ffn,"
                         "decode")
    ap.add_argument("--traffic", default="", help="HBM bytes per dense launch (FETCH+WRITE), from rocprofv3; "
                    "default: profiles/traffic.json")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="first fill a 1 GiB tensor and negate it once: the known-size kernels rocprofv3 counters are "
                         "scaled by")
    ap.add_argument("--warm-seconds", type=float, default=1.0,
                    help="seconds of untimed back-to-back calls before each leg's warm-up steps")
    ap.add_argument("--sweep", action="store_true",
                    help="also time the dense 8192^3 matmul over spec tiles tm x tn x tk from {128..2048}^3 (BASELINE.json "
                         "config 2's sweep) and print the table to stderr")
    ap.add_argument("--regions", action="store_true",
                    help="also profile each leg's kernel rebuilt with trace regions: where its time goes, and the "
                         "shader clock it ran at, measured in the kernel")
    args = ap.parse_args()
    WARM_S[0] = args.warm_seconds
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for {args.gpus}): this build has no multi-GPU path",
              file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU (MI355X)", file=sys.stderr)
        return 2

    from examples.causal_matmul import causal_matmul
    from examples.matmul import MatmulTiles, matmul

    if args.calibrate_copy:
        # kernels of known size for scaling rocprofv3's FETCH_SIZE / WRITE_SIZE: a 1 GiB fill (writes 1 GiB)
        # and a negation of it (reads 1 GiB and writes 1 GiB; no other leg runs torch.neg)
        src = torch.ones(1 << 29, dtype=torch.bfloat16, device="cuda")  # 1 GiB
        dst = torch.neg(src)
        torch.cuda.synchronize()
        del src, dst

    legs = set(args.only.split(",")) if args.only else {"dense", "causal", "rmsnorm", "attention", "moe", "ffn", "decode"}
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(0)
    xh = torch.randn(N_DENSE, N_DENSE, generator=g).to(torch.bfloat16)
    g = torch.Generator().manual_seed(1)
    yh = torch.randn(N_DENSE, N_DENSE, generator=g).to(torch.bfloat16)
    x, y = xh.to(dev), yh.to(dev)
    flop = 2.0 * N_DENSE**3
    tiles = MatmulTiles(*(int(v) for v in args.tiles.split(",")))
    out = {}
    # Each leg's CPU baseline, run after the GPU legs: (leg, what, call, work, unit, calls)
    cpu_jobs = [("dense", f"kernel.reference of the headline on x[:512] @ y (a band of 512 rows, 1/16 of it), {tiles}",
                 lambda: matmul.reference(xh[:512], yh, tiles), 2.0 * 512 * N_DENSE * N_DENSE, "TFLOP/s", 1)]

    _log(f"dense matmul {N_DENSE}^3 tiles {tiles}: lowering")
    lowered = matmul.lower(x, y, tiles)
    _log(f"  hardware: {lowered.program.notes}")
    check = check_dense(lowered.run(x, y), x, y)
    _log(f"  checked against a float32 product: {check}")
    ms, per = time_kernel(lambda: lowered.run(x, y), args.steps, args.warmup)
    tflops = flop / (ms * 1e-3) / 1e12
    launch_ms = statistics.mean(per)
    _log(f"  {ms * 1e3:.1f} us/call, {tflops:.1f} TFLOP/s ({100 * tflops / PEAK_TFLOPS:.1f}% of peak)")
    out["dense"] = {"tiles": [tiles.tm, tiles.tn, tiles.tk], "us": round(ms * 1e3, 2),
                    "tflops": round(tflops, 2), "hw": lowered.program.notes, "check": check}
    if args.regions:
        out["dense"]["regions"] = leg_regions(matmul, lowered, (x, y))

    if "library" in legs or not args.only:
        # the vendor library on the same inputs, for comparison: torch.matmul (hipBLASLt), bf16 out
        _log(f"torch.matmul {N_DENSE}^3 (hipBLASLt)")
        msl, _ = time_kernel(lambda: torch.matmul(x, y), args.steps, args.warmup)
        out["dense_library"] = {"what": "torch.matmul(x, y), hipBLASLt", "us": round(msl * 1e3, 2),
                                "tflops": round(flop / (msl * 1e-3) / 1e12, 2)}
        _log(f"  {msl * 1e3:.1f} us/call, {flop / (msl * 1e-3) / 1e12:.1f} TFLOP/s")

    if "dense2" in legs or not args.only:
        t2 = MatmulTiles(1024, 2048, 1024)
        _log(f"dense matmul {N_DENSE}^3 tiles {t2}: lowering")
        l2 = matmul.lower(x, y, t2)
        ms2, _ = time_kernel(lambda: l2.run(x, y), args.steps, args.warmup)
        _log(f"  {ms2 * 1e3:.1f} us/call, {flop / (ms2 * 1e-3) / 1e12:.1f} TFLOP/s")
        out["dense_1024x2048x1024"] = {"tiles": [t2.tm, t2.tn, t2.tk], "us": round(ms2 * 1e3, 2),
                                       "tflops": round(flop / (ms2 * 1e-3) / 1e12, 2),
                                       "frac_peak": round(flop / (ms2 * 1e-3) / 1e12 / PEAK_TFLOPS, 4)}

    if "config1" in legs or not args.only:
        # 1024^3 at MatmulTiles(512, 512, 512), the spec run as `matmul.fn` on the CPU (the
        # function as written, the reference's plain-JAX path) and the kernel's output verified against it
        t1 = MatmulTiles(512, 512, 512)
        g = torch.Generator().manual_seed(0)
        x1h = torch.randn(1024, 1024, generator=g).to(torch.bfloat16)
        y1h = torch.randn(1024, 1024, generator=g).to(torch.bfloat16)
        x1, y1 = x1h.to(dev), y1h.to(dev)
        l1 = matmul.lower(x1, y1, t1)
        got1 = l1.run(x1, y1).cpu()
        from tilejax_amd.api import compare

        fn_out = matmul.fn(x1h, y1h, t1)
        diff1 = compare("config 1: the kernel against matmul.fn", got1, fn_out, inputs=(x1h.dtype, y1h.dtype))
        ms1, _ = time_kernel(lambda: l1.run(x1, y1), args.steps, args.warmup)
        flop1 = 2.0 * 1024**3
        _log(f"config 1 (1024^3, {t1}): {ms1 * 1e3:.1f} us, {flop1 / (ms1 * 1e-3) / 1e12:.1f} TFLOP/s; the kernel "
             f"against matmul.fn on the CPU: largest difference {diff1:.3g}")
        out["config1"] = {"shape": [1024] * 3, "tiles": [512, 512, 512], "us": round(ms1 * 1e3, 2),
                          "tflops": round(flop1 / (ms1 * 1e-3) / 1e12, 2),
                          "frac_peak": round(flop1 / (ms1 * 1e-3) / 1e12 / PEAK_TFLOPS, 4), "vs_fn_max_abs_diff": diff1}
        cpu_jobs.append(("config1", f"matmul.fn (the function as written, plain-JAX semantics) on the whole 1024^3 "
                         f"workload, {t1}", lambda: matmul.fn(x1h, y1h, t1), flop1, "TFLOP/s", 3))

    if args.sweep:
        _log(f"dense matmul {N_DENSE}^3, spec tiles swept:")
        sweep = []
        for tm_, tn_, tk_ in SWEEP_TILES:
            st = MatmulTiles(tm_, tn_, tk_)
            sl = matmul.lower(x, y, st)
            sms, _ = time_kernel(lambda: sl.run(x, y), args.steps, args.warmup)
            hw_ = sl.program.notes
            sweep.append({"tiles": [tm_, tn_, tk_], "us": round(sms * 1e3, 2),
                          "tflops": round(flop / (sms * 1e-3) / 1e12, 2), "hw_tile": list(hw_["hw_tile"]),
                          "waves": hw_["waves"], "stages": hw_["stages"]})
            _log(f"  {tm_:5d} x {tn_:5d} x {tk_:5d}: {sms * 1e3:7.1f} us {flop / (sms * 1e-3) / 1e12:7.1f} TFLOP/s "
                 f"(workgroup tile {hw_['hw_tile']}, {hw_['waves']} waves, {hw_['stages']} stages)")
        out["dense_tile_sweep"] = sweep

    if "causal" in legs:
        ct = MatmulTiles(*(int(v) for v in args.causal_tiles.split(",")))
        _log(f"causal matmul {N_DENSE}^3 tiles {ct}: lowering")
        cl = causal_matmul.lower(x, y, ct)
        cms, _ = time_kernel(lambda: cl.run(x, y), args.steps, args.warmup)
        _log(f"  {cms * 1e3:.1f} us/call = {cms / ms:.3f} x dense")
        # the work the kernel executes: its computed workgroup tiles (whole ones, and those cut into K-chunks)
        notes, items = cl.program.notes, cl.program.tables["items"].reshape(-1, 3)
        bm, bn, _ = notes["hw_tile"]
        computed = int(((items[:, 1] >> 16) == 0).sum()) + (notes["split"][0] if notes["split"] else 0)
        exec_tf = 2.0 * computed * bm * bn * N_DENSE / (cms * 1e-3) / 1e12
        out["causal"] = {"tiles": [ct.tm, ct.tn, ct.tk], "us": round(cms * 1e3, 2), "vs_dense": round(cms / ms, 4),
                         "tflops_dense_equiv": round(flop / (cms * 1e-3) / 1e12, 2),
                         "computed_tiles": computed, "tflops_executed": round(exec_tf, 2),
                         "frac_peak": round(exec_tf / PEAK_TFLOPS, 4)}
        if args.regions:
            out["causal"]["regions"] = leg_regions(causal_matmul, cl, (x, y))
        cpu_jobs.append(("causal", f"kernel.reference of the whole 8192^3 causal matmul, {ct} (rate on the dense "
                         "FLOP count, as the GPU leg's tflops_dense_equiv)",
                         lambda: causal_matmul.reference(xh, yh, ct), flop, "TFLOP/s", 1))

    if "rmsnorm" in legs:
        try:
            from examples.rmsnorm_matmul import NormMatmulTiles, rmsnorm_matmul

            g = torch.Generator().manual_seed(2)
            gh = (1 + 0.1 * torch.randn(1, N_DENSE, generator=g)).to(torch.bfloat16)
            gamma = gh.to(dev)
            nt = NormMatmulTiles(tiles.tm, tiles.tn, tiles.tk)
            rl = rmsnorm_matmul.lower(x, gamma, y, nt)
            cpu_jobs.append(("rmsnorm_matmul", f"kernel.reference on rows 0..511 of the 8192^3 workload, {nt}",
                             lambda: rmsnorm_matmul.reference(xh[:512], gh, yh, nt), 2.0 * 512 * N_DENSE * N_DENSE,
                             "TFLOP/s", 1))
            rms_, _ = time_kernel(lambda: rl.run(x, gamma, y), args.steps, args.warmup)
            _log(f"RMSNorm + matmul {N_DENSE}^3: {rms_ * 1e3:.1f} us = {rms_ / ms:.3f} x dense")
            out["rmsnorm_matmul"] = {"shape": [N_DENSE] * 3, "us": round(rms_ * 1e3, 2), "vs_dense": round(rms_ / ms, 4),
                                     "tflops": round(flop / (rms_ * 1e-3) / 1e12, 2),
                                     "frac_peak": round(flop / (rms_ * 1e-3) / 1e12 / PEAK_TFLOPS, 4)}
        except Exception as e:  # reported, not hidden
            _log(f"RMSNorm + matmul: not measured ({type(e).__name__}: {str(e).splitlines()[0]})")
            out["rmsnorm_matmul"] = {"error": f"{type(e).__name__}: {str(e).splitlines()[0][:200]}"}

    if "attention" in legs:
        try:
            from examples.causal_attention import AttentionBlocks, causal_attention

            for key, (B, H, S, D) in (("attention", (4, 16, 2048, 128)), ("attention_4096", (1, 16, 4096, 128))):
                gens = [torch.Generator().manual_seed(s) for s in (0, 1, 2)]
                qh, kh, vh = (torch.randn(B, H, S, D, generator=gg).to(torch.bfloat16) for gg in gens)
                qh = (qh.float() * D**-0.5).to(torch.bfloat16)
                q, k, v = qh.to(dev), kh.to(dev), vh.to(dev)
                blocks = AttentionBlocks(512, 512)
                hs = 2  # the CPU sample: batch 0, heads 0 and 1 (each head is its own tiles of the nest)
                cpu_jobs.append((key, f"kernel.reference on batch 0, heads 0..{hs - 1} of ({B}, {H}, {S}, {D}), {blocks}",
                                 lambda qs=qh[:1, :hs].clone(), ks=kh[:1, :hs].clone(), vs=vh[:1, :hs].clone(), b=blocks:
                                 causal_attention.reference(qs, ks, vs, b), 2.0 * hs * S * S * D, "TFLOP/s", 1))
                al = causal_attention.lower(q, k, v, blocks)
                ams, _ = time_kernel(lambda: al.run(q, k, v), args.steps, args.warmup)
                aflop = 2.0 * B * H * S * S * D  # algorithmic causal count (QK^T and PV over the lower triangle)
                atf = aflop / (ams * 1e-3) / 1e12
                _log(f"causal MHA {B}x{H}x{S}x{D}: {ams * 1e3:.1f} us, {atf:.1f} TFLOP/s")
                out[key] = {"shape": [B, H, S, D], "blocks": [512, 512], "us": round(ams * 1e3, 2),
                            "tflops": round(atf, 2), "frac_peak": round(atf / PEAK_TFLOPS, 4)}
                lib = library_attention(q, k, v, al.run(q, k, v), args)
                if lib:
                    out[key]["library"] = lib
                    _log(f"  {lib['what']}: {lib['us']:.1f} us, {aflop / (lib['us'] * 1e-6) / 1e12:.1f} TFLOP/s")
                if args.regions:
                    out[key]["regions"] = leg_regions(causal_attention, al, (q, k, v))
                del q, k, v
        except Exception as e:  # not lowered yet: reported, not hidden
            _log(f"causal MHA: not measured ({type(e).__name__}: {str(e).splitlines()[0]})")
            out["attention"] = {"error": f"{type(e).__name__}: {str(e).splitlines()[0][:200]}"}

    if "moe" in legs:
        try:
            from examples.moe import GroupTiles, grouped_matmul

            g = torch.Generator().manual_seed(0)
            counts = torch.multinomial(torch.full((8,), 1 / 8), 64, replacement=True, generator=g).bincount(minlength=8)
            geh = torch.repeat_interleave(torch.arange(8), counts).to(torch.int32)
            xsh = torch.randn(16384, 4096, generator=g).to(torch.bfloat16)
            wh = (torch.randn(8, 4096, 14336, generator=g) * 0.02).to(torch.bfloat16)
            ge, xs, w = geh.to(dev), xsh.to(dev), wh.to(dev)
            gt = GroupTiles(512, 512)
            gl = grouped_matmul.lower(xs, w, ge, gt)
            cpu_jobs.append(("moe", f"kernel.reference on groups 0 and 1 (512 rows) of config 4, all 8 experts, {gt}",
                             lambda: grouped_matmul.reference(xsh[:512], wh, geh[:2], gt), 2.0 * 512 * 4096 * 14336,
                             "TFLOP/s", 1))
            mms, _ = time_kernel(lambda: gl.run(xs, w, ge), args.steps, args.warmup)
            mflop = 2.0 * 16384 * 4096 * 14336
            mtf = mflop / (mms * 1e-3) / 1e12
            _log(f"MoE grouped GEMM 16384x4096x14336 (8 experts): {mms * 1e3:.1f} us, {mtf:.1f} TFLOP/s")
            out["moe"] = {"shape": [16384, 4096, 14336, 8], "tiles": [512, 512], "us": round(mms * 1e3, 2),
                          "tflops": round(mtf, 2), "frac_peak": round(mtf / PEAK_TFLOPS, 4)}
            if args.regions:
                out["moe"]["regions"] = leg_regions(grouped_matmul, gl, (xs, w, ge))
            del xs, w
        except Exception as e:
            _log(f"MoE: not measured ({type(e).__name__}: {str(e).splitlines()[0]})")
            out["moe"] = {"error": f"{type(e).__name__}: {str(e).splitlines()[0][:200]}"}

    if "ffn" in legs:
        # The MoE expert layer (examples/moe.py `expert_ffn`, the reference's examples/moe.py:167-187) at Mixtral
        # 8x7B's width: config 4's 16384 routed rows in 64 tiles of 256 with the same seeded expert counts,
        # D = 4096, F = 14336, 8 experts; gate, up and down products, 6 * 16384 * 4096 * 14336 FLOP per call.
        try:
            from examples.moe import ExpertTiles, expert_ffn

            g = torch.Generator().manual_seed(0)
            counts = torch.multinomial(torch.full((8,), 1 / 8), 64, replacement=True, generator=g).bincount(minlength=8)
            teh = torch.repeat_interleave(torch.arange(8), counts).to(torch.int32)
            xsh = torch.randn(16384, 4096, generator=g).to(torch.bfloat16)
            wsh = [(torch.randn(8, *shape, generator=g) * 0.02).to(torch.bfloat16)
                   for shape in ((4096, 14336), (4096, 14336), (14336, 4096))]
            fargs = (xsh.to(dev), *(w_.to(dev) for w_ in wsh), teh.to(dev))
            et = ExpertTiles(256)
            fl = expert_ffn.lower(*fargs, et)
            cpu_jobs.append(("ffn", f"kernel.reference on tiles 0 and 1 (512 rows), all 8 experts' weights, {et}",
                             lambda: expert_ffn.reference(xsh[:512], *wsh, teh[:2], et), 6.0 * 512 * 4096 * 14336,
                             "TFLOP/s", 1))
            fms, _ = time_kernel(lambda: fl.run(*fargs), args.steps, args.warmup)
            fflop = 6.0 * 16384 * 4096 * 14336
            ftf = fflop / (fms * 1e-3) / 1e12
            _log(f"MoE expert layer (expert_ffn) 16384 rows, 4096 -> 14336 -> 4096, 8 experts: {fms * 1e3:.1f} us, "
                 f"{ftf:.1f} TFLOP/s ({100 * ftf / PEAK_TFLOPS:.1f}% of peak)")
            out["ffn"] = {"shape": [16384, 4096, 14336, 8], "tiles": [256], "us": round(fms * 1e3, 2),
                          "tflops": round(ftf, 2), "frac_peak": round(ftf / PEAK_TFLOPS, 4),
                          "kernels": [launch.symbol for launch in fl.program.launches]}
            if args.regions:
                out["ffn"]["regions"] = leg_regions(expert_ffn, fl, fargs)
            del fargs
        except Exception as e:
            _log(f"expert_ffn: not measured ({type(e).__name__}: {str(e).splitlines()[0]})")
            out["ffn"] = {"error": f"{type(e).__name__}: {str(e).splitlines()[0][:200]}"}

    if "decode" in legs:
        try:
            from examples.decode import paged_gqa_decode

            B, H, Hkv, D, P, pages = 64, 32, 8, 128, 16, 512
            g = torch.Generator().manual_seed(0)
            lengths = torch.randint(128, 8193, (B,), generator=g, dtype=torch.int32)
            qh = (torch.randn(B, 1, H, D, generator=g) * D**-0.5).to(torch.bfloat16)
            tableh = torch.randperm(B * pages, generator=g).reshape(B, pages).to(torch.int32)
            kph = torch.randn(B * pages, P, Hkv * D, generator=g).to(torch.bfloat16)
            vph = torch.randn(B * pages, P, Hkv * D, generator=g).to(torch.bfloat16)
            q, table, kp, vp, ln = qh.to(dev), tableh.to(dev), kph.to(dev), vph.to(dev), lengths.to(dev)
            nb = 8  # the CPU sample: sequences 0..7 over the whole page pool
            sample_bytes = int(lengths[:nb].sum()) * Hkv * D * 2 * 2
            cpu_jobs.append(("decode", f"kernel.reference on sequences 0..{nb - 1} of config 5 (their valid K and V rows "
                             f"through the page table: {sample_bytes} bytes)",
                             lambda: paged_gqa_decode.reference(qh[:nb], kph, vph, tableh[:nb], lengths[:nb]),
                             sample_bytes, "GB/s", 1))
            from tilejax_amd.tune import Config

            dsig = paged_gqa_decode.signature(q, kp, vp, table, ln)
            dl = paged_gqa_decode.lowered(dsig, paged_gqa_decode.default_config(dsig))
            # the two ways of finding the steps: device step tables, or a cursor in the attention kernel
            dc = paged_gqa_decode.lowered(paged_gqa_decode.signature(q, kp, vp, table, ln),
                                          Config(dl.config.tunable, dl.config.pipeline, True))
            tms, _ = time_kernel(lambda: dl.run(q, kp, vp, table, ln), args.steps, args.warmup)
            cms, _ = time_kernel(lambda: dc.run(q, kp, vp, table, ln), args.steps, args.warmup)
            dms = min(tms, cms)
            # the valid K and V rows, plus queries, outputs, the page table and the lengths
            dbytes = int(lengths.sum()) * Hkv * D * 2 * 2 + 2 * q.numel() * 2 + table.numel() * 4 + B * 4
            gbs = dbytes / (dms * 1e-3) / 1e9
            _log(f"paged GQA decode 64 seqs, 32/8 heads, 16-token pages: {tms * 1e3:.1f} us with step tables, "
                 f"{cms * 1e3:.1f} us with a cursor; {gbs:.0f} GB/s")
            out["decode"] = {"sequences": B, "heads": [H, Hkv], "page": P, "sum_lengths": int(lengths.sum()),
                             "us": round(dms * 1e3, 2), "us_tables": round(tms * 1e3, 2),
                             "us_cursor": round(cms * 1e3, 2), "bytes": dbytes, "gbs": round(gbs, 1),
                             "frac_hbm_peak": round(gbs / 8000.0, 4)}
            if args.regions:
                out["decode"]["regions"] = leg_regions(paged_gqa_decode, dl, (q, kp, vp, table, ln))
            del kp, vp
            # the contiguous cache (the reference's gqa_decode): the same 64 sequences over 8192 positions
            from examples.decode import DecodeTiles, gqa_decode

            S = pages * P
            kch = torch.randn(B, S, Hkv * D, generator=g).to(torch.bfloat16)
            vch = torch.randn(B, S, Hkv * D, generator=g).to(torch.bfloat16)
            kc, vc = kch.to(dev), vch.to(dev)
            gl = gqa_decode.lower(q, kc, vc, ln, DecodeTiles(512))
            cblocks = int(sum(-(-int(n) // 512) for n in lengths[:nb])) * 512 * Hkv * D * 2 * 2
            cpu_jobs.append(("decode_contiguous", f"kernel.reference on sequences 0..{nb - 1} ({cblocks} bytes of "
                             "whole 512-position blocks)",
                             lambda: gqa_decode.reference(qh[:nb], kch[:nb].clone(), vch[:nb].clone(), lengths[:nb],
                                                          DecodeTiles(512)), cblocks, "GB/s", 1))
            gc = gqa_decode.lowered(gqa_decode.signature(q, kc, vc, ln), Config(DecodeTiles(512), gl.config.pipeline, True))
            gms = min(time_kernel(lambda: gl.run(q, kc, vc, ln), args.steps, args.warmup)[0],
                      time_kernel(lambda: gc.run(q, kc, vc, ln), args.steps, args.warmup)[0])
            # whole 512-position blocks are read up to each sequence's end
            blocks = int(sum(-(-int(n) // 512) for n in lengths)) * 512
            gbytes = blocks * Hkv * D * 2 * 2 + 2 * q.numel() * 2 + B * 4
            _log(f"contiguous GQA decode 64 x 8192, block_kv 512: {gms * 1e3:.1f} us, {gbytes / (gms * 1e-3) / 1e9:.0f} GB/s")
            out["decode_contiguous"] = {"sequences": B, "cache": S, "block_kv": 512, "us": round(gms * 1e3, 2),
                                        "bytes": gbytes, "gbs": round(gbytes / (gms * 1e-3) / 1e9, 1),
                                        "frac_hbm_peak": round(gbytes / (gms * 1e-3) / 1e9 / 8000.0, 4)}
            del kc, vc
        except Exception as e:
            _log(f"decode: not measured ({type(e).__name__}: {str(e).splitlines()[0]})")
            out["decode"] = {"error": f"{type(e).__name__}: {str(e).splitlines()[0][:200]}"}

    achieved = flop / (launch_ms * 1e-3) / 1e12
    traffic = float(args.traffic) if args.traffic else _measured_traffic(out["dense"]["tiles"], lowered.source)
    result = {
        "metric": "bf16 TFLOP/s + % MFMA peak: 8192^3 matmul; causal MHA B4 H16 S2048 D128",
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: x, y ~N(0,1) bf16 from torch seeds 0 and 1, resident in HBM",
        "config": {"workload": f"dense matmul x @ y, M=N=K={N_DENSE}, bf16 in, f32 accumulate, bf16 out, "
                               f"MatmulTiles{tuple(out['dense']['tiles'])}"},
        "frac_peak": round(tflops / PEAK_TFLOPS, 4),
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_TFLOPS, 4), "traffic": traffic},
        "legs": out,
    }
    result["warmup_s"] = WARM_S[0]
    if not args.no_cpu:
        _log("cpu baseline ...")
        result["cpu_baseline"] = cpu_baseline()
        for leg, what, call, work, unit, calls in cpu_jobs:
            if leg not in out or "error" in out[leg]:
                continue
            try:
                out[leg]["cpu_baseline"] = cpu_leg(what, call, work, unit, calls)
                _log(f"  cpu {leg}: {out[leg]['cpu_baseline']['value']} {unit}")
            except Exception as e:  # reported, not hidden
                out[leg]["cpu_baseline"] = {"error": f"{type(e).__name__}: {str(e).splitlines()[0][:200]}"}
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
