"""Benchmark: ms per Sinkhorn iteration (f half-step + g half-step) on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
    python bench.py --profile [--reps R]     # for rocprofv3: R loop iterations, then a 256 MiB copy
    python bench.py --profile --workload stress-65k [--reps R]   # the same on the 65k d 128 stress clouds
    python bench.py --profile --workload {single-cell, single-cell-pipeline} [--reps R]   # and the d 30 workloads
    python bench.py --workload {single-cell, single-cell-pipeline, stress-65k} [--no-cpu]

Workload: synthetic balanced 10,000 x 10,000, d = 64, fp32, x ~ N(0, 1) (seed 0), y ~ N(0, 1) + 0.5
(seed 1), uniform weights, squared-Euclidean cost, no normalisation, eps = 0.1 (the reference's
examples/sinkhorn_benchmark.py --flashsinkhorn setup). A "step" is one iteration of the on-device loop
(f half-step, g half-step, loop control), inputs resident in HBM: two launches of the fused partial kernel
(lse_partial_kernel), each merging its own row groups. W untimed iterations, then exactly K timed iterations
between two device synchronisations (defaults 100 and 200: the first ~100 iterations of a process run ~8 %
slower while the GPU's clocks settle).

Also reported on the same JSON line:
* roofline -- the dominant kernel, lse_partial_kernel (every launch of the timed region is one): its average
  launch time from HIP events recorded on its stream around the timed region, divided by the 2 K launches.
  `achieved` is the algorithmic work of one launch, the augmented contraction [x, 1].[2y/eps, g/eps + log b],
  2 n m (d + 1) FLOP (1.30e10 at 10k, d 64), over that time, against the 2.5 PFLOP/s fp16 dense peak of the pipe
  the kernel runs on. The kernel forms that contraction fp32-accurately as three fp16 products of a two-piece
  split of the coordinates: `executed` counts those (3 x 2 x n m kp per launch, padding excluded, about 2.95
  times the algorithmic count) against the same peak. `exp` gives the n m exponentials per launch against the
  1.966e13/s transcendental peak (v_exp_f32 at half rate on gfx950, measured: 256 CUs x 4 SIMDs x 8 lanes at
  2.4 GHz; the quarter rate of earlier CDNA parts would be 9.83e12/s), and `fp32_equivalent` the algorithmic
  FLOP against the 157.3 TFLOP/s fp32 MFMA peak (a ratio above 1: the contraction does not run on that pipe). `traffic` is the HBM bytes per launch from the committed
  counter summary (FETCH_SIZE and WRITE_SIZE passes, scaled by a plain copy's readings);
* iteration_roofline -- per iteration, max(executed fp16 MFMA FLOP / 2.5e15, 2 n m / 1.966e13) seconds over the
  measured ms/iteration (the exp + MFMA roofline the metric names, on the pipe the kernel runs on), and beside
  it the fp32-MFMA form max(4 n m (d + 1) / 157.3e12, 2 n m / 1.966e13) as a ratio;
* cpu_baseline -- the reference's plain-PyTorch CPU path (the oracle's restatement, float32, block 2048,
  all host cores) on the same workload: best of 3 runs of 10 fixed iterations after 1 warm-up iteration;
* end_to_end_s -- sinkhorn() wall time for 10 fixed iterations, host arrays in, float64 potentials out
  (setup, H2D, packing, loop, read-back): best of 3 after 2 warm-up calls.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "trainium-sinkhorn_amd"))

N, M, D, EPS = 10_000, 10_000, 64, 0.1
MFMA_F32_PEAK = 157.3e12
MFMA_F16_PEAK = 2.5e15
EXP_PEAK = 1.966e13   # v_exp_f32 lanes/s: 32 per clock per CU (half rate on gfx950) x 256 CUs x 2.4 GHz
PRODUCTS = 3          # fp16 piece products per K chunk of the half-step contraction


def profiled_traffic():
    """HBM bytes per launch of the dominant kernel from the committed counter summary (FETCH_SIZE and
    WRITE_SIZE passes, scaled by the copy calibration), or None if the summary is absent."""
    import re
    p = ROOT / "profiles" / "loop_10k_d64_counters.md"
    m = re.search(r"traffic_bytes_per_launch:\s*(\d+)", p.read_text()) if p.exists() else None
    return int(m.group(1)) if m else None


def make_inputs():
    import numpy as np
    x = np.random.default_rng(0).standard_normal((N, D))
    y = np.random.default_rng(1).standard_normal((M, D)) + 0.5
    return x, y


def _loop(n_iters):
    """The benchmark's on-device loop, initialised (x's log2-unit copy made, the state written)."""
    import numpy as np
    import torch
    from trnopt import hip_sinkhorn as hk

    hk.lib()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    x, y = make_inputs()
    X = hk.HipCloud(x, np.full(N, -np.log(N)), dev, role=0)
    Y = hk.HipCloud(y, np.full(M, -np.log(M)), dev, role=1)
    loop = hk.DeviceLoop(X, Y, eps=EPS, rho_x=None, rho_y=None, sched=[], stages=[], tol=1e-4, stage_tol=1e-5,
                         max_iters=n_iters, check_every=10, stage_max_iters=1000, fixed_iters=True, balanced=True)
    loop.init()
    return x, y, loop


def gpu_run(steps, warmup):
    import torch
    from trnopt import hip_sinkhorn as hk

    x, y, loop = _loop(warmup + steps + 1)
    loop.capture()                       # with TRNOPT_HIP_GRAPH=1: the graph of a batch, before any timing
    loop.enqueue(warmup)
    stream = torch.cuda.current_stream()   # the stream every loop kernel is launched on
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record(stream)
    loop.enqueue(steps)
    ev1.record(stream)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_per_it = (t1 - t0) * 1e3 / steps
    kernel_ms = ev0.elapsed_time(ev1) / (2 * steps)     # two lse_partial_kernel launches per iteration
    st = loop.read_state()
    assert st.it == warmup + steps and not st.done, (st.it, st.done)

    # end to end: sinkhorn() with host arrays, 10 fixed iterations
    from trnopt import Backend, SinkhornOptions, sinkhorn
    o = SinkhornOptions(eps=EPS, normalize=False, max_iters=10, fixed_iters=True, kernel="hip",
                        backend=Backend.preset("rocm"))
    for _ in range(2):                   # warm-up: the caching allocator and pinned buffers settle
        sinkhorn(x, y, opts=o)
    torch.cuda.synchronize()
    e2e = float("inf")
    for _ in range(3):                   # best of 3, each from host arrays to float64 potentials on the host
        te = time.perf_counter()
        sinkhorn(x, y, opts=o)
        e2e = min(e2e, time.perf_counter() - te)
    return dict(ms_per_it=ms_per_it, kernel_ms=kernel_ms, e2e=e2e, kp=hk.pad_dim(D))


def profile_run(reps):
    """What the rocprofv3 summaries are taken from: `reps` iterations of the benchmark's on-device loop (2 reps
    launches of the dominant kernel), then one plain device copy of 256 MiB (two copy dispatches of 128 MiB),
    whose FETCH_SIZE / WRITE_SIZE calibrate the counters (each dispatch reads and writes exactly 131072 KiB)."""
    import torch
    _, _, loop = _loop(reps + 1)
    loop.enqueue(reps)
    src = torch.ones(64 << 20, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    print(f"profile: {reps} loop iterations of {N} x {M} d {D}, then a 256 MiB copy", flush=True)


def profile_stress(reps, eps=0.01):
    """The stress counterpart of profile_run: `reps` iterations of the on-device loop on the 65,536 x 65,536 d 128
    mixture clouds (median-normalised, uniform weights) at one eps (the staged partial kernel, kp 128), then the
    same 256 MiB copy."""
    import numpy as np
    import torch
    from trnopt import hip_sinkhorn as hk
    from trnopt.sinkhorn import normalization

    hk.lib()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    x, y = stress_inputs()
    center, scale = normalization(x, y, how="median")
    xs, ys = (x - center) / np.sqrt(scale), (y - center) / np.sqrt(scale)
    n = len(xs)
    X = hk.HipCloud(xs, np.full(n, -np.log(n)), dev, role=0)
    Y = hk.HipCloud(ys, np.full(n, -np.log(n)), dev, role=1)
    loop = hk.DeviceLoop(X, Y, eps=eps, rho_x=None, rho_y=None, sched=[], stages=[], tol=1e-4, stage_tol=1e-5,
                         max_iters=reps + 1, check_every=10, stage_max_iters=1000, fixed_iters=True, balanced=True)
    loop.init()
    loop.enqueue(reps)
    src = torch.ones(64 << 20, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    print(f"profile: {reps} loop iterations of {n} x {n} d 128 at eps {eps}, then a 256 MiB copy", flush=True)


def profile_single_cell(reps):
    """The single-cell counterpart of profile_run: one sinkhorn(kernel="hip") call of the single-cell workload
    (7,355 x 8,962, d 30, eps 0.05, rho (1, 50), median-normalised cost, wot formulation) held to `reps` fixed
    iterations (the streamed partial kernel at kp 32 and a merge kernel per half-step: both passes have fewer than
    40 row groups), then the same 256 MiB copy."""
    import numpy as np
    import torch
    from trnopt import Backend, SinkhornOptions, sinkhorn
    x, y, w = single_cell_inputs()
    I, J = len(x), len(y)
    a, b = np.full(I, 1.0 / I), np.full(J, 1.0 / J)
    o = SinkhornOptions(eps=0.05, rho=(1.0, 50.0), normalize="median", tol=1e-6, max_iters=reps, fixed_iters=True,
                        kernel="hip", backend=Backend.preset("rocm"))
    r = sinkhorn(x, y, a, b, o, a_target=w, b_target=b)
    src = torch.ones(64 << 20, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    print(f"profile: {r.iterations} iterations of the {I} x {J} d 30 single-cell solve, then a 256 MiB copy",
          flush=True)


def profile_pipeline(reps):
    """The batched pipeline's counterpart of profile_run: the 38 pairs of the pipeline workload (median-normalised,
    wot's formulation with uniform targets, as a first growth iteration) as one sinkhorn_batch held to `reps`
    fixed iterations at eps 0.05 (the grouped partial kernel, kp 32: each launch one half-step of every pair), then
    the same 256 MiB copy."""
    import numpy as np
    import torch
    from trnopt import Backend, SinkhornOptions
    from trnopt.sinkhorn import sinkhorn_batch
    sizes = pipeline_sizes()
    o = SinkhornOptions(eps=0.05, rho=(1.0, 50.0), normalize="median", max_iters=reps, fixed_iters=True,
                        kernel="hip", backend=Backend.preset("rocm"))
    qs = []
    for t in range(len(sizes) - 1):
        x0, x1 = single_cell_inputs(n=int(sizes[t]), m=int(sizes[t + 1]), t0=t, t1=t + 1)[:2]
        I, J = len(x0), len(x1)
        qs.append(dict(x=x0, y=x1, a=np.full(I, 1.0 / I), b=np.full(J, 1.0 / J), opts=o,
                       a_target=np.full(I, 1.0 / I), b_target=np.full(J, 1.0 / J)))
    res = sinkhorn_batch(qs)
    src = torch.ones(64 << 20, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    print(f"profile: {res[0].iterations} batched iterations of the {len(qs)} pipeline pairs, then a 256 MiB copy",
          flush=True)


def _cpu_model():
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


def cpu_baseline(iters=10, reps=3):
    """The reference's plain-PyTorch CPU path (oracle restatement), float32, block 2048, all host cores:
    best of `reps` runs of `iters` fixed iterations, after one untimed warm-up iteration."""
    import torch
    sys.path.insert(0, str(ROOT))
    from oracle.reference import sinkhorn_ref
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    x, y = make_inputs()
    o = dict(eps=EPS, normalize=False, fixed_iters=True, block=2048, dtype=torch.float32)
    sinkhorn_ref(x, y, max_iters=1, **o)
    best = min(sinkhorn_ref(x, y, max_iters=iters, **o).seconds for _ in range(reps))
    return dict(value=round(best * 1e3 / iters, 3), unit="ms/iteration", cores=cores, kind="port",
                sample=f"best of {reps} runs of {iters} fixed iterations of the 10k x 10k d64 workload (block 2048), "
                       f"after 1 warm-up iteration; torch {torch.__version__} CPU float32 on {cores} threads of "
                       f"{_cpu_model()}")


# ---------------------------------------------------------------------------------------------------------
# Other workloads of the reference's benchmark set (opt-in with --workload; the headline is the default line).
# Each prints one JSON line: GPU wall time, and beside it the CPU port on a bounded sample, extrapolated.

def single_cell_inputs(n=7355, m=8962, d=30, t0=0, t1=1):
    """Anisotropic Gaussians (per-axis std 1/sqrt(k+1), PCA-like), cloud t offset by 0.3 sigma t, and
    lognormal(0, 0.5) source growth weights normalised to 1."""
    import numpy as np
    sig = 1.0 / np.sqrt(np.arange(d) + 1.0)
    x = np.random.default_rng(t0).standard_normal((n, d)) * sig + 0.3 * sig * t0
    y = np.random.default_rng(t1).standard_normal((m, d)) * sig + 0.3 * sig * t1
    w = np.random.default_rng(2).lognormal(0.0, 0.5, n)
    return x, y, w / w.sum()


def _cpu_per_iteration(x, y, a, b, center, scale, iters=3, **kw):
    """Seconds per iteration of the float32 CPU port (block 2048, all host cores) over `iters` fixed iterations."""
    import torch
    sys.path.insert(0, str(ROOT))
    from oracle.reference import sinkhorn_ref
    torch.set_num_threads(len(os.sched_getaffinity(0)))
    r = sinkhorn_ref(x, y, a, b, normalize=(center, scale), max_iters=iters, fixed_iters=True, dtype=torch.float32,
                     block=2048, **kw)
    return r.seconds / iters


def _host_median_seconds(x, y):
    sys.path.insert(0, str(ROOT))
    from oracle.reference import normalization as ref_normalization
    t = time.perf_counter()
    ref_normalization(x, y, how="median")
    return time.perf_counter() - t


def workload_single_cell(cpu):
    """One unbalanced single-cell-shaped solve to convergence (7,355 x 8,962, d 30, eps 0.05, KL weights 1 and
    50, median-normalised cost, wot formulation: uniform reference, growth-weighted row target), end to end."""
    import numpy as np
    import torch
    from trnopt import Backend, SinkhornOptions, sinkhorn
    from trnopt.sinkhorn import normalization
    x, y, w = single_cell_inputs()
    I, J = len(x), len(y)
    a, b = np.full(I, 1.0 / I), np.full(J, 1.0 / J)
    o = SinkhornOptions(eps=0.05, rho=(1.0, 50.0), normalize="median", tol=1e-6, max_iters=50_000,
                        kernel="hip", backend=Backend.preset("rocm"))
    sinkhorn(x, y, a, b, o, a_target=w, b_target=b)
    torch.cuda.synchronize()
    t = time.perf_counter()
    r = sinkhorn(x, y, a, b, o, a_target=w, b_target=b)
    e2e = time.perf_counter() - t
    t = time.perf_counter()
    center, scale = normalization(x, y, how="median", device="cuda")
    med = time.perf_counter() - t
    line = {"metric": "end-to-end seconds, single-cell-shaped unbalanced solve to tol 1e-6", "value": round(e2e, 4),
            "unit": "s", "higher_is_better": False, "n_gpus": 1, "dtype": "f32", "data": "synthetic",
            "iterations": r.iterations, "converged": r.converged,
            "ms_per_iteration": round(r.seconds * 1e3 / max(r.iterations, 1), 4), "gpu_median_s": round(med, 4),
            "config": {"workload": "unbalanced 7355 x 8962, d 30, eps 0.05, rho (1, 50), median cost, tol 1e-6"}}
    # the exp + MFMA roofline of an iteration (both half-steps): the algorithmic augmented contraction
    # 2 x 2 I J (d + 1) FLOP and 2 I J exponentials, beside the three-product fp16 contraction executed at kp 32
    t_it = r.seconds / max(r.iterations, 1)
    exps_it = 2.0 * I * J
    alg_it = 2 * 2.0 * I * J * (30 + 1)
    flop_it = 2 * PRODUCTS * 2.0 * I * J * 32
    line["roofline"] = {"bound": "mfma", "achieved": round(alg_it / t_it / 1e12, 1), "peak": MFMA_F16_PEAK / 1e12,
                        "unit": "TFLOP/s", "frac": round(alg_it / t_it / MFMA_F16_PEAK, 4),
                        "executed": {"achieved": round(flop_it / t_it / 1e12, 1),
                                     "frac": round(flop_it / t_it / MFMA_F16_PEAK, 4)},
                        "exp": {"achieved": round(exps_it / t_it / 1e12, 3), "peak": EXP_PEAK / 1e12, "unit": "Texp/s",
                                "frac": round(exps_it / t_it / EXP_PEAK, 4)},
                        "basis": "algorithmic augmented-contraction FLOP (executed: the three fp16 products) and "
                                 "exponentials of both half-steps per iteration over the iteration time"}
    if cpu:
        hm = _host_median_seconds(x, y)
        per = _cpu_per_iteration(x, y, a, b, center, scale, eps=0.05, rho=(1.0, 50.0), a_target=w, b_target=b)
        line["cpu_baseline"] = {"value": round(hm + per * r.iterations, 2), "unit": "s",
                                "cores": len(os.sched_getaffinity(0)), "kind": "port",
                                "sample": f"host median {hm:.2f} s + 3 fixed float32 iterations "
                                          f"({per * 1e3:.1f} ms each) x the GPU's {r.iterations} iterations"}
    return line


def pipeline_sizes(n_points=39, total=175_000):
    import numpy as np
    s = np.exp(np.random.default_rng(3).uniform(np.log(1500), np.log(9000), n_points))
    return np.maximum(np.round(s * total / s.sum()).astype(int), 2)


PIPELINE_STREAMS = 4      # pairs in flight at once in the streams form (one HIP stream each); 4 the fastest


def workload_pipeline(cpu):
    """38 consecutive wot transport maps (39 time points, log-uniform sizes in [1,500, 9,000] summing to
    ~175,000, d 30), each with median normalisation, wot's eps stages and 3 growth iterations, end to end:
    batched (wot_transport_maps(batch=True): each growth iteration of all the pairs in one batched loop), the
    value, timed after one untimed run of the same pipeline (the first run of a process also pays the host's
    first touch of its arrays and the allocators' growth: reported as first_run_s); for comparison the pairs
    PIPELINE_STREAMS at a time on their own streams and one pair after the other (these two bit-identical,
    checked here; the batched maps against the one-at-a-time ones to float32 rounding, the largest relative
    difference reported)."""
    import numpy as np
    import torch
    from trnopt import Backend, SinkhornOptions
    from trnopt.singlecell import wot_transport_map, wot_transport_maps
    sizes = pipeline_sizes()
    o = SinkhornOptions(check_every=5, max_iters=50_000, kernel="hip", backend=Backend.preset("rocm"))
    clouds = [single_cell_inputs(n=int(sizes[t]), m=int(sizes[t + 1]), t0=t, t1=t + 1)[:2]
              for t in range(len(sizes) - 1)]
    wot_transport_map(*clouds[0], growth_iters=1, opts=o)          # warm-up of the one-pair path
    kw = dict(growth_iters=3, tol=1e-6, stage_tol=1e-6, opts=o)
    torch.cuda.synchronize()
    t = time.perf_counter()
    wot_transport_maps(clouds, batch=True, **kw)                    # warm-up: the same pipeline, untimed
    first = time.perf_counter() - t
    torch.cuda.synchronize()
    t = time.perf_counter()
    maps = wot_transport_maps(clouds, batch=True, **kw)
    total = time.perf_counter() - t
    work = iters = 0
    for k, ((x0, x1), tm) in enumerate(zip(clouds, maps)):
        iters += tm.iterations
        work += tm.iterations * len(x0) * len(x1)
        print(f"pair {k}: {len(x0)} x {len(x1)}, {tm.iterations} iterations (batched)", file=sys.stderr, flush=True)
    torch.cuda.synchronize()
    t = time.perf_counter()
    flight = wot_transport_maps(clouds, streams=PIPELINE_STREAMS, batch=False, **kw)
    flight_s = time.perf_counter() - t
    torch.cuda.synchronize()
    t = time.perf_counter()
    seq = wot_transport_maps(clouds, streams=1, batch=False, **kw)
    seq_s = time.perf_counter() - t
    same = all(np.array_equal(a.result.f, b.result.f) and np.array_equal(a.result.g, b.result.g) and
               a.iterations == b.iterations for a, b in zip(flight, seq))
    rel = max(max(np.abs(a.result.f - b.result.f).max() / np.abs(b.result.f).max(),
                  np.abs(a.result.g - b.result.g).max() / np.abs(b.result.g).max()) for a, b in zip(maps, seq))
    line = {"metric": "total seconds, 38-pair wot pipeline (3 growth iterations each)", "value": round(total, 3),
            "unit": "s", "higher_is_better": False, "n_gpus": 1, "dtype": "f32", "data": "synthetic",
            "pairs": len(clouds), "iterations": iters, "points": int(sizes.sum()), "first_run_s": round(first, 3),
            "streams_s": round(flight_s, 3), "sequential_s": round(seq_s, 3),
            "streams_bit_identical_to_sequential": same, "batched_max_rel_diff_to_sequential": float(f"{rel:.3g}"),
            "sequential_iterations": sum(tm.iterations for tm in seq),
            "config": {"workload": "39 time points, d 30, eps 0.05, rho (1, 50), wot stages, tol 1e-6, growth 3",
                       "form": "batched (each growth iteration of all the pairs in one loop)",
                       "streams_pairs_in_flight": PIPELINE_STREAMS}}
    # the fp16 pipe over the whole batched run (host steps, medians and read-backs included)
    alg = 2 * 2.0 * work * (30 + 1)
    flop = 2 * PRODUCTS * 2.0 * work * 32
    line["roofline"] = {"bound": "mfma", "achieved": round(alg / total / 1e12, 1), "peak": MFMA_F16_PEAK / 1e12,
                        "unit": "TFLOP/s", "frac": round(alg / total / MFMA_F16_PEAK, 4),
                        "executed": {"achieved": round(flop / total / 1e12, 1),
                                     "frac": round(flop / total / MFMA_F16_PEAK, 4)},
                        "basis": "algorithmic augmented-contraction FLOP of every pair's half-steps (iterations x "
                                 "2 x 2 n0 n1 (d + 1); executed: the three fp16 products at kp 32) over the "
                                 "pipeline's end-to-end time"}
    if cpu:
        x0, x1 = clouds[0]
        I, J = len(x0), len(x1)
        sys.path.insert(0, str(ROOT))
        from oracle.reference import normalization as ref_normalization
        c, sc = ref_normalization(x0, x1, how="median")
        per = _cpu_per_iteration(x0, x1, np.full(I, 1 / I), np.full(J, 1 / J), c, sc, eps=0.05, rho=(1.0, 50.0))
        medians = sum(_host_median_seconds(a_, b_) for a_, b_ in clouds[:3]) / 3 * len(clouds)
        est = medians + per / (I * J) * work
        line["cpu_baseline"] = {"value": round(est, 1), "unit": "s", "cores": len(os.sched_getaffinity(0)),
                                "kind": "port",
                                "sample": f"3 fixed float32 iterations of the first pair ({I} x {J}) scaled by the "
                                          f"GPU run's sum of iterations x n0 n1, plus host medians of 3 pairs "
                                          f"scaled to {len(clouds)}"}
    return line


def stress_inputs(n=65_536, d=128):
    import numpy as np
    r = np.random.default_rng(0)
    mu = 2.0 * r.standard_normal((8, d))
    x = mu[r.integers(8, size=n)] + 0.5 * r.standard_normal((n, d))
    r1 = np.random.default_rng(1)
    y = mu[r1.integers(8, size=n)] + 0.5 * r1.standard_normal((n, d))
    return x, y


def workload_stress(cpu):
    """65,536 x 65,536, d 128, 8-component Gaussian mixtures, median-normalised cost (sampled pairs), eps
    annealed 1.0 -> 0.01 by 0.7 per stage, 20 iterations per stage, 280 iterations in all."""
    import numpy as np
    import torch
    from trnopt import Backend, SinkhornOptions, sinkhorn
    x, y = stress_inputs()
    o = SinkhornOptions(eps=0.01, eps_stages=tuple(0.7 ** k for k in range(13)), stage_max_iters=20,
                        check_every=20, fixed_iters=True, max_iters=280, normalize="median", kernel="hip",
                        backend=Backend.preset("rocm"))
    sinkhorn(x[:4096], y[:4096], opts=o)
    torch.cuda.synchronize()
    t = time.perf_counter()
    r = sinkhorn(x, y, opts=o)
    e2e = time.perf_counter() - t
    line = {"metric": "end-to-end seconds, 65k x 65k d 128 eps-scaling stress solve (280 iterations)",
            "value": round(e2e, 3), "unit": "s", "higher_is_better": False, "n_gpus": 1, "dtype": "f32",
            "data": "synthetic", "iterations": r.iterations,
            "ms_per_iteration": round(r.seconds * 1e3 / max(r.iterations, 1), 3),
            "config": {"workload": "balanced 65536 x 65536, d 128, eps 1.0 -> 0.01 (0.7 per stage), 280 its"}}
    # the fp16 pipe the kernel runs on, over whole iterations (both half-steps, merges and control included)
    t_it = r.seconds / max(r.iterations, 1)
    alg_it = 2 * 2.0 * len(x) * len(y) * (128 + 1)
    flop_it = 2 * PRODUCTS * 2.0 * len(x) * len(y) * 128
    line["roofline"] = {"bound": "mfma", "achieved": round(alg_it / t_it / 1e12, 1), "peak": MFMA_F16_PEAK / 1e12,
                        "unit": "TFLOP/s", "frac": round(alg_it / t_it / MFMA_F16_PEAK, 4),
                        "executed": {"achieved": round(flop_it / t_it / 1e12, 1),
                                     "frac": round(flop_it / t_it / MFMA_F16_PEAK, 4)},
                        "basis": "algorithmic augmented-contraction FLOP of both half-steps per iteration (executed: "
                                 "the three fp16 products) over the iteration time"}
    if cpu:
        per = _cpu_per_iteration(x, y, None, None, r.center, r.cost_scale, iters=2, eps=0.01)
        line["cpu_baseline"] = {"value": round(per * 280, 1), "unit": "s", "cores": len(os.sched_getaffinity(0)),
                                "kind": "port",
                                "sample": f"2 fixed float32 iterations at eps 0.01 ({per:.2f} s each) x 280"}
    return line


WORKLOADS = {"single-cell": workload_single_cell, "single-cell-pipeline": workload_pipeline,
             "stress-65k": workload_stress}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-iters", type=int, default=10)
    ap.add_argument("--cpu-reps", type=int, default=3)
    ap.add_argument("--profile", action="store_true", help="only the launches the rocprofv3 summaries use")
    ap.add_argument("--reps", type=int, default=20)
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default=None,
                    help="one of the other benchmark workloads instead of the headline line")
    a = ap.parse_args()
    if a.gpus != 1:
        print("bench.py measures one GPU: this build's path is single-GPU (the multi-GPU row split is a design "
              "only); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if a.profile:
        if a.workload == "stress-65k":
            profile_stress(a.reps)
        elif a.workload == "single-cell":
            profile_single_cell(a.reps)
        elif a.workload == "single-cell-pipeline":
            profile_pipeline(a.reps)
        elif a.workload is None:
            profile_run(a.reps)
        else:
            sys.exit("--profile takes the headline, --workload single-cell, single-cell-pipeline or stress-65k")
        return
    if a.workload is not None:
        print(json.dumps(WORKLOADS[a.workload](not a.no_cpu)), flush=True)
        return
    g = gpu_run(a.steps, a.warmup)
    cpu = None if a.no_cpu else cpu_baseline(a.cpu_iters, a.cpu_reps)
    kp = g["kp"]
    t_launch = g["kernel_ms"] * 1e-3
    executed = PRODUCTS * 2.0 * N * M * kp            # fp16 MFMA FLOP of one launch's contraction (no padding)
    alg = 2.0 * N * M * (D + 1)                       # the augmented fp32 contraction of one half-step
    exps = float(N * M)
    t_it = g["ms_per_it"] * 1e-3
    t_roof = max(2 * executed / MFMA_F16_PEAK, 2 * exps / EXP_PEAK)
    t_roof32 = max(2 * alg / MFMA_F32_PEAK, 2 * exps / EXP_PEAK)
    line = {
        "metric": "ms/iteration, 10k x 10k d=64 fp32 Sinkhorn; fraction of exp+MFMA roofline",
        "value": round(g["ms_per_it"], 5),
        "unit": "ms/iteration",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(g["ms_per_it"], 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded N(0,1) clouds, y shifted by 0.5)",
        "config": {"workload": "balanced Sinkhorn 10000 x 10000, d 64, eps 0.1, fixed iterations", "n": N, "m": M,
                   "d": D, "eps": EPS},
        "roofline": {"bound": "mfma", "achieved": round(alg / t_launch / 1e12, 1), "peak": MFMA_F16_PEAK / 1e12,
                     "unit": "TFLOP/s", "frac": round(alg / t_launch / MFMA_F16_PEAK, 4),
                     "traffic": profiled_traffic(),
                     "kernel": "lse_partial_kernel (fp16 MFMA three-product contraction, row groups merged in-kernel)",
                     "kernel_ms": round(g["kernel_ms"], 5), "flop_per_launch": alg,
                     "executed": {"flop_per_launch": executed, "achieved": round(executed / t_launch / 1e12, 1),
                                  "frac": round(executed / t_launch / MFMA_F16_PEAK, 4),
                                  "note": "the three fp16 products of the fp32-accurate two-piece contraction"},
                     "exp": {"per_launch": exps, "achieved": round(exps / t_launch / 1e12, 3), "peak": EXP_PEAK / 1e12,
                             "unit": "Texp/s", "frac": round(exps / t_launch / EXP_PEAK, 4)},
                     "fp32_equivalent": {"flop_per_launch": alg, "achieved": round(alg / t_launch / 1e12, 1),
                                         "peak": MFMA_F32_PEAK / 1e12, "ratio": round(alg / t_launch / MFMA_F32_PEAK, 4)}},
        "iteration_roofline": {"t_roof_ms": round(t_roof * 1e3, 5), "frac": round(t_roof / t_it, 4),
                               "fp32_mfma_t_roof_ms": round(t_roof32 * 1e3, 5),
                               "fp32_mfma_ratio": round(t_roof32 / t_it, 4)},
        "end_to_end_s": round(g["e2e"], 4),
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
