"""Benchmark: ms per Sinkhorn iteration (f half-step + g half-step) on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
    python bench.py --profile [--reps R]     # for rocprofv3: R half-steps, then a 256 MiB copy

Workload: synthetic balanced 10,000 x 10,000, d = 64, fp32, x ~ N(0, 1) (seed 0), y ~ N(0, 1) + 0.5
(seed 1), uniform weights, squared-Euclidean cost, no normalisation, eps = 0.1 (the reference's
examples/sinkhorn_benchmark.py --flashsinkhorn setup). A "step" is one iteration of the on-device loop
(f half-step, g half-step, loop control: four kernel launches), inputs resident in HBM. W untimed iterations, then
exactly K timed iterations between two device synchronisations.

Also reported on the same JSON line:
* roofline -- the dominant kernel pair, sk_half_step_f32 (lse_partial_kernel, then merge_kernel), timed with
  HIP events on the stream it runs on. `achieved` is the algorithmic count 2 n m (d + 1) of one half-step
  (the augmented fp32 contraction) per second, against the 157.3 TFLOP/s fp32 MFMA peak; `frac` exceeds 1
  because the fp32-accurate contraction runs on the fp16 matrix pipe (three products of a two-piece split of
  the coordinates). `mfma_f16` gives the executed fp16 MFMA work (3 x 2 x n_pad m_pad kp per half-step)
  against the 2.5 PFLOP/s fp16 dense peak, `exp` the exponentials (n m per half-step) against the
  9.83e12/s transcendental peak (quarter rate on 256 CUs x 4 SIMDs x 16 lanes at 2.4 GHz); `traffic` is the
  fabric bytes per half-step from the committed counter summary;
* iteration_roofline_frac -- max(4 n m (d + 1) / 157.3e12, 2 n m / 9.83e12) seconds over the measured
  ms/iteration: the exp + fp32-MFMA roofline fraction the metric names;
* cpu_baseline -- the reference's plain-PyTorch CPU path (the oracle's restatement, float32, block 2048,
  all host cores) on a bounded sample of the same workload;
* end_to_end_s -- sinkhorn() wall time for 10 fixed iterations, host arrays in, float64 potentials out
  (setup, H2D, packing, loop, read-back).
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
EXP_PEAK = 9.83e12
PRODUCTS = 3          # fp16 piece products per K chunk of the half-step contraction


def profiled_traffic():
    """Fabric bytes per half-step from the committed counter summary (FETCH_SIZE and WRITE_SIZE passes,
    scaled by the copy calibration), or None if the summary is absent."""
    import re
    p = ROOT / "profiles" / "half_step_10k_d64_counters.md"
    m = re.search(r"traffic_bytes_per_launch:\s*(\d+)", p.read_text()) if p.exists() else None
    return int(m.group(1)) if m else None


def make_inputs():
    import numpy as np
    x = np.random.default_rng(0).standard_normal((N, D))
    y = np.random.default_rng(1).standard_normal((M, D)) + 0.5
    return x, y


def gpu_run(steps, warmup, kernel_reps=50):
    import numpy as np
    import torch
    from trnopt import hip_sinkhorn as hk

    hk.lib()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    x, y = make_inputs()
    la, lb = np.full(N, -np.log(N)), np.full(M, -np.log(M))
    X = hk.HipCloud(x, la, dev, role=0)
    Y = hk.HipCloud(y, lb, dev, role=1)
    loop = hk.DeviceLoop(X, Y, eps=EPS, rho_x=None, rho_y=None, sched=[], stages=[], tol=1e-4, stage_tol=1e-5,
                         max_iters=warmup + steps + 1, check_every=10, stage_max_iters=1000, fixed_iters=True,
                         balanced=True)
    loop.init()
    loop.enqueue(warmup)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    loop.enqueue(steps)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_per_it = (t1 - t0) * 1e3 / steps
    st = loop.read_state()
    assert st.it == warmup + steps and not st.done, (st.it, st.done)

    # dominant kernel pair: one half-step (f update), HIP events on the current stream
    sc = hk.scalars(EPS, 1.0, dev)
    out = torch.empty(X.npad, dtype=torch.float32, device=dev)
    for _ in range(3):
        hk.half_step(X, Y, loop.gh, sc, out=out)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    ev0.record()
    for _ in range(kernel_reps):
        hk.half_step(X, Y, loop.gh, sc, out=out)
    ev1.record()
    torch.cuda.synchronize()
    half_ms = ev0.elapsed_time(ev1) / kernel_reps
    flop = 2.0 * N * M * (D + 1)
    achieved = flop / (half_ms * 1e-3)
    executed = PRODUCTS * 2.0 * X.npad * Y.npad * hk.pad_dim(D)

    # end to end: sinkhorn() with host arrays, 10 fixed iterations
    from trnopt import Backend, SinkhornOptions, sinkhorn
    o = SinkhornOptions(eps=EPS, normalize=False, max_iters=10, fixed_iters=True, kernel="hip",
                        backend=Backend.preset("rocm"))
    sinkhorn(x, y, opts=o)
    torch.cuda.synchronize()
    te = time.perf_counter()
    r = sinkhorn(x, y, opts=o)
    e2e = time.perf_counter() - te
    return dict(ms_per_it=ms_per_it, half_ms=half_ms, achieved=achieved, flop=flop, executed=executed, e2e=e2e,
                loop_s=r.seconds)


def profile_run(reps):
    """What the rocprofv3 summaries are taken from: `reps` half-steps (f update) of the workload, then one
    plain device copy of 256 MiB (two copy dispatches of 128 MiB), whose FETCH_SIZE / WRITE_SIZE calibrate the
    counters (each dispatch reads and writes exactly 131072 KiB)."""
    import numpy as np
    import torch
    from trnopt import hip_sinkhorn as hk

    hk.lib()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    x, y = make_inputs()
    X = hk.HipCloud(x, np.full(N, -np.log(N)), dev, role=0)
    Y = hk.HipCloud(y, np.full(M, -np.log(M)), dev, role=1)
    gh = torch.zeros(Y.npad, dtype=torch.float32, device=dev)
    sc = hk.scalars(EPS, 1.0, dev)
    out = torch.empty(X.npad, dtype=torch.float32, device=dev)
    for _ in range(reps):
        hk.half_step(X, Y, gh, sc, out=out)
    src = torch.ones(64 << 20, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    print(f"profile: {reps} half-steps of {N} x {M} d {D}, then a 256 MiB copy", flush=True)


def cpu_baseline(iters=2):
    """The reference's plain-PyTorch CPU path (oracle restatement), float32, block 2048, all host cores:
    `iters` fixed iterations after one untimed warm-up iteration, best of 2."""
    import torch
    sys.path.insert(0, str(ROOT))
    from oracle.reference import sinkhorn_ref
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    x, y = make_inputs()
    o = dict(eps=EPS, normalize=False, fixed_iters=True, block=2048, dtype=torch.float32)
    sinkhorn_ref(x, y, max_iters=1, **o)
    best = min(sinkhorn_ref(x, y, max_iters=iters, **o).seconds for _ in range(2))
    return dict(value=best * 1e3 / iters, unit="ms/iteration", cores=cores, kind="port",
                sample=f"{iters} fixed iterations of the 10k x 10k d64 workload (block 2048), best of 2, "
                       f"after 1 warm-up iteration; torch {torch.__version__} CPU float32")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-iters", type=int, default=2)
    ap.add_argument("--profile", action="store_true", help="only the launches the rocprofv3 summaries use")
    ap.add_argument("--reps", type=int, default=20)
    a = ap.parse_args()
    if a.gpus != 1:
        print("bench.py measures one GPU: this build's path is single-GPU (the multi-GPU row split is a design "
              "only); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if a.profile:
        profile_run(a.reps)
        return
    g = gpu_run(a.steps, a.warmup)
    cpu = None if a.no_cpu else cpu_baseline(a.cpu_iters)
    t_roof = max(4.0 * N * M * (D + 1) / MFMA_F32_PEAK, 2.0 * N * M / EXP_PEAK)
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
        "roofline": {"bound": "mfma", "achieved": round(g["achieved"] / 1e12, 3), "peak": MFMA_F32_PEAK / 1e12,
                     "unit": "TFLOP/s", "frac": round(g["achieved"] / MFMA_F32_PEAK, 4), "traffic": profiled_traffic(),
                     "kernel": "sk_half_step_f32 (lse_partial_kernel + merge_kernel)",
                     "kernel_ms": round(g["half_ms"], 5), "flop_per_launch": g["flop"],
                     "mfma_f16": {"executed_flop_per_launch": g["executed"],
                                  "achieved": round(g["executed"] / (g["half_ms"] * 1e-3) / 1e12, 1),
                                  "peak": MFMA_F16_PEAK / 1e12,
                                  "frac": round(g["executed"] / (g["half_ms"] * 1e-3) / MFMA_F16_PEAK, 4)},
                     "exp": {"per_launch": N * M, "frac": round(N * M / (g["half_ms"] * 1e-3) / EXP_PEAK, 4)}},
        "iteration_roofline_frac": round(t_roof * 1e3 / g["ms_per_it"], 4),
        "end_to_end_s": round(g["e2e"], 4),
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
