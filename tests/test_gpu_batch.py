"""The batched on-device loop (sk_loop_run_batch_f32 through DeviceLoopBatch, sinkhorn_batch and
wot_transport_maps(batch=True)): each launch runs one half-step of every problem, each on its own share of the
GPU's workgroups, merged inside the launch.

* One problem: the batch gives it the split of its own launches, so sinkhorn_batch returns sinkhorn()'s
  potentials, masses and iteration counts bit for bit (fixed iterations, an eps schedule, an unbalanced solve
  stopped by its checks).
* Several problems of different sizes and formulations in one batch (balanced and unbalanced, schedules, stages,
  one stopped early by its max_iters while the others go on): each agrees with its own sinkhorn() to float32
  rounding, and with the oracle's float64 run within the solver sweep's bar.
* The wot pipeline batched against the same pairs one at a time: the same maps to float32 rounding.
* More loops than CUs (300 small problems): one workgroup per pass, every loop as its own to float32 rounding.
"""

import numpy as np
import pytest
import torch

from oracle import reference as ref
from conftest import inf_rel

from trnopt import Backend
from trnopt.sinkhorn import SinkhornOptions, sinkhorn, sinkhorn_batch

pytestmark = pytest.mark.gpu
ROCM = Backend.preset("rocm")


def _clouds(n, m, d, seed):
    rng = np.random.default_rng(seed)
    x = rng.normal(size=(n, d))
    y = rng.normal(size=(m, d)) * 0.9 + 0.4
    return x, y, rng


@pytest.mark.parametrize("case", ["fixed", "schedule", "unbalanced"])
def test_batch_of_one_problem_is_sinkhorn_bit_for_bit(case):
    """2,048 x 1,900, d 64 (8 row groups: the loop alone merges with the merge kernel, the batch inside its launch;
    the two forms are bit-identical), so that only the batch machinery differs."""
    x, y, rng = _clouds(2048, 1900, 64, 71)
    kw = {}
    if case == "fixed":
        o = dict(eps=0.1, max_iters=40, fixed_iters=True)
    elif case == "schedule":
        o = dict(eps=0.05, eps_start=1.0, eps_decay=0.8, max_iters=60, fixed_iters=True)
    else:
        o = dict(eps=0.05, rho=(1.0, 50.0), tol=1e-6, normalize="median", check_every=5, max_iters=3000,
                 eps_stages=(1.0, 0.4, 0.15))
        kw = dict(a_target=rng.uniform(0.5, 1.5, 2048) / 2048, b_target=np.full(1900, 1.0 / 1900))
    opts = SinkhornOptions(kernel="hip", backend=ROCM, **o)
    print(f"batch of one, {case}", flush=True)
    alone = sinkhorn(x, y, opts=opts, **kw)
    (got,) = sinkhorn_batch([dict(x=x, y=y, opts=opts, **kw)])
    assert got.iterations == alone.iterations and got.converged == alone.converged
    np.testing.assert_array_equal(got.f, alone.f)
    np.testing.assert_array_equal(got.g, alone.g)
    if alone.row_mass is not None:
        np.testing.assert_array_equal(got.row_mass, alone.row_mass)
        np.testing.assert_array_equal(got.col_mass, alone.col_mass)


# Problems of one batch (d 20): sizes, the options for sinkhorn(), whether marginal targets are drawn.
PROBLEMS = [
    (1500, 1200, dict(eps=0.1, max_iters=30, fixed_iters=True), False),
    (300, 900, dict(eps=0.05, rho=1.0, max_iters=25, fixed_iters=True, normalize="median"), True),
    (1100, 70, dict(eps=0.2, eps_start=2.0, eps_decay=0.7, max_iters=35, fixed_iters=True), False),
    (650, 650, dict(eps=0.05, rho=(1.0, 50.0), eps_stages=(1.0, 0.3, 0.1), stage_max_iters=5, check_every=5,
                    max_iters=40, fixed_iters=True), True),
    (40, 1300, dict(eps=0.1, max_iters=15, fixed_iters=True), False),        # done long before the others
    (900, 1000, dict(eps=0.1, rho=2.0, max_iters=30, fixed_iters=True, normalize=False), False),
]


def test_batch_of_problems_matches_each_alone_and_float64():
    qs = []
    for k, (n, m, o, targets) in enumerate(PROBLEMS):
        x, y, rng = _clouds(n, m, 20, 300 + k)
        a = rng.uniform(0.5, 1.5, n)
        b = rng.uniform(0.5, 1.5, m)
        a, b = a / a.sum(), b / b.sum()
        q = dict(x=x, y=y, a=a, b=b, opts=SinkhornOptions(kernel="hip", backend=ROCM, **o))
        if targets:
            q.update(a_target=a * rng.uniform(0.5, 1.5, n), b_target=b * rng.uniform(0.5, 1.5, m))
        qs.append((q, o))
    print(f"batch of {len(qs)} problems", flush=True)
    batch = sinkhorn_batch([q for q, _ in qs])
    for k, ((q, o), got) in enumerate(zip(qs, batch)):
        alone = sinkhorn(**q)
        ex = {key: q[key] for key in ("a_target", "b_target") if key in q}
        want = ref.sinkhorn_ref(q["x"], q["y"], q["a"], q["b"], **o, **ex)
        ef, eg = inf_rel(got.f, want.f), inf_rel(got.g, want.g)
        af, ag = inf_rel(got.f, alone.f), inf_rel(got.g, alone.g)
        print(f"  problem {k}: {len(q['x'])} x {len(q['y'])}, {got.iterations} iterations; against float64 "
              f"{ef:.2e} / {eg:.2e}, against sinkhorn() {af:.2e} / {ag:.2e}", flush=True)
        assert got.iterations == alone.iterations == want.iterations == o["max_iters"]
        assert af < 2e-6 and ag < 2e-6
        if ef >= 1e-5 or eg >= 1e-5:
            w32 = ref.sinkhorn_ref(q["x"], q["y"], q["a"], q["b"], **o, **ex, dtype=torch.float32)
            rf, rg = inf_rel(w32.f, want.f), inf_rel(w32.g, want.g)
            assert ef <= max(1e-5, 1.5 * rf) and eg <= max(1e-5, 1.5 * rg), (ef, eg, rf, rg)


def test_wot_transport_maps_batched_match_one_at_a_time():
    """The pairs of a small pipeline (7 time points, d 30, wot stages, tol 1e-6, 2 growth iterations): each
    growth iteration of all the pairs as one batch against each pair solved alone. Every pair converges; the
    potentials agree to float32 rounding at the convergence floor (the two forms may stop a check apart), the
    learned growth within 1e-3."""
    from trnopt.singlecell import wot_transport_maps
    sizes = [1500, 2400, 900, 3100, 2000, 700, 2600]
    sig = 1.0 / np.sqrt(np.arange(30) + 1.0)
    pts = [np.random.default_rng(40 + t).standard_normal((s, 30)) * sig + 0.3 * sig * t for t, s in enumerate(sizes)]
    pairs = list(zip(pts[:-1], pts[1:]))
    gpu = SinkhornOptions(kernel="hip", backend=ROCM, check_every=5, max_iters=50_000)
    kw = dict(growth_iters=2, tol=1e-6, stage_tol=1e-6, opts=gpu)
    print("pairs batched", flush=True)
    batched = wot_transport_maps(pairs, batch=True, **kw)
    print("pairs one at a time", flush=True)
    one = wot_transport_maps(pairs, streams=1, batch=False, **kw)
    for k, (a, b) in enumerate(zip(batched, one)):
        ef, eg = inf_rel(a.result.f, b.result.f), inf_rel(a.result.g, b.result.g)
        print(f"  pair {k}: {a.iterations} / {b.iterations} iterations, f {ef:.2e}, g {eg:.2e}", flush=True)
        assert a.result.converged and b.result.converged, k
        assert abs(a.iterations - b.iterations) <= 2 * 5 * 2, k
        assert ef < 2e-5 and eg < 2e-5, (k, ef, eg)
        for Ga, Gb in zip(a.learned_growth, b.learned_growth):
            np.testing.assert_allclose(Ga, Gb, rtol=1e-3)


def test_batch_of_more_loops_than_cus():
    """300 small problems (24-120 points a side, d 8, balanced and unbalanced): more loops than the GPU has CUs, so
    every pass gets one workgroup (its own single-workgroup split) and a launch runs 300 of them; each loop agrees
    with its own sinkhorn() to float32 rounding."""
    rng = np.random.default_rng(505)
    qs = []
    for k in range(300):
        n, m = int(rng.integers(24, 121)), int(rng.integers(24, 121))
        x = rng.normal(size=(n, 8))
        y = rng.normal(size=(m, 8)) + 0.2
        o = dict(eps=0.1, max_iters=int(rng.integers(8, 25)), fixed_iters=True)
        if k % 3 == 1:
            o["rho"] = 1.0
        qs.append(dict(x=x, y=y, opts=SinkhornOptions(kernel="hip", backend=ROCM, **o)))
    print("batch of 300 small problems", flush=True)
    batch = sinkhorn_batch(qs)
    worst = 0.0
    for q, got in zip(qs, batch):
        alone = sinkhorn(**q)
        assert got.iterations == alone.iterations == q["opts"].max_iters
        worst = max(worst, inf_rel(got.f, alone.f), inf_rel(got.g, alone.g))
    print(f"  largest difference from the loops alone {worst:.2e}", flush=True)
    assert worst < 2e-6


def test_batch_refusals_leave_every_problem_as_it_was():
    """sinkhorn_batch refuses problems of different d and options the fused path does not take; a batch's
    solve(targets) refuses the wrong number of targets, targets for a problem made without them and a bad target
    of a later problem, each before any problem's offsets change: the next plain solve repeats the first bit for
    bit."""
    from trnopt.sinkhorn import _HipBatch
    x, y, _ = _clouds(300, 280, 8, 5)
    x2, y2, _ = _clouds(200, 220, 9, 6)
    ok = SinkhornOptions(kernel="hip", backend=ROCM, eps=0.1, rho=1.0, max_iters=30, fixed_iters=True)
    with pytest.raises(ValueError, match="one d"):
        sinkhorn_batch([dict(x=x, y=y, opts=ok), dict(x=x2, y=y2, opts=ok)])
    with pytest.raises(ValueError, match="fused kernels"):
        sinkhorn_batch([dict(x=x, y=y, opts=SinkhornOptions(kernel="torch", backend=ROCM))])
    at, bt = np.full(300, 1 / 300), np.full(280, 1 / 280)
    at2, bt2 = np.full(100, 1.2 / 100), np.full(90, 1 / 90)
    for second in (dict(), dict(a_target=at2, b_target=bt2)):
        batch = _HipBatch([dict(x=x, y=y, opts=ok, a_target=at, b_target=bt),
                           dict(x=x[:100], y=y[:90], opts=ok, **second)])
        first = batch.solve()
        with pytest.raises(ValueError, match="1 targets for 2"):
            batch.solve([(at * 1.1, bt)])
        with pytest.raises(ValueError, match="without marginal targets" if not second else "positive"):
            batch.solve([(at * 1.1, bt), (-at2, bt2)])
        again = batch.solve()
        for r0, r1 in zip(first, again):
            np.testing.assert_array_equal(r0.f, r1.f)
            np.testing.assert_array_equal(r0.g, r1.g)
            assert r0.iterations == r1.iterations == 30
