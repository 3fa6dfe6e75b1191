"""Plans from potentials (trnopt.plan): row / column sums and the pull-back P v, against the dense float64 plan
(transport_plan, src/trnopt/sinkhorn.py:397-403) and the oracle's chunked marginals
(examples/sinkhorn_libs_compare.py:43-56). CPU tests use kernel="torch"; the `gpu` ones run the fused kernel."""

import numpy as np
import pytest
import torch

from oracle import brute, data

from trnopt import Backend
from trnopt.plan import plan_marginals, pull_back
from trnopt.sinkhorn import SinkhornOptions, sinkhorn, transport_plan

CPU = SinkhornOptions(kernel="torch", backend=Backend.preset("cpu"))
F32 = SinkhornOptions(kernel="torch", backend=Backend.preset("cpu-float32"))
ROCM = SinkhornOptions(kernel="hip", backend=Backend.preset("rocm"))


def _rel(a, b):
    return float(np.max(np.abs(a - b) / np.abs(b)))


def _solved(n=140, m=97, d=6, unbalanced=False, weights=False, seed=3):
    x, y = data.clouds(n=n, m=m, d=d, seed=seed)
    rng = np.random.default_rng(seed)
    a = b = None
    if weights:
        a = rng.uniform(0.5, 1.5, n)
        a /= a.sum()
        b = rng.uniform(0.5, 1.5, m)
        b /= b.sum()
    kw = dict(eps=0.1, max_iters=3000, tol=1e-9, backend=Backend.preset("cpu"))
    if unbalanced:
        kw["rho"] = (1.0, 5.0)
    res = sinkhorn(x, y, a, b, opts=SinkhornOptions(kernel="torch", **kw))
    return x, y, a, b, res


@pytest.mark.parametrize("unbalanced", [False, True])
@pytest.mark.parametrize("weights", [False, True])
def test_marginals_equal_the_dense_plan(unbalanced, weights):
    x, y, a, b, res = _solved(unbalanced=unbalanced, weights=weights)
    P = transport_plan(x, y, res, a, b)
    rows, cols = plan_marginals(x, y, res, a, b, opts=CPU)
    assert _rel(rows, P.sum(axis=1)) < 1e-10
    assert _rel(cols, P.sum(axis=0)) < 1e-10
    if unbalanced:
        # the solver's own masses are the same quantity (src/trnopt/sinkhorn.py:381-389)
        assert _rel(rows, res.row_mass) < 1e-10 and _rel(cols, res.col_mass) < 1e-10


def test_marginals_equal_the_oracle_chunked_routine():
    x, y, a, b, res = _solved(n=300, m=211, d=9, unbalanced=True, weights=True, seed=5)
    root = np.sqrt(res.cost_scale)
    xs, ys = (x - res.center) / root, (y - res.center) / root
    r0, c0 = brute.plan_marginals(xs, ys, a, b, res.f, res.g, res.eps, chunk=64)
    rows, cols = plan_marginals(x, y, res, a, b, opts=CPU)
    assert _rel(rows, r0) < 1e-10 and _rel(cols, c0) < 1e-10


def test_balanced_marginals_are_the_weights():
    x, y, a, b, res = _solved(weights=True)
    rows, cols = plan_marginals(x, y, res, a, b, opts=CPU)
    assert np.abs(cols - b).max() < 1e-9          # the last update is g's: columns exact
    assert np.abs(rows - a).max() < 1e-6


def test_pull_back_equals_dense_plan_times_v():
    x, y, a, b, res = _solved(unbalanced=True, weights=True)
    v = np.zeros(len(y))
    v[::3] = np.random.default_rng(0).uniform(0.1, 1.0, len(v[::3]))     # a set of cells, the others zero
    P = transport_plan(x, y, res, a, b)
    want = P @ v
    want = np.log(want / want.sum())
    got = pull_back(x, y, res, v, a, b, opts=CPU)
    assert np.abs(got - want).max() < 1e-10


def test_pull_back_rejects_bad_vectors():
    x, y, a, b, res = _solved()
    with pytest.raises(ValueError, match="non-negative"):
        pull_back(x, y, res, np.zeros(len(y)), opts=CPU)
    with pytest.raises(ValueError, match="non-negative"):
        pull_back(x, y, res, -np.ones(len(y)), opts=CPU)
    with pytest.raises(ValueError, match="potentials"):
        plan_marginals(x[:-1], y, res, opts=CPU)


# --------------------------------------------------------------------------------------------------------
# the fused kernel

@pytest.mark.gpu
@pytest.mark.parametrize("unbalanced", [False, True])
def test_gpu_marginals_match_float64(hip, unbalanced):
    """Two sk_half_step_f32 launches (scores in log2 units: x's copy made for the result's eps) against the float64
    torch path on the same potentials, within 1.5 times the error of the same computation in float32 (the
    reference's float32 op sequence: measured 3.1e-6 / 1.8e-6 relative, the kernel 3.1e-6 / 2.1e-6), and 1e-6
    absolute."""
    x, y = data.balanced_gaussian(n=2048, m=1500, d=32)
    opts = dict(eps=0.05, normalize="median", max_iters=400, tol=1e-6)
    if unbalanced:
        opts["rho"] = (1.0, 50.0)
    res = sinkhorn(x, y, opts=SinkhornOptions(kernel="hip", backend=Backend.preset("rocm"), **opts))
    r64, c64 = plan_marginals(x, y, res, opts=CPU)
    r32, c32 = plan_marginals(x, y, res, opts=F32)
    print("marginals on the fused kernel, unbalanced", unbalanced, flush=True)
    rows, cols = plan_marginals(x, y, res, opts=ROCM)
    print(f"  relative {_rel(rows, r64):.2e} {_rel(cols, c64):.2e} (float32 sequence {_rel(r32, r64):.2e} "
          f"{_rel(c32, c64):.2e}); absolute {np.abs(rows - r64).max():.2e} {np.abs(cols - c64).max():.2e}", flush=True)
    assert _rel(rows, r64) <= 1.5 * _rel(r32, r64) and _rel(cols, c64) <= 1.5 * _rel(c32, c64), \
        (_rel(rows, r64), _rel(cols, c64), _rel(r32, r64), _rel(c32, c64))
    assert np.abs(rows - r64).max() <= 1e-6 and np.abs(cols - c64).max() <= 1e-6
    if unbalanced:
        assert _rel(rows, res.row_mass) < 2e-5


@pytest.mark.gpu
def test_gpu_pull_back_matches_float64(hip):
    """wot's ancestor pull-back on the fused kernel against float64, within 1.5 times the float32 sequence's
    error (measured 3.0e-6 of the largest probability; the kernel 2.4e-6)."""
    x, y = data.balanced_gaussian(n=1000, m=1200, d=16)
    res = sinkhorn(x, y, opts=SinkhornOptions(kernel="hip", backend=Backend.preset("rocm"), eps=0.05,
                                             normalize="median", max_iters=300, tol=1e-6))
    v = np.zeros(len(y))
    v[:300] = 1.0
    want = pull_back(x, y, res, v, opts=CPU)
    g32 = pull_back(x, y, res, v, opts=F32)
    print("pull-back on the fused kernel", flush=True)
    got = pull_back(x, y, res, v, opts=ROCM)

    def err(p):
        return np.abs(np.exp(p) - np.exp(want)).max() / np.exp(want).max()

    print(f"  pull-back max error {err(got):.2e} of max p (float32 sequence {err(g32):.2e})", flush=True)
    assert err(got) <= 1.5 * err(g32), (err(got), err(g32))


# --------------------------------------------------------------------------------------------------------
# the per-pair result file (examples/singlecell_wot.py:112-117) and the pull-back from it

def test_pair_file_round_trip_without_pickle(tmp_path):
    from trnopt.singlecell import PAIR_KEYS, load_pair, pair_result, save_pair, wot_transport_map
    x0, x1, w = data.single_cell_like(n=180, m=150, d=5)
    tm = wot_transport_map(x0, x1, growth=w * len(x0), growth_iters=2, tol=1e-8,
                           opts=SinkhornOptions(kernel="torch", backend=Backend.preset("cpu"), max_iters=20000))
    cells0 = np.array([f"D0_{i}" for i in range(len(x0))], dtype=object)       # names as the reference keeps them
    p = tmp_path / "pair_0_1.npz"
    save_pair(p, tm, x0, x1, cells0=cells0)
    with np.load(p, allow_pickle=False) as z:                                  # no pickled objects inside
        assert sorted(z.files) == sorted(PAIR_KEYS)
        assert z["learned_growth"].shape == (2, len(x0))
        assert z["cells0"][7] == "D0_7" and z["cells1"][3] == "3"
    zz = load_pair(p)
    r = pair_result(zz)
    np.testing.assert_array_equal(r.f, tm.result.f)
    np.testing.assert_array_equal(r.row_mass, tm.result.row_mass)
    assert r.eps == tm.result.eps and r.cost_scale == tm.result.cost_scale
    # the reference's pull-back from the saved potentials (examples/singlecell_figures.py:35-47), restated in
    # float64 on the dense cost: uniform weights, so it equals pull_back on the loaded result
    from scipy.special import logsumexp
    s = np.sqrt(zz["cost_scale"])
    a0, a1 = (zz["x0"] - zz["center"]) / s, (zz["x1"] - zz["center"]) / s
    C = (a0 * a0).sum(1)[:, None] + (a1 * a1).sum(1)[None, :] - 2.0 * a0 @ a1.T
    v = np.zeros(len(x1))
    v[:40] = 1.0 / 40
    with np.errstate(divide="ignore"):
        lv = np.log(v)
    want = logsumexp((zz["g"][None, :] - C) / zz["eps"] + lv[None, :], axis=1) + zz["f"] / zz["eps"]
    want -= logsumexp(want)
    got = pull_back(zz["x0"], zz["x1"], r, v, opts=CPU)
    assert np.abs(got - want).max() < 1e-9


def test_load_pair_refuses_other_files(tmp_path):
    from trnopt.singlecell import load_pair
    p = tmp_path / "x.npz"
    np.savez(p, f=np.zeros(3))
    with pytest.raises(ValueError, match="not a pair file"):
        load_pair(p)


def test_wot_eps_stages_closed_form():
    """wot's stage schedule (src/trnopt/singlecell.py:46-50) against its closed form: eps0 eps^(e / scalings) for
    e = 0 .. scalings - 1 (sf = eps^(-1 / scalings)), so 1, 0.5493, 0.3017, 0.1657, 0.0910 at eps 0.05."""
    from trnopt.singlecell import wot_eps_stages
    st = wot_eps_stages(0.05)
    np.testing.assert_allclose(st, [0.05 ** (e / 5) for e in range(5)], rtol=1e-14)
    np.testing.assert_allclose(st, [1.0, 0.5493, 0.3017, 0.1657, 0.0910], atol=5e-5)
    np.testing.assert_allclose(wot_eps_stages(0.01, eps0=2.0, scalings=4), [2.0 * 0.01 ** (e / 4) for e in range(4)],
                               rtol=1e-14)
    assert all(e > 0.05 for e in st)           # every stage lies above the final eps: the solver keeps them all


def test_wot_transport_maps_equal_the_per_pair_maps():
    """wot_transport_maps runs a pipeline's independent pairs (on the fused path several at once); on the torch
    path it runs them in order, and every map equals wot_transport_map's for its pair, with per-pair growth and
    time steps. Mismatched per-pair arguments are refused."""
    from trnopt.singlecell import wot_transport_map, wot_transport_maps
    opts = SinkhornOptions(kernel="torch", backend=Backend.preset("cpu"), max_iters=20000)
    sig = 1.0 / np.sqrt(np.arange(4) + 1.0)
    pts = [np.random.default_rng(s).standard_normal((n, 4)) * sig + 0.3 * s * sig for n, s in ((90, 1), (110, 2), (70, 3))]
    pairs = [(pts[0], pts[1]), (pts[1], pts[2])]
    growth = [np.linspace(0.5, 1.5, len(pts[0])), None]
    maps = wot_transport_maps(pairs, growth=growth, delta_days=[1.0, 0.5], streams=4, growth_iters=2, tol=1e-7,
                              opts=opts)
    for (x0, x1), G, dd, tm in zip(pairs, growth, [1.0, 0.5], maps):
        one = wot_transport_map(x0, x1, G, dd, growth_iters=2, tol=1e-7, opts=opts)
        assert tm.iterations == one.iterations
        np.testing.assert_array_equal(tm.result.f, one.result.f)
        np.testing.assert_array_equal(tm.result.g, one.result.g)
        for a, b in zip(tm.learned_growth, one.learned_growth):
            np.testing.assert_array_equal(a, b)
    with pytest.raises(ValueError, match="one entry per pair"):
        wot_transport_maps(pairs, growth=[None], opts=opts)
    with pytest.raises(ValueError, match="one entry per pair"):
        wot_transport_maps(pairs, delta_days=[1.0, 2.0, 3.0], opts=opts)
