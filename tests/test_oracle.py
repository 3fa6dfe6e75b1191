"""Pins of the oracle (oracle/reference.py, oracle/brute.py) on the CPU.

The oracle is what every GPU parity test compares against, so it is checked here against what does not come
from it: the reference's published float64 result (results/sinkhorn_trn1.2xlarge_2026-10-30.csv:5,10), the
dense float64 brute force that uses neither shifted potentials, padding nor blocks (the algebra of
src/trnopt/sinkhorn.py:28-33, 108-119 in closed form), wot's scaling-form iteration
(tests/test_sinkhorn.py:186-205 of the reference), closed forms of the row log-sum-exp, and invariants of the
plan. Mutation tests plant a plausible mistake in the oracle (a sign, a dropped term, a transposed operand, the
wrong initial potential) and require one of the pins to fail.
"""

import json
from pathlib import Path

import numpy as np
import pytest
import torch
from scipy.special import logsumexp

from oracle import brute, data
from oracle import reference as ref

GOLDEN = Path(__file__).resolve().parent / "golden"


def _normed(x, y, how="mean"):
    c, s = ref.normalization(x, y, how=how)
    return (x - c) / np.sqrt(s), (y - c) / np.sqrt(s)


def _iterate_gap(res, hist, X_sq, Y_sq):
    """Largest relative gap between the oracle's recorded iterates (shifted, padded) and the brute force's."""
    worst = 0.0
    for (it, fh, gh), (f, g) in zip(res.history, hist):
        fo = fh[:len(f)] + X_sq[:len(f)]
        go = gh[:len(g)] + Y_sq[:len(g)]
        worst = max(worst, np.abs(fo - f).max() / np.abs(f).max(), np.abs(go - g).max() / np.abs(g).max())
    return worst


def _sq(p):
    return (p * p).sum(1)


# ---------------------------------------------------------------------------------------------------------
# Published end-to-end numbers of the reference

def _published():
    return json.loads((GOLDEN / "published.json").read_text())


@pytest.mark.slow
def test_published_float64_cost_10k():
    """The reference's float64 CPU run (preset "cpu", torch half-step, block 2048) on the mixture clouds
    10k x 10k d 64, eps 0.05, mean normalisation, tol 1e-4: 20 iterations, cost 0.8971549234175153
    (results/sinkhorn_trn1.2xlarge_2026-10-30.csv:5). The restated driver, normalisation, init, check cadence
    and half-step must reproduce it to BLAS rounding."""
    pub = _published()["mixture_10k_eps0.05"]
    x = data.mixture(10_000, 64, k=20, seed=0)
    y = data.mixture(10_000, 64, k=20, seed=1, shift=0.3)
    r = ref.sinkhorn_ref(x, y, eps=0.05, tol=1e-4, max_iters=2000, block=2048, dtype=torch.float64)
    assert r.converged and r.iterations == pub["iterations"]
    assert abs(r.cost - pub["cost_float64"]) <= 1e-12 * abs(pub["cost_float64"]), r.cost


@pytest.mark.slow
def test_published_float32_cost_10k():
    """The same problem in float32 (preset "cpu-float32"): the reference's float32 runs converged in 20
    iterations with costs 0.8971549341961733 (torch), 0.8971549319624892 (NKI, 1 core), 0.8971549320295445
    (NKI, 2 cores) and final errors 5.8e-8, 5.2e-8, 6.2e-8 (results/sinkhorn_trn1.2xlarge_2026-10-30.csv:5,10,17):
    all within 1.2e-8 relative of the float64 cost. The float32 oracle (another BLAS, another summation order)
    must land in that band: 20 iterations, cost within 1.5e-8 of both the float64 and the float32 torch cost,
    final error of the same order."""
    pub = _published()["mixture_10k_eps0.05"]
    x = data.mixture(10_000, 64, k=20, seed=0)
    y = data.mixture(10_000, 64, k=20, seed=1, shift=0.3)
    r = ref.sinkhorn_ref(x, y, eps=0.05, tol=1e-4, max_iters=2000, block=2048, dtype=torch.float32)
    assert r.converged and r.iterations == pub["iterations"]
    c64, c32 = pub["cost_float64"], pub["cost_float32_torch"]
    assert abs(c32 - c64) <= 1.5e-8 * c64 and abs(pub["cost_float32_nki"] - c64) <= 1.5e-8 * c64
    assert abs(r.cost - c64) <= 1.5e-8 * c64, r.cost
    assert abs(r.cost - c32) <= 1.5e-8 * c64, r.cost
    assert pub["error_float32_nki"] / 3 <= r.error <= pub["error_float32_torch"] * 3, r.error


def test_eps_schedule_closed_form():
    """The eps_start schedule (src/trnopt/sinkhorn.py:313-320) against its closed form, not against itself:
    eps_start decay^k for k = 0, 1, ... while the value exceeds eps (strictly), at most max_iters values;
    eps_stages above eps replace it. Both the oracle's and the product's (trnopt.sinkhorn._prepare) schedules.
    A schedule that kept the first value <= eps, or started at eps_start decay, fails here."""
    from trnopt.sinkhorn import SinkhornOptions, _prepare
    x, y = data.clouds(n=20, m=15, d=3, seed=1)

    def product(eps, max_iters, eps_start, decay, stages=None):
        p = _prepare(x, y, None, None, SinkhornOptions(eps=eps, max_iters=max_iters, eps_start=eps_start,
                                                       eps_decay=decay, eps_stages=stages), None, None)
        return p.sched, p.stages

    for sched_fn in (ref.eps_schedule, product):
        sched, stages = sched_fn(0.05, 100, 1.0, 0.7)
        assert stages == [] and len(sched) == 9                      # 0.7^8 = 0.0576 > 0.05 > 0.7^9 = 0.0404
        np.testing.assert_allclose(sched, [0.7 ** k for k in range(9)], rtol=1e-15, atol=0)
        assert sched_fn(0.25, 100, 1.0, 0.5) == ([1.0, 0.5], [])     # 0.25 = eps exactly: not scheduled
        sched, _ = sched_fn(0.05, 5, 1.0, 0.7)                       # the max_iters cap
        np.testing.assert_allclose(sched, [0.7 ** k for k in range(5)], rtol=1e-15, atol=0)
        assert sched_fn(0.05, 100, 0.05, 0.7) == ([], [])            # eps_start not above eps
        assert sched_fn(0.05, 100, None, 0.7) == ([], [])
        assert sched_fn(0.05, 100, 1.0, 0.7, (1.0, 0.5, 0.05, 0.01)) == ([], [1.0, 0.5])
        sched, _ = sched_fn(0.01, 1000, 2.0, 0.8)
        k = np.arange(len(sched))
        np.testing.assert_allclose(sched, 2.0 * 0.8 ** k, rtol=1e-14, atol=0)
        assert sched[-1] > 0.01 >= sched[-1] * 0.8 and len(sched) == int(np.ceil(np.log(0.01 / 2.0) / np.log(0.8)))


def test_published_float64_cost_needs_reference_init():
    """The same solve's first iterate from g0 = |y|^2 (the reference's init) differs from g0 = 0 (the
    reference's test oracle's init): the fixed-iteration workloads depend on the distinction."""
    x, y = data.clouds(n=60, m=50, d=4, seed=5)
    xs, ys = _normed(x, y)
    f1, g1, _ = brute.sinkhorn_dense(xs, ys, 0.1, iters=1)
    f0, g0, _ = brute.sinkhorn_dense(xs, ys, 0.1, iters=1, g0=np.zeros(len(ys)))
    r = ref.sinkhorn_ref(x, y, eps=0.1, max_iters=1, fixed_iters=True)
    assert np.abs(r.f - f1).max() < 1e-12 * np.abs(f1).max()
    assert np.abs(r.f - f0).max() > 1e-3


# ---------------------------------------------------------------------------------------------------------
# Iterate-by-iterate equality with the dense brute force

CASES = {
    "balanced": dict(opts=dict(eps=0.1), brute=dict()),
    "balanced_blocks": dict(opts=dict(eps=0.1, block=32, block_y=40), brute=dict()),
    "weighted": dict(opts=dict(eps=0.2), brute=dict(), weights=True),
    "unbalanced_targets": dict(opts=dict(eps=0.1, rho=(1.0, 50.0), block=50), brute=dict(rho_x=1.0, rho_y=50.0),
                               targets=True),
    "eps_start": dict(opts=dict(eps=0.05, eps_start=1.0, eps_decay=0.7), brute=dict(), sched=True),
}


def _run_case(name, iters=12, half_step=None, monkeypatch=None):
    c = CASES[name]
    x, y = data.clouds(n=137, m=91, d=5, seed=0)
    rng = np.random.default_rng(4)
    a = b = None
    if c.get("weights"):
        a = rng.uniform(0.2, 1.0, len(x)); a /= a.sum()
        b = rng.uniform(0.2, 1.0, len(y)); b /= b.sum()
    at = bt = None
    if c.get("targets"):
        at = rng.uniform(0.5, 1.5, len(x)) / len(x)
        bt = np.full(len(y), at.mean())
    if half_step is not None:
        monkeypatch.setattr(ref, "half_step", half_step)
    r = ref.sinkhorn_ref(x, y, a, b, max_iters=iters, fixed_iters=True, record=True, dtype=torch.float64,
                         a_target=at, b_target=bt, **c["opts"])
    xs, ys = _normed(x, y)
    o = c["opts"]
    if c.get("sched"):
        sched, _ = ref.eps_schedule(o["eps"], iters, o["eps_start"], o["eps_decay"])
        eps_of = lambda it: sched[it] if it < len(sched) else o["eps"]   # noqa: E731
    else:
        eps_of = o["eps"]
    kw = dict(c["brute"])
    if c.get("targets"):
        kw.update(off_x=np.log(at) - np.log(np.full(len(x), 1 / len(x))),
                  off_y=np.log(bt) - np.log(np.full(len(y), 1 / len(y))))
    _, _, hist = brute.sinkhorn_dense(xs, ys, eps_of, a=a, b=b, iters=iters, **kw)
    return _iterate_gap(r, hist, _sq(np.vstack([xs, np.zeros((200, xs.shape[1]))])),
                        _sq(np.vstack([ys, np.zeros((200, ys.shape[1]))])))


@pytest.mark.parametrize("name", list(CASES))
def test_iterates_equal_dense_brute_force(name):
    assert _run_case(name) < 1e-10


def test_staged_iterates_equal_dense_brute_force():
    """wot-style stages with a stage_tol no iterate meets: each stage lasts exactly stage_max_iters."""
    x, y = data.clouds(n=80, m=60, d=3, seed=9)
    stages = (1.0, 0.5, 0.25)
    r = ref.sinkhorn_ref(x, y, eps=0.1, eps_stages=stages, stage_tol=0.0, stage_max_iters=4, check_every=2,
                         max_iters=15, fixed_iters=True, record=True, rho=5.0)
    xs, ys = _normed(x, y)
    eps_of = lambda it: stages[it // 4] if it < 12 else 0.1   # noqa: E731
    _, _, hist = brute.sinkhorn_dense(xs, ys, eps_of, rho_x=5.0, rho_y=5.0, iters=15)
    assert _iterate_gap(r, hist, _sq(xs), _sq(ys)) < 1e-10


# Planted mistakes: each must break the iterate equality.
def _mut_sign_gh(x_blk, xsq_blk, off_blk, yT, gh, log_b, inv_eps, eps, kappa):
    z = (2.0 * (x_blk @ yT) - gh[None, :]) * inv_eps + log_b[None, :]
    zmax = z.amax(dim=1, keepdim=True)
    lse = zmax[:, 0] + torch.log(torch.exp(z - zmax).sum(dim=1))
    return kappa * (xsq_blk + eps * off_blk - eps * lse) - xsq_blk


def _mut_drop_logb(x_blk, xsq_blk, off_blk, yT, gh, log_b, inv_eps, eps, kappa):
    z = (2.0 * (x_blk @ yT) + gh[None, :]) * inv_eps
    zmax = z.amax(dim=1, keepdim=True)
    lse = zmax[:, 0] + torch.log(torch.exp(z - zmax).sum(dim=1))
    return kappa * (xsq_blk + eps * off_blk - eps * lse) - xsq_blk


def _mut_factor(x_blk, xsq_blk, off_blk, yT, gh, log_b, inv_eps, eps, kappa):
    z = ((x_blk @ yT) + gh[None, :]) * inv_eps + log_b[None, :]
    zmax = z.amax(dim=1, keepdim=True)
    lse = zmax[:, 0] + torch.log(torch.exp(z - zmax).sum(dim=1))
    return kappa * (xsq_blk + eps * off_blk - eps * lse) - xsq_blk


def _mut_kappa_outside(x_blk, xsq_blk, off_blk, yT, gh, log_b, inv_eps, eps, kappa):
    z = (2.0 * (x_blk @ yT) + gh[None, :]) * inv_eps + log_b[None, :]
    zmax = z.amax(dim=1, keepdim=True)
    lse = zmax[:, 0] + torch.log(torch.exp(z - zmax).sum(dim=1))
    return kappa * (xsq_blk + eps * off_blk - eps * lse - xsq_blk)


def _mut_off_sign(x_blk, xsq_blk, off_blk, yT, gh, log_b, inv_eps, eps, kappa):
    z = (2.0 * (x_blk @ yT) + gh[None, :]) * inv_eps + log_b[None, :]
    zmax = z.amax(dim=1, keepdim=True)
    lse = zmax[:, 0] + torch.log(torch.exp(z - zmax).sum(dim=1))
    return kappa * (xsq_blk - eps * off_blk - eps * lse) - xsq_blk


@pytest.mark.parametrize("mutant,case", [(_mut_sign_gh, "balanced"), (_mut_drop_logb, "weighted"),
                                         (_mut_factor, "balanced"), (_mut_kappa_outside, "unbalanced_targets"),
                                         (_mut_off_sign, "unbalanced_targets")])
def test_planted_mistake_breaks_iterate_pin(mutant, case, monkeypatch):
    assert _run_case(case, iters=3, half_step=mutant, monkeypatch=monkeypatch) > 1e-4


# ---------------------------------------------------------------------------------------------------------
# Converged answers and invariants

def test_converged_plan_matches_brute_force_and_row_sums():
    """tests/test_sinkhorn.py:78-88 of the reference, against the oracle (float64)."""
    x, y = data.clouds()
    r = ref.sinkhorn_ref(x, y, eps=0.1, tol=1e-7, max_iters=5000)
    assert r.converged
    xs, ys = _normed(x, y)
    f, g, _ = brute.sinkhorn_dense(xs, ys, 0.1, g0=np.zeros(len(ys)), iters=20000, tol=1e-12)
    P = ref.transport_plan(x, y, r)
    Q = brute.dense_plan(xs, ys, f, g, 0.1)
    assert np.abs(P - Q).max() / Q.max() < 1e-6
    np.testing.assert_allclose(P.sum(0), 1 / len(y), rtol=1e-9)     # the last update was g's: columns exact
    np.testing.assert_allclose(P.sum(1), 1 / len(x), rtol=1e-5)


def test_raw_cost_plan_matches_log_domain_solver():
    """tests/test_sinkhorn.py:143-152 of the reference (the raw cost, eps 0.5, tol 1e-9, plan within 1e-6), with
    POT's log-domain solver, which is not installed here, replaced by the same textbook iteration on the dense
    float64 C (uniform marginals, g from zero), run to 1e-13."""
    x, y = data.clouds(n=120, m=80, d=4, seed=5)
    r = ref.sinkhorn_ref(x, y, eps=0.5, normalize=False, tol=1e-9, max_iters=10_000)
    assert r.converged
    f, g, _ = brute.sinkhorn_dense(x, y, 0.5, g0=np.zeros(len(y)), iters=20_000, tol=1e-13)
    Q = brute.dense_plan(x, y, f, g, 0.5)
    assert np.abs(ref.transport_plan(x, y, r) - Q).max() / Q.max() < 1e-6


def test_float32_oracle_close_to_float64():
    x, y = data.clouds(n=400, m=350, d=10, seed=3)
    o = dict(eps=0.05, tol=1e-5, max_iters=3000)
    r64 = ref.sinkhorn_ref(x, y, dtype=torch.float64, **o)
    r32 = ref.sinkhorn_ref(x, y, dtype=torch.float32, **o)
    assert r32.converged and abs(r32.iterations - r64.iterations) <= 10
    P, Q = ref.transport_plan(x, y, r32), ref.transport_plan(x, y, r64)
    assert np.abs(P - Q).max() / Q.max() < 2e-3


@pytest.mark.parametrize("staged", [False, True])
def test_wot_formulation_matches_wot_scaling(staged):
    """tests/test_sinkhorn.py:208-226 of the reference against the oracle (float64)."""
    from trnopt.singlecell import wot_eps_stages
    x, y = data.clouds(n=90, m=70, d=4, seed=7)
    G = np.random.default_rng(8).uniform(0.5, 2.0, len(x))
    eps, l1, l2 = 0.2, 1.0, 50.0
    I, J = len(x), len(y)
    r = ref.sinkhorn_ref(x, y, np.full(I, 1 / I), np.full(J, 1 / J), eps=eps, rho=(l1, l2), normalize="median",
                         tol=1e-10, max_iters=50_000, check_every=5, eps_stages=wot_eps_stages(eps) if staged else None,
                         a_target=G / I, b_target=np.full(J, G.mean() / J))
    assert r.converged
    T = I * ref.transport_plan(x, y, r, np.full(I, 1 / I), np.full(J, 1 / J))
    R = brute.wot_scaling(x, y, eps, l1, l2, G)
    assert np.abs(T - R).max() / R.max() < 1e-6
    np.testing.assert_allclose(I * r.row_mass, R.sum(1), rtol=1e-6)
    np.testing.assert_allclose(I * r.col_mass, R.sum(0), rtol=1e-6)


def test_unbalanced_masses_are_plan_marginals():
    """row_mass / col_mass from the two extra balanced half-steps equal the dense plan's sums."""
    x, y = data.clouds(n=70, m=50, d=3, seed=2)
    a = np.random.default_rng(3).uniform(0.5, 1.5, len(x)) / len(x)
    r = ref.sinkhorn_ref(x, y, a=a, eps=0.1, rho=2.0, tol=1e-9, max_iters=5000)
    P = ref.transport_plan(x, y, r, a=a)
    np.testing.assert_allclose(r.row_mass, P.sum(1), rtol=1e-10)
    np.testing.assert_allclose(r.col_mass, P.sum(0), rtol=1e-10)
    rows, cols = brute.plan_marginals(*_normed(x, y), a, np.full(len(y), 1 / len(y)), r.f, r.g, 0.1, chunk=16)
    np.testing.assert_allclose(rows, P.sum(1), rtol=1e-12)
    np.testing.assert_allclose(cols, P.sum(0), rtol=1e-12)


def test_balanced_plan_invariant_to_neutral_shift():
    x, y = data.clouds(n=30, m=20, d=3)
    r = ref.sinkhorn_ref(x, y, eps=0.1, tol=1e-8, max_iters=2000)
    P = ref.transport_plan(x, y, r)
    r.f, r.g = r.f + 0.37, r.g - 0.37
    np.testing.assert_allclose(ref.transport_plan(x, y, r), P, rtol=1e-12)


def test_padding_contributes_nothing():
    """Blocks that pad rows and columns (log weight -1e9) give the unblocked answer."""
    x, y = data.clouds()
    o = dict(eps=0.1, max_iters=15, fixed_iters=True)
    full = ref.sinkhorn_ref(x, y, **o)
    blk = ref.sinkhorn_ref(x, y, block=32, block_y=40, **o)
    np.testing.assert_allclose(blk.f, full.f, rtol=0, atol=1e-12 * np.abs(full.f).max())
    np.testing.assert_allclose(blk.g, full.g, rtol=0, atol=1e-12 * np.abs(full.g).max())


def test_check_cadence_and_convergence_flags():
    """Checks only every check_every iterations: the converged iteration count is a multiple of it, and a
    max_iters that is not stops unconverged with the error of the last check."""
    x, y = data.clouds()
    r = ref.sinkhorn_ref(x, y, eps=0.1, tol=1e-6, max_iters=5000, check_every=7)
    assert r.converged and r.iterations % 7 == 0
    r2 = ref.sinkhorn_ref(x, y, eps=0.1, tol=1e-30, max_iters=23, check_every=7)
    assert not r2.converged and r2.iterations == 23 and np.isfinite(r2.error)
    r3 = ref.sinkhorn_ref(x, y, eps=0.1, max_iters=5, fixed_iters=True)
    assert r3.iterations == 5 and np.isnan(r3.error)


def test_float32_floors():
    """fp32 floors (src/trnopt/sinkhorn.py:340-344): unbalanced tol >= 5e-6."""
    x, y = data.clouds()
    o = dict(eps=0.1, rho=1.0, tol=1e-9, max_iters=5000)
    r32 = ref.sinkhorn_ref(x, y, dtype=torch.float32, **o)
    assert r32.converged and r32.error < 5e-6


# ---------------------------------------------------------------------------------------------------------
# The kernel-level known answers

def test_row_lse_closed_forms():
    rng = np.random.default_rng(0)
    xa = rng.normal(size=(7, 5))
    ya = rng.normal(size=(1, 5))
    np.testing.assert_allclose(brute.row_lse(xa, ya), (xa @ ya.T)[:, 0], rtol=1e-14)      # m = 1
    yb = np.repeat(ya, 9, axis=0)
    np.testing.assert_allclose(brute.row_lse(xa, yb), (xa @ ya.T)[:, 0] + np.log(9), rtol=1e-14)  # identical columns
    yc = rng.normal(size=(300, 5))
    direct = np.array([np.log(sum(np.exp(sum(xa[i, k] * yc[j, k] for k in range(5))) for j in range(300)))
                       for i in range(7)])
    np.testing.assert_allclose(brute.row_lse(xa, yc, chunk=3), direct, rtol=1e-12)


def test_half_step_known_answer_equals_one_dense_update():
    """half_step_f64's epilogue = one f update of the dense iteration (balanced and with kappa, offset)."""
    x, y = data.clouds(n=40, m=30, d=4, seed=1)
    rng = np.random.default_rng(2)
    lb = np.log(rng.uniform(0.5, 1.5, len(y)) / len(y))
    g = rng.normal(size=len(y))
    off = rng.normal(scale=0.2, size=len(x))
    eps, kappa = 0.15, 0.8
    fh = brute.half_step_f64(x, _sq(x), off, y, g - _sq(y), lb, eps, kappa)
    C = brute.sq_dist(x, y)
    f = kappa * (eps * off - eps * logsumexp(lb[None, :] + (g[None, :] - C) / eps, axis=1))
    np.testing.assert_allclose(fh + _sq(x), f, rtol=1e-12, atol=1e-12)


def test_normalization_median_exact_and_sampled():
    x, y = data.clouds(n=50, m=40, d=3)
    c, s = ref.normalization(x, y, how="median")
    np.testing.assert_allclose(c, np.vstack([x, y]).mean(0))
    assert s == pytest.approx(np.median(brute.sq_dist(x - c, y - c)), rel=1e-12)
    c2, s2 = ref.normalization(x, y)           # sampled mean over 20k pairs, seed 0
    assert abs(s2 / brute.sq_dist(x, y).mean() - 1) < 0.05
