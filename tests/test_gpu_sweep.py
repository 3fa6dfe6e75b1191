"""A seeded random sweep of the fused half-step (sk_half_step_f32) against the float64 known answer on the same
float32 inputs (examples/nki_sinkhorn_check.py:60-73, brute.half_step_f64).

Each case draws the row and column counts (1 to 3,000, log-uniform: ragged, single points, many padding
rows and columns), the dimension (1 to 128: every K chunk count, the ring of column chunks above kp 64 included), the
two clouds' scales independently (1e-3 to 1e3: mixed scales put the column terms far above the dot products
in the kernel's units), eps relative to the typical cost (1e-3 to 1e2: from a single dominant score per row
to nearly flat rows), kappa (1 or in (0.5, 1)), offsets or none, random weights and column potentials. Both
directions run (the f update with the first cloud's rows, the g update with the second's), each with and
without the first cloud's log2-unit copy.

The tolerance is the float32 error budget of the half-step, per row: the contraction (at least as accurate as
an fp32 dot product: a few 2^-24 of sum_k |x_k| |y_k| and of the scaled pieces' quantum), the column term's
own rounding, the exp2 / log2 of the log-sum-exp, and the final rounding of the result.
"""

import os

import numpy as np
import pytest
import torch

from oracle import brute

pytestmark = pytest.mark.gpu
DEV = "cuda"
# The default sweep; SK_SWEEP_CASES=N runs N seeded cases instead (a longer one-off sweep), from case
# SK_SWEEP_FIRST on (default 0).
N_CASES = int(os.environ.get("SK_SWEEP_CASES", "160"))
FIRST_CASE = int(os.environ.get("SK_SWEEP_FIRST", "0"))


def _case(k, shape=None):
    rng = np.random.default_rng(7000 + k)
    rows = int(np.exp(rng.uniform(0.0, np.log(3000.0))))
    m = int(np.exp(rng.uniform(0.0, np.log(3000.0))))
    d = int(rng.integers(1, 129))
    if shape is not None:
        rows, m, d = shape
    sx, sy = np.exp(rng.uniform(np.log(1e-3), np.log(1e3), 2))
    x = rng.normal(size=(rows, d)) * sx
    y = rng.normal(size=(m, d)) * sy + 0.3 * sy
    cost = d * (sx * sx + sy * sy)
    eps = float(cost * np.exp(rng.uniform(np.log(1e-3), np.log(1e2))))
    kappa = 1.0 if rng.uniform() < 0.5 else float(rng.uniform(0.5, 1.0))
    gh = -(y * y).sum(1) + rng.normal(scale=0.2 * cost, size=m)     # column potential g - |y|^2
    fh = -(x * x).sum(1) + rng.normal(scale=0.2 * cost, size=rows)  # row potential f - |x|^2
    la = np.log(rng.uniform(0.2, 1.8, rows) / rows)
    lb = np.log(rng.uniform(0.2, 1.8, m) / m)
    offx = rng.normal(scale=0.3, size=rows) if rng.uniform() < 0.5 else None
    offy = rng.normal(scale=0.3, size=m) if rng.uniform() < 0.5 else None
    return dict(rows=rows, m=m, d=d, sx=sx, sy=sy, eps=eps, kappa=kappa, x=x, y=y, gh=gh, fh=fh, la=la, lb=lb,
                offx=offx, offy=offy)


def _budget(r32, c32, col_term, eps, kappa, want):
    """Per-row float32 error budget of a half-step with rows r32 and columns c32 (see the module docstring)."""
    r = np.abs(r32.astype(np.float64))
    c = np.abs(c32.astype(np.float64))
    dots = np.zeros(len(r))
    for s in range(0, len(r), 1024):
        dots[s:s + 1024] = (r[s:s + 1024] @ c.T).max(axis=1)
    quantum = 2.0 ** -21 * r.max() * c.max() * r.shape[1]      # the scaled fp16 pieces' resolution
    contraction = 2.0 * (4.0 * 2.0 ** -24 * np.sqrt(r.shape[1]) * dots + quantum)
    column = 4.0 * 2.0 ** -24 * np.abs(col_term).max()
    lse = 8.0 * 2.0 ** -24 * eps * (1.0 + np.log(len(c)))
    return kappa * (contraction + column + lse) + 4.0 * 2.0 ** -24 * np.abs(want) + 1e-30


@pytest.mark.parametrize("k", range(FIRST_CASE, FIRST_CASE + N_CASES))
def test_half_step_random_sweep(hip, k):
    _check_case(hip, _case(k), f"sweep case {k}")


# A few points against a large cloud and the reverse, up to a million points: one row group whose columns are
# split over every workgroup (256 partial slots per row for the merge), and hundreds to thousands of row groups
# against a single column tile; d 100 (the ring of column chunks) and d 1-2 as well.
EXTREME = [(5, 150_000, 16), (150_000, 5, 16), (3, 60_000, 100), (60_000, 3, 100), (2, 200_000, 2),
           (40_000, 1, 64), (1_000_000, 7, 16), (9, 1_000_000, 4)]


@pytest.mark.parametrize("i", range(len(EXTREME)))
def test_half_step_extreme_aspect_ratios(hip, i):
    _check_case(hip, _case(500 + i, EXTREME[i]), f"extreme case {EXTREME[i]}")


def _check_case(hip, c, label):
    rows, m, d, eps, kappa = c["rows"], c["m"], c["d"], c["eps"], c["kappa"]
    print(f"{label}: rows {rows} m {m} d {d} scales {c['sx']:.3g} {c['sy']:.3g} eps {eps:.3g} "
          f"kappa {kappa:.3f}", flush=True)
    X = hip.HipCloud(c["x"], c["la"], DEV, off=c["offx"], role=0)
    Y = hip.HipCloud(c["y"], c["lb"], DEV, off=c["offy"], role=1)
    sc = hip.scalars(eps, kappa, DEV)
    x32, y32 = c["x"].astype(np.float32), c["y"].astype(np.float32)
    xsq32 = (c["x"] ** 2).sum(1).astype(np.float32)
    ysq32 = (c["y"] ** 2).sum(1).astype(np.float32)
    zx = np.zeros(rows) if c["offx"] is None else c["offx"]
    zy = np.zeros(m) if c["offy"] is None else c["offy"]
    k32 = float(np.float32(kappa))
    # the f update (rows x) and the g update (rows y), float64 answers on the float32 inputs
    gh32, fh32 = c["gh"].astype(np.float32), c["fh"].astype(np.float32)
    la32, lb32 = c["la"].astype(np.float32), c["lb"].astype(np.float32)
    want_f = brute.half_step_f64(x32, xsq32, zx.astype(np.float32), y32, gh32, lb32, eps, k32)
    want_g = brute.half_step_f64(y32, ysq32, zy.astype(np.float32), x32, fh32, la32, eps, k32)
    tol_f = _budget(x32, y32, gh32.astype(np.float64) + eps * lb32, eps, k32, want_f)
    tol_g = _budget(y32, x32, fh32.astype(np.float64) + eps * la32, eps, k32, want_g)
    gh_t = torch.zeros(Y.npad, dtype=torch.float32, device=DEV)
    gh_t[:m] = torch.from_numpy(gh32).to(DEV)
    fh_t = torch.zeros(X.npad, dtype=torch.float32, device=DEV)
    fh_t[:rows] = torch.from_numpy(fh32).to(DEV)
    worst = 0.0
    for copy in (False, True):
        if copy:                                     # the first cloud's log2-unit copy for this eps
            hip.bake_log2(X, Y, sc)
        got_f = hip.half_step(X, Y, gh_t, sc).cpu().numpy()[:rows].astype(np.float64)
        got_g = hip.half_step(Y, X, fh_t, sc).cpu().numpy()[:m].astype(np.float64)
        for got, want, tol, what in ((got_f, want_f, tol_f, "f"), (got_g, want_g, tol_g, "g")):
            assert np.all(np.isfinite(got)), (what, copy)
            ratio = float((np.abs(got - want) / tol).max())
            worst = max(worst, ratio)
            assert ratio <= 1.0, (what, copy, ratio, float(np.abs(got - want).max()))
    print(f"  worst error / budget {worst:.3f}", flush=True)
