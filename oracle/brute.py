"""Independent float64 checks for the Sinkhorn path (test infrastructure: see oracle/__init__.py).

Nothing here uses the shifted-potential rewrite, padding or blocking of the reference: the cost matrix is
formed densely and every update is scipy's logsumexp, so these functions check the reference's algebra
(src/trnopt/sinkhorn.py:28-33, 108-119) as well as its iteration.

  sinkhorn_dense   -- tests/test_sinkhorn.py:54-71 (the reference's own float64 oracle), extended with the
                      reference driver's initial potential g0 = |y|^2 in the normalised frame (sinkhorn.py:336,
                      gh = 0), its per-iteration eps (sched / stages, sinkhorn.py:313-320, 347-350), per-side
                      kappa (rho_x, rho_y) and row/column offsets (sinkhorn.py:262-263), so iterates can be
                      compared one by one.
  wot_scaling      -- tests/test_sinkhorn.py:186-205 (wot's scaling-form update), float64.
  row_lse          -- examples/nki_sinkhorn_check.py:22-35: logsumexp(xa @ ya^T, axis=1) in float64.
  half_step_f64    -- examples/nki_sinkhorn_check.py:60-73: the half-step epilogue on that row-LSE.
  plan_marginals   -- examples/sinkhorn_libs_compare.py:43-56: plan row / column sums from potentials in float64,
                      chunked (no dense plan).
"""

from __future__ import annotations

import numpy as np
from scipy.special import logsumexp


def sq_dist(x, y):
    return ((x[:, None, :] - y[None, :, :]) ** 2).sum(axis=2)


def sinkhorn_dense(x, y, eps_per_iter, *, a=None, b=None, rho_x=None, rho_y=None, off_x=None, off_y=None,
                   g0=None, iters=None, tol=None):
    """Log-domain Sinkhorn on the dense C = |x - y|^2 (float64), x, y already normalised.

    eps_per_iter: a float (every iteration) or a callable it -> eps (it = iterations done). g0: initial g (the
    reference starts from |y|^2; the reference's test oracle from 0). Runs `iters` iterations, or until
    max |g_new - g| < tol. Returns (f, g, history) with history = [(f, g)] after every iteration."""
    x = np.asarray(x, dtype=np.float64)
    y = np.asarray(y, dtype=np.float64)
    n, m = len(x), len(y)
    la = np.log(a) if a is not None else np.full(n, -np.log(n))
    lb = np.log(b) if b is not None else np.full(m, -np.log(m))
    ox = np.zeros(n) if off_x is None else np.asarray(off_x, dtype=np.float64)
    oy = np.zeros(m) if off_y is None else np.asarray(off_y, dtype=np.float64)
    C = sq_dist(x, y)
    g = (y * y).sum(1) if g0 is None else np.asarray(g0, dtype=np.float64).copy()
    f = np.zeros(n)
    eps_of = eps_per_iter if callable(eps_per_iter) else (lambda it: eps_per_iter)
    hist = []
    it = 0
    while True:
        if iters is not None and it >= iters:
            break
        e = eps_of(it)
        kx = 1.0 if rho_x is None else rho_x / (rho_x + e)
        ky = 1.0 if rho_y is None else rho_y / (rho_y + e)
        # f_i = kappa (eps off_i - eps LSE_j(log b_j + (g_j - C_ij) / eps))
        f = kx * (e * ox - e * logsumexp(lb[None, :] + (g[None, :] - C) / e, axis=1))
        g_new = ky * (e * oy - e * logsumexp(la[:, None] + (f[:, None] - C) / e, axis=0))
        done = tol is not None and np.abs(g_new - g).max() < tol
        g = g_new
        it += 1
        hist.append((f.copy(), g.copy()))
        if done:
            break
    return f, g, hist


def dense_plan(x, y, f, g, eps, a=None, b=None):
    n, m = len(x), len(y)
    la = np.log(a) if a is not None else np.full(n, -np.log(n))
    lb = np.log(b) if b is not None else np.full(m, -np.log(m))
    return np.exp(la[:, None] + lb[None, :] + (f[:, None] + g[None, :] - sq_dist(x, y)) / eps)


def wot_scaling(x, y, eps, lam1, lam2, G, iters=50_000, tol=1e-13):
    """wot's scaling-form update (tests/test_sinkhorn.py:186-205): returns I * P for the median-normalised cost."""
    C = sq_dist(np.asarray(x, dtype=np.float64), np.asarray(y, dtype=np.float64))
    C = C / np.median(C)
    I, J = C.shape
    dx, dy = np.ones(I) / I, np.ones(J) / J
    p, q = G, np.ones(J) * G.mean()
    K = np.exp(-C / eps)
    a1, a2 = lam1 / (lam1 + eps), lam2 / (lam2 + eps)
    u, v = np.ones(I), np.ones(J)
    for _ in range(iters):
        u = (p / K.dot(v * dy)) ** a1
        v_new = (q / K.T.dot(u * dx)) ** a2
        done = np.abs(v_new / v - 1).max() < tol
        v = v_new
        if done:
            break
    return (K.T * u).T * v / J


def row_lse(xa, ya, chunk=2048):
    """lse_i = log sum_j exp(xa_i . ya_j) in float64 (examples/nki_sinkhorn_check.py:33), row-chunked."""
    xa = np.asarray(xa, dtype=np.float64)
    ya = np.asarray(ya, dtype=np.float64)
    out = np.empty(len(xa))
    for s in range(0, len(xa), chunk):
        out[s:s + chunk] = logsumexp(xa[s:s + chunk] @ ya.T, axis=1)
    return out


def half_step_f64(x, xsq, off, y, gh, log_b, eps, kappa, chunk=2048):
    """fh = kappa (xsq + eps off - eps lse) - xsq with lse over (2 x.y + gh) / eps + log b, float64
    (examples/nki_sinkhorn_check.py:60-73; src/trnopt/nki_sinkhorn.py:16-19)."""
    x = np.asarray(x, dtype=np.float64)
    y = np.asarray(y, dtype=np.float64)
    xa = np.hstack([x, np.ones((len(x), 1))])
    ya = np.hstack([2.0 / eps * y, (np.asarray(gh, np.float64) / eps + np.asarray(log_b, np.float64))[:, None]])
    lse = row_lse(xa, ya, chunk)
    xsq = np.asarray(xsq, dtype=np.float64)
    return kappa * (xsq + eps * np.asarray(off, np.float64) - eps * lse) - xsq


def plan_marginals(x, y, a, b, f, g, eps, chunk=2048):
    """Row and column sums of P = a b^T exp((f + g - C) / eps) in float64, chunked over rows
    (examples/sinkhorn_libs_compare.py:43-56)."""
    x, y, a, b, f, g = (np.asarray(v, dtype=np.float64) for v in (x, y, a, b, f, g))
    y2 = (y * y).sum(1)
    rows = np.empty(len(x))
    cols = np.full(len(y), -np.inf)
    for i in range(0, len(x), chunk):
        xb = x[i:i + chunk]
        S = (f[i:i + chunk][:, None] + g[None, :] - ((xb * xb).sum(1)[:, None] + y2[None, :] - 2 * xb @ y.T)) / eps
        S += np.log(a[i:i + chunk])[:, None] + np.log(b)[None, :]
        rows[i:i + chunk] = np.exp(logsumexp(S, axis=1))
        cols = np.logaddexp(cols, logsumexp(S, axis=0))
    return rows, np.exp(cols)
