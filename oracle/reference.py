"""The reference's plain-PyTorch Sinkhorn restated on the CPU (test infrastructure: see oracle/__init__.py).

Follows /root/reference/src/trnopt/sinkhorn.py (cited as sinkhorn.py:line):
  PAD_LOG_WEIGHT, _DELTA_CAP        :59-60
  half_step                         :108-119   (the op sequence is kept: it fixes float32 rounding)
  pad_cloud                         :131-158   (torch path only; no NKI blocks, no cores)
  log_weights                       :211-217
  normalization                     :220-238
  sinkhorn_ref                      :241-394   (validation 254-271, schedule 313-320, floors 340-344, loop
                                                346-378, read-back 379-380, masses 381-389, cost 391)
  transport_plan                    :397-403
dtype float64 is the reference's "cpu" preset, float32 its "cpu-float32" preset (backend.py:35-36).
"""

from __future__ import annotations

import time
from dataclasses import dataclass

import numpy as np
import torch

PAD_LOG_WEIGHT = -1e9
_DELTA_CAP = 50.0


@dataclass
class RefResult:
    f: np.ndarray
    g: np.ndarray
    iterations: int
    error: float
    converged: bool
    cost: float
    seconds: float
    center: np.ndarray
    cost_scale: float
    eps: float
    row_mass: np.ndarray | None
    col_mass: np.ndarray | None
    history: list            # (iteration, fh, gh) snapshots when record=True (float64 numpy, padded)


def half_step(x_blk, xsq_blk, off_blk, yT, gh, log_b, inv_eps, eps, kappa):
    """sinkhorn.py:108-119."""
    z = (2.0 * (x_blk @ yT) + gh[None, :]) * inv_eps + log_b[None, :]
    zmax = z.amax(dim=1, keepdim=True)
    lse = zmax[:, 0] + torch.log(torch.exp(z - zmax).sum(dim=1))
    return kappa * (xsq_blk + eps * off_blk - eps * lse) - xsq_blk


def log_weights(w, n, name):
    """sinkhorn.py:211-217."""
    if w is None:
        return np.full(n, -np.log(n))
    w = np.asarray(w, dtype=np.float64)
    if w.shape != (n,) or np.any(w <= 0):
        raise ValueError(f"{name} must be {n} positive weights")
    return np.log(w)


def normalization(x, y, samples=20_000, seed=0, how="mean"):
    """sinkhorn.py:220-238."""
    center = np.concatenate([x, y]).mean(axis=0)
    if how == "median" and len(x) * len(y) <= 100_000_000:
        xc, yc = x - center, y - center
        C = ((xc * xc).sum(1)[:, None] + (yc * yc).sum(1)[None, :] - 2.0 * (xc @ yc.T)).ravel()
        s = float(np.median(np.maximum(C, 0.0)))
        return center, (s if s > 0 else 1.0)
    rng = np.random.default_rng(seed)
    i, j = rng.integers(len(x), size=samples), rng.integers(len(y), size=samples)
    dd = ((x[i] - y[j]) ** 2).sum(axis=1)
    s = float(np.median(dd) if how == "median" else dd.mean())
    return center, (s if s > 0 else 1.0)


class _Padded:
    """sinkhorn.py:138-158 (torch path): padded points, |p|^2 in float64 then cast, log weights, weights."""

    def __init__(self, pts, log_w, block, dtype, off=None):
        n, d = pts.shape
        nb = -(-n // block)
        npad = nb * block
        P = np.zeros((npad, d))
        P[:n] = pts
        L = np.full(npad, PAD_LOG_WEIGHT)
        L[:n] = log_w
        O = np.zeros(npad)
        if off is not None:
            O[:n] = off
        t = lambda a: torch.as_tensor(np.asarray(a), dtype=dtype)   # noqa: E731  (Backend.tensor, backend.py:70-72)
        self.n, self.npad, self.block = n, npad, block
        x = t(P)
        self.xT = x.T.contiguous()
        self.sq = t((P * P).sum(axis=1))
        ot, oz = t(O), t(np.zeros(npad))
        self.blocks = [(x[s:s + block].contiguous(), self.sq[s:s + block].contiguous(),
                        ot[s:s + block].contiguous(), oz[s:s + block].contiguous()) for s in range(0, npad, block)]
        self.log_w = t(L)
        self.w = t(np.exp(L))


def eps_schedule(eps, max_iters, eps_start=None, eps_decay=0.9, eps_stages=None):
    """sinkhorn.py:313-320: (sched, stages)."""
    stages = [e for e in (eps_stages or ()) if e > eps]
    sched = []
    if not stages and eps_start is not None and eps_start > eps:
        e = eps_start
        while e > eps and len(sched) < max_iters:
            sched.append(e)
            e *= eps_decay
    return sched, stages


def sinkhorn_ref(x, y, a=None, b=None, *, eps=0.05, rho=None, max_iters=2000, tol=1e-4, check_every=10,
                 block=None, block_y=None, eps_start=None, eps_decay=0.9, eps_stages=None, stage_tol=1e-6,
                 stage_max_iters=1000, normalize=True, fixed_iters=False, dtype=torch.float64,
                 a_target=None, b_target=None, record=False, threads=None) -> RefResult:
    """sinkhorn.py:241-394 with kernel="torch", cores=1, on the CPU."""
    if threads is not None:
        torch.set_num_threads(int(threads))
    x = np.asarray(x, dtype=np.float64)
    y = np.asarray(y, dtype=np.float64)
    log_a, log_b = log_weights(a, len(x), "a"), log_weights(b, len(y), "b")
    balanced = rho is None
    if balanced and abs(np.exp(log_a).sum() - np.exp(log_b).sum()) > 1e-9 * np.exp(log_a).sum():
        raise ValueError("balanced OT needs sum(a) == sum(b); pass rho for unbalanced")
    if balanced and (a_target is not None or b_target is not None):
        raise ValueError("a_target / b_target are for unbalanced OT (pass rho)")
    rho_x, rho_y = (None, None) if balanced else (tuple(rho) if isinstance(rho, (tuple, list)) else (rho, rho))
    off_x = None if a_target is None else log_weights(a_target, len(x), "a_target") - log_a
    off_y = None if b_target is None else log_weights(b_target, len(y), "b_target") - log_b
    if isinstance(normalize, tuple):
        center, scale = np.asarray(normalize[0], dtype=np.float64), float(normalize[1])
    elif normalize:
        center, scale = normalization(x, y, how=normalize if isinstance(normalize, str) else "mean")
    else:
        center, scale = np.zeros(x.shape[1]), 1.0
    xs, ys = (x - center) / np.sqrt(scale), (y - center) / np.sqrt(scale)
    bx = block or len(x)
    by = block_y or block or len(y)
    X = _Padded(xs, log_a, bx, dtype, off_x)
    Y = _Padded(ys, log_b, by, dtype, off_y)
    sched, stages = eps_schedule(eps, max_iters, eps_start, eps_decay, eps_stages)

    cache = {}

    def consts(e, r):                                    # sinkhorn.py:323-334 (torch part)
        if (e, r) not in cache:
            kappa = 1.0 if r is None else r / (r + e)
            cache[(e, r)] = tuple(torch.tensor(v, dtype=dtype) for v in (1.0 / e, e, kappa))
        return cache[(e, r)]

    def sweep(side, other, other_h, c, use_off=True):    # sinkhorn.py:170-174 (torch path)
        return torch.cat([half_step(xb, sqb, ob if use_off else zb, other.xT, other_h, other.log_w, *c)
                          for xb, sqb, ob, zb in side.blocks])

    gh = torch.zeros(Y.npad, dtype=dtype)
    fh = gh
    err, converged, it = float("nan"), False, 0
    stage, stage_it = 0, 0
    f32 = dtype == torch.float32
    stage_tol_eff = max(stage_tol, 1e-5 if f32 else 0.0)
    tol_eff = max(tol, 5e-6) if (f32 and not balanced) else tol
    history = []
    t0 = time.perf_counter()
    while it < max_iters:
        if stages:
            e = stages[stage] if stage < len(stages) else eps
        else:
            e = sched[it] if it < len(sched) else eps
        cx, cy = consts(e, rho_x), consts(e, rho_y)
        inv_eps = cx[0]
        fh = sweep(X, Y, gh, cx)
        gh_new = sweep(Y, X, fh, cy)
        it += 1
        stage_it += 1
        if record:
            history.append((it, fh.double().numpy().copy(), gh_new.double().numpy().copy()))
        if stages and stage < len(stages):
            if stage_it % check_every == 0:
                ch = float((((gh_new - gh)[:Y.n].abs().amax()) * inv_eps).item())
                if ch < stage_tol_eff or stage_it >= stage_max_iters:
                    stage, stage_it = stage + 1, 0
            gh = gh_new
            continue
        check = (not fixed_iters and (stages or it > len(sched))
                 and (stage_it % check_every == 0 or it == max_iters))
        if check:
            if balanced:
                delta = ((gh - gh_new) * inv_eps).clamp(max=_DELTA_CAP)
                err_t = (Y.w * (torch.exp(delta) - 1.0)).abs().sum()
            else:
                err_t = ((gh_new - gh)[:Y.n].abs().amax()) * inv_eps
            err = float(err_t.item())
        gh = gh_new
        if check and err < tol_eff:
            converged = True
            break
    f = (fh + X.sq)[:X.n].to(torch.float64).numpy()
    g = (gh + Y.sq)[:Y.n].to(torch.float64).numpy()
    row_mass = col_mass = None
    if not balanced:
        c1 = consts(eps, None)
        fb = (sweep(X, Y, gh, c1, use_off=False) + X.sq)[:X.n].to(torch.float64).numpy()
        gb = (sweep(Y, X, fh, c1, use_off=False) + Y.sq)[:Y.n].to(torch.float64).numpy()
        row_mass = np.exp(log_a + (f - fb) / eps)
        col_mass = np.exp(log_b + (g - gb) / eps)
    seconds = time.perf_counter() - t0
    cost = float(np.exp(log_a) @ f + np.exp(log_b) @ g) if balanced else float("nan")
    return RefResult(f=f, g=g, iterations=it, error=err, converged=converged, cost=cost, seconds=seconds,
                     center=center, cost_scale=scale, eps=eps, row_mass=row_mass, col_mass=col_mass,
                     history=history)


def transport_plan(x, y, res, a=None, b=None):
    """sinkhorn.py:397-403 (float64, dense)."""
    x = (np.asarray(x, dtype=np.float64) - res.center) / np.sqrt(res.cost_scale)
    y = (np.asarray(y, dtype=np.float64) - res.center) / np.sqrt(res.cost_scale)
    la, lb = log_weights(a, len(x), "a"), log_weights(b, len(y), "b")
    C = ((x[:, None, :] - y[None, :, :]) ** 2).sum(axis=2)
    return np.exp(la[:, None] + lb[None, :] + (res.f[:, None] + res.g[None, :] - C) / res.eps)
