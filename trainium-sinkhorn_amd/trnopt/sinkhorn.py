"""Entropic optimal transport between point clouds by log-domain Sinkhorn, with a fused HIP half-step.

The public API is the reference's (src/trnopt/sinkhorn.py): sinkhorn(x, y, a, b, opts, a_target, b_target)
-> SinkhornResult, SinkhornOptions, normalization(), transport_plan(), with the same fields, defaults,
validation errors and numerics. What is new is where the work runs:

* kernel="hip" (and kernel="auto" on Backend.preset("rocm")): the half-steps are the fused gfx950 kernels of
  hip_sinkhorn.py, which never materialise the n x m scores, and the iteration loop itself (eps schedule or
  stages, the f then g updates, convergence checks) runs on the GPU. The host enqueues batches of iterations
  and reads a small state block once per batch instead of synchronising on every check.
* kernel="torch": the plain PyTorch half-step (the reference's own, src/trnopt/sinkhorn.py:108-119) and the
  host loop, on any device and dtype. This is the path the fused kernels are checked against.
* kernel="nki" is recognised and refused (no NeuronCore in this build).

Problem and conventions (src/trnopt/sinkhorn.py:1-47). Plan P_ij = a_i b_j exp((f_i + g_j - C_ij) / eps),
C_ij = |x_i - y_j|^2. One iteration is the f update then the g update,

    f_i = -kappa_x eps LSE_j(log b_j + (g_j - C_ij) / eps),  g_j likewise with the roles swapped,

kappa = rho / (rho + eps) when unbalanced (1 when balanced). The state carried is the shifted potential
fh = f - |x|^2 (gh = g - |y|^2), so a half-step is a matrix product plus a column term and a row-wise
log-sum-exp; the loop starts from gh = 0 (g = |y|^2).
"""

from __future__ import annotations

import time
from dataclasses import dataclass
from types import SimpleNamespace

import numpy as np
import torch

from .backend import Backend

PAD_LOG_WEIGHT = -1e9          # log weight of a padding point: exactly zero weight, and finite (sinkhorn.py:59)
_DELTA_CAP = 50.0              # cap on (g_old - g_new) / eps in the balanced check, so exp stays finite (:60)
KERNELS = ("auto", "torch", "hip", "nki")


@dataclass
class SinkhornOptions:
    eps: float = 0.05              # entropic blur, in cost units (after normalisation: of the typical cost)
    rho: float | tuple | None = None   # None: balanced; else the KL marginal penalty, one value or (rho_x, rho_y)
    max_iters: int = 2000
    tol: float = 1e-4              # balanced: L1 column-marginal error; unbalanced: max potential change / eps
                                   #   (float32 unbalanced: at least 5e-6)
    check_every: int = 10          # iterations between convergence checks
    block: int | None = None       # torch kernel: rows of x per block in the f update (None: all at once).
                                   #   The fused HIP kernel streams every row and column, so it ignores blocks.
    block_y: int | None = None     # torch kernel: rows of y per block in the g update (None: same as block)
    eps_start: float | None = None # eps-scaling: start here, multiply by eps_decay each iteration down to eps
    eps_decay: float = 0.9
    eps_stages: tuple | None = None  # wot-style stages: each eps in turn until the max potential change / eps
    stage_tol: float = 1e-6        #   < stage_tol (at least 1e-5 in float32) or stage_max_iters; then eps to tol
    stage_max_iters: int = 1000
    normalize: bool | str | tuple = True  # True / "mean", "median", False, or a precomputed (center, cost_scale)
    fixed_iters: bool = False      # run exactly max_iters, no checks (benchmarks)
    cores: int = 1                 # the reference's NeuronCore row split; this build runs on one GPU (1 only)
    kernel: str = "auto"           # "auto" (hip on a ROCm GPU in float32 with d <= 128, else torch), "hip",
                                   #   "torch", or "nki" (refused: no Neuron device here)
    backend: Backend = Backend.preset("cpu")


@dataclass
class SinkhornResult:
    f: np.ndarray                  # potentials, float64, normalised cost units (times cost_scale: original)
    g: np.ndarray
    iterations: int
    error: float                   # last convergence measure; nan if never checked
    converged: bool
    cost: float                    # balanced: <a, f> + <b, g>; nan if unbalanced
    seconds: float                 # wall time of the iteration loop (including read-back and masses)
    eps: float
    rho: float | tuple | None
    center: np.ndarray             # x_used = (x - center) / sqrt(cost_scale)
    cost_scale: float
    row_mass: np.ndarray | None = None   # unbalanced: the plan's actual row and column sums
    col_mass: np.ndarray | None = None


# ---------------------------------------------------------------------------------------------------------
# The plain PyTorch half-step and its host loop (kernel="torch")

def _half_step(x_blk, xsq_blk, off_blk, yT, gh, log_b, inv_eps, eps, kappa):
    """The f update of one block of rows in shifted form: the reference's op sequence
    (src/trnopt/sinkhorn.py:116-119), scores materialised (k, m). Scalars are 0-d tensors so a compiled
    version does not specialise on eps."""
    scores = (2.0 * (x_blk @ yT) + gh[None, :]) * inv_eps + log_b[None, :]
    top = scores.amax(dim=1, keepdim=True)
    lse = top[:, 0] + torch.log(torch.exp(scores - top).sum(dim=1))
    return kappa * (xsq_blk + eps * off_blk - eps * lse) - xsq_blk


class _TorchCloud:
    """A cloud padded to whole blocks for the torch half-step, as _Cloud does (src/trnopt/sinkhorn.py:131-158)."""

    def __init__(self, pts: np.ndarray, log_w: np.ndarray, block: int, be: Backend, off: np.ndarray | None):
        n, d = pts.shape
        npad = -(-n // block) * block
        P = np.zeros((npad, d))
        P[:n] = pts
        L = np.full(npad, PAD_LOG_WEIGHT)
        L[:n] = log_w
        O = np.zeros(npad)
        if off is not None:
            O[:n] = off
        self.n, self.npad = n, npad
        pts_t = be.tensor(P)
        self.xT = pts_t.T.contiguous()
        self.sq = be.tensor((P * P).sum(axis=1))              # float64 sums, then cast
        off_t, zero_t = be.tensor(O), be.tensor(np.zeros(npad))
        self.blocks = [(pts_t[s:s + block].contiguous(), self.sq[s:s + block].contiguous(),
                        off_t[s:s + block].contiguous(), zero_t[s:s + block].contiguous())
                       for s in range(0, npad, block)]
        self.log_w = be.tensor(L)
        self.w = be.tensor(np.exp(L))                           # padding weight exactly 0


def _solve_torch(p, opts: SinkhornOptions):
    be = opts.backend
    X = _TorchCloud(p.xs, p.log_a, opts.block or len(p.xs), be, p.off_x)
    Y = _TorchCloud(p.ys, p.log_b, opts.block_y or opts.block or len(p.ys), be, p.off_y)
    step = be.compile_fn(_half_step)
    scal: dict = {}

    def consts(e, rho):
        """(1/eps, eps, kappa) as 0-d tensors, each computed in double then rounded (sinkhorn.py:323-334)."""
        key = (e, rho)
        if key not in scal:
            kappa = 1.0 if rho is None else rho / (rho + e)
            if len(scal) > 8:
                scal.clear()
            scal[key] = tuple(torch.tensor(v, dtype=be.dtype, device=be.device) for v in (1.0 / e, e, kappa))
        return scal[key]

    def sweep(side, other, other_h, c, use_off=True):
        inv_eps, eps_t, kappa = c
        return torch.cat([step(xb, sqb, ob if use_off else zb, other.xT, other_h, other.log_w, inv_eps, eps_t, kappa)
                          for xb, sqb, ob, zb in side.blocks])

    gh = torch.zeros(Y.npad, dtype=be.dtype, device=be.device)
    fh = torch.zeros(X.npad, dtype=be.dtype, device=be.device)
    err, converged, it = float("nan"), False, 0
    stage, stage_it = 0, 0
    stages, sched = p.stages, p.sched
    t0 = time.perf_counter()
    while it < opts.max_iters:
        if stages:
            e = stages[stage] if stage < len(stages) else opts.eps
        else:
            e = sched[it] if it < len(sched) else opts.eps
        cx, cy = consts(e, p.rho_x), consts(e, p.rho_y)
        inv_eps = cx[0]
        fh = sweep(X, Y, gh, cx)
        gh_new = sweep(Y, X, fh, cy)
        it += 1
        stage_it += 1
        if stages and stage < len(stages):
            # an intermediate stage: move on once the potentials settle (or after stage_max_iters)
            if stage_it % opts.check_every == 0:
                ch = float((((gh_new - gh)[:Y.n].abs().amax()) * inv_eps).item())
                if ch < p.stage_tol or stage_it >= opts.stage_max_iters:
                    stage, stage_it = stage + 1, 0
            gh = gh_new
            continue
        check = (not opts.fixed_iters and (bool(stages) or it > len(sched))
                 and (stage_it % opts.check_every == 0 or it == opts.max_iters))
        if check:
            if p.balanced:
                # column sums of the plan with (new f, old g) are b_j exp((g_old_j - g_new_j) / eps)
                delta = ((gh - gh_new) * inv_eps).clamp(max=_DELTA_CAP)
                err = float((Y.w * (torch.exp(delta) - 1.0)).abs().sum().item())
            else:
                err = float((((gh_new - gh)[:Y.n].abs().amax()) * inv_eps).item())
        gh = gh_new
        if check and err < p.tol:
            converged = True
            break
    f = (fh + X.sq)[:X.n].detach().to("cpu", torch.float64).numpy()
    g = (gh + Y.sq)[:Y.n].detach().to("cpu", torch.float64).numpy()
    fb = gb = None
    if not p.balanced:
        c1 = consts(opts.eps, None)
        fb = (sweep(X, Y, gh, c1, use_off=False) + X.sq)[:X.n].detach().to("cpu", torch.float64).numpy()
        gb = (sweep(Y, X, fh, c1, use_off=False) + Y.sq)[:Y.n].detach().to("cpu", torch.float64).numpy()
    return f, g, fb, gb, it, err, converged, t0


# ---------------------------------------------------------------------------------------------------------
# The fused HIP path (kernel="hip")

def _hip_setup(p, opts: SinkhornOptions, dev, state=None):
    """The device side of one solve on the fused path: both clouds packed, the loop set up (not run)."""
    from . import hip_sinkhorn as hk
    X = hk.HipCloud(p.xs, p.log_a, dev, p.off_x, role=0)
    Y = hk.HipCloud(p.ys, p.log_b, dev, p.off_y, role=1)
    loop = hk.DeviceLoop(X, Y, eps=opts.eps, rho_x=p.rho_x, rho_y=p.rho_y, sched=p.sched, stages=p.stages,
                         tol=p.tol, stage_tol=p.stage_tol, max_iters=opts.max_iters,
                         check_every=opts.check_every, stage_max_iters=opts.stage_max_iters,
                         fixed_iters=opts.fixed_iters, balanced=p.balanced, state=state)
    c1 = None if p.balanced else hk.scalars(opts.eps, 1.0, dev)     # requested before the loop's launches
    return SimpleNamespace(X=X, Y=Y, loop=loop, c1=c1)


def _hip_finish(p, s, st):
    """f = fh + |x|^2 in float32 on the device, then float64, as the reference reads it back (:379-380); unbalanced,
    also one balanced half-step each way (kappa = 1, no offset) at the final eps (:381-389). One read-back."""
    from . import hip_sinkhorn as hk
    X, Y, loop = s.X, s.Y, s.loop
    parts = [(loop.fh + X.sq)[:X.n], (loop.gh + Y.sq)[:Y.n]]
    if not p.balanced:
        parts.append((hk.half_step(X, Y, loop.gh, s.c1, use_off=False) + X.sq)[:X.n])
        parts.append((hk.half_step(Y, X, loop.fh, s.c1, use_off=False) + Y.sq)[:Y.n])
    host = torch.cat(parts).to("cpu", torch.float64).numpy()
    f, g = host[:X.n], host[X.n:X.n + Y.n]
    fb = gb = None
    if not p.balanced:
        fb, gb = host[X.n + Y.n:2 * X.n + Y.n], host[2 * X.n + Y.n:]
    return f, g, fb, gb, int(st.it), float(st.err), bool(st.converged)


def _hip_finish_many(ps, setups, states) -> list:
    """_hip_finish for several solves at once: every solve's potentials (and unbalanced half-steps) enqueued,
    then one read-back for all of them instead of one each."""
    from . import hip_sinkhorn as hk
    parts, spans = [], []
    for p, s, st in zip(ps, setups, states):
        X, Y, loop = s.X, s.Y, s.loop
        q = [(loop.fh + X.sq)[:X.n], (loop.gh + Y.sq)[:Y.n]]
        if not p.balanced:
            q.append((hk.half_step(X, Y, loop.gh, s.c1, use_off=False) + X.sq)[:X.n])
            q.append((hk.half_step(Y, X, loop.fh, s.c1, use_off=False) + Y.sq)[:Y.n])
        spans.append((len(parts), X.n, Y.n))
        parts.extend(q)
    host = torch.cat(parts).to("cpu", torch.float64).numpy()
    out, pos = [], 0
    for (p, _, st), (_, n, m) in zip(zip(ps, setups, states), spans):
        f, g = host[pos:pos + n], host[pos + n:pos + n + m]
        pos += n + m
        fb = gb = None
        if not p.balanced:
            fb, gb = host[pos:pos + n], host[pos + n:pos + n + m]
            pos += n + m
        out.append((f, g, fb, gb, int(st.it), float(st.err), bool(st.converged)))
    return out


def _solve_hip(p, opts: SinkhornOptions):
    dev = _gpu_device(opts)
    with torch.cuda.device(dev):
        s = _hip_setup(p, opts, dev)
        t0 = time.perf_counter()
        st = s.loop.run()
        f, g, fb, gb, it, err, converged = _hip_finish(p, s, st)
    return f, g, fb, gb, it, err, converged, t0


def _use_hip(opts: SinkhornOptions, d: int) -> bool:
    """Kernel selection, the counterpart of _use_nki (src/trnopt/sinkhorn.py:196-208). The fused kernels need a
    ROCm GPU, float32 and d <= 128. kernel="hip" outside that is an error; so is a missing kernel library
    whenever the fused kernels are selected (there is no silent fallback)."""
    if opts.kernel not in KERNELS:
        raise ValueError(f"unknown kernel {opts.kernel!r}; choose from {KERNELS}")
    if opts.kernel == "torch":
        return False
    if opts.kernel == "nki":
        raise ValueError("kernel='nki' needs a Neuron device; this build's fused kernel is kernel='hip'")
    from . import hip_sinkhorn as hk
    be = opts.backend
    ok = be.is_rocm_gpu and be.dtype == torch.float32 and hk.pad_dim(d) <= hk.KP_MAX
    if opts.kernel == "hip" and not ok:
        raise ValueError("kernel='hip' needs a ROCm GPU device (Backend.preset('rocm')), float32 and d <= 128")
    if ok:
        hk.lib()                     # ImportError if libtrnopt_hip.so is missing
    return ok


# ---------------------------------------------------------------------------------------------------------
# Inputs, normalisation, driver

def _cloud_dim(x, y) -> int:
    """d of two clouds x (n, d) and y (m, d), checked: 2-D, one d >= 1, at least one point each. (The reference
    fails later on such input, inside numpy or torch; here before any device work.)"""
    sx, sy = np.shape(x), np.shape(y)
    if len(sx) != 2 or len(sy) != 2 or sx[1] != sy[1] or sx[1] < 1:
        raise ValueError(f"x (n, d) and y (m, d) must be 2-D with the same d >= 1, got {sx} and {sy}")
    if sx[0] == 0 or sy[0] == 0:
        raise ValueError(f"x and y need at least one point each, got {sx[0]} and {sy[0]}")
    return int(sx[1])


def _log_weights(w, n: int, name: str) -> np.ndarray:
    if w is None:
        return np.full(n, -np.log(n))
    w = np.asarray(w, dtype=np.float64)
    if w.shape != (n,) or np.any(w <= 0):
        raise ValueError(f"{name} must be {n} positive weights")
    return np.log(w)


def normalization(x: np.ndarray, y: np.ndarray, samples: int = 20_000, seed: int = 0,
                  how: str = "mean", device=None) -> tuple[np.ndarray, float]:
    """(center, cost_scale) as the reference computes them (src/trnopt/sinkhorn.py:220-238): center = mean of all
    points; cost_scale = the mean squared x-y distance over `samples` random pairs (rng seed `seed`), or with
    how="median" the median over all pairs when n m <= 1e8 (else over the random pairs). 1 if that is 0.

    device: a ROCm GPU device to take the exact median there (sk_cost_median_f64: radix select over the cost
    recomputed on the fly, no n x m array); None computes it on the host like the reference."""
    x = np.asarray(x, dtype=np.float64)
    y = np.asarray(y, dtype=np.float64)
    center = np.concatenate([x, y]).mean(axis=0)
    if how == "median" and len(x) * len(y) <= 100_000_000:
        xc, yc = x - center, y - center
        if device is not None:
            from . import hip_sinkhorn as hk
            scale = hk.cost_median(xc, yc, device)
            return center, (scale if scale > 0 else 1.0)
        C = ((xc * xc).sum(1)[:, None] + (yc * yc).sum(1)[None, :] - 2.0 * (xc @ yc.T)).ravel()
        scale = float(np.median(np.maximum(C, 0.0)))
    else:
        rng = np.random.default_rng(seed)
        i, j = rng.integers(len(x), size=samples), rng.integers(len(y), size=samples)
        dd = ((x[i] - y[j]) ** 2).sum(axis=1)
        scale = float(np.median(dd) if how == "median" else dd.mean())
    return center, (scale if scale > 0 else 1.0)


def median_normalizations(pairs, device, samples: int = 20_000, seed: int = 0) -> list:
    """normalization(x, y, how="median", device=device) for every (x, y) of `pairs`, the exact medians of all of
    them enqueued on the GPU and read back with one synchronisation (a pipeline's pairs, each otherwise a round
    trip of its own). The same (center, cost_scale) as the one-pair call, pair by pair."""
    from . import hip_sinkhorn as hk
    out, pending = [], []
    for x, y in pairs:
        x = np.asarray(x, dtype=np.float64)
        y = np.asarray(y, dtype=np.float64)
        if len(x) * len(y) > 100_000_000:
            out.append(normalization(x, y, samples=samples, seed=seed, how="median", device=device))
            continue
        center = np.concatenate([x, y]).mean(axis=0)
        pending.append((len(out), hk.cost_median_enqueue(x - center, y - center, device)))
        out.append(center)
    if pending:
        scales = torch.cat([t for _, t in pending]).cpu().numpy()
        for (k, _), scale in zip(pending, scales):
            out[k] = (out[k], float(scale) if scale > 0 else 1.0)
    return out


def _gpu_device(opts: SinkhornOptions):
    dev = torch.device(opts.backend.device)
    return torch.device("cuda", torch.cuda.current_device()) if dev.index is None else dev


def _prepare(x, y, a, b, opts: SinkhornOptions, a_target, b_target, hip: bool = False):
    """Validation, weights, normalisation and the eps schedule (src/trnopt/sinkhorn.py:250-320, 340-344). With
    the HIP path selected, an exact median normalisation runs on the GPU."""
    be = opts.backend
    x = np.asarray(x, dtype=np.float64)
    y = np.asarray(y, dtype=np.float64)
    _cloud_dim(x, y)
    log_a, log_b = _log_weights(a, len(x), "a"), _log_weights(b, len(y), "b")
    balanced = opts.rho is None
    if balanced and abs(np.exp(log_a).sum() - np.exp(log_b).sum()) > 1e-9 * np.exp(log_a).sum():
        raise ValueError("balanced OT needs sum(a) == sum(b); pass rho for unbalanced")
    if balanced and (a_target is not None or b_target is not None):
        raise ValueError("a_target / b_target are for unbalanced OT (pass rho)")
    if balanced:
        rho_x = rho_y = None
    elif isinstance(opts.rho, (tuple, list)):
        rho_x, rho_y = tuple(opts.rho)
    else:
        rho_x = rho_y = opts.rho
    off_x = None if a_target is None else _log_weights(a_target, len(x), "a_target") - log_a
    off_y = None if b_target is None else _log_weights(b_target, len(y), "b_target") - log_b
    if isinstance(opts.normalize, tuple):
        center, scale = np.asarray(opts.normalize[0], dtype=np.float64), float(opts.normalize[1])
    elif opts.normalize:
        how = opts.normalize if isinstance(opts.normalize, str) else "mean"
        center, scale = normalization(x, y, how=how,
                                      device=_gpu_device(opts) if hip and x.shape[1] <= 128 else None)
    else:
        center, scale = np.zeros(x.shape[1]), 1.0
    root = np.sqrt(scale)
    if np.any(center != 0.0) or root != 1.0:
        xs, ys = (x - center) / root, (y - center) / root
    else:                                   # (x - 0) / 1 is x exactly: no copies
        xs, ys = x, y
    stages = [e for e in (opts.eps_stages or ()) if e > opts.eps]
    sched = []
    if not stages and opts.eps_start is not None and opts.eps_start > opts.eps:
        e = opts.eps_start
        while e > opts.eps and len(sched) < opts.max_iters:
            sched.append(e)
            e *= opts.eps_decay
    f32 = be.dtype == torch.float32
    # float32 rounding noise in the potentials' change sits near 1e-6 of eps: floor the thresholds (:340-344)
    stage_tol = max(opts.stage_tol, 1e-5 if f32 else 0.0)
    tol = max(opts.tol, 5e-6) if (f32 and not balanced) else opts.tol
    return SimpleNamespace(x=x, y=y, xs=xs, ys=ys, log_a=log_a, log_b=log_b, off_x=off_x, off_y=off_y,
                           rho_x=rho_x, rho_y=rho_y, balanced=balanced, center=center, scale=scale,
                           stages=stages, sched=sched, tol=tol, stage_tol=stage_tol)


def sinkhorn(x, y, a=None, b=None, opts: SinkhornOptions | None = None, a_target=None,
             b_target=None) -> SinkhornResult:
    """Entropic OT between clouds x (n, d) and y (m, d) with weights a, b (default uniform).

    a, b are the reference measure of the entropy term eps KL(P | a b^T). Unbalanced (rho given), the penalties
    rho KL(P 1 | a_target) and rho KL(P^T 1 | b_target) pull the plan's sums toward a_target and b_target (default
    a and b): wot's formulation is a uniform reference, a_target = growth / I, b_target = mean growth / J."""
    opts = opts or SinkhornOptions()
    hip = _use_hip(opts, _cloud_dim(x, y))
    p = _prepare(x, y, a, b, opts, a_target, b_target, hip)
    if max(1, int(opts.cores)) > 1:
        raise ValueError("cores > 1 split rows across NeuronCores in the reference; this build runs on one GPU")
    if hip:
        f, g, fb, gb, it, err, converged, t0 = _solve_hip(p, opts)
    else:
        f, g, fb, gb, it, err, converged, t0 = _solve_torch(p, opts)
    return _result(p, opts, f, g, fb, gb, it, err, converged, t0)


def _result(p, opts: SinkhornOptions, f, g, fb, gb, it, err, converged, t0) -> SinkhornResult:
    row_mass = col_mass = None
    if not p.balanced:
        # the plan's marginals: row_i = a_i exp((f_i - fb_i) / eps), fb one balanced f update from g
        row_mass = np.exp(p.log_a + (f - fb) / opts.eps)
        col_mass = np.exp(p.log_b + (g - gb) / opts.eps)
    seconds = time.perf_counter() - t0
    cost = float(np.exp(p.log_a) @ f + np.exp(p.log_b) @ g) if p.balanced else float("nan")
    return SinkhornResult(f=f, g=g, iterations=it, error=err, converged=converged, cost=cost, seconds=seconds,
                          eps=opts.eps, rho=opts.rho, center=p.center, cost_scale=p.scale, row_mass=row_mass,
                          col_mass=col_mass)


def sinkhorn_batch(problems) -> list:
    """sinkhorn() for several independent problems at once on the fused path: `problems` is a list of dicts of
    sinkhorn()'s arguments (x, y and optionally a, b, opts, a_target, b_target), all with kernel "hip" selected (or
    "auto" on a ROCm GPU), one device and one d. Their loops run together (DeviceLoopBatch: each launch one pass of
    every problem, on the GPU's workgroups in proportion to each problem's work), so that problems too small to
    fill the GPU alone share it. Each result is sinkhorn()'s for its problem to float32 rounding (the partial
    sums of a half-step are split over fewer workgroups; with one problem, bit for bit); `seconds` is the whole
    batch's time. The reference solves such problems one after another (examples/singlecell_wot.py:84-89)."""
    problems = list(problems)
    return _HipBatch(problems).solve() if problems else []


class _HipBatch:
    """The problems of sinkhorn_batch, prepared, packed and set up once, then solved together, again whenever
    asked with new marginal targets (wot's growth iterations: the same points, weights, normalisation and
    options, only the targets change): each solve writes the new target offsets into the packed clouds and starts
    every loop afresh (potentials zero, state initialised)."""

    def __init__(self, problems):
        from . import hip_sinkhorn as hk
        prepared = []
        for q in problems:
            opts = q.get("opts") or SinkhornOptions()
            if not _use_hip(opts, _cloud_dim(q["x"], q["y"])):
                raise ValueError("sinkhorn_batch runs the fused kernels: kernel 'hip' on a ROCm GPU, float32, d <= 128")
            if max(1, int(opts.cores)) > 1:
                raise ValueError("cores > 1 split rows across NeuronCores in the reference; this build runs on one GPU")
            p = _prepare(q["x"], q["y"], q.get("a"), q.get("b"), opts, q.get("a_target"), q.get("b_target"), True)
            prepared.append((p, opts))
        if len({str(_gpu_device(o)) for _, o in prepared}) != 1 or len({p.xs.shape[1] for p, _ in prepared}) != 1:
            raise ValueError("sinkhorn_batch: every problem must run on one device with one d")
        self.prepared = prepared
        self.dev = dev = _gpu_device(prepared[0][1])
        with torch.cuda.device(dev):
            states = hk.DeviceLoopBatch.state_block(len(prepared), dev)
            self.setups = [_hip_setup(p, o, dev, state=states[k]) for k, (p, o) in enumerate(prepared)]
            self.batch = hk.DeviceLoopBatch([su.loop for su in self.setups], states)
        self._fresh = True

    def solve(self, targets=None) -> list:
        """Solve every problem; targets: one (a_target, b_target) per problem replacing its own (both given where
        the problem had them), or None for the problems as given."""
        offs = None
        if targets is not None:
            targets = list(targets)
            if len(targets) != len(self.prepared):
                raise ValueError(f"solve(targets): {len(targets)} targets for {len(self.prepared)} problems")
            # every target checked before any problem's offsets change
            offs = []
            for (p, _), (at, bt) in zip(self.prepared, targets):
                if p.off_x is None or p.off_y is None:
                    raise ValueError("solve(targets): the problem was made without marginal targets")
                offs.append((_log_weights(at, len(p.xs), "a_target") - p.log_a,
                             _log_weights(bt, len(p.ys), "b_target") - p.log_b))
        with torch.cuda.device(self.dev):
            if offs is not None:
                for (p, _), su, (ox, oy) in zip(self.prepared, self.setups, offs):
                    p.off_x, p.off_y = ox, oy
                    su.X.set_off(ox)
                    su.Y.set_off(oy)
            if not self._fresh:
                for su in self.setups:
                    su.loop.fh.zero_()
                    su.loop.gh.zero_()              # g0 = |y|^2 (sinkhorn.py:336)
            self._fresh = False
            t0 = time.perf_counter()
            sts = self.batch.run()
            fin = _hip_finish_many([p for p, _ in self.prepared], self.setups, sts)
            return [_result(p, o, *r, t0) for (p, o), r in zip(self.prepared, fin)]


def transport_plan(x, y, res: SinkhornResult, a=None, b=None) -> np.ndarray:
    """The dense plan P (n x m, float64) of a result, for small problems and tests (src/trnopt/sinkhorn.py:397-403)."""
    root = np.sqrt(res.cost_scale)
    x = (np.asarray(x, dtype=np.float64) - res.center) / root
    y = (np.asarray(y, dtype=np.float64) - res.center) / root
    log_a, log_b = _log_weights(a, len(x), "a"), _log_weights(b, len(y), "b")
    C = ((x[:, None, :] - y[None, :, :]) ** 2).sum(axis=2)
    return np.exp(log_a[:, None] + log_b[None, :] + (res.f[:, None] + res.g[None, :] - C) / res.eps)
