"""Waddington-OT transport maps between consecutive time points, solved with this package's Sinkhorn.

The interface of the reference's src/trnopt/singlecell.py (wot, Schiebinger et al. 2019, OTModel defaults):

* input: each time point's cells in a per-pair embedding (the reference computes it with sklearn PCA from the
  expression data, src/trnopt/singlecell.py:30-43; that step needs the data and is left to the caller);
* cost: squared Euclidean distance divided by its median (normalize="median"), computed once per pair;
* formulation: uniform reference (1/I, 1/J), row target G / I (the cells' growth), column target
  mean(G) / J, KL penalties (lambda1, lambda2), entropy eps;
* eps stages as wot's duality-gap solver: eps0 * sf^-e for e = 0 .. scalings - 1, sf = eps^(-1/scalings);
* growth_iters: re-solve with the row target set to the previous plan's row sums (wot's learned growth).

wot's tmap is I * P, whose rows sum to the learned growth I * row_mass.

save_pair / load_pair write and read the per-pair result file of the reference's pipeline
(examples/singlecell_wot.py:112-117: f, g, eps, center, cost_scale, row_mass, col_mass, learned_growth,
cells0, cells1, x0, x1), with the cell names stored as fixed-width strings so the file loads without pickle;
pair_result turns a loaded file back into a SinkhornResult for trnopt.plan.
"""

from __future__ import annotations

import time
from dataclasses import dataclass, replace

import numpy as np

from .sinkhorn import (SinkhornOptions, SinkhornResult, _cloud_dim, _gpu_device, _use_hip, normalization, sinkhorn,
                       transport_plan)

PAIR_KEYS = ("f", "g", "eps", "center", "cost_scale", "row_mass", "col_mass", "learned_growth", "cells0",
             "cells1", "x0", "x1")


def wot_eps_stages(eps: float, eps0: float = 1.0, scalings: int = 5) -> tuple:
    """The intermediate eps values of wot's solver (src/trnopt/singlecell.py:46-50); the last stage is eps."""
    sf = np.exp(-np.log(eps) / scalings)
    return tuple(float(eps0 / sf ** e) for e in range(scalings))


@dataclass
class TransportMap:
    result: SinkhornResult             # the last growth iteration's solve
    learned_growth: list               # per growth iteration, the row target used (wot's G)
    seconds: float                     # median normalisation + all solves
    iterations: int                    # Sinkhorn iterations over all growth iterations


def wot_transport_map(x0: np.ndarray, x1: np.ndarray, growth: np.ndarray | None = None, delta_days: float = 1.0,
                      eps: float = 0.05, lambda1: float = 1.0, lambda2: float = 50.0, growth_iters: int = 1,
                      tol: float = 1e-6, stage_tol: float = 1e-6, opts: SinkhornOptions | None = None) -> TransportMap:
    """One wot transport map between x0 (I cells) and x1 (J cells) (src/trnopt/singlecell.py:61-86). opts
    supplies backend, kernel, check_every and max_iters; eps, rho, normalize and the stages are set here."""
    w = _WotPair(x0, x1, growth, delta_days, eps, lambda1, lambda2, tol, stage_tol, opts)
    for _ in range(growth_iters):
        t = time.perf_counter()
        w.take(sinkhorn(**w.problem()), time.perf_counter() - t)
    return w.transport_map()


class _WotPair:
    """One pair's wot solve across its growth iterations (src/trnopt/singlecell.py:61-86): the median
    normalisation once, then per growth iteration the problem for sinkhorn() and the learned growth from its
    result."""

    def __init__(self, x0, x1, growth, delta_days, eps, lambda1, lambda2, tol, stage_tol, opts, norm=None,
                 norm_seconds=0.0):
        self.x0, self.x1 = x0, x1
        self.I, self.J = I, J = len(x0), len(x1)
        self.G = np.ones(I) if growth is None else np.power(np.asarray(growth, dtype=np.float64), delta_days)
        opts = opts or SinkhornOptions()
        d = _cloud_dim(x0, x1)
        hip = _use_hip(opts, d)
        t = time.perf_counter()
        # once per pair (the cost does not change across growth iterations); on the GPU when the fused path runs
        # (norm: already taken, with several pairs' medians at once, in norm_seconds)
        if norm is None:
            norm = normalization(x0, x1, how="median",
                                 device=_gpu_device(opts) if hip and d <= 128 else None)
        self.seconds = time.perf_counter() - t + norm_seconds
        self.base = replace(opts, eps=eps, rho=(lambda1, lambda2), normalize=norm, eps_stages=wot_eps_stages(eps),
                            stage_tol=stage_tol, tol=tol, eps_start=None, fixed_iters=False)
        self.a, self.b = np.full(I, 1.0 / I), np.full(J, 1.0 / J)
        self.learned, self.iters, self.res = [], 0, None

    def problem(self) -> dict:
        """sinkhorn()'s arguments for the next growth iteration (the row target from the last result's row sums)."""
        if self.res is not None:
            self.G = self.I * self.res.row_mass
        self.learned.append(self.G)
        return dict(x=self.x0, y=self.x1, a=self.a, b=self.b, opts=self.base, a_target=self.G / self.I,
                    b_target=np.full(self.J, self.G.mean() / self.J))

    def take(self, res: SinkhornResult, seconds: float) -> None:
        self.res = res
        self.seconds += seconds
        self.iters += res.iterations

    def transport_map(self) -> TransportMap:
        return TransportMap(result=self.res, learned_growth=self.learned, seconds=self.seconds, iterations=self.iters)


def wot_transport_maps(pairs, growth=None, delta_days=1.0, streams: int = 4, batch: bool = True, **kw) -> list:
    """wot_transport_map for every (x0, x1) of `pairs` -- the consecutive time points of a pipeline, whose maps
    are independent -- solved together on the GPU (the reference's example runs them one after the other,
    examples/singlecell_wot.py:84-89).

    growth: None or one growth array per pair; delta_days: a number or one per pair; kw: wot_transport_map's
    other arguments (eps, lambda1, lambda2, growth_iters, tol, stage_tol, opts). On the fused path:
      batch=True (default): each growth iteration of every pair in one batched solve (sinkhorn_batch: each launch
        one half-step of every pair, each on its share of the GPU's workgroups), the pairs' maps equal to
        wot_transport_map's to float32 rounding;
      batch=False: up to `streams` pairs in flight, each on its own HIP stream driven by its own host thread; a
        pair's kernels, work split and host steps do not depend on what runs beside it, so every map equals
        wot_transport_map's for that pair bit for bit.
    With streams=1 and batch=False, or on the torch path, the pairs run in order. Returns the TransportMaps in the
    order of `pairs`."""
    import torch
    pairs = list(pairs)
    n = len(pairs)
    growths = [None] * n if growth is None else list(growth)
    days = list(delta_days) if np.ndim(delta_days) else [float(delta_days)] * n
    if len(growths) != n or len(days) != n:
        raise ValueError("growth and delta_days need one entry per pair")
    opts = kw.get("opts") or SinkhornOptions()
    streams = max(1, int(streams))

    def one(k):
        x0, x1 = pairs[k]
        return wot_transport_map(x0, x1, growths[k], days[k], **kw)

    dims = [_cloud_dim(x0, x1) for x0, x1 in pairs]
    fused = n >= 2 and all(_use_hip(opts, d) for d in dims)
    if fused and batch and len(set(dims)) == 1:
        return _wot_maps_batched(pairs, growths, days, **kw)
    if streams == 1 or not fused:
        return [one(k) for k in range(n)]
    import threading
    from concurrent.futures import ThreadPoolExecutor
    from . import hip_sinkhorn as hk
    hk.lib()                                     # loaded once, before the threads
    dev = _gpu_device(opts)
    with torch.cuda.device(dev):
        caller = torch.cuda.current_stream()
        pool = [torch.cuda.Stream() for _ in range(min(streams, n))]
        for s in pool:
            s.wait_stream(caller)
    free, lock, local = list(pool), threading.Lock(), threading.local()

    def run(k):
        if not hasattr(local, "stream"):        # one stream per worker thread, for all its pairs
            with lock:
                local.stream = free.pop()
        with torch.cuda.device(dev), torch.cuda.stream(local.stream):
            return one(k)

    with ThreadPoolExecutor(len(pool)) as ex:
        maps = list(ex.map(run, range(n)))
    for s in pool:
        caller.wait_stream(s)
    return maps


def _wot_maps_batched(pairs, growths, days, eps: float = 0.05, lambda1: float = 1.0, lambda2: float = 50.0,
                      growth_iters: int = 1, tol: float = 1e-6, stage_tol: float = 1e-6,
                      opts: SinkhornOptions | None = None) -> list:
    """wot_transport_maps' batched form: every pair's normalisation, then each growth iteration of all the pairs as
    one batched solve (sinkhorn_batch's), the pairs' clouds prepared and packed once for all growth iterations
    (only the row and column targets change between them). A pair's `seconds` is its normalisation plus the whole
    of each batch it took part in."""
    from .sinkhorn import _HipBatch, median_normalizations
    t = time.perf_counter()
    norms = median_normalizations(pairs, _gpu_device(opts or SinkhornOptions()))
    dt = time.perf_counter() - t
    ws = [_WotPair(x0, x1, growths[k], days[k], eps, lambda1, lambda2, tol, stage_tol, opts, norm=norms[k],
                   norm_seconds=dt) for k, (x0, x1) in enumerate(pairs)]
    batch = None
    for _ in range(growth_iters):
        t = time.perf_counter()
        problems = [w.problem() for w in ws]
        if batch is None:
            batch = _HipBatch(problems)
            results = batch.solve()
        else:
            results = batch.solve([(q["a_target"], q["b_target"]) for q in problems])
        dt = time.perf_counter() - t
        for w, r in zip(ws, results):
            w.take(r, dt)
    return [w.transport_map() for w in ws]


def wot_tmap(x0, x1, tm: TransportMap) -> np.ndarray:
    """The dense map in wot's normalisation (I * P), small pairs only."""
    I, J = len(x0), len(x1)
    return I * transport_plan(x0, x1, tm.result, np.full(I, 1.0 / I), np.full(J, 1.0 / J))


def save_pair(path, tm: TransportMap, x0: np.ndarray, x1: np.ndarray, cells0=None, cells1=None) -> None:
    """Write one pair's result in the reference's format (examples/singlecell_wot.py:112-117). cells0 / cells1
    default to the point indices; every array is numeric or a fixed-width string, so np.load needs no pickle."""
    r = tm.result
    I, J = len(x0), len(x1)
    cells0 = np.arange(I) if cells0 is None else cells0
    cells1 = np.arange(J) if cells1 is None else cells1
    c0, c1 = np.asarray(cells0).astype(str), np.asarray(cells1).astype(str)
    if c0.shape != (I,) or c1.shape != (J,):
        raise ValueError("cells0 / cells1 must name every point of x0 / x1")
    nan = lambda n: np.full(n, np.nan)                                            # noqa: E731
    np.savez(path, f=np.asarray(r.f, np.float64), g=np.asarray(r.g, np.float64), eps=np.float64(r.eps),
             center=np.asarray(r.center, np.float64), cost_scale=np.float64(r.cost_scale),
             row_mass=nan(I) if r.row_mass is None else np.asarray(r.row_mass, np.float64),
             col_mass=nan(J) if r.col_mass is None else np.asarray(r.col_mass, np.float64),
             learned_growth=np.array(tm.learned_growth, dtype=np.float64), cells0=c0, cells1=c1,
             x0=np.asarray(x0, np.float64), x1=np.asarray(x1, np.float64))


def load_pair(path) -> dict:
    """The arrays of a pair file (written by save_pair or by the reference's pipeline), scalars as floats.
    Loads without pickle; a file whose cell names were stored as Python objects needs the reference's own
    np.load(..., allow_pickle=True) instead and is refused here."""
    with np.load(path, allow_pickle=False) as z:
        missing = [k for k in PAIR_KEYS if k not in z.files]
        if missing:
            raise ValueError(f"{path}: not a pair file (missing {missing})")
        out = {k: z[k] for k in PAIR_KEYS}
    out["eps"], out["cost_scale"] = float(out["eps"]), float(out["cost_scale"])
    return out


def pair_result(z: dict) -> SinkhornResult:
    """A SinkhornResult holding a loaded pair's potentials and normalisation (iterations etc. are unknown)."""
    rm = None if np.all(np.isnan(z["row_mass"])) else z["row_mass"]
    cm = None if np.all(np.isnan(z["col_mass"])) else z["col_mass"]
    return SinkhornResult(f=z["f"], g=z["g"], iterations=0, error=float("nan"), converged=True, cost=float("nan"),
                          seconds=0.0, eps=z["eps"], rho=None, center=z["center"], cost_scale=z["cost_scale"],
                          row_mass=rm, col_mass=cm)
