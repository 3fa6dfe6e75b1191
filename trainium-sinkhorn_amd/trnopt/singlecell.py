"""Waddington-OT transport maps between consecutive time points, solved with this package's Sinkhorn.

The interface of the reference's src/trnopt/singlecell.py (wot, Schiebinger et al. 2019, OTModel defaults):

* local_pca_coords: per pair, PCA of both time points' centred expression (sklearn PCA on the transpose),
  components scaled by the singular values (wot.ot.compute_pca + compute_default_cost_matrix);
* cost: squared Euclidean distance divided by its median (normalize="median"), computed once per pair;
* formulation: uniform reference (1/I, 1/J), row target G / I (the cells' growth), column target
  mean(G) / J, KL penalties (lambda1, lambda2), entropy eps;
* eps stages as wot's duality-gap solver: eps0 * sf^-e for e = 0 .. scalings - 1, sf = eps^(-1/scalings);
* growth_iters: re-solve with the row target set to the previous plan's row sums (wot's learned growth).

wot's tmap is I * P, whose rows sum to the learned growth I * row_mass.
"""

from __future__ import annotations

import time
from dataclasses import dataclass, replace

import numpy as np

from .sinkhorn import SinkhornOptions, SinkhornResult, normalization, sinkhorn, transport_plan


def local_pca_coords(X0, X1, n_components: int = 30) -> tuple[np.ndarray, np.ndarray]:
    """wot's per-pair embedding (src/trnopt/singlecell.py:30-43): (cells0 x k, cells1 x k)."""
    import scipy.sparse as sp
    from sklearn.decomposition import PCA
    a = X0.toarray() if sp.issparse(X0) else np.asarray(X0)
    b = X1.toarray() if sp.issparse(X1) else np.asarray(X1)
    both = np.vstack([a, b]).astype(np.float64)
    both -= both.mean(axis=0)
    k = min(n_components, both.shape[0])
    pca = PCA(n_components=k, random_state=58951).fit(both.T)
    coords = pca.components_.T * pca.singular_values_[None, :]
    return coords[:len(a)], coords[len(a):]


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
    I, J = len(x0), len(x1)
    G = np.ones(I) if growth is None else np.power(np.asarray(growth, dtype=np.float64), delta_days)
    t = time.perf_counter()
    norm = normalization(x0, x1, how="median")
    seconds = time.perf_counter() - t
    base = replace(opts or SinkhornOptions(), eps=eps, rho=(lambda1, lambda2), normalize=norm,
                   eps_stages=wot_eps_stages(eps), stage_tol=stage_tol, tol=tol, eps_start=None, fixed_iters=False)
    a, b = np.full(I, 1.0 / I), np.full(J, 1.0 / J)
    learned, iters, res = [], 0, None
    for i in range(growth_iters):
        if i > 0:
            G = I * res.row_mass
        learned.append(G)
        t = time.perf_counter()
        res = sinkhorn(x0, x1, a, b, base, a_target=G / I, b_target=np.full(J, G.mean() / J))
        seconds += time.perf_counter() - t
        iters += res.iterations
    return TransportMap(result=res, learned_growth=learned, seconds=seconds, iterations=iters)


def wot_tmap(x0, x1, tm: TransportMap) -> np.ndarray:
    """The dense map in wot's normalisation (I * P), small pairs only."""
    I, J = len(x0), len(x1)
    return I * transport_plan(x0, x1, tm.result, np.full(I, 1.0 / I), np.full(J, 1.0 / J))
