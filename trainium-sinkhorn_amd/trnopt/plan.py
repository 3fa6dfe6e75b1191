"""The plan of a Sinkhorn result without forming it: its marginals and its action on a vector.

P_ij = a_i b_j exp((f_i + g_j - C_ij) / eps) on the result's normalised coordinates (the dense form is
transport_plan, src/trnopt/sinkhorn.py:397-403). Both functions here are log-sum-exps over one side's scores,

    log (P v)_i = log a_i + (f_i - |x_i|^2) / eps + LSE_j((2 x_i . y_j + g_j - |y_j|^2) / eps + log b_j + log v_j),

which is the half-step's log-sum-exp with kappa = 1 and no offset: on the GPU each is one sk_half_step_f32 call
per side (the fused kernel, scores never stored), elsewhere a blocked PyTorch computation in the backend's
dtype. They serve what the reference computes on the host in float64 from saved potentials: the plan's row and
column sums (examples/sinkhorn_libs_compare.py:43-56, and the unbalanced masses of sinkhorn.py:381-389) and
wot's ancestor pull-back p_t0 ∝ P p_t1 (examples/singlecell_figures.py:35-47).
"""

from __future__ import annotations

import numpy as np
import torch

from .sinkhorn import SinkhornOptions, SinkhornResult, _log_weights, _use_hip

_NEG = -1.0e9          # log of a zero weight: exactly zero after exp, finite (src/trnopt/sinkhorn.py:59)


def _normalised(x, y, res: SinkhornResult):
    root = np.sqrt(res.cost_scale)
    x = (np.asarray(x, dtype=np.float64) - res.center) / root
    y = (np.asarray(y, dtype=np.float64) - res.center) / root
    if x.ndim != 2 or y.ndim != 2 or x.shape[1] != y.shape[1]:
        raise ValueError("x (n, d) and y (m, d) must share d")
    if len(res.f) != len(x) or len(res.g) != len(y):
        raise ValueError("the result's potentials do not match x and y")
    return x, y


def _log_vector(v, m: int) -> np.ndarray:
    v = np.asarray(v, dtype=np.float64)
    if v.shape != (m,) or np.any(v < 0) or not np.any(v > 0):
        raise ValueError(f"v must be {m} non-negative values, not all zero")
    with np.errstate(divide="ignore"):
        return np.where(v > 0, np.log(np.where(v > 0, v, 1.0)), _NEG)


def _lse_torch(rows, cols, h_cols, log_w_cols, eps, be, block=2048) -> np.ndarray:
    """LSE_j((2 r_i . c_j + h_j) / eps + log_w_j) for every row, blocked, in the backend's dtype."""
    dev = torch.device(be.device)
    R = torch.as_tensor(rows, dtype=be.dtype, device=dev)
    cT = torch.as_tensor(cols.T.copy(), dtype=be.dtype, device=dev)
    h = torch.as_tensor(h_cols, dtype=be.dtype, device=dev)
    lw = torch.as_tensor(log_w_cols, dtype=be.dtype, device=dev)
    out = np.empty(len(rows))
    for s in range(0, len(rows), block):
        z = (2.0 * (R[s:s + block] @ cT) + h) / eps + lw
        out[s:s + block] = torch.logsumexp(z, dim=1).to("cpu", torch.float64).numpy()
    return out


def _lse_hip(rows, log_w_rows, cols, h_cols, log_w_cols, eps, opts: SinkhornOptions, role: int) -> np.ndarray:
    """The same on the fused kernel: one sk_half_step_f32 with |x|^2 = 0, no offset, kappa = 1, so that its
    output is exactly -eps lse, with the scores in log2 units from the matrix cores (the first cloud's log2-unit
    copy made for this eps first)."""
    from . import hip_sinkhorn as hk
    dev = torch.device(opts.backend.device)
    if dev.index is None:
        dev = torch.device("cuda", torch.cuda.current_device())
    with torch.cuda.device(dev):
        R = hk.HipCloud(rows, log_w_rows, dev, role=role)
        C = hk.HipCloud(cols, log_w_cols, dev, role=1 - role)
        h = torch.zeros(C.npad, dtype=torch.float32, device=dev)
        h[:C.n] = torch.as_tensor(h_cols, dtype=torch.float32)
        R.sq = torch.zeros_like(R.sq)
        out = hk.half_step(R, C, h, hk.scalars(eps, 1.0, dev), use_off=False, log2=True)
        return (-out[:R.n].to("cpu", torch.float64) / eps).numpy()


def _side_lse(rows, log_w_rows, cols, g_cols, log_w_cols, eps, opts, role):
    h = g_cols - (cols * cols).sum(axis=1)          # shifted potential of the column side, float64
    if _use_hip(opts, rows.shape[1]):
        return _lse_hip(rows, log_w_rows, cols, h, log_w_cols, eps, opts, role)
    return _lse_torch(rows, cols, h, log_w_cols, eps, opts.backend)


def plan_marginals(x, y, res: SinkhornResult, a=None, b=None,
                   opts: SinkhornOptions | None = None) -> tuple[np.ndarray, np.ndarray]:
    """Row and column sums (float64) of the plan of `res` between x (n, d) and y (m, d) with weights a, b
    (default uniform), without forming the n x m plan. opts selects backend and kernel as for sinkhorn():
    kernel="hip" (or "auto" on a ROCm GPU) runs two fused half-step launches."""
    opts = opts or SinkhornOptions()
    xs, ys = _normalised(x, y, res)
    log_a, log_b = _log_weights(a, len(xs), "a"), _log_weights(b, len(ys), "b")
    f, g, eps = np.asarray(res.f, np.float64), np.asarray(res.g, np.float64), float(res.eps)
    lse_r = _side_lse(xs, log_a, ys, g, log_b, eps, opts, role=0)
    lse_c = _side_lse(ys, log_b, xs, f, log_a, eps, opts, role=1)
    rows = np.exp(log_a + (f - (xs * xs).sum(axis=1)) / eps + lse_r)
    cols = np.exp(log_b + (g - (ys * ys).sum(axis=1)) / eps + lse_c)
    return rows, cols


def pull_back(x, y, res: SinkhornResult, v, a=None, b=None, opts: SinkhornOptions | None = None) -> np.ndarray:
    """log of P v, normalised to a distribution over x's points (log p with sum p = 1): wot's ancestor step
    p_t0 ∝ T_t0,t1 p_t1 for a distribution v (m,) on y's points. With uniform a, b it is the reference's
    pull_back_potentials (examples/singlecell_figures.py:35-47)."""
    opts = opts or SinkhornOptions()
    xs, ys = _normalised(x, y, res)
    log_a, log_b = _log_weights(a, len(xs), "a"), _log_weights(b, len(ys), "b")
    log_bv = np.maximum(log_b + _log_vector(v, len(ys)), _NEG)
    f, g, eps = np.asarray(res.f, np.float64), np.asarray(res.g, np.float64), float(res.eps)
    lse = _side_lse(xs, log_a, ys, g, log_bv, eps, opts, role=0)
    out = log_a + (f - (xs * xs).sum(axis=1)) / eps + lse
    mx = out.max()
    return out - (mx + np.log(np.exp(out - mx).sum()))
