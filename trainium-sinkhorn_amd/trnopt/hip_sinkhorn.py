"""The fused Sinkhorn half-step on AMD Instinct MI355X (gfx950): ctypes binding of libtrnopt_hip.so.

This module plays the part nki_sinkhorn.py plays in the reference (src/trnopt/nki_sinkhorn.py): it holds the
device kernels' entry points and their calling conventions, and sinkhorn.py dispatches to it. The kernels
are hand-written HIP (trainium-sinkhorn_amd/csrc), built ahead of time by trnopt._build into
trnopt/_lib/libtrnopt_hip.so; nothing here compiles at run time. The C ABI is declared in
include/trnopt_hip.h.

What the kernels compute (same as the NKI kernels, src/trnopt/nki_sinkhorn.py:5-22):

    row_lse:    lse_i = log sum_j exp(xa_i . ya_j)
    half_step:  fh_i = kappa * (|x_i|^2 + eps * off_i - eps * lse_i) - |x_i|^2,
                lse_i = LSE_j((2 x_i . y_j + gh_j) / eps + log b_j)

without materialising the scores. On top of that, DeviceLoop runs the whole Sinkhorn iteration loop of
src/trnopt/sinkhorn.py:346-378 on the device (eps schedule / stages, convergence checks), and the host
only reads the loop state back once per batch of iterations.

Memory comes from PyTorch (device tensors, the caching allocator), work goes on PyTorch's current stream.
If the library is missing every entry point raises: there is no fallback to another implementation.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import numpy as np
import torch

PAD_LOG_WEIGHT = -1e9                    # src/trnopt/sinkhorn.py:59
TILE = 32                                 # SK_TILE
KP_ALIGN = 16                             # SK_KP_ALIGN
KP_MAX = 128                              # SK_KP_MAX
PACKED_BYTES_PER_COORD = 8                # SK_PACKED_BYTES_PER_COORD: two fp16 pieces, own scale and log2 copy
PACKED_HEADER_BYTES = 256                 # SK_PACKED_HEADER_BYTES
MAX_ABS_COORDINATE = 7.0e13               # larger coordinates do not fit the kernels' scaled fp16 pieces
LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libtrnopt_hip.so"

_c_float_p = ctypes.c_void_p             # device pointers travel as integers


class SkCloud(ctypes.Structure):
    _fields_ = [("pk", ctypes.c_void_p), ("sq", ctypes.c_void_p), ("log_w", ctypes.c_void_p),
                ("w", ctypes.c_void_p), ("off", ctypes.c_void_p), ("n", ctypes.c_int), ("npad", ctypes.c_int),
                ("log_w_lo", ctypes.c_void_p)]


class SkState(ctypes.Structure):
    _fields_ = [("eps", ctypes.c_double), ("err", ctypes.c_double), ("it", ctypes.c_int),
                ("stage", ctypes.c_int), ("stage_it", ctypes.c_int), ("done", ctypes.c_int),
                ("converged", ctypes.c_int), ("checks", ctypes.c_int),
                ("sc_x", ctypes.c_float * 4), ("sc_y", ctypes.c_float * 4)]


class SkLoop(ctypes.Structure):
    _fields_ = [("x", SkCloud), ("y", SkCloud), ("d", ctypes.c_int),
                ("fh", ctypes.c_void_p), ("gh", ctypes.c_void_p), ("state", ctypes.c_void_p),
                ("sched", ctypes.c_void_p), ("n_sched", ctypes.c_int),
                ("stages", ctypes.c_void_p), ("n_stages", ctypes.c_int),
                ("eps", ctypes.c_double), ("rho_x", ctypes.c_double), ("rho_y", ctypes.c_double),
                ("tol", ctypes.c_double), ("stage_tol", ctypes.c_double),
                ("max_iters", ctypes.c_int), ("check_every", ctypes.c_int), ("stage_max_iters", ctypes.c_int),
                ("fixed_iters", ctypes.c_int), ("balanced", ctypes.c_int),
                ("ws", ctypes.c_void_p), ("ws_bytes", ctypes.c_size_t)]


# name -> (restype, argtypes); the exported symbols of include/trnopt_hip.h
_SIGS = {
    "sk_version": (ctypes.c_int, []),
    "sk_last_error": (ctypes.c_char_p, []),
    "sk_pad_points": (ctypes.c_int, [ctypes.c_int]),
    "sk_pad_dim": (ctypes.c_int, [ctypes.c_int]),
    "sk_packed_bytes": (ctypes.c_size_t, [ctypes.c_int, ctypes.c_int]),
    "sk_pack_cloud_f32": (ctypes.c_int, [_c_float_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                         ctypes.c_void_p]),
    "sk_bake_log2_f32": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, _c_float_p,
                                        ctypes.c_void_p]),
    "sk_row_lse_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    "sk_row_lse_f32": (ctypes.c_int, [_c_float_p, _c_float_p, _c_float_p, ctypes.c_int, ctypes.c_int,
                                      ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "sk_half_step_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    "sk_half_step_meas_count": (ctypes.c_int, [ctypes.c_int]),
    "sk_half_step_f32": (ctypes.c_int, [ctypes.c_void_p, _c_float_p, _c_float_p, ctypes.c_int, ctypes.c_void_p,
                                        _c_float_p, _c_float_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, _c_float_p,
                                        ctypes.c_void_p, _c_float_p, _c_float_p, _c_float_p, ctypes.c_int,
                                        ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "sk_half_step_noalloc_f32": (ctypes.c_int, [ctypes.c_void_p, _c_float_p, _c_float_p, ctypes.c_int, ctypes.c_void_p,
                                                _c_float_p, _c_float_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                                _c_float_p, ctypes.c_void_p, _c_float_p, _c_float_p, _c_float_p,
                                                ctypes.c_int, ctypes.c_void_p]),
    "sk_loop_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    "sk_loop_init_f32": (ctypes.c_int, [ctypes.POINTER(SkLoop), ctypes.c_void_p]),
    "sk_loop_run_f32": (ctypes.c_int, [ctypes.POINTER(SkLoop), ctypes.c_int, ctypes.c_void_p]),
    "sk_loop_batch_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int]),
    "sk_loop_batch_plan": (ctypes.c_int, [ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int), ctypes.c_int,
                                          ctypes.c_int, ctypes.POINTER(ctypes.c_int)]),
    "sk_loop_batch_init_f32": (ctypes.c_int, [ctypes.POINTER(ctypes.POINTER(SkLoop)), ctypes.c_int, ctypes.c_void_p,
                                              ctypes.c_size_t, ctypes.POINTER(ctypes.c_int), ctypes.c_void_p]),
    "sk_loop_run_batch_f32": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.POINTER(ctypes.c_int),
                                             ctypes.c_int, ctypes.c_void_p]),
    "sk_cost_median_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    "sk_cost_median_f64": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                          ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
}
SYMBOLS = tuple(_SIGS)

_lib = None
_load_error: str | None = None


def _load():
    """The library at LIB_PATH, or the build named by TRNOPT_HIP_LIBRARY (another build of the same sources,
    e.g. to compare two versions)."""
    global _lib, _load_error
    if _lib is not None or _load_error is not None:
        return _lib
    path = Path(os.environ.get("TRNOPT_HIP_LIBRARY", str(LIB_PATH)))
    if not path.exists():
        _load_error = f"{path} is not built (run trnopt._build.build() or __graft_entry__.build())"
        return None
    try:
        lib = ctypes.CDLL(str(path))
        for name, (res, args) in _SIGS.items():
            fn = getattr(lib, name)
            fn.restype, fn.argtypes = res, args
    except OSError as e:                 # pragma: no cover - depends on the machine
        _load_error = f"cannot load {path}: {e}"
        return None
    _lib = lib
    return lib


def available() -> bool:
    """True if libtrnopt_hip.so is built and loads (says nothing about a GPU being present)."""
    return _load() is not None


def lib():
    """The loaded library; raises ImportError (naming the reason) if it is not there."""
    lb = _load()
    if lb is None:
        raise ImportError(f"the HIP kernels are not available: {_load_error}")
    return lb


def _check(status: int, what: str) -> None:
    if status != 0:
        msg = lib().sk_last_error().decode(errors="replace")
        if status < 0:
            raise ValueError(f"{what}: {msg} (status {status})")
        raise RuntimeError(f"{what}: {msg} (hipError {status})")


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def pad_points(n: int) -> int:
    return -(-n // TILE) * TILE


def pad_dim(d: int) -> int:
    return -(-d // KP_ALIGN) * KP_ALIGN


def _require_device_f32(name: str, t: torch.Tensor, numel: int | None = None) -> None:
    if not isinstance(t, torch.Tensor) or t.device.type != "cuda" or t.dtype != torch.float32:
        raise ValueError(f"{name} must be a float32 tensor on the GPU")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if numel is not None and t.numel() < numel:
        raise ValueError(f"{name} has {t.numel()} elements, needs {numel}")


def _workspace(nbytes: int, device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=device)


# ---------------------------------------------------------------------------------------------------------
# Kernel-level entry points (the NKI module's make_row_lse_kernel / make_half_step_kernel)

def packed_bytes(n: int, d: int) -> int:
    return PACKED_HEADER_BYTES + pad_points(n) * pad_dim(d) * PACKED_BYTES_PER_COORD


def _check_range(name: str, max_abs: float) -> None:
    if not np.isfinite(max_abs) or max_abs > MAX_ABS_COORDINATE:
        raise ValueError(f"{name}: coordinates must be finite with |x| <= {MAX_ABS_COORDINATE:g} "
                         f"(max |x| = {max_abs:g})")


def pack_cloud(pts: torch.Tensor) -> torch.Tensor:
    """(n, d) float32 device points -> the packed layout as bytes (packed_bytes(n, d),): a header with the
    cloud's power-of-two scale, then each scaled coordinate as two fp16 pieces."""
    _require_device_f32("pts", pts)
    if pts.dim() != 2:
        raise ValueError("pts must be (n, d)")
    n, d = pts.shape
    if pad_dim(d) > KP_MAX:
        raise ValueError(f"d = {d} is above the kernels' limit ({KP_MAX})")
    out = torch.empty(packed_bytes(n, d), dtype=torch.uint8, device=pts.device)
    _check(lib().sk_pack_cloud_f32(pts.data_ptr(), n, d, pts.stride(0), out.data_ptr(), _stream()),
           "sk_pack_cloud_f32")
    return out


def row_lse(xa: torch.Tensor, ya: torch.Tensor) -> torch.Tensor:
    """lse_i = log sum_j exp(xa_i . ya_j) for xa (rows, K), ya (m, K) float32 on the GPU.

    Replaces make_row_lse_kernel(K, rows, m)(xa_T, ya_T) (src/trnopt/nki_sinkhorn.py:150-172); takes the
    row-major (rows, K) / (m, K) arrays instead of their transposes."""
    _require_device_f32("xa", xa)
    _require_device_f32("ya", ya)
    if xa.dim() != 2 or ya.dim() != 2 or xa.shape[1] != ya.shape[1]:
        raise ValueError("xa (rows, K) and ya (m, K) must share K")
    rows, K = xa.shape
    m = ya.shape[0]
    if rows and m:
        _check_range("xa", float(xa.abs().max()))
        _check_range("ya", float(ya.abs().max()))
    lb = lib()
    ws = _workspace(lb.sk_row_lse_workspace_bytes(rows, m, K), xa.device)
    out = torch.empty(rows, dtype=torch.float32, device=xa.device)
    _check(lb.sk_row_lse_f32(xa.data_ptr(), ya.data_ptr(), out.data_ptr(), rows, m, K, ws.data_ptr(), ws.numel(),
                             _stream()), "sk_row_lse_f32")
    return out


def scalars(eps: float, kappa: float, device) -> torch.Tensor:
    """{2/eps, 1/eps, eps, kappa}: each computed in double and rounded once to float32, as consts() does
    (src/trnopt/sinkhorn.py:331-332)."""
    return torch.tensor([2.0 / eps, 1.0 / eps, eps, kappa], dtype=torch.float32, device=device)


class HipCloud:
    """One point cloud on the GPU in the kernels' layout: the counterpart of _Cloud (src/trnopt/sinkhorn.py:131-167).

    Padded to a multiple of 32 points with log weight PAD_LOG_WEIGHT (weight exactly 0) and zero coordinates,
    |p|^2 summed in float64 and cast, coordinates packed once (they never change during a solve). `role` is 0
    for the first cloud of a solve (x) and 1 for the second (y): a half-step with this cloud as rows passes it
    to the kernel, so that the f and g updates form bit-identical x_i . y_j."""

    def __init__(self, pts: np.ndarray, log_w: np.ndarray, device, off: np.ndarray | None = None, role: int = 0):
        n, d = pts.shape
        if pad_dim(d) > KP_MAX:
            raise ValueError(f"d = {d} is above the HIP kernels' limit (d <= {KP_MAX})")
        if role not in (0, 1):
            raise ValueError("role must be 0 (first cloud) or 1 (second cloud)")
        pts = np.asarray(pts, dtype=np.float64)
        _check_range("points", max(float(pts.max()), -float(pts.min())) if pts.size else 0.0)   # no |pts| copy
        npad = pad_points(n)
        self.n, self.npad, self.d, self.device, self.role = n, npad, d, device, role
        # |p|^2 (float64 sums), log w, w, the low part of log w and the offset in one host array and one copy to
        # the device; padding points have |p|^2 = 0, log weight PAD_LOG_WEIGHT (weight exactly 0) and no offset.
        # log_w_lo = log w - fp32(log w) lets the on-device loop carry the log weights to float64 precision, so
        # that the two marginals' total masses agree (a mismatch of a few 1e-8 from fp32 log weights moves a
        # balanced iteration's potentials by eps times it per iteration).
        vec = np.zeros((4 if off is None else 5, npad), dtype=np.float32)
        vec[0, :n] = np.einsum("ij,ij->i", pts, pts)   # float64 sums, as the reference's, then cast
        L = np.full(npad, PAD_LOG_WEIGHT)
        L[:n] = log_w
        vec[1] = L
        vec[2] = np.exp(L)
        with np.errstate(invalid="ignore"):
            lo = L[:n] - vec[1, :n].astype(np.float64)
        vec[3, :n] = np.where(np.isfinite(lo), lo, 0.0)      # (a log weight of -inf has no low part)
        if off is not None:
            vec[4, :n] = off
        dv = torch.from_numpy(vec).to(device)
        self.sq, self.log_w, self.w, self.log_w_lo = dv[0], dv[1], dv[2], dv[3]
        self.off = dv[4] if off is not None else None
        # the points unpadded (the packing pads them to npad x kp with zeros), cast to float32 on the host and
        # copied from pageable memory (a pinned staging buffer for every cloud size bought nothing)
        self.pk = pack_cloud(torch.from_numpy(pts.astype(np.float32)).to(device))

    def c_struct(self) -> SkCloud:
        return SkCloud(self.pk.data_ptr(), self.sq.data_ptr(), self.log_w.data_ptr(), self.w.data_ptr(),
                       _ptr(self.off), self.n, self.npad, self.log_w_lo.data_ptr())

    def set_off(self, off: np.ndarray) -> None:
        """A new offset log(target / weight) in place (the cloud was made with one), for a new solve on the same
        points and weights: loops set up on this cloud keep their pointers."""
        if self.off is None:
            raise ValueError("set_off: the cloud was made without an offset")
        v = np.zeros(self.npad, dtype=np.float32)
        v[:self.n] = off
        self.off.copy_(torch.from_numpy(v))


def bake_log2(first: HipCloud, second: HipCloud, sc: torch.Tensor) -> None:
    """Make the first cloud's log2-unit copy for sc[0] = 2/eps against `second` (sk_bake_log2_f32): half-steps
    of this pair at that eps then take their scores in log2 units from the matrix cores. Any other eps, or a
    copy that does not fit fp16's range, falls back to scaling on the VALU; the results agree to rounding."""
    _require_device_f32("sc", sc, 4)
    if first.role != 0 or second.role != 1 or first.d != second.d:
        raise ValueError("bake_log2 pairs a first cloud (role 0) with a second (role 1) of the same dimension")
    _check(lib().sk_bake_log2_f32(first.pk.data_ptr(), second.pk.data_ptr(), first.n, first.d, sc.data_ptr(),
                                  _stream()), "sk_bake_log2_f32")


def half_step(side: HipCloud, other: HipCloud, other_h: torch.Tensor, sc: torch.Tensor, use_off: bool = True,
              out: torch.Tensor | None = None, log2: bool = False) -> torch.Tensor:
    """One fused half-step: the new shifted potential of `side`'s points (side.npad,) against `other`.

    The counterpart of _NkiStep.__call__ (src/trnopt/sinkhorn.py:185-193) and of make_half_step_kernel's
    kernel (src/trnopt/nki_sinkhorn.py:175-228): sc = {2/eps, 1/eps, eps, kappa} on the device. The scores come
    in log2 units from the matrix cores when the first cloud of the pair carries its log2-unit copy for sc[0]
    (bake_log2; the on-device loop keeps one for its current eps), else they are scaled on the VALU. log2=True
    makes that copy first (one more launch over the first cloud), for callers with no copy of their own."""
    _require_device_f32("other_h", other_h, other.npad)
    _require_device_f32("sc", sc, 4)
    if side.d != other.d:
        raise ValueError("clouds of different dimension")
    if side.role == other.role:
        raise ValueError("a half-step pairs a first cloud (role 0) with a second (role 1)")
    if log2:
        first, second = (side, other) if side.role == 0 else (other, side)
        bake_log2(first, second, sc)
    lb = lib()
    ws = _workspace(lb.sk_half_step_workspace_bytes(side.npad, other.npad, side.d), side.device)
    if out is None:
        out = torch.empty(side.npad, dtype=torch.float32, device=side.device)
    off = side.off if use_off else None
    _check(lb.sk_half_step_f32(side.pk.data_ptr(), side.sq.data_ptr(), _ptr(off), side.npad, other.pk.data_ptr(),
                               other_h.data_ptr(), other.log_w.data_ptr(), other.npad, side.d, side.role,
                               sc.data_ptr(), None, out.data_ptr(), None, None, side.n, ws.data_ptr(), ws.numel(),
                               _stream()), "sk_half_step_f32")
    return out


MEDIAN_D_MAX = 128                        # SK_MEDIAN_D_MAX


def cost_median(xc: np.ndarray, yc: np.ndarray, device) -> float:
    """median over all pairs of max(|xc_i|^2 + |yc_j|^2 - 2 xc_i . yc_j, 0) in float64, np.median's definition,
    on the GPU (sk_cost_median_f64): the exact-median branch of normalization(how="median")
    (src/trnopt/sinkhorn.py:229-233) without the n x m matrix. xc, yc: centred float64 (n, d), (m, d)."""
    return float(cost_median_enqueue(xc, yc, device).item())


def cost_median_enqueue(xc: np.ndarray, yc: np.ndarray, device) -> torch.Tensor:
    """cost_median enqueued on the current stream, not waited for: its (1,) float64 device result. Several
    pairs' medians enqueued back to back are read with one synchronisation (the inputs and workspace go back to
    the caching allocator, which hands them out again only to work ordered after this on the same stream)."""
    xc = np.ascontiguousarray(xc, dtype=np.float64)
    yc = np.ascontiguousarray(yc, dtype=np.float64)
    if xc.ndim != 2 or yc.ndim != 2 or xc.shape[1] != yc.shape[1]:
        raise ValueError("xc (n, d) and yc (m, d) must share d")
    (n, d), m = xc.shape, yc.shape[0]
    lb = lib()
    X = torch.as_tensor(xc).to(device)
    Y = torch.as_tensor(yc).to(device)
    out = torch.empty(1, dtype=torch.float64, device=device)
    ws = _workspace(lb.sk_cost_median_workspace_bytes(n, m, d), device)
    _check(lb.sk_cost_median_f64(X.data_ptr(), Y.data_ptr(), n, m, d, out.data_ptr(), ws.data_ptr(), ws.numel(),
                                 _stream()), "sk_cost_median_f64")
    return out


# ---------------------------------------------------------------------------------------------------------
# The on-device loop

class DeviceLoop:
    """The iteration loop of src/trnopt/sinkhorn.py:346-378 on the GPU.

    Each enqueued iteration is two partial-kernel launches (each merging its own row groups from 40 row
    groups up, followed by a merge-kernel launch below that): f update (X rows
    against Y; counts the iteration), g update (Y rows against X, which also reduces the convergence measures;
    the last row group's merge runs the reference's checks at its cadence, sets `done` and writes the next
    eps's scalars). Kernels enqueued after
    `done` return at once, so the host enqueues batches and reads the 72-byte state once per batch, with the
    next batch already queued behind it (no per-iteration synchronisation).

    With TRNOPT_HIP_GRAPH=1, whole batches of GRAPH_BATCH iterations are replayed from one captured HIP graph
    (20 to 40 kernels, no memset nodes): fewer host calls, for callers whose host enqueue is the bottleneck. Graph
    and eager launches run the same kernels with the same arguments, so the results are bit-identical. The
    default is eager: the GPU-bound loop measured no faster from graphs, and each solve would pay a capture
    (host enqueue at 3,000 x 3,500 d 30: 10.6-12.7 us per iteration eager, 5.2-5.3 us replayed, after a first
    capture of about 4.4 ms). Graphs are used in the main thread only (graphs_enabled)."""

    GRAPH_BATCH = 10

    def __init__(self, X: HipCloud, Y: HipCloud, *, eps: float, rho_x, rho_y, sched, stages, tol: float,
                 stage_tol: float, max_iters: int, check_every: int, stage_max_iters: int, fixed_iters: bool,
                 balanced: bool, state: torch.Tensor | None = None):
        dev = X.device
        lb = lib()
        self.X, self.Y = X, Y
        self.fh = torch.zeros(X.npad, dtype=torch.float32, device=dev)
        self.gh = torch.zeros(Y.npad, dtype=torch.float32, device=dev)      # gh = 0: g0 = |y|^2 (sinkhorn.py:336)
        if state is None:                  # (a DeviceLoopBatch keeps its loops' states in one block: a row of it)
            state = torch.zeros(ctypes.sizeof(SkState), dtype=torch.uint8, device=dev)
        if state.numel() != ctypes.sizeof(SkState) or state.dtype != torch.uint8 or state.data_ptr() % 8:
            raise ValueError("state must be the loop's own 8-byte aligned uint8 block of sizeof(SkState) bytes")
        self.state = state
        self._sched = torch.tensor(list(sched), dtype=torch.float64, device=dev) if len(sched) else None
        self._stages = torch.tensor(list(stages), dtype=torch.float64, device=dev) if len(stages) else None
        self.ws = _workspace(lb.sk_loop_workspace_bytes(X.npad, Y.npad, X.d), dev)
        self.max_iters = int(max_iters)
        self.check_every = max(1, int(check_every))
        self.fixed_iters = bool(fixed_iters)
        L = SkLoop()
        L.x, L.y, L.d = X.c_struct(), Y.c_struct(), X.d
        L.fh, L.gh, L.state = self.fh.data_ptr(), self.gh.data_ptr(), self.state.data_ptr()
        L.sched, L.n_sched = _ptr(self._sched), len(sched)
        L.stages, L.n_stages = _ptr(self._stages), len(stages)
        L.eps = float(eps)
        L.rho_x = float(rho_x) if rho_x is not None else -1.0
        L.rho_y = float(rho_y) if rho_y is not None else -1.0
        L.tol, L.stage_tol = float(tol), float(stage_tol)
        L.max_iters, L.check_every, L.stage_max_iters = self.max_iters, self.check_every, int(stage_max_iters)
        L.fixed_iters, L.balanced = int(bool(fixed_iters)), int(bool(balanced))
        L.ws, L.ws_bytes = self.ws.data_ptr(), self.ws.numel()
        self._L = L
        self._pinned = None                   # two pinned state buffers, made by the first run (a batch has its own)
        self._graph = None

    def init(self) -> None:
        _check(lib().sk_loop_init_f32(ctypes.byref(self._L), _stream()), "sk_loop_init_f32")

    @staticmethod
    def graphs_enabled() -> bool:
        """TRNOPT_HIP_GRAPH=1, and only in the main thread. A capture in one host thread and a graph released in
        another (or a device synchronisation there) cannot overlap: the HIP runtime refuses the release while any
        stream captures, and torch's graph destructor then terminates the process. Worker threads -- such as
        wot_transport_maps' pairs in flight -- therefore launch eagerly, which is also the faster form there."""
        return os.environ.get("TRNOPT_HIP_GRAPH", "0") == "1" and threading.current_thread() is threading.main_thread()

    def capture(self) -> None:
        """Capture the graph of GRAPH_BATCH iterations now (enqueue would do it on first use). Capturing launches
        nothing and does not synchronise the device: the capture is thread-local, so that other host threads
        (wot_transport_maps drives one pair per thread) keep launching on their own streams meanwhile. (The
        torch.cuda.graph context would synchronise the whole device first, which another thread's capture
        forbids.)"""
        if self._graph is not None or not self.graphs_enabled():
            return
        cur = torch.cuda.current_stream()
        side = torch.cuda.Stream(device=self.X.device)
        side.wait_stream(cur)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(side):
            g.capture_begin(capture_error_mode="thread_local")
            try:
                st = lib().sk_loop_run_f32(ctypes.byref(self._L), self.GRAPH_BATCH, _stream())
            finally:
                g.capture_end()
        _check(st, "sk_loop_run_f32")
        cur.wait_stream(side)
        self._graph = g

    def enqueue(self, iters: int) -> None:
        iters = int(iters)
        if iters >= self.GRAPH_BATCH and self.graphs_enabled():
            self.capture()
            for _ in range(iters // self.GRAPH_BATCH):
                self._graph.replay()
            iters %= self.GRAPH_BATCH
        if iters > 0:
            _check(lib().sk_loop_run_f32(ctypes.byref(self._L), iters, _stream()), "sk_loop_run_f32")

    def read_state(self) -> SkState:
        """Synchronous read of the current state (waits for everything enqueued)."""
        host = self.state.to("cpu")
        return SkState.from_buffer_copy(host.numpy().tobytes())

    def run(self, batch: int | None = None) -> SkState:
        """Run to `done` (converged or max_iters). Returns the final state."""
        self.init()
        if self.fixed_iters:
            self.enqueue(self.max_iters)
            return self.read_state()
        batch = max(1, int(batch or max(self.check_every, 10)))
        if self._pinned is None:
            self._pinned = [torch.empty(ctypes.sizeof(SkState), dtype=torch.uint8, pin_memory=True) for _ in range(2)]
        queued = 0
        inflight = []                         # (pinned buffer, event) per enqueued batch, oldest first
        slot = 0
        while True:
            if queued < self.max_iters:
                k = min(batch, self.max_iters - queued)
                self.enqueue(k)
                queued += k
                buf = self._pinned[slot % 2]
                slot += 1
                buf.copy_(self.state, non_blocking=True)
                ev = torch.cuda.Event()
                ev.record()
                inflight.append((buf, ev))
                if len(inflight) < 2 and queued < self.max_iters:
                    continue                  # keep a second batch queued behind the one we wait on
            buf, ev = inflight.pop(0)
            ev.synchronize()
            st = SkState.from_buffer_copy(buf.numpy().tobytes())
            if st.done:
                return st                     # final: the launches still queued return at once, changing nothing
            if not inflight and queued >= self.max_iters:  # pragma: no cover - done must be set by then
                return self.read_state()




class DeviceLoopBatch:
    """Several DeviceLoops of one d run together (sk_loop_run_batch_f32): each iteration is two launches, the f
    updates of all the loops and then their g updates, each loop's pass on its own share of the GPU's workgroups
    (in proportion to its work) and merged in the launch, each loop's control as in its own loop. For independent
    small solves, such as the pairs of a wot pipeline, which alone leave most of the GPU idle during a launch's
    latencies. A loop's splits are coarser than its own launches', so its potentials agree with DeviceLoop.run's to
    float32 rounding (with one loop, bit for bit). The loops' states are rows of one device block (`states`, given
    to each DeviceLoop as its `state`), read back in one copy per batch of iterations; a loop that is done idles
    while the others go on."""

    @staticmethod
    def state_block(n: int, device) -> torch.Tensor:
        """A zeroed (n, sizeof(SkState)) uint8 block whose row k is loop k's state."""
        return torch.zeros((n, ctypes.sizeof(SkState)), dtype=torch.uint8, device=device)

    def __init__(self, loops: list[DeviceLoop], states: torch.Tensor):
        if not loops:
            raise ValueError("DeviceLoopBatch needs at least one loop")
        n = len(loops)
        if states.shape != (n, ctypes.sizeof(SkState)) or any(
                l.state.data_ptr() != states[k].data_ptr() for k, l in enumerate(loops)):
            raise ValueError("each loop's state must be its row of `states` (DeviceLoopBatch.state_block)")
        lb = lib()
        self.loops, self.states = loops, states
        self.ws = _workspace(lb.sk_loop_batch_workspace_bytes(n), loops[0].X.device)
        self._ptrs = (ctypes.POINTER(SkLoop) * n)(*[ctypes.pointer(l._L) for l in loops])
        self._launch = (ctypes.c_int * 3)()
        self.max_iters = max(l.max_iters for l in loops)
        self.check_every = min(l.check_every for l in loops)
        self._pinned = [torch.empty(states.numel(), dtype=torch.uint8, pin_memory=True) for _ in range(2)]

    def init(self) -> None:
        for l in self.loops:
            l.init()
        _check(lib().sk_loop_batch_init_f32(self._ptrs, len(self.loops), self.ws.data_ptr(), self.ws.numel(),
                                            self._launch, _stream()), "sk_loop_batch_init_f32")

    def enqueue(self, iters: int) -> None:
        _check(lib().sk_loop_run_batch_f32(self.ws.data_ptr(), self.ws.numel(), len(self.loops), self._launch,
                                           int(iters), _stream()), "sk_loop_run_batch_f32")

    def _parse(self, buf: torch.Tensor) -> list[SkState]:
        raw = buf.numpy().tobytes()
        sz = ctypes.sizeof(SkState)
        return [SkState.from_buffer_copy(raw[k * sz:(k + 1) * sz]) for k in range(len(self.loops))]

    def run(self, batch: int | None = None) -> list[SkState]:
        """Run every loop to `done`. Returns the final states, in the loops' order. As DeviceLoop.run: batches of
        iterations with the next one queued while the states of the one before are read."""
        self.init()
        batch = max(1, int(batch or max(self.check_every, 10)))
        queued, slot, inflight = 0, 0, []
        while True:
            if queued < self.max_iters:
                k = min(batch, self.max_iters - queued)
                self.enqueue(k)
                queued += k
                buf = self._pinned[slot % 2]
                slot += 1
                buf.copy_(self.states.view(-1), non_blocking=True)
                ev = torch.cuda.Event()
                ev.record()
                inflight.append((buf, ev))
                if len(inflight) < 2 and queued < self.max_iters:
                    continue
            buf, ev = inflight.pop(0)
            ev.synchronize()
            sts = self._parse(buf)
            if all(st.done for st in sts):
                return sts
            if not inflight and queued >= self.max_iters:  # pragma: no cover - done must be set by then
                return self._parse(self.states.view(-1).to("cpu"))