"""The no-allocation half-step (sk_half_step_noalloc_f32) against sk_half_step_f32 through the C ABI: the same
kernels with the partial slots in the library's static device scratch instead of a caller workspace, so the
outputs must be bit-identical, on two calls in a row (the second smaller, over the slots the first left behind),
and replayed from a captured HIP graph."""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _pair(hip, rows, m, d, seed):
    rng = np.random.default_rng(seed)
    x = rng.normal(size=(rows, d))
    y = rng.normal(size=(m, d)) * 0.8 + 0.3
    log_b = np.log(rng.uniform(0.5, 1.5, m) / m)
    X = hip.HipCloud(x, np.log(np.full(rows, 1.0 / rows)), DEV, off=rng.normal(scale=0.3, size=rows), role=0)
    Y = hip.HipCloud(y, log_b, DEV, role=1)
    gh = torch.zeros(Y.npad, dtype=torch.float32, device=DEV)
    gh[:m] = torch.as_tensor(rng.normal(scale=2.0, size=m) - 0.5 * (y * y).sum(1), dtype=torch.float32)
    return X, Y, gh


def _both(hip, X, Y, gh, eps, kappa, with_meas):
    """fh from sk_half_step_f32 (caller workspace) and from sk_half_step_noalloc_f32, and their meas."""
    lb = hip.lib()
    sc = hip.scalars(eps, kappa, DEV)
    stream = torch.cuda.current_stream().cuda_stream
    outs = []
    for noalloc in (False, True):
        fh = torch.full((X.npad,), 0.25, dtype=torch.float32, device=DEV)     # old potential for meas
        nmeas = lb.sk_half_step_meas_count(X.npad)
        meas = torch.zeros(2 * nmeas, dtype=torch.float32, device=DEV) if with_meas else None
        w = X.w if with_meas else None
        args = (X.pk.data_ptr(), X.sq.data_ptr(), X.off.data_ptr(), X.npad, Y.pk.data_ptr(), gh.data_ptr(),
                Y.log_w.data_ptr(), Y.npad, X.d, 0, sc.data_ptr(), None, fh.data_ptr(),
                None if meas is None else meas.data_ptr(), None if w is None else w.data_ptr(), X.n)
        if noalloc:
            st = lb.sk_half_step_noalloc_f32(*args, stream)
        else:
            ws = torch.empty(max(256, lb.sk_half_step_workspace_bytes(X.npad, Y.npad, X.d)), dtype=torch.uint8,
                             device=DEV)
            st = lb.sk_half_step_f32(*args, ws.data_ptr(), ws.numel(), stream)
        assert st == 0, lb.sk_last_error()
        torch.cuda.synchronize()
        outs.append((fh.cpu(), None if meas is None else meas.cpu()))
    return outs


@pytest.mark.parametrize("first,second", [((1300, 1700, 50, 0.05, 0.9), (137, 91, 5, 0.1, 1.0)),
                                          ((10000, 10000, 64, 0.1, 1.0), (2048, 2048, 64, 0.1, 1.0))])
def test_noalloc_half_step_matches_the_workspace_entry_point(hip, first, second):
    for k, (rows, m, d, eps, kappa) in enumerate((first, second)):
        print(f"noalloc call {k}: rows={rows} m={m} d={d} eps={eps} kappa={kappa}", flush=True)
        X, Y, gh = _pair(hip, rows, m, d, seed=rows + m + d)
        (a, ma), (b, mb) = _both(hip, X, Y, gh, eps, kappa, with_meas=(k == 0))
        assert torch.isfinite(a).all()
        assert torch.equal(a, b), (a - b).abs().max()
        if ma is not None:
            assert torch.equal(ma, mb)


def test_noalloc_half_step_replays_from_a_captured_graph(hip):
    """For callers under HIP graph capture: after one eager call on the device (which looks up the scratch's
    device address with hipGetSymbolAddress, outside any capture), the no-alloc half-step is captured as its two
    kernel launches (no allocation, no memset node) and replayed; every replay, with the program's own eager work
    and synchronisations between them, gives the eager result bit for bit. (A shape beyond the scratch is refused
    before any launch: checked on the host, tests/test_host_abi.py.)"""
    rows, m, d, eps, kappa = 700, 900, 24, 0.07, 0.95
    X, Y, gh = _pair(hip, rows, m, d, seed=11)
    lb = hip.lib()
    sc = hip.scalars(eps, kappa, DEV)

    def call(fh, stream):
        return lb.sk_half_step_noalloc_f32(X.pk.data_ptr(), X.sq.data_ptr(), X.off.data_ptr(), X.npad,
                                           Y.pk.data_ptr(), gh.data_ptr(), Y.log_w.data_ptr(), Y.npad, X.d, 0,
                                           sc.data_ptr(), None, fh.data_ptr(), None, None, X.n, stream)

    eager = torch.zeros(X.npad, dtype=torch.float32, device=DEV)
    assert call(eager, torch.cuda.current_stream().cuda_stream) == 0, lb.sk_last_error()
    torch.cuda.synchronize()
    assert torch.isfinite(eager).all()
    out = torch.zeros(X.npad, dtype=torch.float32, device=DEV)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        graph.capture_begin(capture_error_mode="thread_local")
        try:
            st = call(out, side.cuda_stream)
        finally:
            graph.capture_end()
    torch.cuda.current_stream().wait_stream(side)
    assert st == 0, lb.sk_last_error()
    for k in range(4):
        print(f"noalloc graph replay {k}", flush=True)
        out.fill_(float(k) + 0.5)                   # eager work between the replays
        eager2 = torch.zeros_like(eager)
        assert call(eager2, torch.cuda.current_stream().cuda_stream) == 0   # the scratch used eagerly meanwhile
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), (out - eager).abs().max()
        assert torch.equal(eager2, eager)
