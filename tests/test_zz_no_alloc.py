"""The no-allocation half-step (sk_half_step_noalloc_f32) against sk_half_step_f32 through the C ABI: the same
kernels with the partial slots in the library's static device scratch instead of a caller workspace, so the
outputs must be bit-identical, on two calls in a row (the second smaller, over the slots the first left behind),
and a shape beyond the scratch must be refused before anything runs."""

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


def test_noalloc_refuses_shapes_beyond_the_scratch(hip):
    """2,097,184 rows need 16 MiB + 256 bytes of slots: refused with SK_E_WORKSPACE (-3) before any launch."""
    lb = hip.lib()
    rows_pad, m_pad, d = (1 << 21) + 32, 32, 4
    assert lb.sk_half_step_workspace_bytes(rows_pad, m_pad, d) > 16 << 20
    buf = torch.zeros(1024, dtype=torch.float32, device=DEV)
    p = buf.data_ptr()
    st = lb.sk_half_step_noalloc_f32(p, p, None, rows_pad, p, p, p, m_pad, d, 0, p, None, p + 1024, None, None, 1,
                                     torch.cuda.current_stream().cuda_stream)
    assert st == -3
    assert b"static scratch" in lb.sk_last_error()
