"""Kernel-level parity of the HIP row-LSE and half-step against float64 known answers and the float32
torch half-step (the reference's examples/nki_sinkhorn_check.py, restated as assertions)."""

import numpy as np
import pytest
import torch

from oracle import brute
from oracle import data
from oracle import reference as ref
from conftest import inf_rel

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _lse_tol(xa, ya):
    # fp32 contraction error bound per row: a few ulps of the largest |score| term sum, plus exp2/log2 ulps
    mag = np.abs(xa.astype(np.float64)) @ np.abs(ya.astype(np.float64)).T
    return 4e-7 * np.sqrt(xa.shape[1]) * mag.max(axis=1) + 2e-6


@pytest.mark.parametrize("rows,m,K", [(1, 1, 1), (5, 7, 3), (33, 31, 8), (64, 300, 65), (300, 1000, 65),
                                      (257, 4097, 31), (1000, 513, 128), (96, 2048, 65), (2, 5000, 17)])
def test_row_lse_matches_float64(hip, rows, m, K):
    rng = np.random.default_rng(rows * 1000 + m + K)
    xa = rng.normal(size=(rows, K)).astype(np.float32)
    ya = (rng.normal(size=(m, K)) * 0.7).astype(np.float32)
    print(f"row_lse rows={rows} m={m} K={K}", flush=True)
    out = hip.row_lse(torch.from_numpy(xa).to(DEV), torch.from_numpy(ya).to(DEV)).cpu().numpy()
    want = brute.row_lse(xa, ya)
    assert np.all(np.abs(out - want) <= _lse_tol(xa, ya)), np.abs(out - want).max()


def test_row_lse_realistic_scores_with_padding(hip):
    """examples/nki_sinkhorn_check.py:22-35: blob points, eps 0.1, a plausible gh, the last 300 columns padding
    (y = 0, gh = 0, log b = -1e9), so padding must contribute exactly nothing."""
    rng = np.random.default_rng(0)
    rows, m, d, eps, real = 256, 4096, 64, 0.1, 4096 - 300
    x = rng.normal(size=(rows, d)) * 0.15
    y = rng.normal(size=(m, d)) * 0.15 + 0.02
    gh = -(y ** 2).sum(1) + rng.normal(scale=0.05, size=m)
    log_b = np.full(m, -np.log(m))
    y[real:], gh[real:], log_b[real:] = 0.0, 0.0, -1e9
    xa = np.hstack([x, np.ones((rows, 1))]).astype(np.float32)
    ya = np.hstack([2.0 / eps * y, (gh / eps + log_b)[:, None]]).astype(np.float32)
    out = hip.row_lse(torch.from_numpy(xa).to(DEV), torch.from_numpy(ya).to(DEV)).cpu().numpy()
    want = brute.row_lse(xa, ya)
    want_real = brute.row_lse(xa, ya[:real])
    np.testing.assert_allclose(want, want_real, rtol=0, atol=1e-12)
    assert np.abs(out - want).max() < 2e-4


def _half_inputs(rows, m, d, eps, seed, pad_rows=0, pad_cols=0):
    rng = np.random.default_rng(seed)
    x = rng.normal(size=(rows, d))
    y = rng.normal(size=(m, d)) * 0.8 + 0.3
    gh = rng.normal(scale=2.0, size=m) - 0.5 * (y * y).sum(1)
    log_b = np.log(rng.uniform(0.5, 1.5, m) / m)
    off = rng.normal(scale=0.3, size=rows)
    return x, y, gh, log_b, off


@pytest.mark.parametrize("rows,m,d,eps,kappa", [(137, 91, 5, 0.1, 1.0), (1300, 1700, 50, 0.05, 0.9),
                                                (2048, 2048, 64, 0.1, 1.0), (333, 4000, 30, 0.05, 50 / 50.05),
                                                (64, 64, 128, 0.5, 0.7), (40, 3000, 1, 0.2, 1.0)])
def test_half_step_matches_float64_and_torch(hip, rows, m, d, eps, kappa):
    x, y, gh, log_b, off = _half_inputs(rows, m, d, eps, seed=rows + m + d)
    X = hip.HipCloud(x, np.zeros(rows), DEV, off=off, role=0)
    Y = hip.HipCloud(y, log_b, DEV, role=1)
    gh_pad = np.zeros(Y.npad)
    gh_pad[:m] = gh
    gh_t = torch.as_tensor(gh_pad, dtype=torch.float32, device=DEV)
    sc = hip.scalars(eps, kappa, DEV)
    print(f"half_step rows={rows} m={m} d={d} eps={eps} kappa={kappa}", flush=True)
    out = hip.half_step(X, Y, gh_t, sc).cpu().numpy()[:rows].astype(np.float64)
    # float64 known answer on the same float32 inputs (padding columns included: weight exactly 0)
    x32, y32 = x.astype(np.float32), y.astype(np.float32)
    xsq32 = (x * x).sum(1).astype(np.float32)
    want = brute.half_step_f64(x32, xsq32, off.astype(np.float32), y32, gh.astype(np.float32),
                               log_b.astype(np.float32), eps, float(np.float32(kappa)))
    # the reference's float32 torch half-step on the same inputs
    t = lambda a: torch.as_tensor(np.asarray(a), dtype=torch.float32)  # noqa: E731
    got32 = ref.half_step(t(x), t(xsq32), t(off), t(y).T.contiguous(), t(gh), t(log_b),
                          torch.tensor(1.0 / eps, dtype=torch.float32), torch.tensor(eps, dtype=torch.float32),
                          torch.tensor(kappa, dtype=torch.float32)).double().numpy()
    scale = np.abs(want).max()
    assert inf_rel(out, want) < 2e-6, (inf_rel(out, want), inf_rel(got32, want))
    assert np.abs(out - got32).max() <= 4 * np.abs(got32 - want).max() + 2e-6 * scale


def test_half_step_convergence_partials(hip):
    """The g update's convergence partials (meas): max |new - old| over real rows and the balanced L1 column
    error sum |w (exp(min((old - new)/eps, 50)) - 1)| (src/trnopt/sinkhorn.py:360, 368-373)."""
    rows, m, d, eps = 1000, 700, 16, 0.1
    x, y, gh, log_b, _ = _half_inputs(rows, m, d, eps, seed=5)
    w = np.full(rows, 1.0 / rows)
    X = hip.HipCloud(x, np.log(w), DEV, role=0)
    Y = hip.HipCloud(y, log_b, DEV, role=1)
    gh_t = torch.zeros(Y.npad, dtype=torch.float32, device=DEV)
    gh_t[:m] = torch.as_tensor(gh, dtype=torch.float32)
    sc = hip.scalars(eps, 1.0, DEV)
    new = hip.half_step(X, Y, gh_t, sc)
    old = new + torch.linspace(-0.3, 0.2, X.npad, device=DEV)
    buf = old.clone()
    lb = hip.lib()
    nmeas = lb.sk_half_step_meas_count(X.npad)
    meas = torch.zeros(2 * nmeas, dtype=torch.float32, device=DEV)
    ws = torch.empty(lb.sk_half_step_workspace_bytes(X.npad, Y.npad, d), dtype=torch.uint8, device=DEV)
    st = lb.sk_half_step_f32(X.pk.data_ptr(), X.sq.data_ptr(), None, X.npad, Y.pk.data_ptr(), gh_t.data_ptr(),
                             Y.log_w.data_ptr(), Y.npad, d, 0, sc.data_ptr(), None, buf.data_ptr(), meas.data_ptr(),
                             X.w.data_ptr(), X.n, ws.data_ptr(), ws.numel(), torch.cuda.current_stream().cuda_stream)
    assert st == 0
    torch.testing.assert_close(buf, new, rtol=0, atol=0)
    mv = meas.view(-1, 2).cpu().double().numpy()
    o, nw = old.cpu().double().numpy(), new.cpu().double().numpy()
    want_max = np.abs(nw - o)[:rows].max()
    delta = np.minimum((o - nw) * np.float32(1 / eps), 50.0)
    want_err = np.abs(X.w.cpu().double().numpy() * (np.exp(delta) - 1.0)).sum()
    assert abs(mv[:, 0].max() - want_max) <= 1e-6 * want_max
    assert abs(mv[:, 1].sum() - want_err) <= 1e-5 * want_err


def test_errors_are_reported_not_fatal(hip):
    lb = hip.lib()
    assert lb.sk_half_step_f32(None, None, None, 32, None, None, None, 32, 4, 0, None, None, None, None, None, 1,
                               None, 0, None) == -1
    assert b"null pointer" in lb.sk_last_error()
    a = torch.zeros(64 * 200, device=DEV)
    assert lb.sk_row_lse_f32(a.data_ptr(), a.data_ptr(), a.data_ptr(), 10, 10, 200, a.data_ptr(), 1 << 20, None) == -2
    with pytest.raises(ValueError):
        hip.row_lse(torch.zeros(3, 200, device=DEV), torch.zeros(4, 200, device=DEV))


def _masked_dots(hip, X, Y, rows_role, k, sc, bake=True):
    """x_i . y_k (rows_role 0) or y_j . x_k (rows_role 1) for all rows, read off a half-step of the pair whose
    column cloud weighs exactly 0 except at column k (log weight 0), with gh = 0 and |rows|^2 = 0: fh = -2 dot.
    With bake, the first cloud's log2-unit copy is made first. Returns the dots and the first cloud's tag."""
    R, C = (X, Y) if rows_role == 0 else (Y, X)
    lw = np.full(C.n, -1e9)
    lw[k] = 0.0
    Ck = hip.HipCloud(C._pts, lw, DEV, role=C.role)
    first, second = (R, Ck) if rows_role == 0 else (Ck, R)
    if bake:
        hip.bake_log2(first, second, sc)
    sq = R.sq.clone()
    R.sq.zero_()
    out = hip.half_step(R, Ck, torch.zeros(Ck.npad, dtype=torch.float32, device=DEV), sc)
    R.sq.copy_(sq)
    return -0.5 * out.cpu().numpy()[:R.n], _log2_tag(first)


@pytest.mark.parametrize("d", [3, 16, 64, 100, 128])
def test_f_and_g_updates_form_bit_identical_dots(hip, d):
    """The f update (rows x, role 0) and the g update (rows y, role 1) of one pair of clouds issue the piece
    products in the same order: x_i . y_j agrees bit for bit in both directions, and is fp32-accurate."""
    rng = np.random.default_rng(d)
    x = rng.normal(size=(70, d))
    y = rng.normal(size=(40, d)) * 1.7 + 0.3
    X = hip.HipCloud(x, np.zeros(70), DEV, role=0)
    Y = hip.HipCloud(y, np.zeros(40), DEV, role=1)
    X._pts, Y._pts = x, y
    sc = hip.scalars(1.0, 1.0, DEV)
    for j in (0, 7, 39):
        f_side, tag = _masked_dots(hip, X, Y, 0, j, sc, bake=False)
        assert tag == 0.0
        for i in (0, 33, 69):
            g_side, _ = _masked_dots(hip, X, Y, 1, i, sc, bake=False)
            assert np.float32(f_side[i]).tobytes() == np.float32(g_side[j]).tobytes(), (i, j, f_side[i], g_side[j])
        exact = x.astype(np.float32).astype(np.float64) @ y[j].astype(np.float32).astype(np.float64)
        bound = np.abs(x) @ np.abs(y[j])
        assert np.all(np.abs(f_side - exact) <= 4e-7 * bound + 1e-30)


def _log2_tag(cloud):
    """The packed header's log2-copy tag: the score scale the copy was made for (0: none)."""
    return float(cloud.pk[8:12].cpu().numpy().view(np.float32)[0])


def _log2_unit(cloud):
    """The packed header's log2-copy unit t (a power of two; 1 for the usual score scales)."""
    return float(cloud.pk[16:20].cpu().numpy().view(np.float32)[0])


@pytest.mark.parametrize("rows,m,d,eps,kappa,mag", [(137, 91, 5, 0.1, 1.0, 1.0), (1300, 1700, 50, 0.05, 0.9, 1.0),
                                                    (2048, 2048, 64, 0.1, 1.0, 1.0), (333, 4000, 30, 0.01, 1.0, 0.3),
                                                    (64, 64, 128, 0.5, 0.7, 1.0), (500, 600, 16, 0.1, 1.0, 1e3),
                                                    (700, 900, 32, 1.0, 1.0, 0.01), (300, 2100, 128, 2.0, 0.8, 0.03),
                                                    (256, 300, 100, 0.02, 1.0, 30.0)])
def test_half_step_with_log2_copy_matches_float64(hip, rows, m, d, eps, kappa, mag):
    """With the first cloud's log2-unit copy the half-step (both directions) meets the same float64 known answer
    as without it and agrees with the VALU-scaled result to rounding. Where max |c x| / s_y leaves [2^-1, 2^15)
    (mag 1e3 at eps 0.1, small clouds at eps 1 and 2, large ones at eps 0.02) the copy carries a power-of-two
    unit t != 1 and the kernel rescales by 1 / t in the exponent's fma."""
    x, y, gh, log_b, off = _half_inputs(rows, m, d, eps, seed=rows + 7 * m + d)
    x, y, gh = x * mag, y * mag, gh * mag * mag
    la = np.log(np.full(rows, 1.0 / rows))
    X = hip.HipCloud(x, la, DEV, off=off, role=0)
    Y = hip.HipCloud(y, log_b, DEV, role=1)
    sc = hip.scalars(eps, kappa, DEV)
    ghp = torch.zeros(Y.npad, dtype=torch.float32, device=DEV)
    ghp[:m] = torch.as_tensor(gh, dtype=torch.float32)
    fhp = torch.zeros(X.npad, dtype=torch.float32, device=DEV)
    fhp[:rows] = torch.as_tensor(np.random.default_rng(rows).normal(scale=2.0, size=rows) * mag * mag - 0.5 * (x * x).sum(1),
                                 dtype=torch.float32)
    print(f"log2 copy rows={rows} m={m} d={d} eps={eps} mag={mag}", flush=True)
    f_vpu = hip.half_step(X, Y, ghp, sc).cpu().numpy()[:rows].astype(np.float64)
    g_vpu = hip.half_step(Y, X, fhp, sc).cpu().numpy()[:m].astype(np.float64)
    hip.bake_log2(X, Y, sc)
    torch.cuda.synchronize()
    assert _log2_tag(X) != 0.0
    unit = _log2_unit(X)
    print(f"  unit {unit}", flush=True)
    assert (unit == 1.0) == (mag in (1.0, 0.3)), unit
    assert unit == 2.0 ** round(np.log2(unit))
    f_l2 = hip.half_step(X, Y, ghp, sc).cpu().numpy()[:rows].astype(np.float64)
    g_l2 = hip.half_step(Y, X, fhp, sc).cpu().numpy()[:m].astype(np.float64)
    x32, y32 = x.astype(np.float32), y.astype(np.float32)
    k32 = float(np.float32(kappa))
    f_want = brute.half_step_f64(x32, (x * x).sum(1).astype(np.float32), off.astype(np.float32), y32,
                                 gh.astype(np.float32), log_b.astype(np.float32), eps, k32)
    g_want = brute.half_step_f64(y32, (y * y).sum(1).astype(np.float32), np.zeros(m), x32,
                                 fhp.cpu().numpy()[:rows], la.astype(np.float32), eps, k32)
    # small clouds leave fh a small difference of O(1) terms: their bar is the float32 floor of those terms
    f_floor = _f32_floor(x32, y32, gh.astype(np.float32), log_b.astype(np.float32), eps, k32,
                         (x * x).sum(1).astype(np.float32), off.astype(np.float32))
    g_floor = _f32_floor(y32, x32, fhp.cpu().numpy()[:rows], la.astype(np.float32), eps, k32,
                         (y * y).sum(1).astype(np.float32), np.zeros(m))
    for got, vpu, want, floor in ((f_l2, f_vpu, f_want, f_floor), (g_l2, g_vpu, g_want, g_floor)):
        bar = max(2e-6 * np.abs(want).max(), floor)
        assert np.abs(got - want).max() <= bar, (np.abs(got - want).max(), np.abs(vpu - want).max(), bar)
        assert np.abs(got - vpu).max() <= bar


@pytest.mark.parametrize("eps,gscale,bake", [(0.1, 1e-3, False), (0.1, 1e-3, True), (0.1, 3e2, True),
                                             (0.01, 3e4, True), (1.0, 1e6, False), (1.0, 1e6, True)])
def test_half_step_column_terms_across_magnitudes(hip, eps, gscale, bake):
    """The matrix pipe adds each column term (gh_j + eps log b_j) / 2, in the kernel's units, as three bf16
    pieces: column terms from 1e-3 to 1e6 times the dot products, and a fifth of the columns masked by
    log b = -1e9 (weight exactly 0), meet the float64 known answer, with and without the log2-unit copy."""
    rows, m, d = 300, 2000, 16
    rng = np.random.default_rng(int(gscale) + int(100 * eps) + bake)
    x = rng.normal(size=(rows, d))
    y = rng.normal(size=(m, d)) * 0.8 + 0.3
    gh = rng.normal(size=m) * gscale * np.exp(rng.uniform(-3, 0, m))    # magnitudes over three decades
    log_b = np.log(rng.uniform(0.5, 1.5, m) / m)
    log_b[rng.random(m) < 0.2] = -1e9
    X = hip.HipCloud(x, np.zeros(rows), DEV, role=0)
    Y = hip.HipCloud(y, log_b, DEV, role=1)
    ghp = torch.zeros(Y.npad, dtype=torch.float32, device=DEV)
    ghp[:m] = torch.as_tensor(gh, dtype=torch.float32)
    sc = hip.scalars(eps, 1.0, DEV)
    if bake:
        hip.bake_log2(X, Y, sc)
        torch.cuda.synchronize()
        assert _log2_tag(X) != 0.0
    print(f"column terms eps={eps} gscale={gscale} bake={bake}", flush=True)
    out = hip.half_step(X, Y, ghp, sc).cpu().numpy()[:rows].astype(np.float64)
    x32, y32 = x.astype(np.float32), y.astype(np.float32)
    xsq32 = (x * x).sum(1).astype(np.float32)
    keep = log_b > -1e8
    want = brute.half_step_f64(x32, xsq32, np.zeros(rows), y32, gh.astype(np.float32),
                               log_b.astype(np.float32), eps, 1.0)
    want_kept = brute.half_step_f64(x32, xsq32, np.zeros(rows), y32[keep], gh.astype(np.float32)[keep],
                                    log_b.astype(np.float32)[keep], eps, 1.0)
    np.testing.assert_allclose(want, want_kept, rtol=1e-13, atol=0)
    assert inf_rel(out, want) < 2e-6, inf_rel(out, want)


def _f32_floor(x, y, gh, log_b, eps, kappa, xsq, off):
    """A float32 half-step's rounding floor on these inputs: a few ulps of the largest score
    |z| = |(2 x.y + gh) / eps + log b| (times eps), plus the epilogue's roundings at |x|^2 and eps |off|."""
    z = np.abs(2.0 * x.astype(np.float64) @ y.astype(np.float64).T + gh[None, :]) / eps + np.abs(log_b)[None, :]
    return 8 * 2.0 ** -24 * (eps * z.max() + np.abs(xsq).max() + eps * np.abs(off).max()) + 1e-30


@pytest.mark.parametrize("case,rows,m,d,eps,kappa", [("tiny", 500, 500, 16, 0.1, 1.0), ("tiny", 333, 777, 5, 0.02, 0.9),
                                                     ("mixed", 300, 470, 64, 0.1, 1.0),
                                                     ("mixed-rows-y", 470, 300, 64, 0.1, 1.0),
                                                     ("mixed", 1000, 2100, 30, 0.05, 50 / 50.05)])
def test_half_step_small_and_mixed_scale_clouds(hip, case, rows, m, d, eps, kappa):
    """normalize=False inputs whose column terms dwarf the dot products in the kernel's units: clouds at 1e-4
    (both scales 2^16, so sigma = 2^32 and eps log b / 2 = -0.31 is -1.3e9 kernel units) and x at 1e-6 against
    y ~ N(0, 1) with gh ~ -|y|^2 (sigma |gh| / 2 ~ 1e9), m not a multiple of 32. The matrix pipe adds each
    column term as three exact bf16 pieces (no range limit): the half-step meets the float64 known answer to
    the float32 floor of its inputs, and the reference's float32 torch half-step as closely. (A column term
    clamped to +-2^30 gave 0.12 here where |fh| ~ 1e-8.)"""
    rng = np.random.default_rng(rows + m + d)
    if case == "tiny":
        x = rng.normal(size=(rows, d)) * 1e-4
        y = rng.normal(size=(m, d)) * 1e-4
        gh = np.zeros(m)
    elif case == "mixed":
        x = rng.normal(size=(rows, d)) * 1e-6
        y = rng.normal(size=(m, d))
        gh = -(y * y).sum(1) + rng.normal(scale=0.05, size=m)
    else:                                              # the g update's direction: rows at N(0, 1), columns tiny
        x = rng.normal(size=(rows, d))
        y = rng.normal(size=(m, d)) * 1e-6
        gh = rng.normal(scale=1e-6, size=m)
    log_b = np.log(rng.uniform(0.5, 1.5, m) / m)
    off = rng.normal(scale=0.3, size=rows) if kappa != 1.0 else np.zeros(rows)
    role = 1 if case == "mixed-rows-y" else 0
    X = hip.HipCloud(x, np.zeros(rows), DEV, off=off, role=role)
    Y = hip.HipCloud(y, log_b, DEV, role=1 - role)
    ghp = torch.zeros(Y.npad, dtype=torch.float32, device=DEV)
    ghp[:m] = torch.as_tensor(gh, dtype=torch.float32)
    sc = hip.scalars(eps, kappa, DEV)
    print(f"small/mixed scales {case} rows={rows} m={m} d={d} eps={eps}", flush=True)
    out = hip.half_step(X, Y, ghp, sc).cpu().numpy()[:rows].astype(np.float64)
    x32, y32 = x.astype(np.float32), y.astype(np.float32)
    xsq32 = (x * x).sum(1).astype(np.float32)
    gh32, lb32, off32 = gh.astype(np.float32), log_b.astype(np.float32), off.astype(np.float32)
    want = brute.half_step_f64(x32, xsq32, off32, y32, gh32, lb32, eps, float(np.float32(kappa)))
    t = lambda a: torch.as_tensor(np.asarray(a), dtype=torch.float32)  # noqa: E731
    got32 = ref.half_step(t(x32), t(xsq32), t(off32), t(y32).T.contiguous(), t(gh32), t(lb32),
                          torch.tensor(1.0 / eps, dtype=torch.float32), torch.tensor(eps, dtype=torch.float32),
                          torch.tensor(kappa, dtype=torch.float32)).double().numpy()
    tol = _f32_floor(x32, y32, gh32, lb32, eps, kappa, xsq32, off32)
    err, err32 = np.abs(out - want).max(), np.abs(got32 - want).max()
    print(f"  |hip - f64| {err:.3e}, |torch f32 - f64| {err32:.3e}, floor {tol:.3e}, |fh| {np.abs(want).max():.3e}")
    assert err <= tol, (err, err32, tol)


@pytest.mark.parametrize("d", [3, 16, 64, 128])
def test_log2_copy_keeps_f_and_g_dots_bit_identical(hip, d):
    """On the log2-unit copy the f update (rows x) and the g update (rows y) of one pair of clouds still form
    every x_i . y_j bit for bit alike (read back through the merge's division by c), fp32-accurate."""
    rng = np.random.default_rng(100 + d)
    x = rng.normal(size=(70, d))
    y = rng.normal(size=(40, d)) * 1.7 + 0.3
    X = hip.HipCloud(x, np.zeros(70), DEV, role=0)
    Y = hip.HipCloud(y, np.zeros(40), DEV, role=1)
    X._pts, Y._pts = x, y
    sc = hip.scalars(0.5, 1.0, DEV)
    for j in (0, 7, 39):
        f_side, tag = _masked_dots(hip, X, Y, 0, j, sc)
        assert tag != 0.0
        for i in (0, 33, 69):
            g_side, tag = _masked_dots(hip, X, Y, 1, i, sc)
            assert tag != 0.0
            assert np.float32(f_side[i]).tobytes() == np.float32(g_side[j]).tobytes(), (i, j, f_side[i], g_side[j])
        exact = x.astype(np.float32).astype(np.float64) @ y[j].astype(np.float32).astype(np.float64)
        bound = np.abs(x) @ np.abs(y[j])
        assert np.all(np.abs(f_side - exact) <= 4e-7 * bound + 1e-30)


@pytest.mark.parametrize("mx,my", [(1e-5, 1e5), (3e-8, 1e4), (1e3, 1e-3), (1.0, 1.0)])
def test_row_lse_with_badly_scaled_clouds(hip, mx, my):
    """Each packed cloud carries its own power-of-two scale: clouds far from unit magnitude keep the row-LSE's
    accuracy (scores x.y of order 1 here)."""
    rng = np.random.default_rng(int(-np.log10(mx) * 10 + 100))
    xa = (rng.normal(size=(300, 40)) * mx).astype(np.float32)
    ya = (rng.normal(size=(700, 40)) * my).astype(np.float32)
    out = hip.row_lse(torch.from_numpy(xa).to(DEV), torch.from_numpy(ya).to(DEV)).cpu().numpy()
    want = brute.row_lse(xa, ya)
    assert np.all(np.abs(out - want) <= _lse_tol(xa, ya)), np.abs(out - want).max()


def test_out_of_range_coordinates_are_rejected(hip):
    with pytest.raises(ValueError, match="coordinates"):
        hip.row_lse(torch.full((4, 3), 1e15, device=DEV), torch.ones(5, 3, device=DEV))
    with pytest.raises(ValueError, match="coordinates"):
        hip.HipCloud(np.full((4, 3), np.inf), np.zeros(4), DEV)


def test_graph_replays_match_eager_launches(hip, monkeypatch):
    """The device loop replays captured 10-iteration HIP graphs; several replays, with the program's own eager
    work and synchronisations between them, give the eager launches' potentials and state bit for bit."""
    import torch
    x, y = data.clouds(n=1000, m=777, d=24, seed=9)
    dev = torch.device("cuda", 0)
    la, lb = np.full(len(x), -np.log(len(x))), np.full(len(y), -np.log(len(y)))
    X = hip.HipCloud(x, la, dev, role=0)
    Y = hip.HipCloud(y, lb, dev, role=1)
    kw = dict(eps=0.05, rho_x=None, rho_y=None, sched=[0.5, 0.3, 0.2], stages=[], tol=1e-9, stage_tol=1e-5,
              max_iters=10_000, check_every=10, stage_max_iters=1000, fixed_iters=False, balanced=True)
    monkeypatch.setenv("TRNOPT_HIP_GRAPH", "1")
    g = hip.DeviceLoop(X, Y, **kw)
    g.init()
    for _ in range(6):
        g.enqueue(10)
        torch.cuda.synchronize()
        assert float((torch.arange(5, device=dev) * 2.0).sum()) == 20.0      # eager work between replays
    assert g._graph is not None
    monkeypatch.setenv("TRNOPT_HIP_GRAPH", "0")
    e = hip.DeviceLoop(X, Y, **kw)
    e.init()
    e.enqueue(60)
    sg, se = g.read_state(), e.read_state()
    assert e._graph is None
    assert (sg.it, sg.stage, sg.checks, sg.done) == (se.it, se.stage, se.checks, se.done)
    assert sg.it == 60 and sg.checks == 6
    assert sg.err == se.err
    assert torch.equal(g.fh, e.fh) and torch.equal(g.gh, e.gh)
