"""CPU emulation of the HIP kernels' index arithmetic (trainium-sinkhorn_amd/csrc).

Every load and store of pack_cloud_kernel, lse_partial_kernel and lse_finalize_kernel is replayed in numpy
with the kernels' own formulas (workgroup renumbering, stream-K ranges, partial slots, tile-interleaved
packing, the v_mfma_f32_32x32x2_f32 operand and accumulator lane mapping), asserting that every index is
inside its buffer and that the emulated result equals a direct float64 log-sum-exp. Run before any kernel
change goes to the GPU; it needs no GPU.
"""

import numpy as np
import pytest
from scipy.special import logsumexp

TILE, WAVES, XCDS = 32, 4, 8
EMPTY = -1.0e30


def pad_points(n):
    return -(-n // TILE) * TILE


def pad_dim(d):
    return -(-d // 8) * 8


def pack(src, n, d, kp):
    """pack_cloud_kernel: dst[idx] for every idx < npad * kp."""
    npad = pad_points(n)
    kq = kp // 8
    idx = np.arange(npad * kp)
    e = idx & 3
    t = idx >> 2
    r = t % 32
    t //= 32
    h = t % 2
    t //= 2
    q = t % kq
    T = t // kq
    row = T * 32 + r
    k = h * (kp // 2) + q * 4 + e
    ok = (row < n) & (k < d)
    src_idx = np.where(ok, row * d + k, 0)
    assert src_idx.max() < src.size
    return np.where(ok, src.ravel()[src_idx], 0.0)


class Split:
    def __init__(self, work, nt, P):
        self.work, self.nt, self.P = work, nt, P

    def owner(self, x):
        return min((((x + 1) * self.P) - 1) // self.work, self.P - 1)

    def first(self, g):
        return self.owner(g * self.nt)

    def last(self, g):
        return self.owner((g + 1) * self.nt - 1)


def plan(rows_pad, m_pad, kp, rb, ncu=256, per_cu=2):
    nrb, nt = rows_pad // TILE, m_pad // TILE
    ngroups = -(-nrb // (WAVES * rb))
    work = ngroups * nt
    P = max(1, min(ncu * per_cu, work))
    s = Split(work, nt, P)
    slots = max(s.last(g) - s.first(g) + 1 for g in range(ngroups))
    return nrb, nt, ngroups, s, slots


def xcd_contiguous(b, P):
    q, r = P // XCDS, P % XCDS
    xcd, i = b % XCDS, b // XCDS
    return xcd * q + min(xcd, r) + i


def emulate_lse(xa, ya, rb=1, ncu=256, per_cu=2, colterm=None, c=np.log2(np.e)):
    """Row LSE (plain mode: alpha = 1 on a 0 / -1e30 mask, beta = 0) through the kernels' index math, with the
    score / max / sum arithmetic in float32 as on the GPU (overflow or NaN raises)."""
    rows, K = xa.shape
    m = ya.shape[0]
    kp, rp, mp = pad_dim(K), pad_points(rows), pad_points(m)
    kq = kp // 8
    xr = pack(xa, rows, K, kp)
    yc = pack(ya, m, K, kp)
    u = np.where(np.arange(mp) < m, 0.0, -1.0e30) if colterm is None else colterm
    nrb, nt, ngroups, s, slots = plan(rp, mp, kp, rb, ncu, per_cu)
    part = np.full((slots, rp, 2), np.nan)
    lane = np.arange(64)
    h = lane >> 5
    seen = np.zeros((ngroups, nt), dtype=int)
    for b in range(s.P):
        p = xcd_contiguous(b, s.P)
        u1 = (p + 1) * s.work // s.P
        uu = p * s.work // s.P
        while uu < u1:
            g = uu // nt
            tb = uu - g * nt
            te = min(nt, tb + (u1 - uu))
            slot = p - s.first(g)
            assert 0 <= slot < slots
            seen[g, tb:te] += 1
            for wv in range(WAVES):
                rb0 = (g * WAVES + wv) * rb
                if rb0 >= nrb:
                    continue
                for bb in range(rb):
                    blk = rb0 + bb if rb0 + bb < nrb else rb0
                    M = np.full(64, EMPTY, dtype=np.float32)
                    S = np.zeros(64, dtype=np.float32)
                    cf = np.float32(c)
                    # xv[q][e] of lane l: xr[blk * 32 * kp + (q * 64 + l) * 4 + e]
                    xi = blk * 32 * kp + (np.arange(kq)[:, None, None] * 64 + lane[None, :, None]) * 4 \
                        + np.arange(4)[None, None, :]
                    assert xi.max() < xr.size
                    xv = xr[xi]                                    # (kq, 64, 4)
                    for t in range(tb, te):
                        yi = t * 64 * kq * 4 + (np.arange(kq)[:, None, None] * 64 + lane[None, :, None]) * 4 \
                            + np.arange(4)[None, None, :]
                        assert yi.max() < yc.size
                        yv = yc[yi]                                # (kq, 64, 4)
                        ui = t * 32 + 8 * np.arange(4)[None, :, None] + 4 * h[:, None, None] + np.arange(4)[None, None, :]
                        assert ui.max() < mp
                        init = u[ui].reshape(64, 16)               # lane, reg = 4 q + e
                        # MFMA: D[mrow][ncol] += sum_k A[mrow][k] B[k][ncol]; A[mrow][k] = yv of lane mrow + 32 k,
                        # B[k][ncol] = xv of lane ncol + 32 k; lane l reg r holds D[8 (r/4) + 4 (l/32) + r%4][l%32]
                        A = yv.transpose(1, 0, 2).reshape(64, kq * 4)       # lane -> its kp/2 operand values
                        Bm = xv.transpose(1, 0, 2).reshape(64, kq * 4)
                        D = A[:32] @ Bm[:32].T + A[32:] @ Bm[32:].T          # (mrow, ncol)
                        r = np.arange(16)
                        mrow = 8 * (r[None, :] // 4) + 4 * (lane[:, None] // 32) + (r[None, :] % 4)
                        # zero-initialised MFMA chain, then the column term on the VALU (accumulator units)
                        acc = D[mrow, (lane % 32)[:, None]].astype(np.float32) + init.astype(np.float32)
                        Mn = np.maximum(M, acc.max(axis=1))
                        cf = np.float32(c)
                        with np.errstate(over="raise", invalid="raise"):
                            S = S * np.exp2(cf * (M - Mn)) + np.exp2(cf * (acc - Mn[:, None])).sum(axis=1)
                        M = Mn
                    Mo, So = M[lane ^ 32], S[lane ^ 32]
                    Mn = np.maximum(M, Mo)
                    with np.errstate(over="raise", invalid="raise"):
                        Sn = S * np.exp2(cf * (M - Mn)) + So * np.exp2(cf * (Mo - Mn))
                    if rb0 + bb < nrb:
                        idx = (rb0 + bb) * 32 + lane[:32]
                        assert idx.max() < rp
                        part[slot, idx, 0], part[slot, idx, 1] = Mn[:32], Sn[:32]
            uu += te - tb
    assert np.all(seen == 1), "every (row group, tile) unit exactly once"
    # finalisation
    out = np.empty(rp)
    rows_per_group = 32 * rb * WAVES
    for i in range(rp):
        g = i // rows_per_group
        p0, p1 = s.first(g), s.last(g)
        assert p1 - p0 + 1 <= slots
        v = part[: p1 - p0 + 1, i]
        assert not np.isnan(v).any(), (i, g, p0, p1)
        Mx = v[:, 0].max()
        out[i] = Mx + np.log(np.sum(v[:, 1] * np.exp2(c * (v[:, 0] - Mx))))
    return out[:rows], dict(slots=slots, P=s.P, work=s.work)


@pytest.mark.parametrize("rows,m,K,rb,ncu", [(1, 1, 1, 1, 256), (1, 1, 1, 2, 256), (2, 5, 3, 1, 256), (33, 31, 8, 1, 256), (64, 300, 65, 1, 256),
                                             (300, 100, 5, 2, 256), (257, 1000, 17, 2, 4), (500, 70, 30, 1, 3),
                                             (129, 4097, 12, 1, 8), (1000, 40, 64, 2, 256)])
def test_emulated_partial_and_finalize_match_logsumexp(rows, m, K, rb, ncu):
    rng = np.random.default_rng(rows + m + K)
    xa = rng.normal(size=(rows, K))
    ya = rng.normal(size=(m, K)) * 0.5
    out, info = emulate_lse(xa, ya, rb=rb, ncu=ncu)
    # float32 score arithmetic as on the GPU (float64 contraction): rounding-level agreement
    np.testing.assert_allclose(out, logsumexp(xa @ ya.T, axis=1), rtol=0, atol=2e-5)


@pytest.mark.parametrize("n,m", [(10_000, 10_000), (7355, 8962), (8962, 7355), (65_536, 65_536), (32, 100_000),
                                 (100_000, 32), (2048, 2048), (1, 5)])
@pytest.mark.parametrize("rb", [1, 2])
@pytest.mark.parametrize("ncu", [256, 304, 80])
def test_split_covers_work_and_slot_bounds(n, m, rb, ncu):
    """The stream-K split at full sizes: units covered once, slot indexes below the planned slot count,
    workgroup renumbering a bijection."""
    rp, mp = pad_points(n), pad_points(m)
    nrb, nt, ngroups, s, slots = plan(rp, mp, 64, rb, ncu)
    P = s.P
    ids = sorted(xcd_contiguous(b, P) for b in range(P))
    assert ids == list(range(P))
    starts = [p * s.work // P for p in range(P + 1)]
    assert starts[0] == 0 and starts[-1] == s.work
    for g in range(ngroups):
        p0, p1 = s.first(g), s.last(g)
        assert starts[p0] <= g * nt < starts[p0 + 1] or starts[p0] == starts[p0 + 1] == g * nt
        assert p1 - p0 + 1 <= slots
        # every workgroup that owns a unit of group g is in [p0, p1]
        lo, hi = g * nt, (g + 1) * nt
        owners = [p for p in range(P) if starts[p] < hi and starts[p + 1] > lo]
        assert owners[0] >= p0 and owners[-1] <= p1
    # workspace the host allocates for the partials is slots * rows_pad float2
    assert slots * rp * 8 < 2 ** 31 * 8


def test_pack_layout_roundtrip():
    rng = np.random.default_rng(1)
    for n, d in [(1, 1), (31, 7), (33, 64), (100, 65), (64, 128)]:
        x = rng.normal(size=(n, d))
        kp = pad_dim(d)
        pk = pack(x, n, d, kp)
        npad = pad_points(n)
        # invert: point T*32 + r, coordinate h*kp/2 + 4q + e at ((T*kq + q)*2 + h)*32 + r)*4 + e
        kq = kp // 8
        back = np.zeros((npad, kp))
        for T in range(npad // 32):
            for q in range(kq):
                for h in range(2):
                    for r in range(32):
                        base = (((T * kq + q) * 2 + h) * 32 + r) * 4
                        back[T * 32 + r, h * kp // 2 + 4 * q: h * kp // 2 + 4 * q + 4] = pk[base: base + 4]
        np.testing.assert_array_equal(back[:n, :d], x)
        assert np.all(back[n:] == 0) and np.all(back[:, d:] == 0)
