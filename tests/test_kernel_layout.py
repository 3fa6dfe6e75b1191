"""CPU emulation of the HIP kernels' index arithmetic (trainium-sinkhorn_amd/csrc).

Every load and store of pack_cloud_kernel, lse_partial_kernel (global loads, LDS staging and reads -- for the
staged variant a replay of its LDS ring with barrier epochs --, partial slots) and the merge of the slots (merge_group, sk_epilogue.h) is replayed in numpy with the kernels' own
formulas (workgroup renumbering,
stream-K ranges, partial slots, the power-of-two scale and two-piece fp16 packing, the
v_mfma_f32_32x32x16_f16 operand and accumulator lane mapping, the product order of both row roles, the
scaled accumulator units), asserting that every index is inside its buffer and that the emulated result
equals a direct float64 log-sum-exp. It needs no GPU.
"""

import numpy as np
import pytest
from scipy.special import logsumexp

TILE, WAVES, XCDS, RB, BLOCK = 32, 4, 8, 2, 256   # streamed variant: 4 waves of 2 row blocks
WAVES_K, RB_K, BLOCK_K = 4, 2, 256                 # staged variant: the same 4 waves of 2 row blocks
STREAM_MAX_CHUNKS, COL_TILES = 4, 256        # bf16 row-LSE streams up to nc 4 (fp16: every nc); terms per 256 tiles
FOLD_COL_TILES = 192                         # ... per 192 tiles with the f16x2 contraction (folded, 16 B each)
SEG_COST_NARROW, SEG_COST_WIDE = 6, 4       # cost of a row-group boundary in tiles, kp <= 64 / above (make_plan)
ROWS_PER_GROUP = TILE * RB * WAVES
EMPTY = -1.0e30
FIRST = [0, 0, 1]              # fp16x2 (half-steps): (first-cloud piece, second-cloud piece) of the products
SECOND = [0, 1, 0]
FIRST3 = [0, 0, 1, 0, 1, 2]    # bf16x3 (general row log-sum-exp)
SECOND3 = [0, 1, 0, 2, 1, 0]
CONTRACTIONS = {"f16x2": (2, FIRST, SECOND), "bf16x3": (3, FIRST3, SECOND3)}
PAD_SCORE = np.float32(-1.0e30)


def pad_points(n):
    return -(-n // TILE) * TILE


def pad_dim(d):
    return -(-d // 16) * 16


def pack_scale(m):
    """The power-of-two scale of a cloud with max |coordinate| m: m * s in [2^4, 2^5), clamped."""
    if not m > 0:
        return np.float32(1.0)
    e = np.frexp(np.float32(m))[1]                      # m in [2^(e-1), 2^e)
    k = -32 if e > 37 else (40 if e < -35 else 5 - e)
    return np.float32(np.ldexp(1.0, k))


def split2(v):
    """float32 (already scaled) -> two fp16 pieces, as float32."""
    v = np.asarray(v, dtype=np.float32)
    a0 = v.astype(np.float16).astype(np.float32)
    a1 = (v - a0).astype(np.float32).astype(np.float16).astype(np.float32)
    return a0, a1


def bf16_rne(v):
    """float32 -> nearest bfloat16 (ties to even), returned as float32."""
    u = np.asarray(v, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def split3(v):
    v = np.asarray(v, dtype=np.float32)
    a0 = bf16_rne(v)
    r1 = (v - a0).astype(np.float32)
    a1 = bf16_rne(r1)
    a2 = bf16_rne((r1 - a1).astype(np.float32))
    return a0, a1, a2


def fold_split(v):
    """The f16x2 contraction's column term v as the A operand of one v_mfma_f32_32x32x16_bf16 against B = 1 in
    k = 0..5 (sk_lse_partial.hip, column_operand): the exact three-way bf16 split q0 + q1 + q2 = v with q0 in four
    equal quarters, (q0 / 4, q0 / 4, q0 / 4, q0 / 4, q1, q2). Returns the six pieces as float32 values."""
    q0, q1, q2 = split3(v)
    qq = bf16_rne((q0 * np.float32(0.25)).astype(np.float32))
    return qq, qq, qq, qq, q1, q2


def fold_b_operand():
    """B of the column MFMA, per lane: ones in k = 0..5 of lanes 0-31, zeros elsewhere."""
    b = np.zeros((64, 8), dtype=np.float32)
    b[:32, :6] = 1.0
    return b


def mfma_bf16_add(acc, pieces):
    """What v_mfma_f32_32x32x16_bf16 returns for the accumulator `acc` (float32 array) plus the products
    `pieces` (bf16 values against B = 1), by the rule measured on gfx950 (4.2 million accumulator / term pairs,
    either sign, |acc| / |term| from 2^-14 to 2^3, every result reproduced): the accumulator is floored onto the
    grid of half an ulp of the largest product, 2^(e - 24) for a largest product in [2^e, 2^(e+1)), products
    below that grid are dropped, and the sum is rounded to the nearest float32."""
    acc = np.asarray(acc, dtype=np.float64)
    ps = np.stack([np.broadcast_to(np.asarray(p, dtype=np.float64), acc.shape) for p in pieces])
    big = np.abs(ps).max(axis=0)
    e = np.floor(np.log2(np.where(big > 0, big, 1.0)))
    grid = np.where(big > 0, 2.0 ** (e - 24), 0.0)
    safe = np.where(grid > 0, grid, 1.0)
    kept = np.where(np.abs(ps) >= grid, ps, 0.0).sum(axis=0)
    floored = np.where(grid > 0, np.floor(acc / safe) * safe, acc)
    return (floored + kept).astype(np.float32)


FP16_FOLD_MAX = np.float32(2.0 ** 30)
FP16_FOLD_SCALES = (2.0 ** 15, 2.0 ** 4, 2.0 ** -7)


def fp16_fold_split(v):
    """An earlier form of the folded column term, kept here as a planted mistake: three fp16 pieces against
    B = (2^15, 2^4, 2^-7), which only reach +-2^30 (terms beyond are clamped)."""
    w = (np.clip(np.asarray(v, dtype=np.float32), -FP16_FOLD_MAX, FP16_FOLD_MAX) * np.float32(2.0 ** -15)
         ).astype(np.float32)
    q0 = w.astype(np.float16).astype(np.float32)
    r1 = ((w - q0) * np.float32(2.0 ** 11)).astype(np.float32)
    q1 = r1.astype(np.float16).astype(np.float32)
    q2 = ((r1 - q1) * np.float32(2.0 ** 11)).astype(np.float32).astype(np.float16).astype(np.float32)
    return q0, q1, q2


def fp16_fold_b_operand():
    b = np.zeros((64, 8), dtype=np.float32)
    b[:32, :3] = FP16_FOLD_SCALES
    return b


def pack(src, n, d, contraction="f16x2"):
    """pack_cloud_kernel (f16x2: header, max |x|, scaled two fp16 pieces) or pack_cloud_bf3_kernel (bf16x3:
    three exact bf16 pieces, scale 1): (scale, the (npad / 32 * nc * pieces * 64, 8) array of 16-byte units as
    8 float32 values)."""
    PIECES = CONTRACTIONS[contraction][0]
    kp = pad_dim(d)
    nc = kp // 16
    npad = pad_points(n)
    if contraction == "f16x2":
        s = pack_scale(np.abs(src[:n, :d]).max() if n * d else 0.0)
    else:
        s = np.float32(1.0)
    out = np.full((npad // TILE * nc * PIECES * 64, 8), np.nan, dtype=np.float32)
    idx = np.arange(npad // TILE * nc * 64)                  # one thread per (tile, chunk, lane)
    lane = idx % 64
    cc = (idx // 64) % nc
    T = idx // (64 * nc)
    r, h = lane & 31, lane >> 5
    row = T * TILE + r
    e = np.arange(8)
    k = 16 * cc[:, None] + 8 * h[:, None] + e[None, :]
    ok = (row[:, None] < n) & (k < d)
    flat = np.where(ok, row[:, None] * d + k, 0)
    assert flat.max() < src.size
    v = (np.where(ok, src.ravel()[flat], 0.0).astype(np.float32) * s).astype(np.float32)
    pieces = split2(v) if contraction == "f16x2" else split3(v)
    base = (T * nc + cc) * (PIECES * 64) + lane
    for p in range(PIECES):
        dst = base + 64 * p
        assert dst.max() < out.shape[0]
        out[dst] = pieces[p]
    assert not np.isnan(out).any(), "every unit written"
    return s, out


class Split:
    """sk_common.h's Split: units on a cost line where every row-group boundary costs alpha positions."""

    def __init__(self, nt, ngroups, P, alpha):
        self.nt, self.ngroups, self.P, self.alpha = nt, ngroups, P, alpha
        self.work = nt * ngroups
        self.ftot = self.work + alpha * (ngroups - 1)
        self.q, self.r = divmod(self.ftot, P)

    def cost_start(self, p):
        return p * self.q + (p * self.r) // self.P

    def unit_at(self, c):
        span = self.nt + self.alpha
        g, rem = divmod(c, span)
        return g * self.nt + min(rem, self.nt)

    def start(self, p):
        return self.unit_at(self.cost_start(p))

    def owner(self, x):
        fx = x + self.alpha * (x // self.nt)
        return min(((fx + 1) * self.P - 1) // self.ftot, self.P - 1)

    def first(self, g):
        return self.owner(g * self.nt)

    def last(self, g):
        return self.owner((g + 1) * self.nt - 1)


def plan(rows_pad, m_pad, ncu=256, per_cu=1, nc=4, alpha=None):
    nrb, nt = rows_pad // TILE, m_pad // TILE
    ngroups = -(-rows_pad // ROWS_PER_GROUP)
    work = ngroups * nt
    P = max(1, min(ncu * per_cu, 1024, work))
    if alpha is None:
        alpha = SEG_COST_NARROW if nc <= STREAM_MAX_CHUNKS else SEG_COST_WIDE
    s = Split(nt, ngroups, P, alpha)
    slots = max(s.last(g) - s.first(g) + 1 for g in range(ngroups))
    return nrb, nt, ngroups, s, slots


def xcd_contiguous(b, P):
    q, r = P // XCDS, P % XCDS
    xcd, i = b % XCDS, b // XCDS
    return xcd * q + min(xcd, r) + i


def mfma_32x32x16(Aop, Bop):
    """v_mfma_f32_32x32x16_f16 on per-lane operands (64, 8): lane l holds A[m = l % 32][k = 8 (l / 32) + e] and
    B[k = 8 (l / 32) + e][n = l % 32]. Returns the (64, 16) accumulator: lane l, register r holds
    D[m = 8 (r / 4) + 4 (l / 32) + r % 4][n = l % 32]."""
    A = np.concatenate([Aop[:32], Aop[32:]], axis=1).astype(np.float64)    # (m, k)
    B = np.concatenate([Bop[:32], Bop[32:]], axis=1).astype(np.float64)    # (n, k)
    D = A @ B.T                                                             # (m, n); fp16 products exact
    lane = np.arange(64)
    r = np.arange(16)
    m = 8 * (r[None, :] // 4) + 4 * (lane[:, None] // 32) + r[None, :] % 4
    return D[m, (lane % 32)[:, None]]


def ring_depth(nc):
    """Register slots of the staged kernel's column-chunk ring (sk_lse_partial.hip ring_depth)."""
    return 4 if (2 * nc) % 4 == 0 else 2


def staged_protocol(segments, nc, pieces, products, ahead=2):
    """Replay the LDS protocol of the staged kernel (sk_lse_partial.hip Staged::run, the bf16 row log-sum-exp above
    kp 64) over the work segments of one workgroup, in program order, with barrier epochs: a write becomes visible
    to the other waves at the next barrier, and waves interleave arbitrarily between barriers. Asserts that every
    read (column chunks into the register ring, the column terms of the previous tile) sees data staged for the
    tile it belongs to (min(t, last)), written in an earlier epoch and not rewritten in the same epoch, and that
    every MFMA takes its chunk from the ring slot holding it. `ahead` is the stage distance in tiles (two in the
    kernel; other values are planted mistakes). Returns the number of barriers."""
    D = ring_depth(nc)
    LA = D - 1
    NS = products * nc * RB_K
    stage_slot = NS // 2
    visible = {}                  # ("y", lds tile buffer) / ("c", column buffer) -> tile id
    pending = {}                  # writes of the current epoch
    reads = set()                 # regions read in the current epoch
    barriers = [0]

    def write(key, tile):
        assert key not in reads, f"write after read in one epoch: {key}"
        pending[key] = tile

    def read(key, tile):
        assert key not in pending, f"read of {key} rewritten in the same epoch"
        assert visible.get(key) == tile, f"{key} holds {visible.get(key)}, expected tile {tile}"
        reads.add(key)

    def barrier():
        visible.update(pending)
        pending.clear()
        reads.clear()
        barriers[0] += 1

    for tb, te in segments:
        last = te - 1
        clamp = lambda t: t if t < te else last                           # noqa: E731
        sets = [None, None]                        # the tile id held by each register set (tile and column inputs)

        def prefetch(sset, t):
            sets[sset] = clamp(t)

        def stage(sset, ybuf, cbuf):
            write(("y", ybuf), sets[sset])
            write(("c", cbuf), sets[sset])

        ring = {}
        yq, cq = 0, 0

        def read_chunk(g, ytile, tile):
            read(("y", ytile), tile)
            ring[g % D] = (tile, g % nc)

        prefetch(0, tb)
        prefetch(1, tb + 1)
        stage(0, 0, 0)
        stage(1, 1, 1)
        prefetch(0, tb + 2)
        prefetch(1, tb + 3)
        barrier()
        for g in range(LA):
            read_chunk(g, 0, clamp(tb))

        def tile(ph, t, prev):
            nonlocal yq, cq
            ynext = (yq + 1) % 3
            for i in range(NS):
                # MFMA slot i: chunk cc, product p, row block b (b innermost, as the kernel issues them)
                cc, p, b = i // (products * RB_K), (i // RB_K) % products, i % RB_K
                g = ph * nc + cc
                if p == 0 and b == 0:
                    if cc + LA < nc:
                        read_chunk((g + LA) % (2 * nc), yq, clamp(t))
                    else:
                        read_chunk((g + LA) % (2 * nc), ynext, clamp(t + 1))
                assert ring[g % D] == (clamp(t), cc), (t, cc, ring[g % D])
                if i == 0 and prev is not None:
                    read(("c", prev[0]), prev[1])                         # the previous tile's column terms
                if i == stage_slot - 2:
                    write(("c", (cq + ahead) % 4), sets[ph])
                if i == stage_slot:
                    write(("y", (yq + ahead) % 3), sets[ph])
                if i == stage_slot + 1:
                    sets[ph] = clamp(t + 4)                               # the tile four ahead, then its column inputs
            yq, cq = (yq + 1) % 3, (cq + 1) % 4
            barrier()
            return ((cq + 3) % 4, clamp(t))

        prev = tile(0, tb, None)
        t = tb + 1
        while te - t >= 2:
            prev = tile(1, t, prev)
            prev = tile(0, t + 1, prev)
            t += 2
        if t < te:
            prev = tile(1, t, prev)
        read(("c", prev[0]), prev[1])                                     # the last update's column terms
        barrier()
    return barriers[0]


def emulate_lse(xa, ya, role=0, ncu=256, per_cu=1, c=np.log2(np.e), contraction="bf16x3", col=None,
                fold_rule=(fold_split, fold_b_operand)):
    """Row LSE (plain mode: alpha = 1 on a 0 / -1e30 mask, beta = 0) through the kernels' index math, the
    score / max / sum arithmetic in float32 as on the GPU (overflow or NaN raises). The product's row-LSE entry
    point uses bf16x3; f16x2 (the half-steps' packing) runs through the same index math here.
    With `col` (pad_points(m) column terms in accumulator units, padding included), the half-step's scores
    c (x.y + col_j) instead: the result is then L_i = M_i + log2(S_i) / c in accumulator units (the plain mode's
    natural-log LSE for c = log2(e)). `fold_rule` is the (pieces, B operand) pair of the folded column term."""
    PIECES, FIRST_, SECOND_ = CONTRACTIONS[contraction]
    rows, K = xa.shape
    m = ya.shape[0]
    kp, rp, mp = pad_dim(K), pad_points(rows), pad_points(m)
    nc = kp // 16
    tile16 = nc * PIECES * 64
    staged_variant = nc > STREAM_MAX_CHUNKS and contraction != "f16x2"   # sk_lse_partial.hip streamed_form
    waves, rbk, block = (WAVES_K, RB_K, BLOCK_K) if staged_variant else (WAVES, RB, BLOCK)
    per_thread = -(-tile16 // block)
    sx, xr = pack(xa, rows, K, contraction)
    sy, yc = pack(ya, m, K, contraction)
    sigma, inv_sigma = np.float32(sx * sy), np.float32((1 / sx) * (1 / sy))
    if col is None:
        u_raw = np.where(np.arange(mp) < m, 0.0, -1.0e30).astype(np.float32)
    else:
        u_raw = np.asarray(col, dtype=np.float32)
        assert u_raw.shape == (mp,)
    with np.errstate(over="ignore"):
        u = np.maximum((u_raw * sigma).astype(np.float32), PAD_SCORE)     # scaled column term, floored
    nrb, nt, ngroups, s, slots = plan(rp, mp, ncu, per_cu, nc=nc)
    fold = contraction == "f16x2"
    part = np.full((slots, rp, 2), np.nan)
    lane = np.arange(64)
    h = lane >> 5
    tid = np.arange(block)
    seen = np.zeros((ngroups, nt), dtype=int)
    cf = np.float32(np.float32(c) * inv_sigma)
    ra, ca = (FIRST_, SECOND_) if role == 0 else (SECOND_, FIRST_)
    for b in range(s.P):
        p = xcd_contiguous(b, s.P)
        u1 = s.start(p + 1)
        uu = s.start(p)
        while uu < u1:
            g = uu // nt
            tb = uu - g * nt
            te = min(nt, tb + (u1 - uu))
            slot = p - s.first(g)
            assert 0 <= slot < slots
            seen[g, tb:te] += 1
            staged = {}
            if not staged_variant:
                # streamed: column terms of runs of col_tiles tiles into LDS; operands straight from memory.
                # Folded (f16x2): 16 bytes per column, the A operand of the column MFMA (lane l: column l % 32).
                col_tiles = FOLD_COL_TILES if fold else COL_TILES
                lds_col = np.full((col_tiles * 32, 8) if fold else col_tiles * 32, np.nan, dtype=np.float32)
                for t0 in range(tb, te, col_tiles):
                    t1 = min(t0 + col_tiles, te)
                    k = np.arange((t1 - t0) * 32)
                    assert k.max() < lds_col.shape[0] and (t0 * 32 + k).max() < mp
                    if fold:
                        lds_col[k] = 0.0
                        for sl, piece in enumerate(fold_rule[0](u[t0 * 32 + k])):
                            lds_col[k, sl] = piece
                    else:
                        lds_col[k] = u[t0 * 32 + k]
                    for t in range(t0, t1):
                        rd = (t - t0) * 32 + (lane & 31 if fold else np.arange(32))
                        assert rd.max() < lds_col.shape[0]
                        gi = t * tile16 + np.arange(tile16)
                        assert gi.max() < yc.shape[0]
                        staged[t] = (yc[gi].copy(), lds_col[rd].copy())
                loads = [min(t + 1, te - 1) for t in range(tb, te)]      # the one-ahead operand loads
                assert max(loads) * tile16 + tile16 - 1 < yc.shape[0]
            if staged_variant:
                # staged: the LDS protocol of the ring (asserted), then each tile's operands and column terms
                staged_protocol([(tb, te)], nc, PIECES, len(FIRST_))
                for k in range(per_thread):
                    idx = np.where(tid + k * block < tile16, tid + k * block, tile16 - 1)
                    assert idx.max() < tile16 and (te - 1) * tile16 + idx.max() < yc.shape[0]
                for t in range(tb, te):
                    assert t * 32 + 31 < mp
                    gi = t * tile16 + np.arange(tile16)
                    staged[t] = (yc[gi].copy(), u[t * 32 + np.arange(32)].copy())
            for wv in range(waves):
                rb0 = (g * waves + wv) * rbk
                for bb in range(rbk):
                    blk = rb0 + bb if rb0 + bb < nrb else nrb - 1
                    xi = blk * tile16 + (np.arange(nc)[:, None, None] * PIECES + np.arange(PIECES)[None, :, None]) * 64 \
                        + lane[None, None, :]
                    assert xi.max() < xr.shape[0]
                    xv = xr[xi]                                    # (nc, 3, 64, 8)
                    M = np.full(64, EMPTY, dtype=np.float32)
                    S = np.zeros(64, dtype=np.float32)
                    for t in range(tb, te):
                        ybuf, cbuf = staged[t]
                        yi = (np.arange(nc)[:, None, None] * PIECES + np.arange(PIECES)[None, :, None]) * 64 \
                            + lane[None, None, :]
                        assert yi.max() < tile16
                        yv = ybuf[yi]
                        acc = np.zeros((64, 16))
                        for cc in range(nc):
                            for pp in range(len(FIRST_)):
                                acc += mfma_32x32x16(yv[cc, ca[pp]], xv[cc, ra[pp]])
                        if fold:                                   # the column MFMA, after the dot product
                            acc += mfma_32x32x16(cbuf, fold_rule[1]())
                            a = acc.astype(np.float32)
                        else:
                            ci = 8 * np.arange(4)[None, :, None] + 4 * h[:, None, None] + np.arange(4)[None, None, :]
                            assert ci.max() < 32
                            col = cbuf[ci].reshape(64, 16)
                            a = (acc.astype(np.float32) + col).astype(np.float32)
                        Mn = np.maximum(M, a.max(axis=1))
                        with np.errstate(over="raise", invalid="raise"):
                            S = S * np.exp2(cf * (M - Mn)) + np.exp2(cf * (a - Mn[:, None])).sum(axis=1)
                        M = Mn
                    Mo, So = M[lane ^ 32], S[lane ^ 32]
                    Mn = np.maximum(M, Mo)
                    with np.errstate(over="raise", invalid="raise"):
                        Sn = S * np.exp2(cf * (M - Mn)) + So * np.exp2(cf * (Mo - Mn))
                    if rb0 + bb < nrb:
                        idx = (rb0 + bb) * 32 + lane[:32]
                        assert idx.max() < rp
                        part[slot, idx, 0] = np.maximum(Mn[:32] * inv_sigma, np.float32(EMPTY))
                        part[slot, idx, 1] = Sn[:32]
            uu += te - tb
    assert np.all(seen == 1), "every (row group, tile) unit exactly once"
    out = np.empty(rp)
    for i in range(rp):
        g = i // ROWS_PER_GROUP
        p0, p1 = s.first(g), s.last(g)
        assert p1 - p0 + 1 <= slots
        v = part[: p1 - p0 + 1, i]
        assert not np.isnan(v).any(), (i, g, p0, p1)
        Mx = v[:, 0].max()
        out[i] = Mx + np.log2(np.sum(v[:, 1] * np.exp2(c * (v[:, 0] - Mx)))) / c
    return out[:rows], dict(slots=slots, P=s.P, work=s.work)


@pytest.mark.parametrize("rows,m,K,ncu,role,ct", [(1, 1, 1, 256, 0, "bf16x3"), (1, 1, 1, 256, 1, "f16x2"),
                                                  (2, 5, 3, 256, 0, "f16x2"), (33, 31, 8, 256, 1, "f16x2"),
                                                  (64, 300, 65, 256, 0, "bf16x3"), (300, 100, 5, 3, 1, "f16x2"),
                                                  (257, 1000, 17, 4, 0, "bf16x3"), (500, 70, 30, 3, 0, "f16x2"),
                                                  (129, 1500, 12, 8, 1, "f16x2"), (600, 40, 128, 256, 0, "f16x2"),
                                                  (40, 9000, 64, 1, 1, "f16x2"), (70, 300, 100, 1, 0, "bf16x3")])
def test_emulated_partial_and_finalize_match_logsumexp(rows, m, K, ncu, role, ct):
    rng = np.random.default_rng(rows + m + K)
    xa = rng.normal(size=(rows, K)).astype(np.float32)
    ya = (rng.normal(size=(m, K)) * 0.5).astype(np.float32)
    out, info = emulate_lse(xa, ya, role=role, ncu=ncu, contraction=ct)
    np.testing.assert_allclose(out, logsumexp(xa.astype(np.float64) @ ya.astype(np.float64).T, axis=1),
                               rtol=0, atol=2e-5)


@pytest.mark.parametrize("n,m", [(10_000, 10_000), (7355, 8962), (8962, 7355), (65_536, 65_536), (32, 100_000),
                                 (100_000, 32), (2048, 2048), (1, 5), (5, 150_000), (150_000, 5), (2, 200_000),
                                 (40_000, 1), (6, 120_000), (120_000, 6), (1_000_000, 7), (9, 1_000_000)])
@pytest.mark.parametrize("ncu,per_cu", [(256, 1), (304, 1), (80, 1), (256, 2)])
def test_split_covers_work_and_slot_bounds(n, m, ncu, per_cu):
    """The stream-K split at full sizes: units covered once and each owned by the workgroup whose range holds
    it, every slot a merge reads written by a workgroup with units in that row group, slot indexes below the
    planned slot count, workgroup renumbering a bijection; all in 32-bit range."""
    rp, mp = pad_points(n), pad_points(m)
    for nc in (4, 8):
        nrb, nt, ngroups, s, slots = plan(rp, mp, ncu, per_cu, nc=nc)
        P = s.P
        assert s.ftot < 2 ** 31 and P <= 1024
        ids = sorted(xcd_contiguous(b, P) for b in range(P))
        assert ids == list(range(P))
        starts = np.array([s.start(p) for p in range(P + 1)])
        assert starts[0] == 0 and starts[-1] == s.work and (np.diff(starts) >= 0).all()
        x = np.arange(s.work)
        fx = x + s.alpha * (x // nt)
        owner = np.minimum(((fx + 1) * P - 1) // s.ftot, P - 1)
        assert (owner == np.searchsorted(starts, x, side="right") - 1).all()
        for g in range(ngroups):
            p0, p1 = s.first(g), s.last(g)
            assert p1 - p0 + 1 <= slots
            lo, hi = g * nt, (g + 1) * nt
            for p in range(p0, p1 + 1):
                assert starts[p] < hi and starts[p + 1] > lo and starts[p + 1] > starts[p], (g, p)
        assert slots * rp * 8 < 2 ** 31 * 8


def _costs(s, starts):
    """Per workgroup: tiles + alpha * (row-group boundaries its range crosses)."""
    out = []
    for p in range(s.P):
        a, b = starts[p], starts[p + 1]
        segs = 0 if b == a else (b - 1) // s.nt - a // s.nt + 1
        out.append(b - a + s.alpha * max(segs - 1, 0))
    return np.array(out)


def make_div(d):
    """sk_common.h make_div: k the smallest with d <= 2^k, m = ceil(2^(31 + k) / d)."""
    k = (d - 1).bit_length()
    return -(-(1 << (31 + k)) // d), k


def div_by(n, md):
    """sk_common.h div_by: floor(2n m / 2^32) >> k, in 32-bit unsigned arithmetic as the kernels do it."""
    m, k = md
    assert 0 <= n < 2 ** 31 and 2 ** 31 <= m < 2 ** 32 or m == 2 ** 31
    return (((2 * n) & 0xFFFFFFFF) * m >> 32) >> k


def test_split_division_by_multiply_high_is_exact():
    """The split's divisions by its per-launch constants (P, nt + alpha, nt, ftot) are one multiply-high each:
    exact for every dividend below 2^31 (the split's positions and owner products, which the planner keeps
    there). Divisors 1 to 2^31 at and around powers of two, the plans' usual sizes and random ones; dividends at
    the multiples of the divisor and around them, the top of the range and random ones."""
    rng = np.random.default_rng(17)
    ds = {1, 2, 3, 7, 31, 32, 33, 313, 319, 1023, 1024, 1025, 2 ** 31 - 1, 2 ** 31}
    ds |= {2 ** e + o for e in range(1, 31) for o in (-1, 0, 1)}
    ds |= set(int(v) for v in rng.integers(1, 2 ** 31, 400))
    for d in sorted(ds):
        md = make_div(d)
        top = (2 ** 31 - 1) // d * d
        ns = {0, 1, d - 1, d, d + 1, 2 * d - 1, 2 * d, top - 1, top, 2 ** 31 - 2, 2 ** 31 - 1}
        ns |= set(int(v) for v in rng.integers(0, 2 ** 31, 60))
        for n in ns:
            if 0 <= n < 2 ** 31:
                assert div_by(n, md) == n // d, (n, d)
    # a planted mistake (m rounded down instead of up) is caught
    d = 3
    m_floor = (1 << (31 + 2)) // d
    assert any((((2 * n) * m_floor >> 32) >> 2) != n // d for n in range(0, 3000))


def test_split_balances_segment_costs():
    """Workgroups whose range crosses a row-group boundary get about alpha fewer tiles: every workgroup's cost
    is within one tile plus alpha of ftot / P, and at 10k x 10k the largest cost is below the equal-tiles
    split's."""
    for n, m in [(10_000, 10_000), (7355, 8962), (65_536, 65_536), (2048, 2048), (300, 100_000)]:
        rp, mp = pad_points(n), pad_points(m)
        nrb, nt, ngroups, s, slots = plan(rp, mp, 256, 1, nc=4)
        starts = [s.start(p) for p in range(s.P + 1)]
        cost = _costs(s, starts)
        assert cost.max() <= s.q + 1 + s.alpha, (n, m, cost.max(), s.q)
        u = Split(nt, ngroups, s.P, 0)
        uniform = _costs(Split(nt, ngroups, s.P, s.alpha), [p * u.work // s.P for p in range(s.P + 1)])
        if (n, m) == (10_000, 10_000):
            assert cost.max() < uniform.max(), (cost.max(), uniform.max())


def test_scale_and_split2_error_bound():
    rng = np.random.default_rng(1)
    for mag in (1.0, 1e-3, 7.3e4, 1e-7, 3e12, 1e-10):  # the full-precision range: max |x| in [2^-35, 7e13]
        x = (rng.normal(size=100_000) * mag).astype(np.float32)
        s = pack_scale(np.abs(x).max())
        scaled_max = np.abs(x).max() * s
        assert ((2.0 ** 4 <= scaled_max < 2.0 ** 5) or (s == 2.0 ** 40 and scaled_max < 2.0 ** 4)
                or (s == 2.0 ** -32 and 2.0 ** 5 <= scaled_max < 2.0 ** 14))
        v = (x * s).astype(np.float32)
        np.testing.assert_array_equal(v.astype(np.float64), x.astype(np.float64) * float(s))   # exact scaling
        a0, a1 = split2(v)
        for a in (a0, a1):                          # each piece is an fp16 value
            np.testing.assert_array_equal(a, a.astype(np.float16).astype(np.float32))
        err = np.abs(a0.astype(np.float64) + a1 - v)
        assert np.all(err <= 2.0 ** -23 * np.abs(v) + 2.0 ** -25)
        assert err.max() <= 2.0 ** -22 * scaled_max                    # relative to the cloud's largest value
    assert pack_scale(7.0e13) * 7.0e13 <= 2.0 ** 14 and pack_scale(0.0) == 1.0
    # below 2^-26 the scale is clamped and the smallest pieces are fp16 subnormals: precision degrades
    x = (rng.normal(size=10_000) * 1e-14).astype(np.float32)
    s = pack_scale(np.abs(x).max())
    a0, a1 = split2((x * s).astype(np.float32))
    assert s == 2.0 ** 40 and np.abs(a0.astype(np.float64) + a1 - x * float(s)).max() <= 2.0 ** -18 * np.abs(x).max() * s


def test_three_products_are_fp32_accurate_and_symmetric():
    """The three piece products reproduce x.y at least as accurately as a float32 dot product, and the
    transposed product order of the other row role adds the same terms in the same order."""
    rng = np.random.default_rng(2)
    x = rng.normal(size=(50, 64)).astype(np.float32)
    y = (rng.normal(size=(40, 64)) + 0.5).astype(np.float32)
    sx, sy = pack_scale(np.abs(x).max()), pack_scale(np.abs(y).max())
    xs, ys = split2(x * sx), split2(y * sy)
    exact = x.astype(np.float64) @ y.astype(np.float64).T
    bound = np.abs(x.astype(np.float64)) @ np.abs(y.astype(np.float64)).T
    approx = sum(xs[FIRST[p]].astype(np.float64) @ ys[SECOND[p]].astype(np.float64).T for p in range(len(FIRST)))
    approx /= float(sx) * float(sy)
    err = np.max(np.abs(approx - exact) / bound)
    assert err < 2.0 ** -22
    assert err < np.max(np.abs((x @ y.T).astype(np.float64) - exact) / bound)    # a float32 dot product

    def accumulate(role, rows, cols, swap_rule=True):
        """float32 sum of the products in issue order, with the kernel's piece choice for `role`."""
        ra, ca = (FIRST, SECOND) if (role == 0 or not swap_rule) else (SECOND, FIRST)
        acc = np.zeros((rows[0].shape[0], cols[0].shape[0]), dtype=np.float32)
        for p in range(len(ra)):
            acc = (acc + (rows[ra[p]].astype(np.float64) @ cols[ca[p]].astype(np.float64).T).astype(np.float32))
        return acc

    f = accumulate(0, xs, ys)            # f update: rows x (role 0)
    g = accumulate(1, ys, xs)            # g update: rows y (role 1)
    np.testing.assert_array_equal(f, g.T)
    # a rule that does not transpose the piece order for role 1 adds the cross terms in another order
    g_wrong = accumulate(1, ys, xs, swap_rule=False)
    assert np.abs(f - g_wrong.T).max() > 0


def bake_log2(xs, sx, sy, mx, c):
    """sk_epilogue.h bake_params / bake_unit: the first cloud's log2-unit copy, pieces of t fl(c x) / s_y where
    x = (x0 + x1) / s_x, and its unit t (1 while max |fl(c x)| / s_y lies in [2^-1, 2^15), else the power of two
    that brings it into [2^4, 2^5), within [2^-40, 2^40]); None where no unit fits."""
    c = np.float32(c)
    wmax = np.float32(np.float32(c * np.float32(mx)) * np.float32(1.0 / sy))
    t = np.float32(1.0)
    if wmax > 0 and not (0.5 <= wmax < 32768.0):
        e = np.frexp(wmax)[1]
        t = np.float32(np.ldexp(1.0, int(np.clip(5 - e, -40, 40))))
    if not (c > 0 and 0.5 <= wmax * t < 32768.0):
        return None
    x = ((xs[0] + xs[1]).astype(np.float32) * np.float32(1.0 / sx)).astype(np.float32)
    w = (((c * x).astype(np.float32) * np.float32(1.0 / sy)).astype(np.float32) * t).astype(np.float32)
    return split2(w), t


@pytest.mark.parametrize("eps,shift", [(0.1, 0.5), (0.01, 0.0), (1.0, 0.0), (0.05, 3.0)])
def test_log2_copy_gives_c_x_dot_y_to_fp32_accuracy(eps, shift):
    """With the first cloud's log2-unit copy, the three piece products against the second cloud's own pieces
    sum to c x.y (c = fp32(2/eps) log2 e, the kernels' score scale) with no scaling left: as accurate as the
    own-scale contraction times c, the transposed product order still adds the same terms in the same order,
    and the per-score VALU form exp2(a - m) equals exp2(c (a_acc - m_acc)) to rounding."""
    rng = np.random.default_rng(3)
    x = rng.normal(size=(60, 64)).astype(np.float32)
    y = (rng.normal(size=(50, 64)) + shift).astype(np.float32)
    sx, sy = pack_scale(np.abs(x).max()), pack_scale(np.abs(y).max())
    xs, ys = split2(x * sx), split2(y * sy)
    c = np.float32(np.float32(2.0 / eps) * np.float32(np.log2(np.e)))
    ws, t = bake_log2(xs, sx, sy, np.abs(x).max(), c)
    assert t == 1.0
    for p in range(2):
        np.testing.assert_array_equal(ws[p], ws[p].astype(np.float16).astype(np.float32))
    exact = float(c) * (x.astype(np.float64) @ y.astype(np.float64).T)
    bound = float(c) * (np.abs(x.astype(np.float64)) @ np.abs(y.astype(np.float64)).T)
    approx = sum(ws[FIRST[p]].astype(np.float64) @ ys[SECOND[p]].astype(np.float64).T for p in range(3))
    err = np.max(np.abs(approx - exact) / bound)
    assert err < 2.0 ** -21, err
    assert err < np.max(np.abs(float(c) * (x @ y.T).astype(np.float64) - exact) / bound)    # c times an fp32 dot

    def accumulate(rows, cols, ra, ca):
        acc = np.zeros((rows[0].shape[0], cols[0].shape[0]), dtype=np.float32)
        for p in range(3):
            acc = (acc + (rows[ra[p]].astype(np.float64) @ cols[ca[p]].astype(np.float64).T).astype(np.float32))
        return acc

    np.testing.assert_array_equal(accumulate(ws, ys, FIRST, SECOND), accumulate(ys, ws, SECOND, FIRST).T)


def test_log2_copy_unit_and_window():
    """The copy's unit: t = 1 while max |fl(c x)| / s_y stays in [2^-1, 2^15) (the pieces then hold the
    copy as before), a power of two bringing it into [2^4, 2^5) outside that window (tiny or huge score
    scales), and no copy only for c = 0 or past the unit's range. With any unit the three piece products
    divided by t give c x.y to fp32 accuracy; without the rescaling (a planted mistake) they are off by t."""
    rng = np.random.default_rng(4)
    y = rng.normal(size=(20, 8)).astype(np.float32)
    sy = pack_scale(np.abs(y).max())
    ys = split2(y * sy)
    for mag, c, unit in [(1.0, 28.85, "one"), (1e-6, 28.85, "up"), (1e6, 288.5, "down"), (30.0, 2.885, "one"),
                         (3e-3, 2.885, "up"), (1.0, 0.0, None), (1e-30, 1e-8, None)]:
        x = (rng.normal(size=(20, 8)) * mag).astype(np.float32)
        sx = pack_scale(np.abs(x).max())
        got = bake_log2(split2(x * sx), sx, sy, np.abs(x).max(), c)
        if unit is None:
            assert got is None, (mag, c)
            continue
        ws, t = got
        wmax = np.float32(np.float32(np.float32(c) * np.abs(x).max()) / sy)
        assert {"one": t == 1.0, "up": t > 1.0, "down": t < 1.0}[unit], (mag, c, t)
        if unit != "one":
            assert 16.0 <= wmax * t < 32.0
        exact = float(np.float32(c)) * (x.astype(np.float64) @ y.astype(np.float64).T)
        bound = float(np.float32(c)) * (np.abs(x.astype(np.float64)) @ np.abs(y.astype(np.float64)).T)
        approx = sum(ws[FIRST[p]].astype(np.float64) @ ys[SECOND[p]].astype(np.float64).T for p in range(3))
        assert np.max(np.abs(approx / t - exact) / bound) < 2.0 ** -21, (mag, c)
        if t != 1.0:
            assert np.max(np.abs(approx - exact) / bound) > 0.4


@pytest.mark.parametrize("ct", ["f16x2", "bf16x3"])
def test_pack_layout_roundtrip(ct):
    rng = np.random.default_rng(1)
    PIECES = CONTRACTIONS[ct][0]
    for n, d in [(1, 1), (31, 7), (33, 64), (100, 65), (64, 128)]:
        x = rng.normal(size=(n, d)).astype(np.float32)
        kp = pad_dim(d)
        nc = kp // 16
        s, pk = pack(x, n, d, ct)
        npad = pad_points(n)
        back = np.zeros((npad, kp))
        for T in range(npad // TILE):
            for cc in range(nc):
                for p in range(PIECES):
                    for lane in range(64):
                        r, h = lane & 31, lane >> 5
                        unit = pk[((T * nc + cc) * PIECES + p) * 64 + lane]
                        back[T * TILE + r, 16 * cc + 8 * h:16 * cc + 8 * h + 8] += unit
        v = x.astype(np.float64) * float(s)
        if ct == "bf16x3":
            np.testing.assert_array_equal(back[:n, :d], v)                  # exact
        else:
            assert np.all(np.abs(back[:n, :d] - v) <= 2.0 ** -23 * np.abs(v) + 2.0 ** -25)
        assert np.all(back[n:] == 0) and np.all(back[:, d:] == 0)


def test_split3_is_exact_over_the_fp32_range():
    """The row-LSE packing: three bf16 pieces reproduce any fp32 value exactly, whatever its magnitude (the
    augmented padding rows hold -1e9 next to values of order 1)."""
    rng = np.random.default_rng(1)
    for scale in (1.0, 1e-3, 7.3e4, 1e-20, 3e30, 1e9):
        v = (rng.normal(size=100_000) * scale).astype(np.float32)
        a0, a1, a2 = split3(v)
        for a in (a0, a1, a2):
            assert np.all((a.view(np.uint32) & 0xFFFF) == 0)
        np.testing.assert_array_equal(a0.astype(np.float64) + a1 + a2, v.astype(np.float64))


def test_fold_split_reproduces_column_terms():
    """The folded column term: its six bf16 pieces summed against B = 1 reproduce every fp32 value of magnitude
    2^-98 or more exactly (bf16 has fp32's exponent range: no clamp, the -1e30 padding floor included), and
    smaller ones within 2^-124 (the quarters and the third piece then fall among bf16's subnormals); a plausible
    slip, a piece dropped or q0 taken whole beside its quarters, is caught."""
    rng = np.random.default_rng(5)
    b = fold_b_operand()[0]
    assert np.all(b[:6] == 1.0) and np.all(b[6:] == 0.0)

    def back(ps):
        return sum(p.astype(np.float64) * b[k] for k, p in enumerate(ps))

    for scale in (1e-35, 1e-29, 1e-9, 1e-3, 0.3, 1.0, 7.3e2, 6.1e4, 1e7, 3e8, 1.3e9, 4e12, 1e30):
        v = (rng.normal(size=200_000) * scale).astype(np.float32)
        ps = fold_split(v)
        assert len(ps) == 6
        for q in ps:
            assert np.all(np.isfinite(q)) and np.all((q.view(np.uint32) & 0xFFFF) == 0)
        big = np.abs(v) >= 2.0 ** -98
        np.testing.assert_array_equal(back(ps)[big], v[big].astype(np.float64))
        assert np.abs(back(ps) - v.astype(np.float64)).max() <= 2.0 ** -124
    edge = np.array([-1e30, 2.0 ** 30, -3e9, 3.0e38], dtype=np.float32)
    np.testing.assert_array_equal(back(fold_split(edge)), edge.astype(np.float64))
    v = (rng.normal(size=1000) * 100).astype(np.float32)
    ps = fold_split(v)
    assert np.abs(back(ps[:5]) - v).max() > 1e-4                        # the third piece dropped
    assert np.abs(back((split3(v)[0],) + ps[1:]) - v).max() > 1.0       # q0 beside its last three quarters


def test_column_mfma_rounding_bias_of_the_quarter_split():
    """By the column MFMA's measured rounding rule (mfma_bf16_add), a dot product much smaller than the column term
    comes out a quarter ulp low on average when the term's leading bf16 piece is one product (the old three-piece
    operand), and a sixteenth of an ulp low with that piece in quarters (the kernel's six-piece operand); a
    compensating piece below the accumulator's grid is dropped and changes nothing. The rule itself reproduces
    the gfx950 results it was measured on bit for bit; here it checks that the split the kernel uses gets the
    bias the measurement found (-0.249 and -0.060 ulp of the result)."""
    rng = np.random.default_rng(17)
    n = 400_000
    q = (2.0 ** rng.uniform(-3, 12, n) * np.where(rng.uniform(size=n) < 0.5, -1, 1)).astype(np.float32)
    acc = (np.abs(q) * 2.0 ** rng.uniform(-14, -6, n) * np.where(rng.uniform(size=n) < 0.5, -1, 1)).astype(np.float32)
    exact = acc.astype(np.float64) + q.astype(np.float64)
    ulp = np.spacing(np.abs(exact.astype(np.float32))).astype(np.float64)

    def bias(pieces):
        return float(((mfma_bf16_add(acc, pieces).astype(np.float64) - exact) / ulp).mean())

    three = split3(q)
    b3, b6 = bias(three), bias(fold_split(q))
    assert -0.27 < b3 < -0.23, b3
    assert -0.075 < b6 < -0.045, b6
    g = 2.0 ** (np.floor(np.log2(np.abs(three[0].astype(np.float64)))) - 24)
    comp = bf16_rne((g / 2).astype(np.float32))
    assert abs(bias(three + (comp,)) - b3) < 1e-3
    # round to nearest (the VALU add) is unbiased; the rule is not just that
    rn = float(((exact.astype(np.float32).astype(np.float64) - exact) / ulp).mean())
    assert abs(rn) < 0.01


def _half_step_lse_f64(x, y, col):
    """float64 L_i = (eps / 2) LSE_j((2 x_i.y_j + gh_j) / eps + log b_j) = LSE in accumulator units
    (a_ij = x_i.y_j + col_j, col_j = (gh_j + eps log b_j) / 2) with c = (2 / eps) log2(e): returned for the
    caller's c as max_j a_ij + log2(sum_j 2^(c (a_ij - max))) / c."""
    a = x.astype(np.float64) @ y.astype(np.float64).T + col[None, :]
    mx = a.max(axis=1)
    return mx, a


@pytest.mark.parametrize("case", ["tiny", "mixed"])
def test_folded_column_terms_cover_small_and_mixed_scale_clouds(case):
    """Regression for the folded column term's range: clouds at 1e-4 scale (d 16, 500 x 500: every cloud scale
    2^16, so sigma = 2^32 and eps log b / 2 = -0.31 becomes -1.3e9 in kernel units) and mixed scales (x at 2e-7,
    y ~ N(0, 1), gh ~ -|y|^2: sigma = 2^27, sigma |gh| / 2 ~ 6e9), normalize=False, m not a multiple of 32. The bf16 fold
    gives the float64 log-sum-exp; the earlier fp16 fold, clamped at +-2^30, loses every column's identity."""
    rng = np.random.default_rng(11)
    eps = 0.1
    c = np.float32(2.0 / eps * np.log2(np.e))
    if case == "tiny":
        n, m, d = 500, 500, 16
        x = (rng.normal(size=(n, d)) * 1e-4).astype(np.float32)
        y = (rng.normal(size=(m, d)) * 1e-4).astype(np.float32)
        gh = np.zeros(m)
    else:
        n, m, d = 300, 470, 64
        x = (rng.normal(size=(n, d)) * 2e-7).astype(np.float32)
        y = rng.normal(size=(m, d)).astype(np.float32)
        gh = -(y.astype(np.float64) ** 2).sum(1) + rng.normal(scale=0.05, size=m)
    log_b = np.log(rng.uniform(0.5, 1.5, m) / m)
    mp = pad_points(m)
    col = np.full(mp, 0.5 * eps * -1e9)                       # padding: gh 0, log weight -1e9
    col[:m] = 0.5 * (gh + eps * log_b)
    col32 = col.astype(np.float32)
    mx, a = _half_step_lse_f64(x, y, col32[:m].astype(np.float64))
    want = mx + np.log2(np.exp2(c * (a - mx[:, None])).sum(1)) / c
    sx = pack_scale(np.abs(x).max())
    sy = pack_scale(np.abs(y).max())
    assert np.abs(col32[:m]).max() * sx * sy > 2.0 ** 30        # the terms the fp16 fold had to clamp
    got, _ = emulate_lse(x, y, col=col32, c=c, contraction="f16x2")
    # (eps / 2) of a float32 half-step's rounding: the float32 scores' ulp, c |a| 2^-24, in accumulator units
    tol = 4 * np.abs(a).max() * 2.0 ** -24 + 1e-12
    assert np.abs(got - want).max() <= tol, (np.abs(got - want).max(), tol)
    bad, _ = emulate_lse(x, y, col=col32, c=c, contraction="f16x2", fold_rule=(fp16_fold_split, fp16_fold_b_operand))
    assert np.abs(bad - want).max() > 1e3 * tol



@pytest.mark.parametrize("nc", [5, 6, 7, 8])
def test_staged_ring_protocol(nc):
    """The staged kernel's LDS ring (the bf16 row log-sum-exp above kp 64: three tile buffers, four column
    buffers, the column chunks read ahead into a register ring) over segments of every length from 1 to 13 tiles,
    one after another in one workgroup as the work split hands them out: every read sees its own tile's data,
    staged in an earlier barrier epoch and not rewritten in its own; one barrier per tile plus two per segment."""
    pieces, first, _ = CONTRACTIONS["bf16x3"]
    lengths = range(1, 14)
    segs, t0 = [], 0
    for n in lengths:
        segs.append((t0, t0 + n))
        t0 += n + 3
    nb = staged_protocol(segs, nc, pieces, len(first))
    assert nb == sum(2 + n for n in lengths)


@pytest.mark.parametrize("nc", [5, 8])
@pytest.mark.parametrize("ahead", [1, 3])
def test_staged_ring_protocol_catches_a_wrong_stage_distance(nc, ahead):
    """Planted mistakes: staging the tile `ahead` tiles ahead instead of two. One ahead writes the buffer whose
    first chunks the current tile's last MFMAs read; three ahead (into buffer q % 3, the current tile's own)
    rewrites operands still being read."""
    pieces, first, _ = CONTRACTIONS["bf16x3"]
    with pytest.raises(AssertionError):
        staged_protocol([(0, 9)], nc, pieces, len(first), ahead=ahead)


def _round_down_f32(v):
    """float64 -> float32 rounded toward -inf (a model of the column MFMA's downward rounding of its sum)."""
    r = v.astype(np.float32)
    below = r.astype(np.float64) > v
    r[below] = np.nextafter(r[below], np.float32(-np.inf))
    return r


def _loop_log2_weights(log_w, n, with_lo=True):
    """The on-device loop's log2 weights of one cloud (loop_log2_kernel, sk_kernels.hip): L0 = rint(log2(e) max
    log w) over the fp32 log weights, and log2(e) (log_w + log_w_lo) - L0 = Lh + Ll as two floats (Ll = 0 on
    padding), from the host's log_w = fp32(log w), log_w_lo = fp32(log w - log_w) (zeros without it)."""
    lw = np.asarray(log_w, dtype=np.float64)
    lw32 = lw.astype(np.float32)
    lo32 = (lw - lw32.astype(np.float64)).astype(np.float32) if with_lo else np.zeros_like(lw32)
    L0 = float(np.float32(np.rint(np.log2(np.e) * float(lw32[:n].max()))))
    L = np.log2(np.e) * (lw32.astype(np.float64) + lo32.astype(np.float64)) - L0
    lh = L.astype(np.float32)
    ll = (L - lh.astype(np.float64)).astype(np.float32)
    ll[n:] = 0.0
    return L0, lh, ll


def _emulate_balanced_loop_drift(x, y, la, lb, eps, iters, weights):
    """A balanced Sinkhorn loop in the kernel's log2 units (R = (c / 2) fh, column terms rounded once to float32 as
    the partial kernel stages them, everything else in float64) against the same loop in float64 throughout;
    returns the mean difference of f. `weights`: "loop" (Lh + fl(R + Ll), the kernel's), "no lo" (the same without
    the host's log_w_lo: float32 log weights), or "fp32" (the column term fl(R + log2(e) fp32(log w)) less the
    offset, the earlier form)."""
    c = 2.0 / eps * np.log2(np.e)
    D = c * (x @ y.T)                                               # the dot part in log2 units
    ys, xs = (y ** 2).sum(1), (x ** 2).sum(1)

    def colterm(R, lw, side):
        if weights == "fp32":
            L0 = float(np.rint(np.log2(np.e) * lw.astype(np.float32).max()))
            return (R.astype(np.float64) + np.log2(np.e) * lw.astype(np.float32).astype(np.float64)).astype(np.float32) \
                .astype(np.float64) - L0, L0
        L0, lh, ll = side
        u2 = (R.astype(np.float64) + ll.astype(np.float64)).astype(np.float32)
        return (lh.astype(np.float64) + u2.astype(np.float64)).astype(np.float32).astype(np.float64), L0

    def step(Dm, R_cols, lw_cols, side):
        q, L0 = colterm(R_cols, lw_cols, side)
        a = Dm + q[None, :]
        M = a.max(1)
        return -(M + L0 + np.log2(np.exp2(a - M[:, None]).sum(1)))

    lo = weights != "no lo"
    sx, sy = _loop_log2_weights(la, len(la), lo), _loop_log2_weights(lb, len(lb), lo)
    Rx, Ry = np.zeros(len(x), np.float32), np.zeros(len(y), np.float32)
    Fx, Fy = np.zeros(len(x)), np.zeros(len(y))                    # the float64 loop (log2 units, exact weights)
    for _ in range(iters):
        Rx = step(D, Ry, lb, sy).astype(np.float32)
        Ry = step(D.T, Rx, la, sx).astype(np.float32)
        Fx = -np.log2(np.exp2(D + (Fy + np.log2(np.e) * lb)[None, :]).sum(1))
        Fy = -np.log2(np.exp2(D.T + (Fx + np.log2(np.e) * la)[None, :]).sum(1))
    k2 = c / 2
    return float(np.mean(Rx.astype(np.float64) / k2 - Fx / k2)), float(np.abs(Fx / k2 + xs).max())


def test_loop_log2_weights_hold_the_balanced_iteration_still_at_large_eps():
    """At an eps far above the cost scale a balanced iteration moves its potentials along the neutral mode by eps
    times the log of the two marginals' effective total masses' ratio, every iteration. Log weights rounded to
    float32 leave that ratio at a few 1e-8 (a float64 run has none), so f drifts linearly; the on-device loop's log2
    weights, log2(e) log w - L0 = Lh + Ll carried to float64 precision with Ll kept in the stored potential and
    the column term Lh + fl(R + Ll) rounded once, keep the drift at rounding level. Emulated on a raw cloud pair at
    eps 20 times the mean cost; leaving out the host's low parts of the log weights (a plausible slip) brings the
    drift back."""
    rng = np.random.default_rng(23)
    n, m, d = 97, 311, 16
    x = rng.normal(size=(n, d))
    y = rng.normal(size=(m, d)) + 0.3
    a = rng.uniform(0.2, 1.8, n)
    b = rng.uniform(0.2, 1.8, m)
    la, lb = np.log(a / a.sum()), np.log(b / b.sum())
    mass32 = np.log(np.exp(lb.astype(np.float32).astype(np.float64)).sum() /
                    np.exp(la.astype(np.float32).astype(np.float64)).sum())
    assert abs(mass32) > 3e-9                                      # the float32 weights' mass mismatch
    L0, lh, ll = _loop_log2_weights(lb, m)
    mass_loop = np.log(np.exp2(lh.astype(np.float64) + ll + L0).sum())
    assert abs(mass_loop) < 1e-13                                   # the loop's weights: float64 masses
    eps = 20.0 * 2.0 * d
    iters = 40
    drift32, fscale = _emulate_balanced_loop_drift(x, y, la, lb, eps, iters, "fp32")
    drift_loop, _ = _emulate_balanced_loop_drift(x, y, la, lb, eps, iters, "loop")
    drift_lh, _ = _emulate_balanced_loop_drift(x, y, la, lb, eps, iters, "no lo")
    expect = iters * eps * abs(mass32)                              # eps log(mass ratio) per iteration
    assert abs(drift32) > 0.3 * expect, (drift32, expect)
    assert abs(drift_lh) > 0.3 * expect, (drift_lh, expect)
    assert abs(drift_loop) < 0.1 * abs(drift32), (drift_loop, drift32)
    assert abs(drift_loop) < 2e-7 * fscale, (drift_loop, fscale)
