// The MFMA partial (max, sum) kernel of the fused Sinkhorn half-step, gfx950.
//
// Built with -fno-honor-nans -mno-amdgpu-ieee: row maxima are taken directly over MFMA results, which in
// IEEE mode would first be canonicalised one by one. No value here is NaN or infinite: padding and empty
// rows use large finite sentinels.
//
// Per row i and column j the kernel forms the dot product D_ij = x_i . y_j with v_mfma_f32_32x32x2_f32
// chains that start from zero (A = 32 columns of the packed y tile, B = 32 rows of packed x held in
// registers), then a_ij = D_ij + alpha u_j + beta v_j on the VALU, and keeps per lane a running (M, S) with
// S = sum_j exp2(c (a_ij - M)).
//
// Why the contraction starts from zero on unscaled coordinates: a v_mfma_f32_32x32x2_f32 chain rounds like
// chained round-to-nearest FMAs, in the same coordinate order whichever cloud is A and which is B, so the
// f update (rows x, columns y) and the g update (rows y, columns x) get bit-identical x_i . y_j. In the cold
// regime (eps much smaller than the cost spread) a row's log-sum-exp is a single dominant score, and any
// rounding that differs between the two directions pushes f_i + g_j of that pair by the difference in every
// iteration: the potentials would drift linearly along the pair's neutral mode. (The reference's PyTorch
// path has the same property: x @ y^T and y @ x^T round alike.) For the same reason the max is subtracted
// before scaling, exp2(c (a - M)): the dominant term is exactly 1.
//
// The tile loop is a two-stage software pipeline: while the MFMAs of tile t run, the loads of tile t + 1
// are in flight and the column term, max, exp and sum of tile t - 1 are issued between the MFMAs.

#include "sk_common.h"

namespace sk {
namespace {

__device__ __forceinline__ float ex2(float x) { return __builtin_amdgcn_exp2f(x); }

// Hardware hands consecutive workgroup ids to the 8 XCDs in turn; renumber so that the workgroups of one
// XCD own one contiguous range of the work (their column tiles then share that XCD's L2).
__device__ __forceinline__ int xcd_contiguous(int b, int P) {
    const int q = P / kXcds, r = P % kXcds;
    const int xcd = b % kXcds, idx = b / kXcds;
    return xcd * q + (xcd < r ? xcd : r) + idx;
}

// Online log-sum-exp update of one lane's row with 16 new scores a = D + colterm (accumulator units).
__device__ __forceinline__ void lse_update(const f32x16& acc, const f32x16& col, float& M, float& S, float c) {
    f32x16 a;
#pragma unroll
    for (int r = 0; r < 16; ++r) a[r] = acc[r] + col[r];
    const float m0 = fmaxf(fmaxf(a[0], a[1]), fmaxf(a[2], a[3]));
    const float m1 = fmaxf(fmaxf(a[4], a[5]), fmaxf(a[6], a[7]));
    const float m2 = fmaxf(fmaxf(a[8], a[9]), fmaxf(a[10], a[11]));
    const float m3 = fmaxf(fmaxf(a[12], a[13]), fmaxf(a[14], a[15]));
    const float Mn = fmaxf(M, fmaxf(fmaxf(m0, m1), fmaxf(m2, m3)));
    float e[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) e[r] = ex2(c * (a[r] - Mn));
    const float s0 = (e[0] + e[1]) + (e[2] + e[3]);
    const float s1 = (e[4] + e[5]) + (e[6] + e[7]);
    const float s2 = (e[8] + e[9]) + (e[10] + e[11]);
    const float s3 = (e[12] + e[13]) + (e[14] + e[15]);
    S = fmaf(S, ex2(c * (M - Mn)), (s0 + s1) + (s2 + s3));
    M = Mn;
}

template <int KQ>
struct Tile {
    const f32x4* y;   // packed columns + lane
    const f32x4* u;   // u + 4 h
    const f32x4* v;   // v + 4 h

    __device__ __forceinline__ void load_y(int t, f32x4 (&out)[KQ]) const {
#pragma unroll
        for (int q = 0; q < KQ; ++q) out[q] = y[(size_t)t * (64 * KQ) + q * 64];
    }
    // Column term inputs of the lane's 16 accumulator rows: columns t * 32 + 8 q + 4 h + (0..3).
    __device__ __forceinline__ void load_uv(int t, f32x4 (&uu)[4], f32x4 (&vv)[4]) const {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            uu[q] = u[t * 8 + q * 2];
            vv[q] = v[t * 8 + q * 2];
        }
    }
};

// Column term of the lane's 16 accumulator rows (columns t * 32 + 8 q + 4 h + e, register 4 q + e).
__device__ __forceinline__ void col_term(f32x16& col, const f32x4 (&uu)[4], const f32x4 (&vv)[4], float alpha,
                                         float beta) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
#pragma unroll
        for (int e = 0; e < 4; ++e) col[4 * q + e] = fmaf(beta, vv[q][e], alpha * uu[q][e]);
    }
}

// D = x . y for RB row blocks against one column tile, from zero.
template <int KQ, int RB>
__device__ __forceinline__ void tile_mfma(f32x16 (&acc)[RB], const f32x4 (&yv)[KQ], const f32x4 (&xv)[RB][KQ]) {
#pragma unroll
    for (int b = 0; b < RB; ++b) acc[b] = f32x16{};
#pragma unroll
    for (int q = 0; q < KQ; ++q) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
#pragma unroll
            for (int b = 0; b < RB; ++b)
                acc[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(yv[q][e], xv[b][q][e], acc[b], 0, 0, 0);
        }
    }
}

template <int RB>
__device__ __forceinline__ void update_all(const f32x16 (&acc)[RB], const f32x16& col, float (&M)[RB], float (&S)[RB],
                                           float c) {
#pragma unroll
    for (int b = 0; b < RB; ++b) lse_update(acc[b], col, M[b], S[b], c);
}

template <int KQ, int RB>
__device__ __forceinline__ void run_segment(const PartialArgs& a, int rb0, int tb, int te, int slot, float alpha,
                                            float beta, float c) {
    constexpr int KP = 8 * KQ;
    const int lane = threadIdx.x & 63;
    const int h = lane >> 5;

    f32x4 xv[RB][KQ];
#pragma unroll
    for (int b = 0; b < RB; ++b) {
        const bool ok = rb0 + b < a.nrb;
        const f32x4* src = reinterpret_cast<const f32x4*>(a.xr + (size_t)(ok ? rb0 + b : rb0) * (32 * KP)) + lane;
#pragma unroll
        for (int q = 0; q < KQ; ++q) xv[b][q] = src[q * 64];
    }

    float M[RB], S[RB];
#pragma unroll
    for (int b = 0; b < RB; ++b) {
        M[b] = kEmpty;
        S[b] = 0.0f;
    }

    Tile<KQ> tl;
    tl.y = reinterpret_cast<const f32x4*>(a.yc) + lane;
    tl.u = reinterpret_cast<const f32x4*>(a.u + 4 * h);
    tl.v = reinterpret_cast<const f32x4*>(a.v + 4 * h);

    f32x4 ya[KQ], yb[KQ], uu[4], vv[4];
    f32x16 accA[RB], accB[RB], colA, colB;
    const int last = te - 1;

    // Phase for tile t: (1) the column term of tile t from loads issued one phase earlier, (2) the loads of
    // tile t + 1, then (3) the MFMAs of tile t interleaved with the update of tile t - 1. The scheduling
    // fences keep the loads a whole MFMA chain ahead of their first use.
    tl.load_y(tb, ya);
    tl.load_uv(tb, uu, vv);
    col_term(colA, uu, vv, alpha, beta);
    {
        const int tn = tb + 1 < te ? tb + 1 : last;
        tl.load_y(tn, yb);
        tl.load_uv(tn, uu, vv);
    }
    __builtin_amdgcn_sched_barrier(0);
    tile_mfma<KQ, RB>(accA, ya, xv);
    __builtin_amdgcn_sched_barrier(0);
    int t = tb + 1;
    while (t + 1 < te) {
        // yb / uu / vv hold tile t; accA / colA hold tile t - 1.
        col_term(colB, uu, vv, alpha, beta);
        tl.load_y(t + 1, ya);
        tl.load_uv(t + 1, uu, vv);
        __builtin_amdgcn_sched_barrier(0);
        tile_mfma<KQ, RB>(accB, yb, xv);
        update_all<RB>(accA, colA, M, S, c);
        __builtin_amdgcn_sched_barrier(0);
        // ya / uu / vv hold tile t + 1; accB / colB hold tile t.
        col_term(colA, uu, vv, alpha, beta);
        {
            const int tn = t + 2 < te ? t + 2 : last;
            tl.load_y(tn, yb);
            tl.load_uv(tn, uu, vv);
        }
        __builtin_amdgcn_sched_barrier(0);
        tile_mfma<KQ, RB>(accA, ya, xv);
        update_all<RB>(accB, colB, M, S, c);
        __builtin_amdgcn_sched_barrier(0);
        t += 2;
    }
    if (t < te) {
        // yb / uu / vv hold tile t (the last); accA / colA hold tile t - 1.
        col_term(colB, uu, vv, alpha, beta);
        tile_mfma<KQ, RB>(accB, yb, xv);
        update_all<RB>(accA, colA, M, S, c);
        update_all<RB>(accB, colB, M, S, c);
    } else {
        update_all<RB>(accA, colA, M, S, c);
    }

    // Lanes l and l + 32 hold the same row over different columns: merge them, then store.
#pragma unroll
    for (int b = 0; b < RB; ++b) {
        const float Mo = __shfl_xor(M[b], 32);
        const float So = __shfl_xor(S[b], 32);
        const float Mn = fmaxf(M[b], Mo);
        const float Sn = S[b] * ex2(c * (M[b] - Mn)) + So * ex2(c * (Mo - Mn));
        if (h == 0 && rb0 + b < a.nrb)
            a.part[(size_t)slot * a.rows_pad + (size_t)(rb0 + b) * 32 + lane] = make_float2(Mn, Sn);
    }
}

template <int KQ, int RB>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(2, 2)))
void lse_partial_kernel(PartialArgs a) {
    if (a.skip != nullptr && *a.skip != 0) return;
    const int wv = threadIdx.x >> 6;
    const int P = a.s.P;
    const int p = xcd_contiguous(blockIdx.x, P);

    // a_ij = x_i . y_j + alpha u_j + beta v_j in accumulator units, scores exp2(c (a - M)):
    // half-step: a = x . y + (gh + eps log b) / 2, c = (2 / eps) log2(e); plain row-LSE: a = xa . ya + mask,
    // c = log2(e).
    float alpha, beta, c;
    if (a.mode == kHalfStep) {
        alpha = 0.5f;
        beta = 0.5f * a.sc[2];
        c = a.sc[0] * kLog2e;
    } else {
        alpha = 1.0f;
        beta = 0.0f;
        c = kLog2e;
    }

    const long long u1 = (long long)(p + 1) * a.s.work / P;
    for (long long u = (long long)p * a.s.work / P; u < u1;) {
        const int g = (int)(u / a.s.nt);
        const int tb = (int)(u - (long long)g * a.s.nt);
        const long long left = u1 - u;
        const int te = left < (long long)(a.s.nt - tb) ? tb + (int)left : a.s.nt;
        const int slot = p - first_wg(g, a.s);
        const int rb0 = (g * kWaves + wv) * RB;
        if (rb0 < a.nrb) run_segment<KQ, RB>(a, rb0, tb, te, slot, alpha, beta, c);
        u += te - tb;
    }
}

template <int KQ>
hipError_t launch_kq(const PartialArgs& a, int rb, hipStream_t st) {
    if (rb == 2)
        hipLaunchKernelGGL((lse_partial_kernel<KQ, 2>), dim3(a.s.P), dim3(kBlock), 0, st, a);
    else
        hipLaunchKernelGGL((lse_partial_kernel<KQ, 1>), dim3(a.s.P), dim3(kBlock), 0, st, a);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_partial(const PartialArgs& a, int kq, int rb, hipStream_t st) {
    switch (kq) {
        case 1: return launch_kq<1>(a, rb, st);
        case 2: return launch_kq<2>(a, rb, st);
        case 3: return launch_kq<3>(a, rb, st);
        case 4: return launch_kq<4>(a, rb, st);
        case 5: return launch_kq<5>(a, rb, st);
        case 6: return launch_kq<6>(a, rb, st);
        case 7: return launch_kq<7>(a, rb, st);
        case 8: return launch_kq<8>(a, rb, st);
        case 9: return launch_kq<9>(a, rb, st);
        case 10: return launch_kq<10>(a, rb, st);
        case 11: return launch_kq<11>(a, rb, st);
        case 12: return launch_kq<12>(a, rb, st);
        case 13: return launch_kq<13>(a, rb, st);
        case 14: return launch_kq<14>(a, rb, st);
        case 15: return launch_kq<15>(a, rb, st);
        case 16: return launch_kq<16>(a, rb, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace sk
