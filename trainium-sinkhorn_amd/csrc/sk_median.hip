// Exact median of the squared-Euclidean cost over all pairs, on the GPU: the normalisation
// "cost / median(cost)" of src/trnopt/sinkhorn.py:229-233 (wot's), which the reference computes on the host
// by materialising the n x m float64 cost matrix (527 MB at 7,355 x 8,962) and calling np.median.
//
//     C_ij = max((|x_i|^2 + |y_j|^2) - 2 x_i . y_j, 0)        in float64, x and y already centred
//     median = (C_(k0) + C_(k1)) / 2,   k0 = floor((N - 1) / 2), k1 = floor(N / 2),  N = n m
//
// (np.median's definition: the middle element for odd N, the mean of the two middle ones for even N.)
//
// Radix select on the fused cost stream: non-negative doubles order like their bit patterns, so the k-th
// smallest cost is found digit by digit from the top (11, 11, 11, 11, 11, 9 bits). A pass recomputes every
// C_ij tile by tile (256 rows x 32 columns per step: one row per thread, the dot products in registers, the
// column coordinates from zero-padded copies through the scalar cache), keeps the pairs whose high bits equal
// the prefix found so far, and histograms their next digit in LDS; a one-workgroup scan then picks the digit
// holding rank k and narrows the prefix. The two ranks k0 and k1 share one histogram while their prefixes
// agree. The third pass also collects the keys that still match a rank's prefix (a small fraction: a 22-bit
// prefix) into the workspace, and the last three passes read only those; when there are more than the
// workspace holds (massive ties), they recompute every cost instead. Every launch goes on the caller's stream
// with no host round trip.

#include <hip/hip_runtime.h>

#include <stdint.h>

#include <algorithm>

#include "sk_common.h"

namespace {

using sk::fail;
using sk::hip_fail;

constexpr int kBins = 2048;                 // 11-bit digits
constexpr int kRowsPerBlock = 256;          // one row per thread
constexpr int kColTile = 32;                // column points per LDS tile
constexpr int kTargetBlocks = 1024;         // workgroups a pass aims for (4 per CU): columns per workgroup follow
constexpr int kChunk = 8;                   // coordinates per register chunk of the row
constexpr int kPasses = 6;
constexpr int kCompactPass = 2;             // this pass also collects the keys matching its prefix ...
constexpr unsigned long long kCandMax = 1ull << 22;   // ... up to this many; later passes read only those
constexpr int kShift[kPasses] = {53, 42, 31, 20, 9, 0};
constexpr int kWidth[kPasses] = {11, 11, 11, 11, 11, 9};

struct SelectState {
    unsigned long long prefix[2];   // bits of the answer known so far (above the current digit)
    unsigned long long k[2];        // rank still to find among the pairs that match the prefix
    int same;                       // 1 while both ranks have the same prefix (one histogram serves both)
    int pad;
};

__global__ void norms_kernel(const double* __restrict__ p, int n, int d, double* __restrict__ out) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const double* r = p + (size_t)i * d;
    double s = 0.0;
    for (int k = 0; k < d; ++k) s = fma(r[k], r[k], s);
    out[i] = s;
}

__global__ void select_init_kernel(SelectState* st, unsigned* __restrict__ hist, unsigned long long* count,
                                   unsigned long long N) {
    for (int b = threadIdx.x; b < 2 * kBins; b += blockDim.x) hist[b] = 0u;
    if (threadIdx.x == 0) {
        *count = 0ull;
        st->prefix[0] = st->prefix[1] = 0ull;
        st->k[0] = (N - 1ull) / 2ull;
        st->k[1] = N / 2ull;
        st->same = 1;
    }
}

__device__ __forceinline__ unsigned long long cost_key(double c) {
    // max(c, 0); -0.0 and +0.0 are the same cost and the same key
    const unsigned long long b = (unsigned long long)__double_as_longlong(c > 0.0 ? c : 0.0);
    return b & 0x7fffffffffffffffull;
}

// Row-major copy of p (n x d) with rows of dp coordinates (zeros after d) and zero rows up to n_pad.
__global__ void pad_kernel(const double* __restrict__ p, int n, int d, int n_pad, int dp, double* __restrict__ out) {
    const long long total = (long long)n_pad * dp;
    for (long long e = (long long)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (long long)gridDim.x * blockDim.x) {
        const long long i = e / dp;
        const int k = (int)(e - i * dp);
        out[e] = i < n && k < d ? p[i * d + k] : 0.0;
    }
}

// How a full pass relates to the candidate keys.
enum PassMode { kPlain = 0, kCollect = 1, kIfOverflow = 2 };

constexpr unsigned kStage = 2048;           // collected keys a workgroup stages in LDS before one reservation

__device__ __forceinline__ unsigned long long readlane64(unsigned long long v, int lane) {
    const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)v, lane);
    const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(v >> 32), lane);
    return ((unsigned long long)hi << 32) | lo;
}

// Collect the wave's lanes with `take`: into the workgroup's LDS stage while it has room (reservations are
// contiguous from 0, so the filled part is [0, *fill)), else straight into cand with a reservation of the
// wave's own. Keys past cap are counted, not stored, so that *count > cap tells the later passes to
// recompute instead.
__device__ __forceinline__ void collect(bool take, unsigned long long key, unsigned long long* stage,
                                        unsigned* reserved, unsigned* fill, unsigned long long* cand,
                                        unsigned long long* count, unsigned long long cap) {
    const unsigned long long bal = __ballot(take);
    if (bal == 0ull) return;
    const int lane = (int)(threadIdx.x & 63);
    const int leader = __ffsll((long long)bal) - 1;
    const unsigned cnt = (unsigned)__popcll(bal);
    const unsigned below = (unsigned)__popcll(bal & ((1ull << lane) - 1ull));
    unsigned sb = 0u;
    if (lane == leader) sb = atomicAdd(reserved, cnt);
    sb = (unsigned)__builtin_amdgcn_readlane((int)sb, leader);
    if (sb + cnt <= kStage) {
        if (take) stage[sb + below] = key;
        if (lane == leader) atomicMax(fill, sb + cnt);
        return;
    }
    unsigned long long base = 0ull;
    if (lane == leader) base = atomicAdd(count, (unsigned long long)cnt);
    const unsigned long long idx = readlane64(base, leader) + below;
    if (take && idx < cap) cand[idx] = key;
}

// One digit pass over the workgroup's block of 256 rows x `cols` columns, on the zero-padded copies (rows of
// dp coordinates, a multiple of 8; the column copy padded to whole tiles of 32 points). Each thread keeps its
// row's dot products with a tile of 32 column points in registers and takes the row's coordinates 8 at a
// time; the column coordinates are the same for every lane, so they come through the scalar cache as
// operands of the fma (no LDS traffic). The dot products sum over k in ascending order, one fma each; the
// padding adds 0 * 0.
// The column copy is read through the constant address space: its addresses are the same for every lane, and
// this keeps them on scalar loads whatever else the kernel stores.
typedef __attribute__((address_space(4))) const double ConstDouble;

template <int MODE>
__global__ __launch_bounds__(kRowsPerBlock) void select_pass_kernel(
    const double* __restrict__ xp, const double* __restrict__ yp, const double* __restrict__ xx,
    const double* __restrict__ yy, int n, int m, int dp, int cols, const SelectState* __restrict__ st,
    unsigned* __restrict__ hist, int shift, int width, unsigned long long* __restrict__ cand,
    unsigned long long* __restrict__ count, unsigned long long cap) {
    __shared__ unsigned h[2][kBins];
    __shared__ unsigned long long stage[MODE == kCollect ? kStage : 1];
    __shared__ unsigned reserved, fill;
    __shared__ unsigned long long stage_base;
    if (MODE == kIfOverflow && *count <= cap) return;     // the candidate pass below does this digit
    const int tid = threadIdx.x;
    if (tid == 0) reserved = fill = 0u;
    const int same = st->same;
    const unsigned long long high = shift + width >= 64 ? 0ull : ~((1ull << (shift + width)) - 1ull);
    const unsigned long long p0 = st->prefix[0] & high, p1 = st->prefix[1] & high;
    const unsigned dmask = (1u << width) - 1u;
    for (int b = tid; b < 2 * kBins; b += kRowsPerBlock) (&h[0][0])[b] = 0u;
    __syncthreads();

    const int i = blockIdx.x * kRowsPerBlock + tid;
    const bool row_ok = i < n;
    const double xi2 = row_ok ? xx[i] : 0.0;
    const double* xr = xp + (size_t)(row_ok ? i : 0) * dp;
    const int j_begin = blockIdx.y * cols;
    const long long j_lim = (long long)j_begin + cols;
    const int j_end = j_lim < m ? (int)j_lim : m;

    for (int j0 = j_begin; j0 < j_end; j0 += kColTile) {
        const int nj = j_end - j0 < kColTile ? j_end - j0 : kColTile;
        const ConstDouble* yt = (const ConstDouble*)(yp + (size_t)j0 * dp);
        double acc[kColTile];
#pragma unroll
        for (int jj = 0; jj < kColTile; ++jj) acc[jj] = 0.0;
        for (int k0 = 0; k0 < dp; k0 += kChunk) {
            double xv[kChunk];
#pragma unroll
            for (int e = 0; e < kChunk; ++e) xv[e] = xr[k0 + e];
#pragma unroll
            for (int jj = 0; jj < kColTile; ++jj) {
                const ConstDouble* yr = yt + (size_t)jj * dp + k0;
                double a = acc[jj];
#pragma unroll
                for (int e = 0; e < kChunk; ++e) a = fma(xv[e], yr[e], a);
                acc[jj] = a;
            }
        }
#pragma unroll
        for (int jj = 0; jj < kColTile; ++jj) {
            const bool ok = row_ok && jj < nj;
            const double c = (xi2 + (jj < nj ? yy[j0 + jj] : 0.0)) - 2.0 * acc[jj];
            const unsigned long long key = cost_key(c);
            const unsigned digit = (unsigned)(key >> shift) & dmask;
            const bool m0 = ok && (key & high) == p0;
            const bool m1 = ok && !same && (key & high) == p1;
            if (m0) atomicAdd(&h[0][digit], 1u);
            if (m1) atomicAdd(&h[1][digit], 1u);
            if (MODE == kCollect) collect(m0 || m1, key, stage, &reserved, &fill, cand, count, cap);
        }
    }
    __syncthreads();
    for (int b = tid; b < 2 * kBins; b += kRowsPerBlock) {
        const unsigned v = (&h[0][0])[b];
        if (v != 0u) atomicAdd(&hist[b], v);
    }
    if (MODE == kCollect) {
        const unsigned nf = fill;                        // the same for every thread (after the barrier)
        if (nf != 0u) {
            if (tid == 0) stage_base = atomicAdd(count, (unsigned long long)nf);
            __syncthreads();
            for (unsigned e = tid; e < nf; e += kRowsPerBlock) {
                const unsigned long long idx = stage_base + e;
                if (idx < cap) cand[idx] = stage[e];
            }
        }
    }
}

// One digit pass over the collected keys (every key that can still hold a rank), when they all fit.
__global__ __launch_bounds__(kRowsPerBlock) void select_cand_kernel(
    const unsigned long long* __restrict__ cand, const unsigned long long* __restrict__ count,
    unsigned long long cap, const SelectState* __restrict__ st, unsigned* __restrict__ hist, int shift,
    int width) {
    __shared__ unsigned h[2][kBins];
    const unsigned long long c = *count;
    if (c > cap) return;                                  // overflowed: the full pass does this digit
    const int tid = threadIdx.x;
    const int same = st->same;
    const unsigned long long high = shift + width >= 64 ? 0ull : ~((1ull << (shift + width)) - 1ull);
    const unsigned long long p0 = st->prefix[0] & high, p1 = st->prefix[1] & high;
    const unsigned dmask = (1u << width) - 1u;
    for (int b = tid; b < 2 * kBins; b += kRowsPerBlock) (&h[0][0])[b] = 0u;
    __syncthreads();
    for (unsigned long long e = (unsigned long long)blockIdx.x * kRowsPerBlock + tid; e < c;
         e += (unsigned long long)gridDim.x * kRowsPerBlock) {
        const unsigned long long key = cand[e];
        const unsigned digit = (unsigned)(key >> shift) & dmask;
        if ((key & high) == p0) atomicAdd(&h[0][digit], 1u);
        if (!same && (key & high) == p1) atomicAdd(&h[1][digit], 1u);
    }
    __syncthreads();
    for (int b = tid; b < 2 * kBins; b += kRowsPerBlock) {
        const unsigned v = (&h[0][0])[b];
        if (v != 0u) atomicAdd(&hist[b], v);
    }
}

// Pick, for each rank, the digit whose bin holds it; narrow the prefix and the rank; clear the histograms.
__global__ __launch_bounds__(1024) void select_scan_kernel(SelectState* st, unsigned* __restrict__ hist, int shift,
                                                           int width) {
    __shared__ unsigned long long part[1024];
    __shared__ int pick[2];
    __shared__ unsigned long long below[2];
    const int tid = threadIdx.x;
    const int bins = 1 << width;
    const int same = st->same;
    for (int s = 0; s < 2; ++s) {
        const unsigned* hs = hist + (same ? 0 : s) * kBins;
        // two bins per thread, then an inclusive scan over the threads (Hillis-Steele)
        const unsigned long long c0 = 2 * tid < bins ? hs[2 * tid] : 0ull;
        const unsigned long long c1 = 2 * tid + 1 < bins ? hs[2 * tid + 1] : 0ull;
        part[tid] = c0 + c1;
        __syncthreads();
        for (int off = 1; off < 1024; off <<= 1) {
            const unsigned long long v = tid >= off ? part[tid - off] : 0ull;
            __syncthreads();
            part[tid] += v;
            __syncthreads();
        }
        const unsigned long long k = st->k[s];
        const unsigned long long before = tid > 0 ? part[tid - 1] : 0ull;
        if (tid == 0) {
            pick[s] = 0;
            below[s] = 0ull;
        }
        __syncthreads();
        if (k >= before && k < before + c0) {
            pick[s] = 2 * tid;
            below[s] = before;
        } else if (k >= before + c0 && k < before + c0 + c1) {
            pick[s] = 2 * tid + 1;
            below[s] = before + c0;
        }
        __syncthreads();
    }
    if (tid == 0) {
        for (int s = 0; s < 2; ++s) {
            st->prefix[s] |= (unsigned long long)pick[s] << shift;
            st->k[s] -= below[s];
        }
        st->same = (same && pick[0] == pick[1]) ? 1 : 0;
    }
    for (int b = tid; b < 2 * kBins; b += 1024) hist[b] = 0u;
}

__global__ void select_finish_kernel(const SelectState* st, double* out) {
    if (threadIdx.x != 0) return;
    const double a = __longlong_as_double((long long)st->prefix[0]);
    const double b = __longlong_as_double((long long)st->prefix[1]);
    *out = (a + b) * 0.5;
}

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }
int padded_dim(int d) { return (d + kChunk - 1) / kChunk * kChunk; }
int padded_cols(int m) { return (m + kColTile - 1) / kColTile * kColTile; }
unsigned long long cand_cap(int n, int m) {
    const unsigned long long N = (unsigned long long)n * (unsigned long long)m;
    return N < kCandMax ? N : kCandMax;
}

}  // namespace

extern "C" {

size_t sk_cost_median_workspace_bytes(int n, int m, int d) {
    if (n < 1 || m < 1 || d < 1 || d > SK_MEDIAN_D_MAX) return 0;
    const size_t dp = (size_t)padded_dim(d);
    return align256(sizeof(SelectState)) + align256(2 * kBins * sizeof(unsigned)) + align256((size_t)n * 8) +
           align256((size_t)m * 8) + align256((size_t)n * dp * 8) + align256((size_t)padded_cols(m) * dp * 8) +
           align256(sizeof(unsigned long long)) + align256((size_t)cand_cap(n, m) * 8);
}

int sk_cost_median_f64(const double* xc, const double* yc, int n, int m, int d, double* out, void* ws,
                       size_t ws_bytes, void* stream) {
    if (xc == nullptr || yc == nullptr || out == nullptr || ws == nullptr)
        return fail(SK_E_ARG, "sk_cost_median_f64: null pointer");
    if (n < 1 || m < 1 || d < 1 || d > SK_MEDIAN_D_MAX)
        return fail(SK_E_SHAPE, "sk_cost_median_f64: need n, m >= 1 and 1 <= d <= SK_MEDIAN_D_MAX");
    if ((unsigned long long)n * (unsigned long long)m > 0xffffffffull)
        return fail(SK_E_SHAPE, "sk_cost_median_f64: n * m must be below 2^32");
    if (ws_bytes < sk_cost_median_workspace_bytes(n, m, d))
        return fail(SK_E_WORKSPACE, "sk_cost_median_f64: workspace too small");
    if (((uintptr_t)ws & 255) != 0) return fail(SK_E_ARG, "sk_cost_median_f64: workspace must be 256-byte aligned");
    char* p = (char*)ws;
    SelectState* st = (SelectState*)p;
    p += align256(sizeof(SelectState));
    unsigned* hist = (unsigned*)p;
    p += align256(2 * kBins * sizeof(unsigned));
    double* xx = (double*)p;
    p += align256((size_t)n * 8);
    double* yy = (double*)p;
    p += align256((size_t)m * 8);
    const int dp = padded_dim(d), mp = padded_cols(m);
    double* xp = (double*)p;
    p += align256((size_t)n * dp * 8);
    double* yp = (double*)p;
    p += align256((size_t)mp * dp * 8);
    unsigned long long* count = (unsigned long long*)p;
    p += align256(sizeof(unsigned long long));
    unsigned long long* cand = (unsigned long long*)p;
    const unsigned long long cap = cand_cap(n, m);
    hipStream_t s = (hipStream_t)stream;
    hipLaunchKernelGGL(norms_kernel, dim3((n + 255) / 256), dim3(256), 0, s, xc, n, d, xx);
    hipLaunchKernelGGL(norms_kernel, dim3((m + 255) / 256), dim3(256), 0, s, yc, m, d, yy);
    hipLaunchKernelGGL(pad_kernel, dim3(1024), dim3(256), 0, s, xc, n, d, n, dp, xp);
    hipLaunchKernelGGL(pad_kernel, dim3(1024), dim3(256), 0, s, yc, m, d, mp, dp, yp);
    hipLaunchKernelGGL(select_init_kernel, dim3(1), dim3(1024), 0, s, st, hist, count,
                       (unsigned long long)n * (unsigned long long)m);
    // 256 rows per workgroup; the columns split into blocks (multiples of a tile) so that a pass has about
    // kTargetBlocks workgroups, each flushing its nonzero bins once.
    const int rb = (n + kRowsPerBlock - 1) / kRowsPerBlock;
    const int want = (kTargetBlocks + rb - 1) / rb;
    int cols = (m + want - 1) / want;
    cols = (cols + kColTile - 1) / kColTile * kColTile;
    const dim3 grid(rb, (m + cols - 1) / cols);
    // Passes up to kCompactPass recompute every cost; that pass also collects the keys matching its prefix,
    // and the later passes histogram only those (unless there were more than cap: then they recompute).
    const int cand_blocks = (int)std::min<unsigned long long>(1024ull, (cap + kRowsPerBlock - 1) / kRowsPerBlock);
    for (int q = 0; q < kPasses; ++q) {
        if (q > kCompactPass)
            hipLaunchKernelGGL(select_cand_kernel, dim3(cand_blocks), dim3(kRowsPerBlock), 0, s, cand, count, cap, st,
                               hist, kShift[q], kWidth[q]);
        auto* pass = q < kCompactPass    ? select_pass_kernel<kPlain>
                     : q == kCompactPass ? select_pass_kernel<kCollect>
                                         : select_pass_kernel<kIfOverflow>;
        hipLaunchKernelGGL(pass, grid, dim3(kRowsPerBlock), 0, s, xp, yp, xx, yy, n, m, dp, cols, st, hist, kShift[q],
                           kWidth[q], cand, count, cap);
        hipLaunchKernelGGL(select_scan_kernel, dim3(1), dim3(1024), 0, s, st, hist, kShift[q], kWidth[q]);
    }
    hipLaunchKernelGGL(select_finish_kernel, dim3(1), dim3(64), 0, s, st, out);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? SK_OK : hip_fail(e, "sk_cost_median_f64");
}

}  // extern "C"
