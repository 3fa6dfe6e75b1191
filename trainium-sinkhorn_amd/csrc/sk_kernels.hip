// Fused log-domain Sinkhorn half-step for AMD Instinct MI355X (gfx950), and the on-device Sinkhorn loop.
//
// What is computed (reference: src/trnopt/sinkhorn.py:108-119 and src/trnopt/nki_sinkhorn.py:175-228):
//
//     fh_i = kappa * (|x_i|^2 + eps * off_i - eps * lse_i) - |x_i|^2
//     lse_i = LSE_j( (2 x_i . y_j + gh_j) / eps + log b_j )
//
// Score layout. With c = (2 / eps) log2(e) and
//
//     a_ij = x_i . y_j + (gh_j + eps * log b_j) / 2           ("accumulator units")
//
// the score is c a_ij in log2 units. x_i . y_j is accumulated by fp16 MFMAs from a two-piece fp16 split of
// the power-of-two scaled fp32 coordinates (sk_lse_partial.hip), bit-identical in the f and g updates; the
// column term is added after it by one more MFMA, as exact bf16 pieces (column_operand in sk_lse_partial.hip;
// on the VALU for the bf16 row-LSE). The running (max, sum) of a row is kept as
//
//     eps * lse_i = 2 M_i + eps ln(2) log2 S_i,   S_i = sum_j exp2(c (a_ij - M_i)),  M_i = max_j a_ij,
//
// or, when x carries its log2-unit copy (bake_log2_kernel), with M_i in log2 units (c a) and the loop's
// potentials in log2 units too (sk_epilogue.h).
//
// Packed cloud layout. A 256-byte header ([0] max |coordinate| as float bits, [1] the scale s, a power of
// two with max |coordinate| * s in [2^4, 2^5), [2], [3] the log2-unit copy's tag), then the tiles: points
// padded to a multiple of 32,
// coordinates to kp = 16 * nc, every scaled coordinate v = s x stored as two fp16 pieces (v0 = fp16(v),
// v1 = fp16(v - v0)). Within tile T, the 16-byte unit ((T * nc + c) * 2 + p) * 64 + 32 h + r holds piece p
// of coordinates [16 c + 8 h, 16 c + 8 h + 8) of point 32 T + r: lane l = 32 h + r reads its
// v_mfma_f32_32x32x16_f16 operand for K chunk c with one coalesced 16-byte load (a wave reads 1 KB
// contiguous). The same layout serves a cloud as rows (one half-step) and as columns (the other).
// 4 kp bytes per point, and as many again for the log2-unit copy that follows.
//
// Work decomposition ("stream-K" over row groups x column tiles). A workgroup is 4 waves, one per SIMD;
// wave w owns 2 row blocks of 32 rows of a row group (256 rows) and all 4 waves walk the same column tiles.
// The (row group, column tile) units are split into contiguous ranges of equal cost, one per workgroup (one
// workgroup per CU; a row-group boundary inside a range costs as much as a few tiles, Split), so every
// workgroup does about the same work whatever n and m are. A range may end inside a row group; each
// (workgroup, row group) segment writes a partial (M, S) per row into its own slot, and the merge pass merges
// the slots of every row and applies the kappa / offset epilogue.
//
// A half-step is two launches: the partial kernel, then the merge kernel, one workgroup per row group, which
// merges the group's slots and applies the epilogue (sk_epilogue.h). The on-device loop
// (src/trnopt/sinkhorn.py:346-378) runs the f and the g update's partial kernels per iteration; in a pass of 40
// row groups or more the last workgroup to finish a row group merges it (per-group arrival counters), and a
// smaller pass launches the merge kernel after its partial kernel (fused_merge below): two to four launches
// per iteration. The f update's merge of group 0 counts the iteration; in the g
// update the merges also produce per-group convergence partials, and at a check, a schedule step or the last
// iteration the last group's merge runs the balanced / unbalanced checks at the reference's cadence, advances
// the stage, sets `done`, and writes the next iteration's eps and {2/eps, 1/eps, eps, kappa} into the device
// state (remaking x's log2-unit copy when eps changes). Every loop kernel returns immediately once `done` is
// set, so the host may enqueue whole batches of iterations.

#include <hip/hip_runtime.h>

#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <mutex>

#include "sk_common.h"
#include "sk_epilogue.h"
#include "trnopt_hip.h"

namespace sk {

// Error reporting shared by the translation units (declared in sk_common.h).
thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int hip_fail(hipError_t e, const char* where) {
    return fail((int)e, "%s: %s", where, hipGetErrorString(e));
}

}  // namespace sk

namespace {

using namespace sk;

constexpr float kMaskOut = -1.0e30f;   // column term of a padding column in the plain row-LSE mode

__device__ __forceinline__ float ex2(float x) { return __builtin_amdgcn_exp2f(x); }

// ---------------------------------------------------------------------------------------------------
// Pack a row-major (n, d) cloud into the tile-interleaved layout.

// Packing is three launches: clear the header, max |coordinate| (one atomic max per block on the float
// bits, which order like the values for non-negative floats), then the pieces.
__global__ void pack_header_kernel(unsigned* __restrict__ header) {
    if (threadIdx.x == 0) {
        header[0] = 0u;
        header[1] = __float_as_uint(1.0f);
        header[2] = 0u;                     // no log2-unit copy yet
        header[3] = 0u;
        header[4] = __float_as_uint(1.0f);  // the copy's unit
        header[5] = 0u;                     // L0, the loop's log2 weight offset (the on-device loop writes it)
    }
}

// Word 5 of a packed cloud's header: the on-device loop's log2 weight offset L0 = rint(log2(e) max log w) over the
// real points, a float (loop_weight_offset in sk_epilogue.h). One workgroup of kWeightMaxThreads, eight loads in
// flight per thread (a cloud of 10,000 points in two rounds).
constexpr int kWeightMaxThreads = 1024;
__global__ __launch_bounds__(kWeightMaxThreads) void weight_offset_kernel(const float* __restrict__ log_w, int n,
                                                                          unsigned* __restrict__ header) {
    __shared__ float s_mx[kWeightMaxThreads / 64];
    float mx = -3.0e38f;
    for (int i0 = 0; i0 < n; i0 += 8 * kWeightMaxThreads) {
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int i = i0 + k * kWeightMaxThreads + (int)threadIdx.x;
            v[k] = i < n ? log_w[i] : -3.0e38f;
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) mx = fmaxf(mx, v[k]);
    }
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    if ((threadIdx.x & 63) == 0) s_mx[threadIdx.x >> 6] = mx;
    __syncthreads();
    if (threadIdx.x == 0) {
        float r = s_mx[0];
        for (int w = 1; w < kWeightMaxThreads / 64; ++w) r = fmaxf(r, s_mx[w]);
        header[5] = __float_as_uint((float)rint(kLog2eD * (double)r));
    }
}

// I: the element index type (32-bit whenever n d fits, so that the row / column split is a 32-bit division).
// Four elements per thread per round, their loads in flight together.
template <typename I>
__global__ __launch_bounds__(256) void absmax_kernel(const float* __restrict__ src, int n, int d, int ld,
                                                     unsigned* __restrict__ header) {
    float mx = 0.0f;
    const I total = (I)n * d, stride = (I)gridDim.x * blockDim.x;
    for (I i0 = (I)blockIdx.x * blockDim.x + threadIdx.x; i0 < total; i0 += 4 * stride) {
        float v[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const I i = i0 + k * stride;
            v[k] = i < total ? fabsf(src[(size_t)(i / d) * ld + (size_t)(i % d)]) : 0.0f;
        }
        mx = fmaxf(fmaxf(mx, fmaxf(v[0], v[1])), fmaxf(v[2], v[3]));
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    __shared__ float red[4];
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    if (threadIdx.x == 0) {
        mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        atomicMax(&header[0], __float_as_uint(mx));
    }
}

// The power-of-two scale for a max |coordinate| m: m * s in [2^4, 2^5), clamped to [2^-32, 2^40] so that
// s_x s_y and the scaled column terms stay well inside the fp32 range (m <= 7e13 < 2^46 keeps m s < 2^14).
// The pieces then hold every coordinate within max(2^-23 |v|, 2^-25) of v = s x: relative to the largest,
// 2^-23 at worst. The target sits low in the fp16 range so that the first cloud's log2-unit copy against
// this scale, fl(c x) / s, lands in fp16's full-precision range for the usual score scales (bake_log2).
__device__ __forceinline__ float pack_scale(float m) {
    if (!(m > 0.0f)) return 1.0f;
    int e;
    frexpf(m, &e);                          // m in [2^(e-1), 2^e)
    const int k = e > 37 ? -32 : (e < -35 ? 40 : 5 - e);
    return ldexpf(1.0f, k);
}

__global__ void pack_cloud_kernel(const float* __restrict__ src, int n, int d, int ld, char* __restrict__ dst,
                                  int npad, int nc) {
    // one thread per (tile, K chunk, lane): 8 coordinates, two pieces each
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const long long total = (long long)(npad / SK_TILE) * nc * 64;
    const float s = pack_scale(__uint_as_float(reinterpret_cast<const unsigned*>(dst)[0]));
    if (idx == 0) reinterpret_cast<float*>(dst)[1] = s;
    if (idx >= total) return;
    const int lane = (int)(idx % 64);
    const int cc = (int)((idx / 64) % nc);
    const long long T = idx / (64 * nc);
    const int r = lane & 31, h = lane >> 5;
    const long long row = T * SK_TILE + r;
    f16x8 p0, p1;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const int k = 16 * cc + 8 * h + e;
        const float v = (row < n && k < d) ? src[row * ld + k] * s : 0.0f;   // exact: s is a power of two
        const _Float16 a0 = (_Float16)v;
        p0[e] = a0;
        p1[e] = (_Float16)(v - (float)a0);       // v - a0 is exact in fp32
    }
    f16x8* o = reinterpret_cast<f16x8*>(dst + kHeaderBytes) + (T * nc + cc) * (2 * 64) + lane;
    o[0] = p0;
    o[64] = p1;
}

// The first cloud's log2-unit copy (bake_params / bake_unit / bake_header, sk_epilogue.h), one unit per thread.
__global__ __launch_bounds__(256) void bake_log2_kernel(char* __restrict__ first, const void* __restrict__ second,
                                                        int npad, int nc, const float* __restrict__ sc) {
    const BakeParams b = bake_params(first, second, sc);
    const long long total = (long long)(npad / SK_TILE) * nc * 64;
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (b.valid && idx < total) bake_unit(first, idx, npad, nc, b);
    if (idx == 0) bake_header(first, second, b);
}

// The general row log-sum-exp's packing: three bf16 pieces per coordinate (exact), no scale (the header
// keeps the scale 1 written by pack_header_kernel).
__global__ void pack_cloud_bf3_kernel(const float* __restrict__ src, int n, int d, int ld, char* __restrict__ dst,
                                      int npad, int nc) {
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const long long total = (long long)(npad / SK_TILE) * nc * 64;
    if (idx >= total) return;
    const int lane = (int)(idx % 64);
    const int cc = (int)((idx / 64) % nc);
    const long long T = idx / (64 * nc);
    const int r = lane & 31, h = lane >> 5;
    const long long row = T * SK_TILE + r;
    bf16x8 p0, p1, p2;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const int k = 16 * cc + 8 * h + e;
        const float v = (row < n && k < d) ? src[row * ld + k] : 0.0f;
        const __bf16 a0 = (__bf16)v;
        const float r1 = v - (float)a0;          // exact: v and a0 share the leading bits
        const __bf16 a1 = (__bf16)r1;
        p0[e] = a0;
        p1[e] = a1;
        p2[e] = (__bf16)(r1 - (float)a1);        // exact: at most 8 significant bits remain
    }
    bf16x8* o = reinterpret_cast<bf16x8*>(dst + kHeaderBytes) + (T * nc + cc) * (3 * 64) + lane;
    o[0] = p0;
    o[64] = p1;
    o[128] = p2;
}

size_t packed_bf3_bytes(int n, int d) {
    return (size_t)kHeaderBytes + (size_t)((n + SK_TILE - 1) / SK_TILE * SK_TILE) *
                                      ((d + SK_KP_ALIGN - 1) / SK_KP_ALIGN * SK_KP_ALIGN) * 6;
}

__global__ void fill_mask_kernel(float* __restrict__ mask, int m, int mpad) {
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j < mpad) mask[j] = j < m ? 0.0f : kMaskOut;
}

// The merge pass: one workgroup per row group, then the loop step (sk_epilogue.h).
__global__ __launch_bounds__(kRowsPerGroup) void merge_kernel(PartialArgs a) {
    const LoopCounters lc = loop_counters(a);
    // The loop's convergence partials are read only by a control that checks: skip them otherwise.
    if (a.state != nullptr && !needs_control(lc.it, lc.stage, lc.stage_it, a.cfg)) a.meas = nullptr;
    if (!merge_group<false, kRowsPerGroup>(a, (int)blockIdx.x)) return;
    loop_step<false, kRowsPerGroup>(a, (int)blockIdx.x, lc, a.counters);
}

// One cloud's part of the on-device loop's log2 state (loop_weight_offset in sk_epilogue.h): its log2 weights
// relative to its offset L0 (header word 5, weight_offset_kernel) as a double-float,
//     log2(e) (log_w + log_w_lo) - L0 = Lh + Ll      (log_w_lo null: zeros; Ll = 0 on padding points),
// and its log2-unit potential R = (c / 2) fh, c = sc[0] log2(e), stored as R + Ll.
struct Log2Side {
    const float* fh;
    const float* log_w;
    const float* log_w_lo;
    const void* pk;
    float* r;
    float* lh;
    float* ll;
    int n, npad;
};
__device__ inline void log2_side(const Log2Side& c, int i, double k2) {
    if (i >= c.npad) return;
    const double L0 = (double)loop_weight_offset(c.pk);
    const double L = kLog2eD * ((double)c.log_w[i] + (c.log_w_lo != nullptr ? (double)c.log_w_lo[i] : 0.0)) - L0;
    const float lh = (float)L;
    const float ll = i < c.n ? (float)(L - (double)lh) : 0.0f;
    c.lh[i] = lh;
    c.ll[i] = ll;
    c.r[i] = (float)((double)c.fh[i] * k2 + (double)ll);
}
__global__ __launch_bounds__(256) void loop_log2_kernel(Log2Side x, Log2Side y, const float* __restrict__ sc) {
    const double k2 = 0.5 * (double)(sc[0] * kLog2e);
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    log2_side(x, i, k2);
    log2_side(y, i, k2);
}

// ---------------------------------------------------------------------------------------------------
// On-device loop control.

__global__ void loop_init_kernel(sk_state* st, LoopCfg c, int* __restrict__ counters, int ncounters) {
    for (int k = threadIdx.x; k < ncounters; k += blockDim.x) counters[k] = 0;
    if (threadIdx.x != 0) return;
    st->it = 0;
    st->stage = 0;
    st->stage_it = 0;
    st->done = c.max_iters <= 0 ? 1 : 0;
    st->converged = 0;
    st->checks = 0;
    st->err = __builtin_nan("");
    set_scalars(st, eps_for(c, 0, 0), c.rho_x, c.rho_y);
}

// ---------------------------------------------------------------------------------------------------
// Host side: errors, device facts, planning, dispatch.

int cu_count() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cached[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cached[dev] = n;
    }
    return cached[dev];
}

int env_int(const char* name, int dflt) {
    const char* v = getenv(name);
    if (v == nullptr || *v == 0) return dflt;
    return atoi(v);
}

struct Plan {
    int nc;
    int nrb, nt, ngroups;
    Split s;
    int slots;       // partial slots per row
    bool ok;         // the split fits 32-bit arithmetic (at most 2^31 - 1 cost positions)
};

// The cost of a row-group boundary in tiles (Split::alpha): what a second segment adds to a workgroup, its
// row operands, column-term staging and stores (about 3 us against 0.7-0.84 us per 32-column tile at kp 64,
// 10k x 10k), and in the on-device loop the arrival count (and maybe merge) of the first row group. Swept on
// the 10k x 10k d 64 loop: 6 tiles, 1.4 % faster than 4, 5 and 7 within 0.3 %. Above kp 64, where a tile takes
// up to twice as long: 4, swept on the 20k x 20k d 128 loop (0.5084-0.5089 ms per iteration against 0.5097-0.5103
// with 2 and 0.5089-0.5096 with 6). TRNOPT_HIP_SEG_COST overrides it.
constexpr int kSegCostNarrow = 6;     // kp <= 64
constexpr int kSegCostWide = 4;       // kp 80 to 128

// P_req > 0: that many workgroups (the grouped launches of sk_loop_run_batch_f32), else one per CU (times
// TRNOPT_HIP_WG_PER_CU); at most 1024 and at most one per unit either way.
Plan make_plan(int rows_pad, int m_pad, int kp, int P_req = 0) {
    Plan pl;
    pl.nc = kp / 16;
    pl.nrb = rows_pad / SK_TILE;
    pl.nt = m_pad / SK_TILE;
    pl.ngroups = (rows_pad + kRowsPerGroup - 1) / kRowsPerGroup;
    const long long work = (long long)pl.ngroups * pl.nt;
    int per_cu = env_int("TRNOPT_HIP_WG_PER_CU", 1);
    if (per_cu < 1 || per_cu > 4) per_cu = 1;
    long long P = P_req > 0 ? P_req : (long long)cu_count() * per_cu;
    if (P > 1024) P = 1024;
    if (P > work) P = work;
    if (P < 1) P = 1;
    int alpha = env_int("TRNOPT_HIP_SEG_COST", pl.nc <= 4 ? kSegCostNarrow : kSegCostWide);
    if (alpha < 0 || alpha > 64) alpha = 0;
    const long long ftot = work + (long long)alpha * (pl.ngroups - 1);
    pl.s.nt = pl.nt;
    pl.s.ngroups = pl.ngroups;
    pl.s.P = (int)P;
    pl.s.alpha = alpha;
    pl.s.ftot = (int)ftot;
    pl.s.q = (int)(ftot / P);
    pl.s.r = (int)(ftot % P);
    pl.ok = ftot < 0x7fffffffLL;
    if (pl.ok) set_divisors(pl.s);
    int slots = 1;
    if (pl.ok)
        for (int g = 0; g < pl.ngroups; ++g) slots = std::max(slots, last_wg(g, pl.s) - first_wg(g, pl.s) + 1);
    pl.slots = slots;
    return pl;
}

size_t align_up(size_t v) { return (v + 255) & ~(size_t)255; }

size_t partial_bytes(const Plan& pl, int rows_pad) { return align_up((size_t)pl.slots * rows_pad * sizeof(float2)); }

// Row groups of rows_pad rows: the number of convergence partials.
int meas_count(int rows_pad) { return (rows_pad + kRowsPerGroup - 1) / kRowsPerGroup; }

// One LSE pass over packed rows and columns: the partial kernel writes the slots, the merge kernel merges them
// (with group_counters the partial kernel's last workgroup of each row group does, and no merge kernel follows).
struct Pass {
    const void* xr;
    int rows_pad;
    const void* yc;
    int m_pad;
    int kp;
    const float* u;
    const float* v;
    float* u2;      // the column cloud's log2-unit potential + Ll (on-device loop), or null
    const float* v2;  // with u2: the column cloud's Lh
    const float* sc;
    const int* skip;
    int mode;
    int rows_role;
    int contraction;
    const float* xsq;
    const float* off;
    float* out;
    float* out2;    // the rows' log2-unit potential + Ll (on-device loop), or null
    const float* rows_l2lo;   // with out2: the rows' Ll
    const float* cols_l2lo;   // with out2: the columns' Ll
    int n_store;
    float2* meas;
    const float* w;
    int n_real;
    float2* part;   // workspace: partial slots
    int* counters;  // with state: one arrival counter, zero on entry and left zero
    int* group_counters;  // or null: per row group arrival counters; the partial kernel merges (no merge launch)
    sk_state* tick;   // the loop's state whose iteration counters the merge advances (f update), or null
    sk_state* state;  // loop control after the merge (g update of the loop), or null
    LoopCfg cfg;
    char* rebake;   // with state: the packed first cloud, whose log2-unit copy the control remakes on a new eps
};

PartialArgs pass_args(const Pass& ps, const Plan& pl) {
    PartialArgs a;
    a.xr = ps.xr;
    a.yc = ps.yc;
    a.u = ps.u;
    a.v = ps.v;
    a.u2 = ps.u2;
    a.v2 = ps.v2;
    a.sc = ps.sc;
    a.skip = ps.skip;
    a.part = ps.part;
    a.nrb = pl.nrb;
    a.rows_pad = ps.rows_pad;
    a.mode = ps.mode;
    a.rows_role = ps.rows_role;
    a.contraction = ps.contraction;
    a.nc = pl.nc;
    a.s = pl.s;
    a.xsq = ps.xsq;
    a.off = ps.off;
    a.out = ps.out;
    a.out2 = ps.out2;
    a.rows_l2lo = ps.rows_l2lo;
    a.cols_l2lo = ps.cols_l2lo;
    a.n_store = ps.n_store;
    a.meas = ps.meas;
    a.w = ps.w;
    a.n_real = ps.n_real;
    a.counters = ps.counters;
    a.group_counters = ps.group_counters;
    a.ngroups = pl.ngroups;
    a.tick = ps.tick;
    a.state = ps.state;
    a.cfg = ps.cfg;
    a.rebake = ps.rebake;
    return a;
}

hipError_t run_pass(const Pass& ps, const Plan& pl, hipStream_t st) {
    const PartialArgs a = pass_args(ps, pl);
    hipError_t e = launch_partial(a, pl.nc, st);
    if (e != hipSuccess || ps.group_counters != nullptr) return e;
    hipLaunchKernelGGL(merge_kernel, dim3(pl.ngroups), dim3(kRowsPerGroup), 0, st, a);
    return hipGetLastError();
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

int check_kp(int d) {
    if (d < 1) return fail(SK_E_SHAPE, "dimension %d must be >= 1", d);
    const int kp = sk_pad_dim(d);
    if (kp > SK_KP_MAX) return fail(SK_E_SHAPE, "dimension %d pads to %d > SK_KP_MAX (%d)", d, kp, SK_KP_MAX);
    return SK_OK;
}

LoopCfg loop_cfg(const sk_loop_f32* L) {
    LoopCfg c;
    c.sched = L->sched;
    c.stages = L->stages;
    c.n_sched = L->sched != nullptr ? L->n_sched : 0;
    c.n_stages = L->stages != nullptr ? L->n_stages : 0;
    c.eps = L->eps;
    c.rho_x = L->rho_x;
    c.rho_y = L->rho_y;
    c.tol = L->tol;
    c.stage_tol = L->stage_tol;
    c.max_iters = L->max_iters;
    c.check_every = L->check_every > 0 ? L->check_every : 1;
    c.stage_max_iters = L->stage_max_iters;
    c.fixed_iters = L->fixed_iters;
    c.balanced = L->balanced;
    return c;
}

int check_cloud(const sk_cloud_f32& c, const char* name) {
    if (c.pk == nullptr || c.sq == nullptr || c.log_w == nullptr || c.w == nullptr)
        return fail(SK_E_ARG, "cloud %s: null pointer", name);
    if (c.n < 1 || c.npad != sk_pad_points(c.n))
        return fail(SK_E_SHAPE, "cloud %s: n %d, npad %d (expected %d)", name, c.n, c.npad, sk_pad_points(c.n));
    if (!aligned16(c.pk) || !aligned16(c.log_w)) return fail(SK_E_ARG, "cloud %s: buffers must be 16-byte aligned", name);
    return SK_OK;
}

// TRNOPT_HIP_LOG2=0 turns the log2-unit copies off (every half-step then scales on the VALU), to compare the paths.
bool log2_enabled() { return env_int("TRNOPT_HIP_LOG2", 1) != 0; }

// Whether a pass of the on-device loop merges its row groups inside the partial kernel or launches the merge
// kernel after it (the form of the single half-step entry points). Merging in the partial kernel saves the
// merge launch and overlaps each group's merge with the other groups' tiles, but adds the arrival (a wait for
// the slot stores and an atomic round trip) and device-coherent slot loads to the tail of every row group.
// Measured on the loop at d 30 and d 64, it breaks even at 40 row groups (10k rows) and costs 1-1.5 us per
// half-step from 2k to 9k rows, so it is taken from 40 row groups up. TRNOPT_HIP_FUSED_MERGE=1 or 0 forces
// either form for every pass.
constexpr int kFuseMinGroups = 40;

bool fused_merge(const Plan& pl) {
    const int v = env_int("TRNOPT_HIP_FUSED_MERGE", -1);
    return v < 0 ? pl.ngroups >= kFuseMinGroups : v != 0;
}

void launch_bake(void* first, const void* second, int npad, int nc, const float* sc, hipStream_t st) {
    if (!log2_enabled()) return;
    const long long total = (long long)(npad / SK_TILE) * nc * 64;
    hipLaunchKernelGGL(bake_log2_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, (char*)first, second,
                       npad, nc, sc);
}

}  // namespace

// ===================================================================================================
// C ABI

extern "C" {

int sk_version(void) { return 500; }   // 0.5.0: sk_cloud_f32.log_w_lo; header word 5 is the loop's log2 weight offset

const char* sk_last_error(void) { return g_err; }

int sk_pad_points(int n) { return n <= 0 ? 0 : (n + SK_TILE - 1) / SK_TILE * SK_TILE; }

int sk_pad_dim(int d) { return d <= 0 ? 0 : (d + SK_KP_ALIGN - 1) / SK_KP_ALIGN * SK_KP_ALIGN; }

size_t sk_packed_bytes(int n, int d) {
    if (n < 1 || d < 1 || sk_pad_dim(d) > SK_KP_MAX) return 0;
    return SK_PACKED_HEADER_BYTES + (size_t)sk_pad_points(n) * sk_pad_dim(d) * SK_PACKED_BYTES_PER_COORD;
}

int sk_bake_log2_f32(void* first_pk, const void* second_pk, int n_first, int d, const float* sc, void* stream) {
    if (first_pk == nullptr || second_pk == nullptr || sc == nullptr)
        return fail(SK_E_ARG, "sk_bake_log2_f32: null pointer");
    if (n_first < 1) return fail(SK_E_SHAPE, "sk_bake_log2_f32: n_first %d", n_first);
    if (int r = check_kp(d)) return r;
    if (!aligned16(first_pk) || !aligned16(second_pk))
        return fail(SK_E_ARG, "sk_bake_log2_f32: packed clouds must be 16-byte aligned");
    launch_bake(first_pk, second_pk, sk_pad_points(n_first), sk_pad_dim(d) / 16, sc, (hipStream_t)stream);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? SK_OK : hip_fail(e, "sk_bake_log2_f32");
}

int sk_pack_cloud_f32(const float* pts, int n, int d, int ld, void* out, void* stream) {
    if (pts == nullptr || out == nullptr) return fail(SK_E_ARG, "sk_pack_cloud_f32: null pointer");
    if (n < 1 || ld < d) return fail(SK_E_SHAPE, "sk_pack_cloud_f32: n %d, d %d, ld %d", n, d, ld);
    if (int r = check_kp(d)) return r;
    if (!aligned16(out)) return fail(SK_E_ARG, "sk_pack_cloud_f32: out must be 16-byte aligned");
    const int npad = sk_pad_points(n), nc = sk_pad_dim(d) / 16;
    const long long total = (long long)(npad / SK_TILE) * nc * 64;
    const int threads = 256;
    const long long blocks = (total + threads - 1) / threads;
    hipStream_t st = (hipStream_t)stream;
    const long long elems = (long long)n * d;
    const long long mblocks = std::min<long long>((elems + threads - 1) / threads, 256);   // one atomic per block
    hipLaunchKernelGGL(pack_header_kernel, dim3(1), dim3(64), 0, st, (unsigned*)out);
    if (elems + 4LL * mblocks * threads < (1LL << 31))
        hipLaunchKernelGGL(absmax_kernel<int>, dim3((unsigned)mblocks), dim3(threads), 0, st, pts, n, d, ld,
                           (unsigned*)out);
    else
        hipLaunchKernelGGL(absmax_kernel<long long>, dim3((unsigned)mblocks), dim3(threads), 0, st, pts, n, d, ld,
                           (unsigned*)out);
    hipLaunchKernelGGL(pack_cloud_kernel, dim3((unsigned)blocks), dim3(threads), 0, st, pts, n, d, ld, (char*)out,
                       npad, nc);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? SK_OK : hip_fail(e, "sk_pack_cloud_f32");
}

size_t sk_row_lse_workspace_bytes(int rows, int m, int K) {
    if (rows < 1 || m < 1 || K < 1 || sk_pad_dim(K) > SK_KP_MAX) return 0;
    const int rp = sk_pad_points(rows), mp = sk_pad_points(m), kp = sk_pad_dim(K);
    const Plan pl = make_plan(rp, mp, kp);
    if (!pl.ok) return 0;
    return align_up(packed_bf3_bytes(rows, K)) + align_up(packed_bf3_bytes(m, K)) + align_up((size_t)mp * 4) +
           partial_bytes(pl, rp);
}

int sk_row_lse_f32(const float* xa, const float* ya, float* lse, int rows, int m, int K, void* ws, size_t ws_bytes,
                   void* stream) {
    if (xa == nullptr || ya == nullptr || lse == nullptr || ws == nullptr)
        return fail(SK_E_ARG, "sk_row_lse_f32: null pointer");
    if (rows < 1 || m < 1) return fail(SK_E_SHAPE, "sk_row_lse_f32: rows %d, m %d", rows, m);
    if (int r = check_kp(K)) return r;
    const size_t need = sk_row_lse_workspace_bytes(rows, m, K);
    if (need == 0) return fail(SK_E_SHAPE, "sk_row_lse_f32: %d x %d is too large for one launch", rows, m);
    if (ws_bytes < need) return fail(SK_E_WORKSPACE, "sk_row_lse_f32: workspace %zu < %zu bytes", ws_bytes, need);
    if (((uintptr_t)ws & 255) != 0) return fail(SK_E_ARG, "sk_row_lse_f32: workspace must be 256-byte aligned");
    const int rp = sk_pad_points(rows), mp = sk_pad_points(m), kp = sk_pad_dim(K);
    const Plan pl = make_plan(rp, mp, kp);
    char* p = (char*)ws;
    void* xpk = p;
    p += align_up(packed_bf3_bytes(rows, K));
    void* ypk = p;
    p += align_up(packed_bf3_bytes(m, K));
    float* mask = (float*)p;
    p += align_up((size_t)mp * 4);
    float2* part = (float2*)p;
    hipStream_t st = (hipStream_t)stream;
    {
        const int nc = kp / 16;
        const long long ux = (long long)(rp / SK_TILE) * nc * 64, uy = (long long)(mp / SK_TILE) * nc * 64;
        hipLaunchKernelGGL(pack_header_kernel, dim3(1), dim3(64), 0, st, (unsigned*)xpk);
        hipLaunchKernelGGL(pack_header_kernel, dim3(1), dim3(64), 0, st, (unsigned*)ypk);
        hipLaunchKernelGGL(pack_cloud_bf3_kernel, dim3((unsigned)((ux + 255) / 256)), dim3(256), 0, st, xa, rows, K, K,
                           (char*)xpk, rp, nc);
        hipLaunchKernelGGL(pack_cloud_bf3_kernel, dim3((unsigned)((uy + 255) / 256)), dim3(256), 0, st, ya, m, K, K,
                           (char*)ypk, mp, nc);
    }
    hipLaunchKernelGGL(fill_mask_kernel, dim3((mp + 255) / 256), dim3(256), 0, st, mask, m, mp);
    Pass ps = {};
    ps.xr = xpk;
    ps.rows_pad = rp;
    ps.yc = ypk;
    ps.m_pad = mp;
    ps.kp = kp;
    ps.u = mask;
    ps.v = mask;
    ps.sc = mask;       // not read in this mode; a valid address all the same
    ps.mode = kPlainLse;
    ps.rows_role = 0;
    ps.contraction = kBF16x3;
    ps.out = lse;
    ps.n_store = rows;
    ps.part = part;
    const hipError_t e = run_pass(ps, pl, st);
    return e == hipSuccess ? SK_OK : hip_fail(e, "sk_row_lse_f32");
}

size_t sk_half_step_workspace_bytes(int rows_pad, int m_pad, int d) {
    if (rows_pad < SK_TILE || m_pad < SK_TILE || d < 1 || sk_pad_dim(d) > SK_KP_MAX) return 0;
    const Plan pl = make_plan(rows_pad, m_pad, sk_pad_dim(d));
    if (!pl.ok) return 0;
    return partial_bytes(pl, rows_pad);
}

int sk_half_step_meas_count(int rows_pad) { return rows_pad < 1 ? 0 : meas_count(rows_pad); }

}  // extern "C"

namespace {

// Argument checks shared by the two half-step entry points (everything but the workspace).
int check_half_step(const char* who, const void* x_pk, const float* xsq, int rows_pad, const void* y_pk,
                    const float* gh, const float* log_b, int m_pad, int d, int rows_role, const float* sc,
                    const float* fh, const float* meas, const float* w) {
    if (x_pk == nullptr || xsq == nullptr || y_pk == nullptr || gh == nullptr || log_b == nullptr || sc == nullptr ||
        fh == nullptr)
        return fail(SK_E_ARG, "%s: null pointer", who);
    if (meas != nullptr && w == nullptr) return fail(SK_E_ARG, "%s: meas needs w", who);
    if (fh == gh) return fail(SK_E_ARG, "%s: fh must not alias gh", who);
    if (rows_pad < SK_TILE || rows_pad % SK_TILE != 0 || m_pad < SK_TILE || m_pad % SK_TILE != 0)
        return fail(SK_E_SHAPE, "%s: rows_pad %d and m_pad %d must be positive multiples of %d", who, rows_pad, m_pad,
                    SK_TILE);
    if (int r = check_kp(d)) return r;
    if (rows_role != 0 && rows_role != 1) return fail(SK_E_ARG, "%s: rows_role %d not 0 or 1", who, rows_role);
    if (!aligned16(x_pk) || !aligned16(y_pk) || !aligned16(gh) || !aligned16(log_b))
        return fail(SK_E_ARG, "%s: packed clouds, gh and log_b must be 16-byte aligned", who);
    if (sk_half_step_workspace_bytes(rows_pad, m_pad, d) == 0)
        return fail(SK_E_SHAPE, "%s: %d x %d is too large for one launch", who, rows_pad, m_pad);
    return SK_OK;
}

// The partial kernel and the merge kernel of one half-step, partial slots at `part`.
hipError_t launch_half_step(const void* x_pk, const float* xsq, const float* off, int rows_pad, const void* y_pk,
                            const float* gh, const float* log_b, int m_pad, int d, int rows_role, const float* sc,
                            const int* skip, float* fh, float* meas, const float* w, int n_real, void* part,
                            hipStream_t stream) {
    const Plan pl = make_plan(rows_pad, m_pad, sk_pad_dim(d));
    Pass ps = {};
    ps.xr = x_pk;
    ps.rows_pad = rows_pad;
    ps.yc = y_pk;
    ps.m_pad = m_pad;
    ps.kp = sk_pad_dim(d);
    ps.u = gh;
    ps.v = log_b;
    ps.sc = sc;
    ps.skip = skip;
    ps.mode = kHalfStep;
    ps.rows_role = rows_role;
    ps.contraction = kF16x2;
    ps.xsq = xsq;
    ps.off = off;
    ps.out = fh;
    ps.n_store = rows_pad;
    ps.meas = (float2*)meas;
    ps.w = w;
    ps.n_real = n_real;
    ps.part = (float2*)part;
    return run_pass(ps, pl, stream);
}

// The no-allocation entry point's partial slots: a file-scope device array, one per GPU. In host code `scratch`
// names a host-side stand-in, not device memory; its device address is looked up once per device
// (hipGetSymbolAddress, with that device current) and only that address is handed to kernels.
constexpr size_t kScratchBytes = SK_NOALLOC_SCRATCH_BYTES;
__device__ __align__(256) char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's copy of `scratch` (looked up on the first call on that device).
int scratch_on_current_device(void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "sk_half_step_noalloc_f32: hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices) return fail(SK_E_DEVICE, "sk_half_step_noalloc_f32: device %d", dev);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_fail(e, "sk_half_step_noalloc_f32: hipGetSymbolAddress(scratch)");
        if (p == nullptr || ((uintptr_t)p & 255) != 0)
            return fail(SK_E_DEVICE, "sk_half_step_noalloc_f32: scratch address %p is not 256-byte aligned", p);
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return SK_OK;
}

}  // namespace

extern "C" {

int sk_half_step_f32(const void* x_pk, const float* xsq, const float* off, int rows_pad, const void* y_pk,
                     const float* gh, const float* log_b, int m_pad, int d, int rows_role, const float* sc,
                     const int* skip, float* fh, float* meas, const float* w, int n_real, void* ws, size_t ws_bytes,
                     void* stream) {
    if (int r = check_half_step("sk_half_step_f32", x_pk, xsq, rows_pad, y_pk, gh, log_b, m_pad, d, rows_role, sc, fh,
                                meas, w))
        return r;
    if (ws == nullptr) return fail(SK_E_ARG, "sk_half_step_f32: null pointer");
    const size_t need = sk_half_step_workspace_bytes(rows_pad, m_pad, d);
    if (ws_bytes < need) return fail(SK_E_WORKSPACE, "sk_half_step_f32: workspace %zu < %zu bytes", ws_bytes, need);
    if (((uintptr_t)ws & 255) != 0) return fail(SK_E_ARG, "sk_half_step_f32: workspace must be 256-byte aligned");
    const hipError_t e = launch_half_step(x_pk, xsq, off, rows_pad, y_pk, gh, log_b, m_pad, d, rows_role, sc, skip, fh,
                                          meas, w, n_real, ws, (hipStream_t)stream);
    return e == hipSuccess ? SK_OK : hip_fail(e, "sk_half_step_f32");
}

int sk_half_step_noalloc_f32(const void* x_pk, const float* xsq, const float* off, int rows_pad, const void* y_pk,
                             const float* gh, const float* log_b, int m_pad, int d, int rows_role, const float* sc,
                             const int* skip, float* fh, float* meas, const float* w, int n_real, void* stream) {
    if (int r = check_half_step("sk_half_step_noalloc_f32", x_pk, xsq, rows_pad, y_pk, gh, log_b, m_pad, d, rows_role,
                                sc, fh, meas, w))
        return r;
    const size_t need = sk_half_step_workspace_bytes(rows_pad, m_pad, d);
    if (need > kScratchBytes)
        return fail(SK_E_WORKSPACE, "sk_half_step_noalloc_f32: %d x %d needs %zu bytes of slots, above the %zu-byte "
                    "static scratch (use sk_half_step_f32 with a workspace)", rows_pad, m_pad, need, kScratchBytes);
    void* part = nullptr;
    if (int r = scratch_on_current_device(&part)) return r;
    const hipError_t e = launch_half_step(x_pk, xsq, off, rows_pad, y_pk, gh, log_b, m_pad, d, rows_role, sc, skip, fh,
                                          meas, w, n_real, part, (hipStream_t)stream);
    return e == hipSuccess ? SK_OK : hip_fail(e, "sk_half_step_noalloc_f32");
}

size_t sk_loop_workspace_bytes(int nx_pad, int ny_pad, int d) {
    if (nx_pad < SK_TILE || ny_pad < SK_TILE || d < 1 || sk_pad_dim(d) > SK_KP_MAX) return 0;
    const int kp = sk_pad_dim(d);
    const Plan pf = make_plan(nx_pad, ny_pad, kp), pg = make_plan(ny_pad, nx_pad, kp);
    if (!pf.ok || !pg.ok) return 0;
    return std::max(partial_bytes(pf, nx_pad), partial_bytes(pg, ny_pad)) +
           align_up((size_t)meas_count(ny_pad) * sizeof(float2)) +
           align_up((size_t)(1 + std::max(pf.ngroups, pg.ngroups)) * sizeof(int)) +
           3 * (align_up((size_t)nx_pad * sizeof(float)) + align_up((size_t)ny_pad * sizeof(float)));
}

namespace {
// The loop's workspace: partial slots (shared by the f and g updates), the g update's per-group convergence
// partials, the arrival counters (zeroed at init, left zero by every launch: [0] the loop control's, then one
// per row group for the merge inside the partial kernel), the two potentials in log2 units that the iteration
// carries when the scores come in log2 units, R = (c / 2) fh stored as R + Ll, and both clouds' log2 weights
// Lh, Ll (loop_weight_offset in sk_epilogue.h).
struct LoopLayout {
    Plan pf, pg;
    float2* part;
    float2* meas;
    int* counters;
    int ncounters;
    float* rf;
    float* rg;
    float *lxh, *lxl, *lyh, *lyl;
};

LoopLayout loop_layout(const sk_loop_f32* L) {
    LoopLayout o;
    const int kp = sk_pad_dim(L->d);
    o.pf = make_plan(L->x.npad, L->y.npad, kp);
    o.pg = make_plan(L->y.npad, L->x.npad, kp);
    const size_t part_sz = std::max(partial_bytes(o.pf, L->x.npad), partial_bytes(o.pg, L->y.npad));
    o.part = (float2*)L->ws;
    o.meas = (float2*)((char*)L->ws + part_sz);
    o.counters = (int*)((char*)o.meas + align_up((size_t)meas_count(L->y.npad) * sizeof(float2)));
    o.ncounters = 1 + std::max(o.pf.ngroups, o.pg.ngroups);
    const size_t bx = align_up((size_t)L->x.npad * sizeof(float)), by = align_up((size_t)L->y.npad * sizeof(float));
    o.rf = (float*)((char*)o.counters + align_up((size_t)o.ncounters * sizeof(int)));
    o.rg = (float*)((char*)o.rf + bx);
    o.lxh = (float*)((char*)o.rg + by);
    o.lxl = (float*)((char*)o.lxh + bx);
    o.lyh = (float*)((char*)o.lxl + bx);
    o.lyl = (float*)((char*)o.lyh + by);
    return o;
}
}  // namespace

int sk_loop_init_f32(const sk_loop_f32* L, void* stream) {
    if (L == nullptr || L->state == nullptr || L->fh == nullptr || L->gh == nullptr || L->ws == nullptr)
        return fail(SK_E_ARG, "sk_loop_init_f32: null pointer");
    if (L->n_sched > 0 && L->sched == nullptr) return fail(SK_E_ARG, "sk_loop_init_f32: n_sched without sched");
    if (L->n_stages > 0 && L->stages == nullptr) return fail(SK_E_ARG, "sk_loop_init_f32: n_stages without stages");
    if (!(L->eps > 0.0)) return fail(SK_E_ARG, "sk_loop_init_f32: eps must be > 0");
    if (int r = check_cloud(L->x, "x")) return r;
    if (int r = check_cloud(L->y, "y")) return r;
    if (int r = check_kp(L->d)) return r;
    const size_t need = sk_loop_workspace_bytes(L->x.npad, L->y.npad, L->d);
    if (need == 0) return fail(SK_E_SHAPE, "sk_loop: %d x %d is too large for one launch", L->x.npad, L->y.npad);
    if (L->ws_bytes < need) return fail(SK_E_WORKSPACE, "sk_loop_init_f32: workspace %zu < %zu bytes", L->ws_bytes, need);
    if (((uintptr_t)L->ws & 255) != 0) return fail(SK_E_ARG, "sk_loop_init_f32: workspace must be 256-byte aligned");
    const LoopLayout lo = loop_layout(L);
    hipLaunchKernelGGL(loop_init_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, L->state, loop_cfg(L),
                       lo.counters, lo.ncounters);
    // both clouds' log2 weight offsets into their headers (each is the column cloud of one half-step)
    hipLaunchKernelGGL(weight_offset_kernel, dim3(1), dim3(kWeightMaxThreads), 0, (hipStream_t)stream, L->x.log_w,
                       L->x.n, (unsigned*)const_cast<void*>(L->x.pk));
    hipLaunchKernelGGL(weight_offset_kernel, dim3(1), dim3(kWeightMaxThreads), 0, (hipStream_t)stream, L->y.log_w,
                       L->y.n, (unsigned*)const_cast<void*>(L->y.pk));
    // x's log2-unit copy for the first iteration's eps, both clouds' log2 weights and both log2-unit potentials
    // (from fh and the caller's gh); the loop control remakes the copy and the potentials when eps changes
    launch_bake(const_cast<void*>(L->x.pk), L->y.pk, L->x.npad, sk_pad_dim(L->d) / 16, L->state->sc_x,
                (hipStream_t)stream);
    const int nmax = std::max(L->x.npad, L->y.npad);
    const Log2Side sx = {L->fh, L->x.log_w, L->x.log_w_lo, L->x.pk, lo.rf, lo.lxh, lo.lxl, L->x.n, L->x.npad};
    const Log2Side sy = {L->gh, L->y.log_w, L->y.log_w_lo, L->y.pk, lo.rg, lo.lyh, lo.lyl, L->y.n, L->y.npad};
    hipLaunchKernelGGL(loop_log2_kernel, dim3((nmax + 255) / 256), dim3(256), 0, (hipStream_t)stream, sx, sy,
                       L->state->sc_x);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? SK_OK : hip_fail(e, "sk_loop_init_f32");
}

}  // extern "C"

namespace {

// The loop's two passes over its workspace layout: the f update (rows x against y; counts the iteration) and the g
// update (rows y against x; convergence partials, loop control).
void loop_passes(const sk_loop_f32* L, const LoopLayout& lo, Pass& f, Pass& g) {
    const int kp = sk_pad_dim(L->d);
    sk_state* st = L->state;
    f = Pass{};
    f.xr = L->x.pk;
    f.rows_pad = L->x.npad;
    f.yc = L->y.pk;
    f.m_pad = L->y.npad;
    f.kp = kp;
    f.u = L->gh;
    f.v = L->y.log_w;
    f.u2 = lo.rg;
    f.v2 = lo.lyh;
    f.sc = st->sc_x;
    f.skip = &st->done;
    f.mode = kHalfStep;
    f.rows_role = 0;
    f.contraction = kF16x2;
    f.xsq = L->x.sq;
    f.off = L->x.off;
    f.out = L->fh;
    f.out2 = lo.rf;
    f.rows_l2lo = lo.lxl;
    f.cols_l2lo = lo.lyl;
    f.n_store = L->x.npad;
    f.tick = st;
    f.part = lo.part;
    f.group_counters = fused_merge(lo.pf) ? lo.counters + 1 : nullptr;

    g = Pass{};
    g.xr = L->y.pk;
    g.rows_pad = L->y.npad;
    g.yc = L->x.pk;
    g.m_pad = L->x.npad;
    g.kp = kp;
    g.u = L->fh;
    g.v = L->x.log_w;
    g.u2 = lo.rf;
    g.v2 = lo.lxh;
    g.sc = st->sc_y;
    g.skip = &st->done;
    g.mode = kHalfStep;
    g.rows_role = 1;
    g.contraction = kF16x2;
    g.xsq = L->y.sq;
    g.off = L->y.off;
    g.out = L->gh;
    g.out2 = lo.rg;
    g.rows_l2lo = lo.lyl;
    g.cols_l2lo = lo.lxl;
    g.n_store = L->y.npad;
    g.meas = lo.meas;
    g.w = L->y.w;
    g.n_real = L->y.n;
    g.part = lo.part;
    g.counters = lo.counters;
    g.state = st;
    g.cfg = loop_cfg(L);
    g.rebake = log2_enabled() ? (char*)const_cast<void*>(L->x.pk) : nullptr;
    g.group_counters = fused_merge(lo.pg) ? lo.counters + 1 : nullptr;
}

int check_loop(const sk_loop_f32* L, const char* where) {
    if (L == nullptr || L->state == nullptr || L->fh == nullptr || L->gh == nullptr || L->ws == nullptr)
        return fail(SK_E_ARG, "%s: null pointer", where);
    if (int r = check_cloud(L->x, "x")) return r;
    if (int r = check_cloud(L->y, "y")) return r;
    if (int r = check_kp(L->d)) return r;
    const size_t need = sk_loop_workspace_bytes(L->x.npad, L->y.npad, L->d);
    if (need == 0) return fail(SK_E_SHAPE, "sk_loop: %d x %d is too large for one launch", L->x.npad, L->y.npad);
    if (L->ws_bytes < need) return fail(SK_E_WORKSPACE, "%s: workspace %zu < %zu bytes", where, L->ws_bytes, need);
    if (((uintptr_t)L->ws & 255) != 0) return fail(SK_E_ARG, "%s: workspace must be 256-byte aligned", where);
    return SK_OK;
}

}  // namespace

extern "C" {

int sk_loop_run_f32(const sk_loop_f32* L, int iters, void* stream) {
    if (int r = check_loop(L, "sk_loop_run_f32")) return r;
    if (iters < 0) return fail(SK_E_ARG, "sk_loop_run_f32: iters %d < 0", iters);
    const LoopLayout lo = loop_layout(L);
    Pass f, g;
    loop_passes(L, lo, f, g);
    hipStream_t hs = (hipStream_t)stream;
    for (int k = 0; k < iters; ++k) {
        hipError_t e = run_pass(f, lo.pf, hs);
        if (e == hipSuccess) e = run_pass(g, lo.pg, hs);
        if (e != hipSuccess) return hip_fail(e, "sk_loop_run_f32");
    }
    return SK_OK;
}

}  // extern "C"

// ---------------------------------------------------------------------------------------------------
// Several loops at once (independent solves of the same d, such as the pairs of a wot pipeline): each launch runs
// one pass of every loop, each on its own share of the workgroups, so that small solves fill the GPU together
// instead of each paying a launch and its latencies per pass.

namespace {

constexpr int kBatchMapEntries = 1024;      // workgroups of one grouped launch, at most
constexpr int kBatchMaxLoops = 1024;

struct BatchLayout {
    size_t args_f, args_g, map_f, map_g, bytes;
};

BatchLayout batch_layout(int count) {
    BatchLayout b;
    const size_t args = align_up((size_t)count * sizeof(PartialArgs));
    const size_t map = align_up((size_t)kBatchMapEntries * sizeof(unsigned));
    b.args_f = 0;
    b.args_g = args;
    b.map_f = 2 * args;
    b.map_g = 2 * args + map;
    b.bytes = 2 * args + 2 * map;
    return b;
}

// Workgroups per pass: P_k = ceil(cost_k / T), with T the smallest per-workgroup cost (tiles, row-group boundaries
// included) at which the P_k add up to at most `total`, so that every workgroup of the launch carries about T
// tiles; then the workgroups left over, one at a time, to the pass with the largest cost per workgroup (while it
// has more tiles than workgroups). Each pass gets one workgroup at least (then the sum is the number of passes if
// that is larger). A single pass gets min(total, cost) workgroups: the split of its own launches.
std::vector<int> share_workgroups(const std::vector<long long>& cost, int total) {
    long long lo = 1, hi = 1;
    for (long long c : cost) hi = std::max(hi, c);
    auto need = [&](long long T) {
        long long n = 0;
        for (long long c : cost) n += std::max(1LL, (c + T - 1) / T);
        return n;
    };
    while (lo < hi) {
        const long long mid = lo + (hi - lo) / 2;
        if (need(mid) <= total) hi = mid; else lo = mid + 1;
    }
    std::vector<int> P(cost.size());
    long long used = 0;
    for (size_t k = 0; k < cost.size(); ++k) {
        P[k] = (int)std::max(1LL, (cost[k] + lo - 1) / lo);
        used += P[k];
    }
    for (; used < total; ++used) {
        size_t best = cost.size();
        for (size_t k = 0; k < cost.size(); ++k)
            if (P[k] < cost[k] && (best == cost.size() || cost[k] * P[best] > cost[best] * P[k])) best = k;
        if (best == cost.size()) break;
        ++P[best];
    }
    return P;
}

// The cost of a pass on the cost line of its split (tiles plus one boundary cost per row group after the first).
long long pass_cost(const Plan& pl) { return (long long)pl.s.ftot; }

// The map of one grouped launch: workgroup b runs workgroup p of pass k, map[b] = k << 16 | p; the passes' workgroups
// are numbered in order and placed as the single-pass kernel places its own (the workgroups of one XCD hold one
// contiguous range, xcd_contiguous); entries past the launch name no pass.
std::vector<unsigned> batch_map(const std::vector<int>& P) {
    std::vector<unsigned> order;
    for (size_t k = 0; k < P.size(); ++k)
        for (int p = 0; p < P[k]; ++p) order.push_back((unsigned)k << 16 | (unsigned)p);
    const int n = (int)order.size();
    std::vector<unsigned> map(kBatchMapEntries, 0xffffffffu);
    const int q = n / kXcds, r = n % kXcds;
    for (int b = 0; b < n; ++b) {
        const int xcd = b % kXcds, idx = b / kXcds;
        map[b] = order[xcd * q + (xcd < r ? xcd : r) + idx];
    }
    return map;
}

}  // namespace

extern "C" {

size_t sk_loop_batch_workspace_bytes(int count) {
    if (count < 1 || count > kBatchMaxLoops) return 0;
    return batch_layout(count).bytes;
}

int sk_loop_batch_plan(const int* nx_pad, const int* ny_pad, int count, int d, int* workgroups) {
    if (nx_pad == nullptr || ny_pad == nullptr || workgroups == nullptr)
        return fail(SK_E_ARG, "sk_loop_batch_plan: null pointer");
    if (count < 1 || count > kBatchMaxLoops) return fail(SK_E_SHAPE, "sk_loop_batch_plan: count %d", count);
    if (int r = check_kp(d)) return r;
    const int kp = sk_pad_dim(d), total = cu_count();
    std::vector<long long> cf(count), cg(count);
    for (int k = 0; k < count; ++k) {
        if (nx_pad[k] < SK_TILE || ny_pad[k] < SK_TILE || nx_pad[k] % SK_TILE || ny_pad[k] % SK_TILE)
            return fail(SK_E_SHAPE, "sk_loop_batch_plan: loop %d: %d x %d", k, nx_pad[k], ny_pad[k]);
        cf[k] = pass_cost(make_plan(nx_pad[k], ny_pad[k], kp));
        cg[k] = pass_cost(make_plan(ny_pad[k], nx_pad[k], kp));
    }
    const std::vector<int> pf = share_workgroups(cf, total), pg = share_workgroups(cg, total);
    for (int k = 0; k < count; ++k) {
        workgroups[2 * k] = std::min(pf[k], 1024);
        workgroups[2 * k + 1] = std::min(pg[k], 1024);
    }
    return SK_OK;
}

int sk_loop_batch_init_f32(const sk_loop_f32* const* loops, int count, void* ws, size_t ws_bytes, int* launch,
                           void* stream) {
    if (loops == nullptr || ws == nullptr || launch == nullptr) return fail(SK_E_ARG, "sk_loop_batch_init_f32: null pointer");
    if (count < 1 || count > kBatchMaxLoops)
        return fail(SK_E_SHAPE, "sk_loop_batch_init_f32: count %d (1 to %d)", count, kBatchMaxLoops);
    const size_t need = sk_loop_batch_workspace_bytes(count);
    if (ws_bytes < need) return fail(SK_E_WORKSPACE, "sk_loop_batch_init_f32: workspace %zu < %zu bytes", ws_bytes, need);
    if (((uintptr_t)ws & 255) != 0) return fail(SK_E_ARG, "sk_loop_batch_init_f32: workspace must be 256-byte aligned");
    const int d = loops[0] != nullptr ? loops[0]->d : 0;
    std::vector<int> nx(count), ny(count), wg(2 * (size_t)count);
    for (int k = 0; k < count; ++k) {
        if (int r = check_loop(loops[k], "sk_loop_batch_init_f32")) return r;
        if (loops[k]->d != d) return fail(SK_E_SHAPE, "sk_loop_batch_init_f32: loop %d has d %d, loop 0 %d", k, loops[k]->d, d);
        nx[k] = loops[k]->x.npad;
        ny[k] = loops[k]->y.npad;
    }
    if (int r = sk_loop_batch_plan(nx.data(), ny.data(), count, d, wg.data())) return r;
    const int kp = sk_pad_dim(d);
    std::vector<PartialArgs> af(count), ag(count);
    std::vector<int> pf(count), pg(count);
    long long nf = 0, ng = 0;
    for (int k = 0; k < count; ++k) {
        const sk_loop_f32* L = loops[k];
        const LoopLayout lo = loop_layout(L);
        const Plan bf = make_plan(L->x.npad, L->y.npad, kp, wg[2 * k]);
        const Plan bg = make_plan(L->y.npad, L->x.npad, kp, wg[2 * k + 1]);
        // the loop's workspace holds the partial slots of its own plans; a plan on fewer workgroups has no more
        if (!bf.ok || !bg.ok || partial_bytes(bf, L->x.npad) > partial_bytes(lo.pf, L->x.npad) ||
            partial_bytes(bg, L->y.npad) > partial_bytes(lo.pg, L->y.npad) ||
            std::max(bf.ngroups, bg.ngroups) + 1 > lo.ncounters)
            return fail(SK_E_SHAPE, "sk_loop_batch_init_f32: loop %d does not fit its workspace on %d / %d workgroups", k,
                        wg[2 * k], wg[2 * k + 1]);
        Pass f, g;
        loop_passes(L, lo, f, g);
        // every row group is merged inside the grouped kernel (its last workgroup), so no merge launch follows
        f.group_counters = lo.counters + 1;
        g.group_counters = lo.counters + 1;
        af[k] = pass_args(f, bf);
        ag[k] = pass_args(g, bg);
        pf[k] = bf.s.P;
        pg[k] = bg.s.P;
        nf += bf.s.P;
        ng += bg.s.P;
    }
    if (nf > kBatchMapEntries || ng > kBatchMapEntries)
        return fail(SK_E_SHAPE, "sk_loop_batch_init_f32: %lld / %lld workgroups > %d", nf, ng, kBatchMapEntries);
    const std::vector<unsigned> mf = batch_map(pf), mg = batch_map(pg);
    const BatchLayout bl = batch_layout(count);
    char* base = (char*)ws;
    hipStream_t hs = (hipStream_t)stream;
    hipError_t e = hipMemcpyAsync(base + bl.args_f, af.data(), af.size() * sizeof(PartialArgs), hipMemcpyHostToDevice, hs);
    if (e == hipSuccess)
        e = hipMemcpyAsync(base + bl.args_g, ag.data(), ag.size() * sizeof(PartialArgs), hipMemcpyHostToDevice, hs);
    if (e == hipSuccess) e = hipMemcpyAsync(base + bl.map_f, mf.data(), mf.size() * sizeof(unsigned), hipMemcpyHostToDevice, hs);
    if (e == hipSuccess) e = hipMemcpyAsync(base + bl.map_g, mg.data(), mg.size() * sizeof(unsigned), hipMemcpyHostToDevice, hs);
    // the host arrays die with this call: the copies complete before it returns
    if (e == hipSuccess) e = hipStreamSynchronize(hs);
    if (e != hipSuccess) return hip_fail(e, "sk_loop_batch_init_f32");
    launch[0] = kp / 16;
    launch[1] = (int)nf;
    launch[2] = (int)ng;
    return SK_OK;
}

int sk_loop_run_batch_f32(const void* ws, size_t ws_bytes, int count, const int* launch, int iters, void* stream) {
    if (ws == nullptr || launch == nullptr) return fail(SK_E_ARG, "sk_loop_run_batch_f32: null pointer");
    if (count < 1 || count > kBatchMaxLoops) return fail(SK_E_SHAPE, "sk_loop_run_batch_f32: count %d", count);
    if (ws_bytes < sk_loop_batch_workspace_bytes(count))
        return fail(SK_E_WORKSPACE, "sk_loop_run_batch_f32: workspace %zu < %zu bytes", ws_bytes,
                    sk_loop_batch_workspace_bytes(count));
    const int nc = launch[0], nf = launch[1], ng = launch[2];
    if (nc < 1 || nc * 16 > SK_KP_MAX || nf < 1 || ng < 1 || nf > kBatchMapEntries || ng > kBatchMapEntries)
        return fail(SK_E_ARG, "sk_loop_run_batch_f32: launch {%d, %d, %d} is not one sk_loop_batch_init_f32 returned",
                    nc, nf, ng);
    if (iters < 0) return fail(SK_E_ARG, "sk_loop_run_batch_f32: iters %d < 0", iters);
    const BatchLayout bl = batch_layout(count);
    const char* base = (const char*)ws;
    const PartialArgs* af = (const PartialArgs*)(base + bl.args_f);
    const PartialArgs* ag = (const PartialArgs*)(base + bl.args_g);
    const unsigned* mf = (const unsigned*)(base + bl.map_f);
    const unsigned* mg = (const unsigned*)(base + bl.map_g);
    hipStream_t hs = (hipStream_t)stream;
    for (int k = 0; k < iters; ++k) {
        hipError_t e = launch_grouped(af, mf, count, nf, nc, 0, hs);
        if (e == hipSuccess) e = launch_grouped(ag, mg, count, ng, nc, 1, hs);
        if (e != hipSuccess) return hip_fail(e, "sk_loop_run_batch_f32");
    }
    return SK_OK;
}

}  // extern "C"
