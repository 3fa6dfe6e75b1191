// Definitions shared by the two translation units of libtrnopt_hip.so: the MFMA partial kernel
// (sk_lse_partial.hip, built without NaN semantics so row maxima need no canonicalisation) and the rest
// (sk_kernels.hip: packing, the merge pass and loop control of sk_epilogue.h, C ABI).
#pragma once

#include <hip/hip_runtime.h>

#include "trnopt_hip.h"

namespace sk {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr float kLog2e = 1.44269504088896340736f;
// log2(e) - kLog2e (1.93e-8): with it, fmaf(kLog2e, v, fmaf(kLog2eLo, v, r)) is r + log2(e) v rounded once
// (kLog2e alone is 1.3e-8 low, a bias of 1.3e-8 |v| that does not average out).
constexpr float kLog2eLo = (float)(1.44269504088896340736 - (double)kLog2e);
constexpr float kLn2 = 0.69314718055994530942f;
constexpr float kEmpty = -1.0e30f;     // running max of a row before its first column (finite on purpose)
constexpr int kWaves = 4;              // waves per workgroup of the partial kernel (one per SIMD)
constexpr int kBlock = kWaves * 64;
constexpr int kRowBlocks = 2;          // 32-row blocks per wave (independent MFMA accumulator chains)
constexpr int kRowsPerGroup = 32 * kRowBlocks * kWaves;   // rows of a row group: one row per thread
constexpr int kXcds = 8;
constexpr int kMaxChunks = 8;          // K chunks of 16 coordinates: kp = 16 * nc <= 128
// The contraction x.y on the matrix cores:
//   kF16x2  -- the half-steps: the cloud's power-of-two scaled coordinates as two fp16 pieces, three products
//              (fp32 accuracy for coordinates within 2^26 of the cloud's largest; 4 bytes per coordinate);
//   kBF16x3 -- the general row log-sum-exp of arbitrary fp32 matrices: each coordinate as three bf16 pieces
//              (exact over the whole fp32 range), six products (6 bytes per coordinate).
enum Contraction { kF16x2 = 0, kBF16x3 = 1 };
constexpr int pieces_of(int ct) { return ct == kF16x2 ? 2 : 3; }
constexpr int kHeaderBytes = 256;      // packed cloud header (layout below, packed_tiles)
constexpr float kMaxAbsCoordinate = 7.0e13f; // above this the scaled coordinates would not fit fp16
constexpr float kPadScore = -1.0e30f;  // floor of a (scaled) column term: padding, never -inf

enum Mode { kHalfStep = 0, kPlainLse = 1 };

// What a kernel reads for its done flag when the call has none: an unconditional load, so that the flag is
// requested together with the launch's other scalars.
__device__ const int kNoSkip = 0;

// n / d for 0 <= n < 2^31 by one multiply-high, d in [1, 2^31] a divisor fixed per launch: with
// 2^(k-1) < d <= 2^k and m = ceil(2^(31 + k) / d) (in [2^31, 2^32)), n m / 2^(31 + k) = n / d + delta with
// 0 <= delta < n / 2^(31 + k) < 2^-k <= 1 / d, which no fraction of n / d reaches 1 with, so
// floor(2n m / 2^32) >> k = floor(n / d) exactly. The prologue's divisions by the split's constants (seven per
// segment, ~30 dependent instructions each on the vector unit) become two scalar instructions each.
struct Div {
    unsigned m;
    int k;
};
inline Div make_div(int d) {
    Div v;
    v.k = 0;
    while ((1LL << v.k) < d) ++v.k;
    v.m = (unsigned)((((unsigned long long)1 << (31 + v.k)) + (unsigned long long)d - 1) / (unsigned long long)d);
    return v;
}
__host__ __device__ inline int div_by(int n, const Div& v) {
    return (int)((unsigned)(((unsigned long long)(2u * (unsigned)n) * v.m) >> 32) >> v.k);
}

// Work split shared by the partial and the merge kernels. The (row group, column tile) units are laid out on a
// cost line: unit x of row group g = x / nt sits at position F(x) = x + alpha g, i.e. every row-group boundary
// costs alpha positions, because a workgroup whose range crosses one starts a second segment (its row
// operands, column terms and stores again: about alpha tiles of time). The line [0, ftot), ftot = work +
// alpha (ngroups - 1), is cut into P equal pieces: workgroup p owns the units whose positions lie in
// [C_p, C_(p+1)), C_p = floor(p ftot / P) = p q + floor(p r / P) with (q, r) = divmod(ftot, P). Everything is
// 32-bit (ftot < 2^31 and P <= 1024, checked by the planner), so a kernel's prologue needs no 64-bit division.
struct Split {
    int nt;          // column tiles per row group
    int ngroups;     // row groups
    int P;           // workgroups
    int alpha;       // cost of a row-group boundary, in tiles
    int ftot;        // ngroups * nt + alpha * (ngroups - 1)
    int q, r;        // ftot = q P + r
    Div dP, dspan, dnt, dftot;   // division by P, nt + alpha, nt and ftot (set_divisors)
};
inline void set_divisors(Split& s) {
    s.dP = make_div(s.P);
    s.dspan = make_div(s.nt + s.alpha);
    s.dnt = make_div(s.nt);
    s.dftot = make_div(s.ftot);
}

// C_p, the first cost position of workgroup p (C_P = ftot; p r < 2^20).
__host__ __device__ inline int cost_start(int p, const Split& s) { return p * s.q + div_by(p * s.r, s.dP); }

// The first unit at or after cost position c: inside a row group's span the unit at c, inside the boundary
// gap after group g the first unit of group g + 1.
__host__ __device__ inline int unit_at(int c, const Split& s) {
    const int span = s.nt + s.alpha;
    const int g = div_by(c, s.dspan), rem = c - g * span;
    return g * s.nt + (rem < s.nt ? rem : s.nt);
}

// Workgroup p owns units [unit_at(C_p), unit_at(C_(p+1))). The owner of unit x is the largest p with
// C_p <= F(x) (unit_at(C) <= x exactly when C <= F(x)), i.e. ((F(x) + 1) P - 1) / ftot.
__host__ __device__ inline int owner_of(int x, const Split& s) {
    const int fx = x + s.alpha * div_by(x, s.dnt);
    const int p = fx < 0x7fffffff / s.P ? div_by((fx + 1) * s.P - 1, s.dftot)
                                        : (int)((((long long)fx + 1) * s.P - 1) / s.ftot);
    return p < s.P - 1 ? p : s.P - 1;
}
__host__ __device__ inline int first_wg(int g, const Split& s) { return owner_of(g * s.nt, s); }
__host__ __device__ inline int last_wg(int g, const Split& s) { return owner_of((g + 1) * s.nt - 1, s); }

// A packed cloud: a 256-byte header of 32-bit words
//     [0] max |coordinate| (float bits), [1] s, the power-of-two scale of the cloud's own pieces (1 for kBF16x3),
//     [2] c_b, the score scale its log2-unit copy was made for (0: no valid copy),
//     [3] the scale of the second cloud that copy was made against, [4] the copy's unit t (a power of two),
//     [5] L0, the integer offset of the cloud's log2 weights in the on-device loop (a float; written at loop
//         init, 0 elsewhere),
// then the tiles of the cloud's own pieces (s x), then (kF16x2 only) the tiles of its log2-unit copy: two fp16
// pieces of t fl(c_b x) / s_2 per coordinate, which the first cloud of a pair carries so that its piece products
// with the second cloud's own pieces sum to t c_b x.y, the half-step's score in log2 units times t (see
// bake_params in sk_epilogue.h).
template <class T>
__host__ __device__ inline const T* packed_tiles(const void* pk) {
    return reinterpret_cast<const T*>(reinterpret_cast<const char*>(pk) + kHeaderBytes);
}
// The log2-unit copy of a kF16x2 cloud of npad points and nc K chunks.
template <class T>
__host__ __device__ inline const T* packed_log2_tiles(const void* pk, int npad, int nc) {
    return packed_tiles<T>(pk) + (size_t)(npad / 32) * nc * 2 * 64;
}
__device__ inline float packed_scale(const void* pk) { return reinterpret_cast<const float*>(pk)[1]; }

// A half-step takes its scores in log2 units from the matrix cores ("log2_ready") when the first cloud's
// log2-unit copy was made for its score scale c = (2 / eps) log2(e) and against its second cloud: header word
// [2] of the first cloud equals c (and is not 0) and word [3] equals the second cloud's scale, word [1]. The
// partial and the merge kernels test this on the same header words.

// The on-device loop's configuration (src/trnopt/sinkhorn.py:313-320, 340-344).
struct LoopCfg {
    const double* sched;
    const double* stages;
    int n_sched, n_stages;
    double eps, rho_x, rho_y, tol, stage_tol;
    int max_iters, check_every, stage_max_iters, fixed_iters, balanced;
};

// Work-item and workgroup ids straight from the hardware registers. threadIdx / blockIdx / blockDim call
// device-library functions, which the compiler stops inlining into kernels as large as the partial kernel;
// every such call makes the kernel spill its scalars around it.
__device__ __forceinline__ int tid_x() { return (int)__builtin_amdgcn_workitem_id_x(); }
__device__ __forceinline__ int wg_x() { return (int)__builtin_amdgcn_workgroup_id_x(); }

struct PartialArgs {
    const void* xr;     // packed rows (header, then two fp16 pieces per scaled coordinate)
    const void* yc;     // packed columns
    const float* u;     // column term = alpha * u + beta * v  (m_pad each)
    const float* v;
    float* u2;          // or null: the column cloud's potential in log2 units (on-device loop), (c / 2) u + Ll
    const float* v2;    // with u2: the column cloud's log2 weights Lh (log2(e) log w - L0 = Lh + Ll, L0 in word 5)
    const float* sc;    // {2/eps, 1/eps, eps, kappa} (half-step mode)
    const int* skip;
    float2* part;       // [slot][rows_pad] partial (M, S): M = max_j a_ij, S = sum_j exp2(c (a_ij - M))
    int nrb;            // row blocks of 32
    int rows_pad;
    int mode;
    int rows_role;      // 0: the rows are the first cloud of the pair, 1: the second (piece order)
    int contraction;    // kF16x2 or kBF16x3 (the packing of both clouds)
    int nc;             // K chunks of 16 coordinates
    Split s;
    // The merge pass (one workgroup per row group):
    const float* xsq;   // |x|^2 (half-step epilogue)
    const float* off;   // log(target / weight) or null
    float* out;         // merged result (fh, or the plain row-LSE)
    float* out2;        // or null: with log2-unit scores, also the result in log2 units, (c / 2) fh + Ll
    const float* rows_l2lo;   // with out2: the rows' Ll (the low part of their log2 weights)
    const float* cols_l2lo;   // with out2 and rebake: the columns' Ll
    int n_store;        // rows of out written
    float2* meas;       // per-group convergence partials (g update of the loop), or null
    const float* w;     // row weights, with meas
    int n_real;         // real rows, with meas
    int* counters;      // with state: one arrival counter, zero on entry and left zero
    int* group_counters;  // or null: per row group arrival counters (zero on entry, left zero); the partial
                          // kernel's last workgroup to finish a row group merges it (no merge kernel)
    int ngroups;
    // ... and, in the last merge workgroup of a g update, the loop control (null: none), which also remakes the
    // log2-unit copy of the first cloud (rebake, the packed first cloud; null: never) when eps changes; the f
    // update's merge advances the state's iteration counters (tick; null: none).
    sk_state* tick;
    sk_state* state;
    LoopCfg cfg;
    char* rebake;
};

// Launch the partial kernel for kp = 16 * nc on P workgroups (nc <= 4: launch_partial_small, else
// launch_partial_large; the two are separate objects built from sk_lse_partial.hip). kBF16x3 exists for
// rows_role 0 only.
// Sets the message that sk_last_error() returns and passes `code` through.
int fail(int code, const char* fmt, ...);
int hip_fail(hipError_t e, const char* where);

hipError_t launch_partial_small(const PartialArgs& a, int nc, hipStream_t stream);
hipError_t launch_partial_large(const PartialArgs& a, int nc, hipStream_t stream);
inline hipError_t launch_partial(const PartialArgs& a, int nc, hipStream_t stream) {
    return nc <= 4 ? launch_partial_small(a, nc, stream) : launch_partial_large(a, nc, stream);
}
// The grouped partial kernel of the fp16 half-steps (rows_role `role` in every pass): nmap workgroups, workgroup b
// running workgroup map[b] & 0xffff of pass map[b] >> 16 of args[0 .. count) (device memory, kp = 16 nc each).
hipError_t launch_grouped_small(const PartialArgs* args, const unsigned* map, int count, int nmap, int nc, int role,
                                hipStream_t stream);
hipError_t launch_grouped_large(const PartialArgs* args, const unsigned* map, int count, int nmap, int nc, int role,
                                hipStream_t stream);
inline hipError_t launch_grouped(const PartialArgs* args, const unsigned* map, int count, int nmap, int nc, int role,
                                 hipStream_t stream) {
    return nc <= 4 ? launch_grouped_small(args, map, count, nmap, nc, role, stream)
                   : launch_grouped_large(args, map, count, nmap, nc, role, stream);
}

}  // namespace sk
