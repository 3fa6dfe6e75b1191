// Definitions shared by the two translation units of libtrnopt_hip.so: the MFMA partial kernel
// (sk_lse_partial.hip, built without NaN semantics so row maxima need no canonicalisation) and the rest
// (sk_kernels.hip: packing, finalisation, loop control, C ABI).
#pragma once

#include <hip/hip_runtime.h>

namespace sk {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr float kLog2e = 1.44269504088896340736f;
constexpr float kLn2 = 0.69314718055994530942f;
constexpr float kEmpty = -1.0e30f;     // running max of a row before its first column (finite on purpose)
constexpr int kWaves = 4;              // waves per workgroup of the partial kernel (one per SIMD)
constexpr int kBlock = kWaves * 64;
constexpr int kRowBlocks = 2;          // 32-row blocks per wave (independent MFMA accumulator chains)
constexpr int kXcds = 8;
constexpr int kMaxChunks = 8;          // K chunks of 16 coordinates: kp = 16 * nc <= 128
constexpr int kPieces = 3;             // bf16 pieces per fp32 coordinate

enum Mode { kHalfStep = 0, kPlainLse = 1 };

// Work split shared by the partial and the finalisation kernels: the (row group, column tile) units are
// cut into P equal contiguous ranges, one per workgroup.
struct Split {
    long long work;  // row groups * column tiles
    int nt;          // column tiles
    int P;           // workgroups
};

// Workgroup p owns units [p * work / P, (p + 1) * work / P). The owner of unit x is the largest p with
// floor(p * work / P) <= x, i.e. ((x + 1) * P - 1) / work.
__host__ __device__ inline int owner_of(long long x, const Split& s) {
    const long long p = ((x + 1) * (long long)s.P - 1) / s.work;
    return (int)(p < s.P - 1 ? p : s.P - 1);
}
__host__ __device__ inline int first_wg(int g, const Split& s) { return owner_of((long long)g * s.nt, s); }
__host__ __device__ inline int last_wg(int g, const Split& s) {
    return owner_of((long long)(g + 1) * s.nt - 1, s);
}

struct PartialArgs {
    const bf16x8* xr;   // packed rows (three bf16 pieces per coordinate)
    const bf16x8* yc;   // packed columns
    const float* u;     // column term = alpha * u + beta * v  (m_pad each)
    const float* v;
    const float* sc;    // {2/eps, 1/eps, eps, kappa} (half-step mode)
    const int* skip;
    float2* part;       // [slot][rows_pad] partial (M, S): M = max_j a_ij, S = sum_j exp2(c (a_ij - M))
    int nrb;            // row blocks of 32
    int rows_pad;
    int mode;
    int rows_role;      // 0: the rows are the first cloud of the pair, 1: the second (piece order)
    Split s;
};

// Launch the partial kernel for kp = 16 * nc on P workgroups (nc <= 4: launch_partial_small, else
// launch_partial_large; the two are separate objects built from sk_lse_partial.hip).
hipError_t launch_partial_small(const PartialArgs& a, int nc, hipStream_t stream);
hipError_t launch_partial_large(const PartialArgs& a, int nc, hipStream_t stream);
inline hipError_t launch_partial(const PartialArgs& a, int nc, hipStream_t stream) {
    return nc <= 4 ? launch_partial_small(a, nc, stream) : launch_partial_large(a, nc, stream);
}

}  // namespace sk
