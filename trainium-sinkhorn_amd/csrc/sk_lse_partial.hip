// The MFMA partial (max, sum) kernel of the fused Sinkhorn half-step, gfx950.
//
// Built with -fno-honor-nans -mno-amdgpu-ieee: row maxima are taken directly over MFMA results, which in
// IEEE mode would first be canonicalised one by one. No value here is NaN or infinite: padding and empty
// rows use large finite sentinels.
//
// Contraction. Every packed cloud carries a power-of-two scale s (max |coordinate| * s in [2^4, 2^5)),
// and every scaled coordinate v = s x is stored as two fp16 pieces v = v0 + v1 (22 significand bits: within
// 2^-23 of v, about one fp32 ulp; sk_kernels.hip packs them). The dot product of two scaled points is
// accumulated in fp32 by v_mfma_f32_32x32x16_f16 from the three products
//
//     x0 y0, x0 y1, x1 y0                          (each fp16 x fp16 product is exact in fp32);
//
// the fourth, x1 y1, is at most 2^-22 |x_k y_k| and left out. This reproduces x.y at least as accurately as
// an fp32 dot product (error ~1e-7 of sum |x_k y_k| on N(0, 1) data; a float32 dot product gives ~2.3e-7,
// the fp32 MFMA chain 3.2e-7). With sigma = s_x s_y, the kernel works in scaled accumulator units
// sigma a = D + sigma (column term) and c / sigma, all exact power-of-two rescalings, and stores M / sigma.
// When the first cloud carries its log2-unit copy (pieces of t fl(c x) / s_y, t a power of two) for this
// launch's c, the same three products of the copy and the second cloud's own pieces give t c x.y: the scores
// are in log2 units times t and the exponentials take them with one fma that subtracts the max and rescales
// by 1 / t exactly (L2 below); M is stored in log2 units.
// On gfx950 the fp16 matrix pipe runs at ~15x the fp32 MFMA rate and, unlike the fp32 MFMA, issues alongside
// VALU work of the same SIMD, so the exp / max / sum epilogue of one tile hides under the MFMAs of the next.
// The general row log-sum-exp of arbitrary fp32 matrices (whose columns may mix magnitudes 1e9 apart, as the
// augmented padding rows do) uses the exact three-way bf16 split instead: v = v0 + v1 + v2, six products
// x0 y0, x0 y1, x1 y0, x0 y2, x1 y1, x2 y0 on v_mfma_f32_32x32x16_bf16, scale 1.
//
// Symmetry. The f update (rows x, columns y) and the g update (rows y, columns x) must form bit-identical
// x_i . y_j: in the cold regime a row's log-sum-exp is one dominant score, and any rounding difference
// between the directions would push f_i + g_j of that pair by the same amount every iteration (a linear
// drift along the pair's neutral mode). The products are exact and the MFMA adds them in k order, so the two
// directions agree when they issue the same (x piece, y piece) pairs in the same order (sigma is the same
// product of the two scales in both directions): `rows_role` says
// whether the rows are the first or the second cloud, and the pair list is transposed accordingly. The
// contraction starts from zero and the column term is added afterwards: by one more MFMA per row block and
// tile with the fp16 contraction (the fp32 term split exactly into bf16 pieces, summed against B = 1:
// exact for every fp32 value, since bf16 has fp32's exponent range, with q's largest piece in quarters so that
// the MFMA's rounding of the sum is nearly unbiased, column_operand; 32 VALU adds per tile fewer), on the VALU
// otherwise. The max is subtracted before scaling, exp2(c (a - M)), so the dominant term
// is exactly 1.
//
// Layout of one workgroup (one row group of 256 rows): 4 waves, one per SIMD, and wave w owns 2 blocks of 32
// rows of the group (its fp16 pieces stay in registers for the whole work segment); all waves walk the same
// column tiles. Two ways to feed the column tiles (streamed_form):
//   - streamed (every fp16 half-step, and the bf16 row log-sum-exp up to kp 64): every wave loads the tile's
//     pieces straight into registers one tile ahead (above kp 64 chunk by chunk, into the registers of the chunk
//     just used); the four waves of the CU read the same addresses at about the same time and share them
//     through L1. The column terms of the whole segment are computed once into LDS
//     (as MFMA operands with the fp16 contraction). No per-tile barrier.
//   - staged (the bf16 row log-sum-exp above kp 64, whose three pieces per coordinate no longer fit in registers
//     twice): the workgroup stages the tiles and their column terms once in LDS through a ring of three tile
//     buffers, two tiles ahead, one barrier per tile; each wave reads its column operands chunk by chunk a few
//     chunks ahead of their MFMAs, once for both of its row blocks.
// MFMA orientation: A = 32 columns, B = 32 rows, so lane l's 16 accumulators all belong to row l % 32
// (columns 8 (r / 4) + 4 (l / 32) + r % 4); row reductions stay inside a lane and lanes l, l + 32 are merged
// once per segment.
//
// This file is compiled twice: SK_PARTIAL_LARGE = 0 builds the instantiations of nc <= 4, SK_PARTIAL_LARGE = 1
// those of nc > 4 (kp 80 to 128), both with MFMA results forced into VGPRs (-mllvm -amdgpu-mfma-vgpr-form: the
// epilogue reads them without copies).

#include <type_traits>
#include <utility>

#include "sk_common.h"
#include "sk_epilogue.h"

#ifndef SK_PARTIAL_LARGE
#define SK_PARTIAL_LARGE 0
#endif

namespace sk {
namespace {

// Waves per workgroup and 32-row blocks per wave, both variants: 4 waves, one per SIMD, 2 row blocks each (two
// accumulator chains per wave, the epilogue interleaved with the MFMAs at compile time). With one wave per SIMD a
// wave may use all 512 registers of its lanes, VGPRs and AGPRs: at kp 128 the streamed variant holds its row
// operands (128 registers), one tile's column operands as a ring of chunks (64), two accumulator sets per row
// block and the epilogue in about 350, the MFMA results in VGPRs and part of the operands in AGPRs, which the
// MFMAs read directly (32 register copies per tile, no scratch).
constexpr int kWavesK = 4, kRowBlocksK = 2, kWavesPerSimd = 1;
constexpr int kBlockK = 64 * kWavesK;
static_assert(32 * kRowBlocksK * kWavesK == kRowsPerGroup, "a row group is 256 rows in both variants");

__device__ __forceinline__ float ex2(float x) { return __builtin_amdgcn_exp2f(x); }

// A workgroup barrier that orders LDS only: the release / acquire fences are restricted to the local address
// space, so that the wave waits for its LDS accesses (lgkmcnt) but not for its global loads in flight. (The
// fences of __syncthreads also cover global memory and made every wave wait for all its outstanding operand
// loads at the barrier.) For barriers that protect LDS buffers only.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Hardware hands consecutive workgroup ids to the 8 XCDs in turn; renumber so that the workgroups of one
// XCD own one contiguous range of the work.
__device__ __forceinline__ int xcd_contiguous(int b, int P) {
    const int q = P / kXcds, r = P % kXcds;
    const int xcd = b % kXcds, idx = b / kXcds;
    return xcd * q + (xcd < r ? xcd : r) + idx;
}

// max(a, b, c) as one v_max3_f32 (the compiler would pair the operands into a tree of two-operand maxima).
// Its operands are always written by VALU instructions (the column-term adds), never directly by an MFMA.
__device__ __forceinline__ float max3(float a, float b, float c) {
    float r;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}

// Compile-time loop: f(integral_constant<int, i>) for i in [B, E).
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

// The online log-sum-exp update of one row block and one tile, as kOps elementary steps:
//   j == 0:        the tile's 16 column terms of this lane from LDS (four 16-byte reads, shared by the row
//                  blocks; costed high so that the adds land a few MFMA slots later, past the LDS latency)
//   j in [1, 17):  a_r = acc_r + col_r
//   j in [17, 25): running max over a pair of scores
//   j in [25, 41): acc_r = exp2(c (a_r - m)), in place
//   j in [41, 56): the sum of the 16 exponentials as a pairwise tree (8 + 4 + 2 + 1 adds), long after the
//                  exponentials were issued, so no add waits on the transcendental unit
//   j == 56:       S = S exp2(c (M - m)) + sum, M = m
// With FOLD the matrix pipe has already added the column terms (one more MFMA per row block and tile, see
// Streamed) and steps 1-16 are empty; step 0 only starts the running max, costed so that the first reads of
// the accumulators come a few MFMA slots after the last MFMA of the tile.
// The max is subtracted before the scaling: a - m is exact for the scores near the maximum, so the dominant
// term is exactly 1 and S is relative to 2^(c M) exactly, which is what the merge of the slots assumes.
// (Folding the offset into one fma, exp2(c a - fl(c m)), would leave S relative to the rounded fl(c M): an
// error of up to half an ulp of c M in the log-sum-exp, which moves with M from one iteration to the next
// and holds float32 Sinkhorn several ulps away from its fixed point. With L2, c is a power of two, c m is
// exact, and the fma is exactly c (a - m).)
// Steps are spread over the MFMA slots of the next tile in proportion to their cost.
constexpr int kOps = 57;
template <bool FOLD>
constexpr int op_cost(int j) {
    return FOLD && j > 0 && j < 17 ? 0 : j == 0 ? (FOLD ? 6 : 8) : (j >= 25 && j < 41) ? 4 : j == 56 ? 4 : 1;
}
template <bool FOLD>
constexpr int block_cost() {
    int s = 0;
    for (int j = 0; j < kOps; ++j) s += op_cost<FOLD>(j);
    return s;
}
// First step of slot i of NS (steps of the row blocks interleaved: step k is step k / RB of block k % RB).
template <int RB, bool FOLD>
constexpr int op_begin(int i, int NS) {
    const int target = (int)((long long)i * RB * block_cost<FOLD>() / NS);
    int cost = 0, k = 0;
    while (k < RB * kOps && cost < target) {
        cost += op_cost<FOLD>(k / RB);
        ++k;
    }
    return k;
}

// col4(q) returns the column terms of accumulators 4q .. 4q + 3 of the tile being updated (unused with FOLD).
// With L2 the scores are in log2 units times the copy's unit t (the first cloud's log2-unit copy) and c = 1 / t,
// a power of two: the max is subtracted and the rescaling applied by one fma, exp2(fma(a, c, -c m)), exact in
// c m and equal to exp2(c (a - m)) bit for bit (for t = 1, exp2(a - m)).
template <int RB, bool L2, bool FOLD = false>
struct Online {
    float m[RB];
    float mc[RB];      // L2: c m
    f32x4 cv[4];
    template <int k, class ColFn>
    __device__ __forceinline__ void step(f32x16 (&acc)[RB], ColFn&& col4, float (&M)[RB], float (&S)[RB], float c) {
        constexpr int j = k / RB, b = k % RB;
        if constexpr (j == 0) {
            if constexpr (b == 0 && !FOLD)
#pragma unroll
                for (int q = 0; q < 4; ++q) cv[q] = col4(q);
            m[b] = M[b];
        } else if constexpr (j < 17) {
            if constexpr (!FOLD) {
                constexpr int r = j - 1;
                acc[b][r] = acc[b][r] + cv[r / 4][r % 4];
            }
        } else if constexpr (j < 25) {
            constexpr int p = j - 17;
            // With FOLD the operands come straight from the MFMAs: a compiler-visible maximum, so that the
            // compiler keeps the wait states between the matrix results and their first VALU read.
            if constexpr (FOLD)
                m[b] = __builtin_fmaxf(__builtin_fmaxf(m[b], acc[b][2 * p]), acc[b][2 * p + 1]);
            else
                m[b] = max3(m[b], acc[b][2 * p], acc[b][2 * p + 1]);
        } else if constexpr (j < 41) {
            constexpr int r = j - 25;
            if constexpr (L2) {
                if constexpr (r == 0) mc[b] = m[b] * c;
                acc[b][r] = ex2(fmaf(acc[b][r], c, -mc[b]));
            } else {
                acc[b][r] = ex2(c * (acc[b][r] - m[b]));
            }
        } else if constexpr (j < 56) {
            // tree level l (stride 2^l) pairs acc[2^(l+1) q] += acc[2^(l+1) q + 2^l]
            constexpr int t = j - 41;
            constexpr int l = t < 8 ? 0 : t < 12 ? 1 : t < 14 ? 2 : 3;
            constexpr int q = t - (l == 0 ? 0 : l == 1 ? 8 : l == 2 ? 12 : 14);
            constexpr int lo = q << (l + 1), hi = lo + (1 << l);
            acc[b][lo] = acc[b][lo] + acc[b][hi];
        } else {
            S[b] = fmaf(S[b], ex2(L2 ? fmaf(M[b], c, -mc[b]) : c * (M[b] - m[b])), acc[b][0]);
            M[b] = m[b];
        }
    }
};

// The contractions: operand type, pieces per coordinate, the products as (first-cloud piece, second-cloud
// piece) in issue order, and the MFMA.
template <int CT>
struct Contract;

template <>
struct Contract<kF16x2> {
    using T = f16x8;
    static constexpr int pieces = 2, products = 3;
    static constexpr int first[3] = {0, 0, 1};               // x0 y0, x0 y1, x1 y0
    static constexpr int second[3] = {0, 1, 0};
    static __device__ __forceinline__ f32x16 mfma(const T& a, const T& b, const f32x16& c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
};

template <>
struct Contract<kBF16x3> {
    using T = bf16x8;
    static constexpr int pieces = 3, products = 6;
    static constexpr int first[6] = {0, 0, 1, 0, 1, 2};     // x0 y0, x0 y1, x1 y0, x0 y2, x1 y1, x2 y0
    static constexpr int second[6] = {0, 1, 0, 2, 1, 0};
    static __device__ __forceinline__ f32x16 mfma(const T& a, const T& b, const f32x16& c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
};

// The A operand of the column MFMA (v_mfma_f32_32x32x16_bf16 against B = 1 in k < kColPieces of every row): the
// column term q as bf16 pieces that sum to it exactly, (q0 / 4, q0 / 4, q0 / 4, q0 / 4, q1, q2, 0, 0) with
// q0 = bf16(q), q1 = bf16(q - q0), q2 = q - q0 - q1 (each piece the nearest bf16 to what the earlier ones leave:
// 8 + 8 + 8 significand bits, all of fp32's; q0 / 4 is exact for |q| >= 2^-124, and bf16 has fp32's exponent
// range, so no term is out of range).
// Why q0 comes in quarters: this MFMA floors its accumulator input onto the grid of half an ulp of its largest
// product, 2^(e - 24) for a largest product in [2^e, 2^(e+1)), and then rounds the sum to nearest; products
// below that grid are dropped. (Measured on gfx950 over 4.2 million (accumulator, term) pairs of either sign and
// magnitude ratios 2^-14 to 2^3: that rule reproduces every result bit for bit.) With q0 whole, an accumulator
// (the dot product) much smaller than the column term therefore comes out a quarter ulp low on average, a bias
// toward -inf that does not average out over a row's scores and, at eps far above the scores' spread, moved
// balanced potentials along their neutral mode. With the largest product q0 / 4 the grid is four times finer and
// the bias a sixteenth of an ulp (measured: -0.060 against -0.249 ulp of the result); a compensating piece
// below the grid would be dropped, so none is added.
constexpr int kColPieces = 6;
__device__ __forceinline__ bf16x8 column_operand(float v) {
    const __bf16 q0 = (__bf16)v;
    const float r1 = v - (float)q0;                       // exact
    const __bf16 q1 = (__bf16)r1;
    const __bf16 q2 = (__bf16)(r1 - (float)q1);           // exact: at most 8 significant bits remain
    const __bf16 qq = (__bf16)((float)q0 * 0.25f);        // exact
    return bf16x8{qq, qq, qq, qq, q1, q2, 0, 0};
}
// The B operand of the column MFMA: 1 in k < kColPieces of every row (lanes 0-31), zeros elsewhere.
__device__ __forceinline__ bf16x8 column_ones(int h) {
    const __bf16 one = h == 0 ? (__bf16)1.0f : (__bf16)0.0f;
    return bf16x8{one, one, one, one, one, one, 0, 0};
}

// End of a work segment: lanes l and l + 32 hold the same row over different columns; merge them and store
// (M / sigma, S) of each row (with L2, sigma is the copy's unit t and M / t is in log2 units).
template <int RB, bool L2>
__device__ __forceinline__ void store_rows(const PartialArgs& a, const float (&M)[RB], const float (&S)[RB], int rb0,
                                           int slot, float c, float inv_sigma, int lane) {
#pragma unroll
    for (int b = 0; b < RB; ++b) {
        const float Mo = __shfl_xor(M[b], 32);
        const float So = __shfl_xor(S[b], 32);
        const float Mn = fmaxf(M[b], Mo);
        const float Sn = S[b] * ex2(c * (M[b] - Mn)) + So * ex2(c * (Mo - Mn));
        if (lane < 32 && rb0 + b < a.nrb) {
            float2* dst = a.part + (size_t)slot * a.rows_pad + (size_t)(rb0 + b) * 32 + lane;
            // (a segment whose columns all have zero weight has M near the -1e30 floor; kept finite when
            // rescaled, as an empty slot)
            const float2 v = make_float2(fmaxf(Mn * inv_sigma, kEmpty), Sn);
            if (a.group_counters != nullptr)
                coh_store(dst, v);           // read back in this launch by the group's last workgroup
            else
                *dst = v;
        }
    }
}

// Register ring of the staged kernel's column operands: chunk g of a pair of tiles (g = 0 .. 2 nc - 1) sits in
// slot g % D, read D - 1 chunks ahead of its MFMAs; D divides 2 nc so that the slots repeat every two tiles.
constexpr int ring_depth(int nc) { return (2 * nc) % 4 == 0 ? 4 : 2; }   // three-piece chunks: at most 48 registers

// The staged kernel: the general row log-sum-exp (three bf16 pieces, six products, ROLE 0, no log2-unit copy)
// above kp 64, where its operands no longer fit in registers twice. (The fp16 half-steps stream at every kp.)
template <int NC, int ROLE, int CT, bool L2>
struct Staged {
    static_assert(CT == kBF16x3 && ROLE == 0 && !L2, "the staged kernel runs the bf16 row log-sum-exp only");
    using C = Contract<CT>;
    using T = typename C::T;
    static constexpr int kPieces = C::pieces;
    static constexpr int kProducts = C::products;
    static constexpr int RB = kRowBlocksK;
    static constexpr int TILE16 = NC * kPieces * 64;   // 16-byte units per packed 32-point tile
    static constexpr int PER_THREAD = (TILE16 + kBlockK - 1) / kBlockK;
    static constexpr int NS = kProducts * NC * RB;     // MFMA slots per tile
    static constexpr int D = ring_depth(NC);           // register slots of column chunks
    static constexpr int LA = D - 1;                   // chunks read ahead
    static constexpr int kStageSlot = NS / 2;          // the MFMA slots from which the tile two ahead is staged

    // Rows rb0 .. rb0 + RB - 1 against column tiles [tb, te); writes one (M, S) per row into `slot`.
    //
    // Pipeline, tile by tile (tile q = tb + q: its operands in LDS buffer q % 3, its column terms in column buffer
    // q % 4):
    //   - from half-way through each tile, spread over a few MFMA slots, tile q + 2 is written to LDS from
    //     registers (its buffer held tile q - 1, which every wave finished before the barrier that ended it) and the
    //     same registers are loaded with tile q + 4 (two register sets, by the parity of q): about two tiles of
    //     latency cover for the global loads;
    //   - the column operands of a tile are read chunk by chunk, LA chunks ahead of their MFMAs, the last ones of a
    //     tile already reading the first chunks of the next (staged at least a tile earlier, visible since the
    //     barrier that ended that tile), so that the matrix pipe does not wait on LDS after a barrier;
    //   - one barrier per tile.
    __device__ __forceinline__ static void run(const PartialArgs& a, int rb0, int tb, int te, int slot, const float* cu,
                                               const float* cv, float alpha, float beta, float beta_lo, float cs,
                                               float c, float inv_sigma, T* lds_y, float* lds_col) {
        const int tid = tid_x();
        const int lane = tid & 63;
        const int h = lane >> 5;
        const T* xt = packed_tiles<T>(a.xr);
        const T* yt = packed_tiles<T>(a.yc);

        T xv[RB][NC][kPieces];
#pragma unroll
        for (int b = 0; b < RB; ++b) {
            const int blk = rb0 + b < a.nrb ? rb0 + b : a.nrb - 1;   // a missing block recomputes the last one
#pragma unroll
            for (int cc = 0; cc < NC; ++cc)
#pragma unroll
                for (int p = 0; p < kPieces; ++p)
                    xv[b][cc][p] = xt[(size_t)blk * TILE16 + (cc * kPieces + p) * 64 + lane];
        }
        float M[RB], S[RB];
#pragma unroll
        for (int b = 0; b < RB; ++b) {
            M[b] = kEmpty;
            S[b] = 0.0f;
        }

        // Staging of one tile. Thread `tid` copies the 16-byte units tid, tid + kBlockK, ... of the tile (clamped:
        // threads mapped to the same unit write the same value), and lane l % 32 of every wave the inputs of the
        // column term of column l % 32 (the lanes and waves write the same values). Branch-free, so that a whole
        // tile is one basic block and the epilogue stays between the MFMAs. The loads land in registers that
        // nothing reads until the stage (the column term itself is formed there), so that no instruction in
        // between waits for them.
        const int last = te - 1;
        const int cl = lane & 31;                           // column of the tile
        unsigned offb[PER_THREAD];                          // byte offsets of this thread's units in a tile
#pragma unroll
        for (int k = 0; k < PER_THREAD; ++k)
            offb[k] = (unsigned)(tid + k * kBlockK < TILE16 ? tid + k * kBlockK : TILE16 - 1) * 16u;
        T pf[2][PER_THREAD];
        float pv[2], pu[2];
        auto prefetch_tile = [&](int s, int t) {
            const char* src = reinterpret_cast<const char*>(yt + (size_t)(t < te ? t : last) * TILE16);
#pragma unroll
            for (int k = 0; k < PER_THREAD; ++k) pf[s][k] = *reinterpret_cast<const T*>(src + offb[k]);
        };
        auto prefetch_cols = [&](int s, int t) {
            const int tc = t < te ? t : last;
            pv[s] = cv[tc * 32 + cl];
            pu[s] = cu[tc * 32 + cl];
        };
        auto stage_tile = [&](int s, int ybuf) {
            char* dst = reinterpret_cast<char*>(lds_y + ybuf * TILE16);
#pragma unroll
            for (int k = 0; k < PER_THREAD; ++k) *reinterpret_cast<T*>(dst + offb[k]) = pf[s][k];
        };
        auto stage_cols = [&](int s, int cbuf) {
            lds_col[cbuf * 32 + cl] = fmaxf(cs * fmaf(beta, pv[s], fmaf(beta_lo, pv[s], alpha * pu[s])), kPadScore);
        };
        auto prefetch = [&](int s, int t) {
            prefetch_tile(s, t);
            prefetch_cols(s, t);
        };
        auto stage = [&](int s, int ybuf, int cbuf) {
            stage_tile(s, ybuf);
            stage_cols(s, cbuf);
        };
        // The ring of column chunks: slot g % D holds chunk g of the current pair of tiles.
        T yr[D][kPieces];
        auto read_chunk = [&](auto G, int ytile) {
            constexpr int g = decltype(G)::value;
            constexpr int cc = g % NC;
#pragma unroll
            for (int p = 0; p < kPieces; ++p) yr[g % D][p] = lds_y[ytile * TILE16 + (cc * kPieces + p) * 64 + lane];
        };

        f32x16 accA[RB], accB[RB];
        Online<RB, false, false> on;
        // Ring positions of the current tile: LDS buffers yq = q % 3 and cq = q % 4.
        int yq = 0, cq = 0;
        auto nxt3 = [](int v) { return v == 2 ? 0 : v + 1; };
        auto nxt4 = [](int v) { return (v + 1) & 3; };
        // Tile t of phase PH (t - tb even: 0, odd: 1): MFMAs into accN from zero, and (epi) the update of the previous
        // tile (accP, its column terms at colp) spread between them, one slot per MFMA, fenced so that the compiler
        // keeps the interleave; tile t + 2 staged and tile t + 4 loaded into register set PH.
        auto tile = [&](auto PH, int t, f32x16 (&accN)[RB], f32x16 (&accP)[RB], const float* colp, bool epi) {
            constexpr int ph = decltype(PH)::value;
            auto col4 = [&](int q) { return *reinterpret_cast<const f32x4*>(colp + 8 * q); };
            const int ynext = nxt3(yq);
#pragma unroll
            for (int b = 0; b < RB; ++b) accN[b] = f32x16{};
            static_for<0, NS>([&](auto I) {
                constexpr int i = decltype(I)::value;
                constexpr int cc = i / (kProducts * RB), p = (i / RB) % kProducts, b = i % RB;
                constexpr int g = ph * NC + cc;           // this chunk's place in the pair of tiles
                if constexpr (p == 0 && b == 0) {
                    // the chunk LA ahead: of this tile, or the first ones of the next
                    if constexpr (cc + LA < NC)
                        read_chunk(std::integral_constant<int, (g + LA) % (2 * NC)>{}, yq);
                    else
                        read_chunk(std::integral_constant<int, (g + LA) % (2 * NC)>{}, ynext);
                }
                accN[b] = C::mfma(yr[g % D][C::second[p]], xv[b][cc][C::first[p]], accN[b]);
                if (epi) {
                    constexpr int k0 = op_begin<RB, false>(i, NS), k1 = op_begin<RB, false>(i + 1, NS);
                    static_for<k0, k1>([&](auto K) { on.template step<decltype(K)::value>(accP, col4, M, S, c); });
                }
                // The staging, spread over a few slots: the tile's units (and the column terms) are written out
                // before the same registers are loaded again.
                if constexpr (i == kStageSlot - 2) stage_cols(ph, nxt4(nxt4(cq)));
                if constexpr (i == kStageSlot) stage_tile(ph, nxt3(nxt3(yq)));
                if constexpr (i == kStageSlot + 1) prefetch_tile(ph, t + 4);
                if constexpr (i == kStageSlot + 2) prefetch_cols(ph, t + 4);
                __builtin_amdgcn_sched_barrier(0);
            });
        };
        auto update = [&](f32x16 (&accP)[RB], const float* colp) {
            auto col4 = [&](int q) { return *reinterpret_cast<const f32x4*>(colp + 8 * q); };
            static_for<0, RB * kOps>([&](auto K) { on.template step<decltype(K)::value>(accP, col4, M, S, c); });
        };
        // Column terms of the tile in column buffer cbuf, as this lane's accumulators take them.
        auto colp_of = [&](int cbuf) { return lds_col + cbuf * 32 + 4 * h; };
        // After a tile: to the next buffers and a barrier there.
        auto advance = [&]() {
            yq = nxt3(yq);
            cq = nxt4(cq);
            __syncthreads();
        };

        // Prologue: tiles tb and tb + 1 staged, tb + 2 and tb + 3 in the register sets, the first chunks of tile tb
        // read. Every prefetch / stage is unconditional (tiles past the last one are the last one again).
        prefetch(0, tb);
        prefetch(1, tb + 1);
        stage(0, 0, 0);
        stage(1, 1, 1);
        prefetch(0, tb + 2);
        prefetch(1, tb + 3);
        __syncthreads();
        static_for<0, LA>([&](auto G) { read_chunk(G, 0); });
        int t = tb;
        tile(std::integral_constant<int, 0>{}, t, accA, accB, nullptr, false);
        advance();
        ++t;
        // Tiles in pairs (phase 1 then phase 0), so that the accumulators keep their registers; the column terms
        // of the tile before are in column buffer cq - 1.
        while (te - t >= 2) {
            tile(std::integral_constant<int, 1>{}, t, accB, accA, colp_of((cq + 3) & 3), true);
            advance();
            tile(std::integral_constant<int, 0>{}, t + 1, accA, accB, colp_of((cq + 3) & 3), true);
            advance();
            t += 2;
        }
        if (t < te) {
            tile(std::integral_constant<int, 1>{}, t, accB, accA, colp_of((cq + 3) & 3), true);
            advance();
            update(accB, colp_of((cq + 3) & 3));
        } else {
            update(accA, colp_of((cq + 3) & 3));
        }
        // The next segment's prologue rewrites the first buffers: every wave is done with them first.
        __syncthreads();
        store_rows<RB, false>(a, M, S, rb0, slot, c, inv_sigma, lane);
    }
};

// Column terms computed into LDS once per run of col_tiles(fold) tiles (streamed variant), 16 bytes per column
// with FOLD (98 KB of LDS), 4 without (33 KB), plus one spare entry (col_sink) that the staging's lanes past the
// run's end write to, so that every staging store is unconditional.
constexpr int col_tiles(bool fold) { return fold ? 192 : 256; }
constexpr int col_sink(bool fold) { return fold ? col_tiles(fold) * 32 : (col_tiles(fold) + 1) * 32; }
constexpr int col_floats(bool fold) { return fold ? (col_sink(fold) + 1) * 4 : col_sink(fold) + 1; }
constexpr int kColBatch = 8;
constexpr int kStreamMaxChunks = 4;
// The streamed kernel serves every fp16 half-step (up to kp 128, where one wave per SIMD holds its row operands and
// two column tiles in VGPRs and AGPRs) and the bf16 row log-sum-exp up to kp 64; the staged one that row
// log-sum-exp above kp 64 (three pieces per coordinate). At kp 128 streaming measured 3.4 % faster than staging the
// fp16 tiles through LDS (4.963-4.968 against 5.140-5.145 ms per iteration, 65,536 x 65,536 stress clouds).
constexpr bool streamed_form(int nc, int ct) { return ct == kF16x2 || nc <= kStreamMaxChunks; }

template <int NC, int ROLE, int CT, bool L2>
struct Streamed {
    using C = Contract<CT>;
    using T = typename C::T;
    static constexpr int kPieces = C::pieces;
    static constexpr int kProducts = C::products;
    static constexpr int RB = kRowBlocksK;
    static constexpr int TILE16 = NC * kPieces * 64;
    static constexpr int NS = kProducts * NC * RB;
    static constexpr bool FOLD = CT == kF16x2;      // column terms added by the matrix pipe
    static constexpr int kColTiles = col_tiles(FOLD);
    // Above kp 64 the next tile's operands come as a ring of chunks instead of a second whole tile: chunk cc of
    // tile t + 1 is loaded into the registers of chunk cc of tile t as soon as the last MFMA of that chunk has
    // issued, one tile ahead as before, in half the registers (350 instead of 388 at kp 128: 0.9 % faster on the
    // 65,536 x 65,536 d 128 stress clouds; at kp 64, where both forms fit, 1 % slower).
    static constexpr bool RING = NC > kStreamMaxChunks;

    __device__ __forceinline__ static void run(const PartialArgs& a, int rb0, int tb, int te, int slot, const float* cu,
                                               const float* cv, float alpha, float beta, float beta_lo, float cs,
                                               float c, float inv_sigma, float* lds_col) {
        const int tid = tid_x();
        const int lane = tid & 63;
        const int h = lane >> 5;
        // With L2 the first cloud of the pair (the rows for ROLE 0, the columns for ROLE 1) is read from its
        // log2-unit copy.
        const T* xt = L2 && ROLE == 0 ? packed_log2_tiles<T>(a.xr, a.nrb * 32, NC) : packed_tiles<T>(a.xr);
        const T* yt = L2 && ROLE == 1 ? packed_log2_tiles<T>(a.yc, a.s.nt * 32, NC) : packed_tiles<T>(a.yc);

        T xv[RB][NC][kPieces];
#pragma unroll
        for (int b = 0; b < RB; ++b) {
            const int blk = rb0 + b < a.nrb ? rb0 + b : a.nrb - 1;   // a missing block recomputes the last one
#pragma unroll
            for (int cc = 0; cc < NC; ++cc)
#pragma unroll
                for (int p = 0; p < kPieces; ++p)
                    xv[b][cc][p] = xt[(size_t)blk * TILE16 + (cc * kPieces + p) * 64 + lane];
        }
        float M[RB], S[RB];
#pragma unroll
        for (int b = 0; b < RB; ++b) {
            M[b] = kEmpty;
            S[b] = 0.0f;
        }

        // Column terms into LDS, tile t at (t - cbase) * 32. Without FOLD: tiles [t0 - 1, t1), one float per
        // column (the update of tile t0 - 1 still runs while tile t0's MFMAs do). With FOLD: tiles [t0, t1), each
        // column term q stored as the A operand of one bf16 MFMA, eight bf16 values whose sum is q exactly
        // (column_operand). Eight column terms per thread per batch, all sixteen loads in flight before the first
        // use (a run of up to 256 tiles takes at most five batches, a typical segment one).
        int cbase = tb - 1;
        auto load_batch = [&](int n, int base, int k0, float (&uu)[kColBatch], float (&vv)[kColBatch]) {
#pragma unroll
            for (int q = 0; q < kColBatch; ++q) {
                const int k = k0 + q * kBlockK + tid, j = base + k;
                const int jc = (k < n && j >= 0) ? j : 0;         // clamped in bounds; not stored
                uu[q] = cu[jc];
                vv[q] = cv[jc];
            }
        };
        // Every store is unconditional (lanes past the run write the spare entry col_sink): behind a branch the
        // compiler moved the first load of each batch into it, where it waited alone.
        auto store_batch = [&](int n, int base, int k0, const float (&uu)[kColBatch], const float (&vv)[kColBatch]) {
#pragma unroll
            for (int q = 0; q < kColBatch; ++q) {
                const int k = k0 + q * kBlockK + tid, j = base + k;
                const int ks = (k < n && j >= 0) ? k : col_sink(FOLD);
                const float v = fmaxf(cs * fmaf(beta, vv[q], fmaf(beta_lo, vv[q], alpha * uu[q])), kPadScore);
                if constexpr (FOLD) {
                    reinterpret_cast<bf16x8*>(lds_col)[ks] = column_operand(v);
                } else {
                    lds_col[ks] = v;
                }
            }
        };
        // The run [t0, t1): the first batch's loads, then `between` (the segment's prologue issues its first
        // operand tiles there), then the barrier that frees the buffer, the stores and any further batches. The
        // loads of the hardware's in-order counter complete in issue order, so the column terms, which the
        // staging needs first, are requested before the operand tiles, and waiting for them does not wait for
        // the tiles. (Inside the loop over a workgroup's segments the compiler also waited for every earlier
        // load at the first batch's loop header when the batches were one loop: the first batch is straight-line.)
        auto stage_cols = [&](int t0, int t1, auto&& between) {
            const int n = (t1 - t0 + (FOLD ? 0 : 1)) * 32, base = (t0 - (FOLD ? 0 : 1)) * 32;
            float uu[kColBatch], vv[kColBatch];
            load_batch(n, base, 0, uu, vv);
            between();
            lds_barrier();          // every wave is done reading the previous run's column terms
            store_batch(n, base, 0, uu, vv);
            for (int k0 = kColBatch * kBlockK; k0 < n; k0 += kColBatch * kBlockK) {
                float u2[kColBatch], v2[kColBatch];
                load_batch(n, base, k0, u2, v2);
                store_batch(n, base, k0, u2, v2);
            }
            lds_barrier();          // the run's column terms are in LDS for every wave
            cbase = t0 - (FOLD ? 0 : 1);
        };
        T yA[NC][kPieces], yB[NC][kPieces];
        // A tile's pieces lie in 1 KB units (one per K chunk and piece). The loads address them from a scalar base
        // plus the lane's offset; each group of four units is one 4 KB immediate-offset range, and the groups
        // after the first take scalar bases of their own, b0 + g ystep (ystep opaque to the compiler, which would
        // otherwise form a 64-bit vector address for them: four more VALU instructions per tile).
        size_t ystep = 4 * 64;                          // opaque once, so that the pointer stays a global one
        if constexpr (NC * kPieces > 4) asm volatile("" : "+s"(ystep));
        auto load_y_chunk = [&](int t, T (&yv)[NC][kPieces], int cc) {
            const T* b0 = yt + (size_t)t * TILE16;
#pragma unroll
            for (int p = 0; p < kPieces; ++p) {
                const int k = cc * kPieces + p;
                yv[cc][p] = (b0 + (k / 4) * ystep)[(k % 4) * 64 + lane];
            }
        };
        auto load_y = [&](int t, T (&yv)[NC][kPieces]) {
#pragma unroll
            for (int cc = 0; cc < NC; ++cc) load_y_chunk(t, yv, cc);
        };
        auto colp_of = [&](int t) { return lds_col + (t - cbase) * 32 + 4 * h; };
        // With FOLD, the A operand of tile t's column MFMA (lane l: column l % 32; lanes 32-63 meet zeros in B)
        // and the B operand (column_ones): the MFMA adds the pieces of column_operand, whose sum is q.
        auto colA_of = [&](int t) { return reinterpret_cast<const bf16x8*>(lds_col)[(t - cbase) * 32 + (lane & 31)]; };
        const bf16x8 colB = column_ones(h);

        f32x16 accA[RB], accB[RB];
        Online<RB, L2, FOLD> on;
        auto tile = [&](f32x16 (&accN)[RB], f32x16 (&accP)[RB], const float* colp, T (&yv)[NC][kPieces], int t,
                        bool epi) {
            auto col4 = [&](int q) { return *reinterpret_cast<const f32x4*>(colp + 8 * q); };
            bf16x8 colA;
            if constexpr (FOLD) colA = colA_of(t);
            const int tn = t + 1 < te ? t + 1 : te - 1;     // RING: the tile whose chunks replace this one's
#pragma unroll
            for (int b = 0; b < RB; ++b) accN[b] = f32x16{};
            static_for<0, NS>([&](auto I) {
                constexpr int i = decltype(I)::value;
                constexpr int cc = i / (kProducts * RB), p = (i / RB) % kProducts, b = i % RB;
                constexpr int rp = ROLE == 0 ? C::first[p] : C::second[p];
                constexpr int cp = ROLE == 0 ? C::second[p] : C::first[p];
                accN[b] = C::mfma(yv[cc][cp], xv[b][cc][rp], accN[b]);
                if (epi) {
                    constexpr int k0 = op_begin<RB, FOLD>(i, NS), k1 = op_begin<RB, FOLD>(i + 1, NS);
                    static_for<k0, k1>([&](auto K) { on.template step<decltype(K)::value>(accP, col4, M, S, c); });
                }
                if constexpr (RING && p == kProducts - 1 && b == RB - 1) load_y_chunk(tn, yv, cc);
                __builtin_amdgcn_sched_barrier(0);
            });
            // The column terms last, after the whole dot product: x.y is formed identically in both directions.
            if constexpr (FOLD) {
#pragma unroll
                for (int b = 0; b < RB; ++b)
                    accN[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(colA, colB, accN[b], 0, 0, 0);
            }
        };
        auto update = [&](f32x16 (&accP)[RB], const float* colp) {
            auto col4 = [&](int q) { return *reinterpret_cast<const f32x4*>(colp + 8 * q); };
            static_for<0, RB * kOps>([&](auto K) { on.template step<decltype(K)::value>(accP, col4, M, S, c); });
        };

        // Tiles in pairs so the accumulator and operand buffers alternate without copies; the operand load of
        // the tile after the last is the last tile again (in bounds, unused).
        const int last = te - 1;
        // The first two operand tiles are requested right behind the first batch of column terms, so that the
        // latencies of the row operands, the column terms and the operands overlap.
        int cend = tb + kColTiles < te ? tb + kColTiles : te;
        int t = tb;
        stage_cols(tb, cend, [&] {
            load_y(t, yA);
            if constexpr (!RING) load_y(t + 1 < te ? t + 1 : last, yB);
        });
        tile(accA, accB, nullptr, yA, t, false);
        ++t;
        if constexpr (RING) {
            // the same loop with the one ring of operands, its next tile loaded inside tile()
            while (t < te) {
                if (__builtin_expect(t >= cend, 0)) {
                    cend = t + kColTiles < te ? t + kColTiles : te;
                    stage_cols(t, cend, [] {});
                }
                tile(accB, accA, colp_of(t - 1), yA, t, true);
                ++t;
                if (__builtin_expect(t >= te, 0)) {
                    update(accB, colp_of(t - 1));
                    goto done;
                }
                if (__builtin_expect(t >= cend, 0)) {
                    cend = t + kColTiles < te ? t + kColTiles : te;
                    stage_cols(t, cend, [] {});
                }
                tile(accA, accB, colp_of(t - 1), yA, t, true);
                ++t;
            }
            update(accA, colp_of(t - 1));
            goto done;
        }
        // The restaging of the column terms (once per kColTiles tiles) and the segment's end are the unlikely
        // branches: laid out of line, so that consecutive tiles fall through with no taken branch between them
        // (with one wave per SIMD a taken branch costs the wave about 25 cycles in which nothing issues).
        while (t < te) {
            if (__builtin_expect(t >= cend, 0)) {
                cend = t + kColTiles < te ? t + kColTiles : te;
                stage_cols(t, cend, [] {});
            }
            load_y(t + 1 < te ? t + 1 : last, yA);
            tile(accB, accA, colp_of(t - 1), yB, t, true);
            ++t;
            if (__builtin_expect(t >= te, 0)) {
                update(accB, colp_of(t - 1));
                goto done;
            }
            if (__builtin_expect(t >= cend, 0)) {
                cend = t + kColTiles < te ? t + kColTiles : te;
                stage_cols(t, cend, [] {});
            }
            load_y(t + 1 < te ? t + 1 : last, yB);
            tile(accA, accB, colp_of(t - 1), yA, t, true);
            ++t;
        }
        update(accA, colp_of(t - 1));
    done:
        store_rows<RB, L2>(a, M, S, rb0, slot, c, inv_sigma, lane);
    }
};

// The kernel's argument block, read where it is used. The merge's and the loop step's fields (epilogue
// vectors, loop configuration) are read through this reference, so that the compiler loads them there and not
// at the kernel's entry, where they would crowd the scalar registers the tile loop needs (spilled and reloaded
// one dependent load at a time).
__device__ __forceinline__ const PartialArgs& kernel_args() {
    return *(const PartialArgs*)__builtin_amdgcn_kernarg_segment_ptr();   // address-space conversion
}

// After a work segment of row group g (every wave has stored its rows of the slot, as device-scope atomic
// stores): count the workgroup's arrival; the last of the group's workgroups merges the group's slots and runs
// the loop step (sk_epilogue.h), so that no merge launch follows. Before the count every wave waits for its
// stores to complete (they are then visible device-wide: sc1 stores are write-through), and the barrier makes
// thread 0's atomic add follow all of them; the last arrival reads the slots with device-scope loads, which
// miss the XCD's L2. No fence: a device-scope one would write back and invalidate the L2 under the operand
// tiles the other workgroups of the XCD are streaming.
template <bool KARG>
__device__ inline void arrive(const PartialArgs& a, const PartialArgs* kp, int g) {
    __shared__ int s_last;
    // The merge's own argument fields (epilogue vectors, loop state and configuration), requested here in one
    // batch through a pointer to the argument block (kp) the compiler cannot follow out of this function, so that
    // they arrive while the stores and the counter make their round trips; the fields the segments use come from
    // `a`, already held. KARG: kp is the kernel argument segment (an empty asm hides it); otherwise an argument
    // block in device memory (the grouped kernel), hidden by taking its two halves through readfirstlane, which
    // the compiler keeps in scalar registers where the asm's register constraint could not.
    if constexpr (KARG) {
        asm volatile("" : "+s"(kp));
    } else {
        const unsigned long long v = (unsigned long long)(uintptr_t)kp;
        const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)v);
        const unsigned hi = __builtin_amdgcn_readfirstlane((unsigned)(v >> 32));
        kp = (const PartialArgs*)(uintptr_t)(((unsigned long long)hi << 32) | lo);
    }
    PartialArgs m = a;
    m.xsq = kp->xsq;
    m.off = kp->off;
    m.out = kp->out;
    m.out2 = kp->out2;
    m.n_store = kp->n_store;
    m.meas = kp->meas;
    m.w = kp->w;
    m.n_real = kp->n_real;
    m.counters = kp->counters;
    m.ngroups = kp->ngroups;
    m.tick = kp->tick;
    m.state = kp->state;
    m.rebake = kp->rebake;
    m.rows_role = kp->rows_role;
    m.contraction = kp->contraction;
    m.cfg.n_sched = kp->cfg.n_sched;
    m.cfg.n_stages = kp->cfg.n_stages;
    m.cfg.max_iters = kp->cfg.max_iters;
    m.cfg.check_every = kp->cfg.check_every;
    m.cfg.fixed_iters = kp->cfg.fixed_iters;
    asm volatile("" ::"s"(m.xsq), "s"(m.off), "s"(m.out), "s"(m.out2), "s"(m.n_store), "s"(m.meas), "s"(m.w),
                 "s"(m.n_real), "s"(m.counters), "s"(m.ngroups), "s"(m.tick), "s"(m.state), "s"(m.rebake),
                 "s"(m.rows_role), "s"(m.contraction), "s"(m.cfg.n_sched), "s"(m.cfg.n_stages),
                 "s"(m.cfg.max_iters), "s"(m.cfg.check_every), "s"(m.cfg.fixed_iters));
    // (the rest of the loop configuration, read only by the control itself, comes from the argument block)
    m.cfg.sched = kp->cfg.sched;
    m.cfg.stages = kp->cfg.stages;
    m.cfg.eps = kp->cfg.eps;
    m.cfg.rho_x = kp->cfg.rho_x;
    m.cfg.rho_y = kp->cfg.rho_y;
    m.cfg.tol = kp->cfg.tol;
    m.cfg.stage_tol = kp->cfg.stage_tol;
    m.cfg.stage_max_iters = kp->cfg.stage_max_iters;
    m.cfg.balanced = kp->cfg.balanced;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid_x() == 0) {
        const int nslots = last_wg(g, a.s) - first_wg(g, a.s) + 1;
        s_last = coh_add(a.group_counters + g, 1) == nslots - 1 ? 1 : 0;
    }
    __syncthreads();
    if (s_last == 0) return;
    if (tid_x() == 0) coh_store(a.group_counters + g, 0);
    // The loop's counters as this launch found them: the control runs only after every group is merged, this
    // one included, so nothing has changed them yet.
    const LoopCounters lc = loop_counters(m);
    if (m.state != nullptr && !needs_control(lc.it, lc.stage, lc.stage_it, m.cfg)) m.meas = nullptr;   // no check
    if (merge_group<true, kBlockK>(m, g)) loop_step<true, kBlockK>(m, g, lc, m.counters);
    __syncthreads();   // the next segment's column staging reuses LDS the merge does not touch; keep waves together
}

// The work segments of workgroup p: a_ij = x_i . y_j + cs (alpha cu_j + (beta + beta_lo) cv_j) in the kernel's
// units (the column term rounded once, then scaled by a power of two), scores exp2(c (a - M)) (with L2:
// exp2(fma(a, c, -c M)), a in log2 units times the copy's unit t = 1 / c).
template <int NC, int ROLE, int CT, bool L2, bool KARG>
__device__ __forceinline__ void segments(const PartialArgs& a, const PartialArgs* kp, int p, int wv, const float* cu,
                                         const float* cv, float alpha, float beta, float beta_lo, float cs, float c,
                                         float inv_sigma, typename Contract<CT>::T* lds_y, float* lds_col) {
    // The segment bounds are 32-bit integer arithmetic (the divisions expand to vector code); their results are
    // the same in every lane, and readfirstlane hands them to the scalar unit, so the tile loop's counters and
    // operand addresses stay in scalar registers.
    const int u1 = __builtin_amdgcn_readfirstlane(unit_at(cost_start(p + 1, a.s), a.s));
    for (int u = __builtin_amdgcn_readfirstlane(unit_at(cost_start(p, a.s), a.s)); u < u1;) {
        const int g = __builtin_amdgcn_readfirstlane(div_by(u, a.s.dnt));
        const int tb = u - g * a.s.nt;
        const int te = u1 - u < a.s.nt - tb ? tb + (u1 - u) : a.s.nt;
        const int slot = __builtin_amdgcn_readfirstlane(p - first_wg(g, a.s));
        // Waves past the last row block recompute it (their rows are not stored) so that every wave takes part
        // in the workgroup's barriers.
        const int rb0 = (g * kWavesK + wv) * kRowBlocksK;
        if constexpr (streamed_form(NC, CT))
            Streamed<NC, ROLE, CT, L2>::run(a, rb0, tb, te, slot, cu, cv, alpha, beta, beta_lo, cs, c, inv_sigma,
                                            lds_col);
        else
            Staged<NC, ROLE, CT, L2>::run(a, rb0, tb, te, slot, cu, cv, alpha, beta, beta_lo, cs, c, inv_sigma, lds_y,
                                          lds_col);
        if (a.group_counters != nullptr) arrive<KARG>(a, kp, g);
        // The segment's stores complete here, as an s_waitcnt the compiler sees (vmcnt(0); expcnt and lgkmcnt
        // unrestricted, gfx9 encoding): otherwise the loop's back edge carries the slot stores, whose address and
        // data registers the next prologue reuses, and the compiler's wait for them there (its counts cannot
        // tell a store from a load) also held back every operand load of the first segment's prologue.
        __builtin_amdgcn_s_waitcnt(0x0F70);
        u += te - tb;
    }
}

// Workgroup p of one pass with arguments a (kp: the same argument block, from which the merge inside the kernel
// reads its own fields late; KARG: the kernel argument segment).
template <int NC, int ROLE, int CT, bool KARG>
__device__ __forceinline__ void partial_pass(const PartialArgs& a, const PartialArgs* kp, int p) {
    // Every scalar this launch needs (the loop's done flag, the eps scalars, both clouds' scales, the first
    // cloud's log2-copy tag) is requested at once, and the done flag tested after: one memory round trip before
    // the work starts.
    const int* skip_p = a.skip != nullptr ? a.skip : &kNoSkip;
    const float* h1 = reinterpret_cast<const float*>(ROLE == 0 ? a.xr : a.yc);   // the first cloud's header
    const float sc0 = a.sc[0], sc2 = a.sc[2];                         // a.sc is valid in both modes
    const float sx = packed_scale(a.xr), sy = packed_scale(a.yc);   // 1 for kBF16x3
    const float cb = h1[2], cb_s2 = h1[3], cb_t = h1[4];
    const int skip = *skip_p;
    // The argument fields the segments need, requested with the first batch of argument loads rather than
    // after the scalars have arrived.
    asm volatile("" ::"s"(a.nrb), "s"(a.rows_pad), "s"(a.mode), "s"(a.s.nt), "s"(a.s.P), "s"(a.s.alpha),
                 "s"(a.s.ftot), "s"(a.s.q), "s"(a.s.r), "s"(a.group_counters), "s"(a.s.dP.m), "s"(a.s.dP.k),
                 "s"(a.s.dspan.m), "s"(a.s.dspan.k), "s"(a.s.dnt.m), "s"(a.s.dnt.k), "s"(a.s.dftot.m),
                 "s"(a.s.dftot.k), "s"(a.u), "s"(a.v), "s"(a.u2), "s"(a.v2), "s"(a.part));
    asm volatile("" ::"s"(sc0), "s"(sc2), "s"(sx), "s"(sy), "s"(cb), "s"(cb_s2), "s"(cb_t), "v"(skip));
    if (skip != 0) return;
    constexpr bool kStream = streamed_form(NC, CT);
    constexpr int kLdsY = kStream ? 1 : 3 * NC * Contract<CT>::pieces * 64;     // staged: three tile buffers
    constexpr int kLdsCol = kStream ? col_floats(CT == kF16x2) : 4 * 32;        // staged: four column buffers
    __shared__ typename Contract<CT>::T lds_y[kLdsY];
    __shared__ __attribute__((aligned(16))) float lds_col[kLdsCol];
    const int wv = __builtin_amdgcn_readfirstlane(tid_x() >> 6);   // one value per wave

    // a_ij = x_i . y_j + alpha u_j + beta v_j in accumulator units, scores exp2(c (a - M)):
    // half-step: a = x . y + (gh + eps log b) / 2, c = (2 / eps) log2(e); plain row-LSE: a = xa . ya + mask,
    // c = log2(e).
    float alpha, beta, c;
    if (a.mode == kHalfStep) {
        alpha = 0.5f;
        beta = 0.5f * sc2;
        c = sc0 * kLog2e;
    } else {
        alpha = 1.0f;
        beta = 0.0f;
        c = kLog2e;
    }
    // With a valid log2-unit copy of the first cloud for this c (log2_ready), the matrix cores produce t c x.y
    // (t, the copy's unit, a power of two; 1 for the usual score scales) and the exponentials take the scores
    // with the exact rescaling by 1 / t fused into the max subtraction. The column term
    // t c (gh / 2 + eps log b / 2) then comes, in the on-device loop (u2), from the column cloud's potential in
    // log2 units plus the low part of its log2 weights, u2 = (c / 2) gh + Ll, and the high part Lh: t (Lh + u2),
    // one rounding, where Lh + Ll = log2(e) log b - L0 carries the log weights to double precision relative to
    // the cloud's integer offset L0 (header word 5; the merge adds it back); otherwise from gh, scaled by t c.
    // Otherwise the kernel works in units scaled by sigma = s_rows s_cols (a power of two): column terms times
    // sigma, c divided by it.
    if constexpr (CT == kF16x2) {
        if (a.mode == kHalfStep && cb != 0.0f && cb == c && cb_s2 == (ROLE == 0 ? sy : sx)) {
            const float it = 1.0f / cb_t;                  // exact
            // The usual unit t = 1 gets its own inlined copy: with c = 1 a constant, each exponential's argument is
            // the two-operand a - m (v_sub_f32) instead of the three-operand fma.
            if (a.u2 != nullptr && cb_t == 1.0f)
                segments<NC, ROLE, CT, true, KARG>(a, kp, p, wv, a.u2, a.v2, 1.0f, 1.0f, 0.0f, 1.0f, 1.0f, 1.0f, lds_y, lds_col);
            else if (a.u2 != nullptr)
                segments<NC, ROLE, CT, true, KARG>(a, kp, p, wv, a.u2, a.v2, 1.0f, 1.0f, 0.0f, cb_t, it, it, lds_y, lds_col);
            else
                segments<NC, ROLE, CT, true, KARG>(a, kp, p, wv, a.u, a.v, alpha, beta, 0.0f, c * cb_t, it, it, lds_y, lds_col);
            return;
        }
    }
    const float sigma = sx * sy, inv_sigma = (1.0f / sx) * (1.0f / sy);
    segments<NC, ROLE, CT, false, KARG>(a, kp, p, wv, a.u, a.v, alpha, beta, 0.0f, sigma, c * inv_sigma, inv_sigma, lds_y,
                                  lds_col);
}

template <int NC, int ROLE, int CT>
__global__ __launch_bounds__(kBlockK) __attribute__((amdgpu_waves_per_eu(kWavesPerSimd, kWavesPerSimd)))
void lse_partial_kernel(PartialArgs a) {
    partial_pass<NC, ROLE, CT, true>(a, &kernel_args(), xcd_contiguous(wg_x(), a.s.P));
}

// The grouped form (sk_loop_run_batch_f32): the passes of several independent loops in one launch, each on its
// own share of the workgroups. Workgroup b runs workgroup p of pass k, map[b] = k << 16 | p, with pass k's
// arguments args[k] in device memory; a workgroup past the map or naming no pass of this kp returns at once.
template <int NC, int ROLE>
__global__ __launch_bounds__(kBlockK) __attribute__((amdgpu_waves_per_eu(kWavesPerSimd, kWavesPerSimd)))
void lse_partial_grouped_kernel(const PartialArgs* __restrict__ args, const unsigned* __restrict__ map, int count,
                                int nmap) {
    const int b = wg_x();
    if (b >= nmap) return;
    const unsigned e = __builtin_amdgcn_readfirstlane(map[b]);    // uniform: one entry per workgroup
    const int k = (int)(e >> 16), p = (int)(e & 0xffffu);
    if (k >= count) return;
    // Through the constant address space, as the kernel argument segment is read: scalar loads, the fields in
    // scalar registers as the pass expects them (the block does not change during the launch).
    using ConstArgs = const __attribute__((address_space(4))) PartialArgs;
    const PartialArgs* ap = (const PartialArgs*)((ConstArgs*)args + k);
    if (ap->nc != NC || p >= ap->s.P) return;
    partial_pass<NC, ROLE, kF16x2, false>(*ap, ap, p);
}

template <int NC>
hipError_t launch_nc(const PartialArgs& a, hipStream_t st) {
    if (a.contraction == kBF16x3) {
        if (a.rows_role != 0) return hipErrorInvalidValue;
        hipLaunchKernelGGL((lse_partial_kernel<NC, 0, kBF16x3>), dim3(a.s.P), dim3(kBlockK), 0, st, a);
    } else if (a.rows_role == 0) {
        hipLaunchKernelGGL((lse_partial_kernel<NC, 0, kF16x2>), dim3(a.s.P), dim3(kBlockK), 0, st, a);
    } else {
        hipLaunchKernelGGL((lse_partial_kernel<NC, 1, kF16x2>), dim3(a.s.P), dim3(kBlockK), 0, st, a);
    }
    return hipGetLastError();
}

template <int NC>
hipError_t launch_grouped_nc(const PartialArgs* args, const unsigned* map, int count, int nmap, int role,
                             hipStream_t st) {
    if (role == 0)
        hipLaunchKernelGGL((lse_partial_grouped_kernel<NC, 0>), dim3(nmap), dim3(kBlockK), 0, st, args, map, count, nmap);
    else
        hipLaunchKernelGGL((lse_partial_grouped_kernel<NC, 1>), dim3(nmap), dim3(kBlockK), 0, st, args, map, count, nmap);
    return hipGetLastError();
}

}  // namespace

#if SK_PARTIAL_LARGE
hipError_t launch_grouped_large(const PartialArgs* args, const unsigned* map, int count, int nmap, int nc, int role,
                                hipStream_t st) {
    switch (nc) {
        case 5: return launch_grouped_nc<5>(args, map, count, nmap, role, st);
        case 6: return launch_grouped_nc<6>(args, map, count, nmap, role, st);
        case 7: return launch_grouped_nc<7>(args, map, count, nmap, role, st);
        case 8: return launch_grouped_nc<8>(args, map, count, nmap, role, st);
        default: return hipErrorInvalidValue;
    }
}
hipError_t launch_partial_large(const PartialArgs& a, int nc, hipStream_t st) {
    switch (nc) {
        case 5: return launch_nc<5>(a, st);
        case 6: return launch_nc<6>(a, st);
        case 7: return launch_nc<7>(a, st);
        case 8: return launch_nc<8>(a, st);
        default: return hipErrorInvalidValue;
    }
}
#else
hipError_t launch_grouped_small(const PartialArgs* args, const unsigned* map, int count, int nmap, int nc, int role,
                                hipStream_t st) {
    switch (nc) {
        case 1: return launch_grouped_nc<1>(args, map, count, nmap, role, st);
        case 2: return launch_grouped_nc<2>(args, map, count, nmap, role, st);
        case 3: return launch_grouped_nc<3>(args, map, count, nmap, role, st);
        case 4: return launch_grouped_nc<4>(args, map, count, nmap, role, st);
        default: return hipErrorInvalidValue;
    }
}
hipError_t launch_partial_small(const PartialArgs& a, int nc, hipStream_t st) {
    switch (nc) {
        case 1: return launch_nc<1>(a, st);
        case 2: return launch_nc<2>(a, st);
        case 3: return launch_nc<3>(a, st);
        case 4: return launch_nc<4>(a, st);
        default: return hipErrorInvalidValue;
    }
}
#endif

}  // namespace sk
