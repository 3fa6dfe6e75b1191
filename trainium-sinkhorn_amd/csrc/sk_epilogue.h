// Device code of the merge pass: the merge of a row group's partial (max, sum) slots with the half-step
// epilogue, and the on-device loop control (src/trnopt/sinkhorn.py:346-378), which runs after the last row
// group of a g update is merged. Two hosts for it: the merge kernel (sk_kernels.hip), a launch of its own after
// the partial kernel; or, in the on-device loop, the partial kernel itself, whose last workgroup to finish a
// row group merges it ("coherent" below). The coherent form passes data between workgroups only through
// device-scope relaxed atomic loads and stores (global_load / global_store with sc1: coherent across the XCDs'
// L2 caches without writing back or invalidating them; device-scope fences would invalidate each XCD's L2 under
// the tiles the other workgroups are still streaming), ordered by the workgroup barrier's wait for the
// workgroup's stores before the arrival counter's atomic add.
#pragma once

#include "sk_common.h"

namespace sk {

constexpr float kDeltaCap = 50.0f;     // cap of (g_old - g_new) / eps in the balanced check (sinkhorn.py:60)
constexpr int kMergeBatch = 16;                      // partial slots a merging thread loads at once (their latencies overlap)
constexpr double kLog2eD = 1.4426950408889634074;   // log2(e) in double
constexpr double kLn2D = 0.69314718055994530942;     // ln(2) in double

__device__ __forceinline__ float ep_ex2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float ep_lg2(float x) { return __builtin_amdgcn_logf(x); }

// log2 S of a row's merged sum of exponentials (S >= 1: the row's largest term is exactly 1), as an exact
// integer part e plus log2 m: the caller adds them in double. The hardware log2 (v_log_f32) truncates instead of
// rounding: on gfx950 its mean error is -0.47 ulp of the result, i.e. about -2e-7 for S near 2^6 and -9e-7 near
// 2^20. Applied to S directly, that biases every half-step's log-sum-exp low by eps ln2 times as much,
// differently in the f and g updates (their rows' S differ), which offsets the cost of a balanced problem (1.6e-8
// of it on the 10k x 10k d 64 mixture clouds at eps 0.05). The exponent is split off exactly and the hardware
// log2 takes only the mantissa, centred on 1, so its error is at most one ulp of a number below 1/2 (2^-25).
struct Log2Split {
    int e;
    float lm;        // log2 m, m in [sqrt(1/2), sqrt(2))
};
__device__ __forceinline__ Log2Split lse_log2(float S) {
    int e;
    float m = frexpf(S, &e);                   // S = m 2^e, m in [1/2, 1)
    if (m < 0.70710678f) {
        m *= 2.0f;                              // exact
        e -= 1;
    }
    return {e, ep_lg2(m)};
}

// Device-scope relaxed atomic accesses (coherent between workgroups on different XCDs within a launch).
__device__ __forceinline__ float2 coh_load(const float2* p) {
    const unsigned long long b =
        __hip_atomic_load(reinterpret_cast<const unsigned long long*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return make_float2(__uint_as_float((unsigned)b), __uint_as_float((unsigned)(b >> 32)));
}
__device__ __forceinline__ void coh_store(float2* p, float2 v) {
    const unsigned long long b =
        (unsigned long long)__float_as_uint(v.x) | ((unsigned long long)__float_as_uint(v.y) << 32);
    __hip_atomic_store(reinterpret_cast<unsigned long long*>(p), b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float coh_load(const float* p) {
    return __uint_as_float(
        __hip_atomic_load(reinterpret_cast<const unsigned*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}
__device__ __forceinline__ void coh_store(float* p, float v) {
    __hip_atomic_store(reinterpret_cast<unsigned*>(p), __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int coh_load(const int* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void coh_store(int* p, int v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int coh_add(int* p, int v) {
    return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <bool COH, class T>
__device__ __forceinline__ T ld(const T* p) {
    if constexpr (COH) return coh_load(p); else return *p;
}
template <bool COH, class T>
__device__ __forceinline__ void st(T* p, T v) {
    if constexpr (COH) coh_store(p, v); else *p = v;
}

// The first cloud's log2-unit copy for score scale c = (2 / eps) log2(e) = sc[0] log2(e), against the second
// cloud's scale s2: every coordinate x, as the cloud's own pieces hold it (x = (v0 + v1) / s1, exact), becomes
// w = t fl(c x) / s2 in two fp16 pieces (w0 = fp16(w), w1 = fp16(w - w0)), with t a power of two, the copy's
// unit. Products with the second cloud's own pieces (s2 y) then sum to t c x.y in fp32: the score in log2 units
// times t, so that the exponentials need no more than an exact power-of-two rescaling, fused with the max
// subtraction (exp2(t^-1 a - t^-1 m), one fma); the f and g updates both use this copy, in the same product
// order, and stay bit-identical. t = 1 while max |fl(c x)| / s2 lies in [2^-1, 2^15) (within fp16's range and
// with w1 normal for the largest coordinates); outside that window t brings max |w| into [2^4, 2^5), as the
// packing scale does for the clouds' own pieces. The copy is valid (header c_b = c, [3] = s2, [4] = t) for
// every c > 0 and every cloud whose max |w| reaches that range with t in [2^-40, 2^40]; otherwise c_b = 0 and
// the half-steps scale on the VALU.
struct BakeParams {
    float c, inv_s1, inv_s2, t;
    bool valid;
};

__device__ inline BakeParams bake_params(const void* first, const void* second, const float* sc) {
    const float* h1 = reinterpret_cast<const float*>(first);
    BakeParams b;
    b.c = sc[0] * kLog2e;                                   // as the half-step kernels form it
    const float s1 = h1[1], s2 = packed_scale(second);
    b.inv_s1 = 1.0f / s1;                                   // powers of two: exact
    b.inv_s2 = 1.0f / s2;
    const float wmax = (b.c * __uint_as_float(reinterpret_cast<const unsigned*>(first)[0])) * b.inv_s2;
    b.t = 1.0f;
    if (wmax > 0.0f && (wmax < 0.5f || wmax >= 32768.0f)) {
        int e;
        frexpf(wmax, &e);                                   // wmax in [2^(e-1), 2^e)
        const int k = 5 - e;
        b.t = ldexpf(1.0f, k < -40 ? -40 : (k > 40 ? 40 : k));
    }
    const float tw = wmax * b.t;                            // exact
    b.valid = b.c > 0.0f && tw >= 0.5f && tw < 32768.0f;
    return b;
}

// One 16-byte unit (8 coordinates of one tile row half, one K chunk) of the copy.
__device__ inline void bake_unit(char* first, long long idx, int npad, int nc, const BakeParams& b) {
    const f16x8* own = reinterpret_cast<const f16x8*>(first + kHeaderBytes);
    f16x8* cp = reinterpret_cast<f16x8*>(first + kHeaderBytes) + (size_t)(npad / SK_TILE) * nc * 2 * 64;
    const int lane = (int)(idx % 64);
    const long long tc = idx / 64;                          // tile * nc + chunk
    const f16x8 p0 = own[tc * 128 + lane], p1 = own[tc * 128 + 64 + lane];
    f16x8 q0, q1;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float x = ((float)p0[e] + (float)p1[e]) * b.inv_s1;
        const float w = ((b.c * x) * b.inv_s2) * b.t;     // one rounding (c x), then exact scalings
        const _Float16 a0 = (_Float16)w;
        q0[e] = a0;
        q1[e] = (_Float16)(w - (float)a0);
    }
    cp[tc * 128 + lane] = q0;
    cp[tc * 128 + 64 + lane] = q1;
}

__device__ inline void bake_header(char* first, const void* second, const BakeParams& b) {
    float* h = reinterpret_cast<float*>(first);
    h[2] = b.valid ? b.c : 0.0f;
    h[3] = packed_scale(second);
    h[4] = b.valid ? b.t : 1.0f;
}

// The on-device loop's log2 weights. In log2 units a column term is R_j + log2(e) log w_j (R_j = (c / 2) gh_j,
// the column cloud's potential). The loop carries each cloud's log2 weights as a double-float relative to an
// integer offset, log2(e) log w_j - L0 = Lh_j + Ll_j (made at loop init from the caller's log weights and their
// low parts, log_w + log_w_lo = log w to double precision; L0 = rint(log2(e) max log w) in header word 5), keeps
// Ll inside the stored potential (u2 = fl(R + Ll)) and stages the column term as t fl(Lh + u2): one rounding at
// the magnitude of the term relative to the largest weight. The merge adds L0 back to each row's maximum in
// double. Why the precision: at an eps far above the cost scale every half-step's log-sum-exp is nearly the
// weights' own log-sum-exp, and a balanced iteration moves its potentials along the neutral mode (f + s, g - s)
// by eps times the log of the two marginals' effective total masses' ratio each iteration. Log weights rounded
// to float32 change those masses by a few 1e-8 (relative), so at eps ten times the typical cost the potentials
// drifted by 1e-6 of their size per iteration (3.6e-4 per iteration at eps 9,746 on a 144 x 435 d 126 raw
// cloud pair, against none for the float64 run). The reference's float32 op sequence has the same mismatch but
// no drift: its float32 log of each row's sum, nearly the same number for every row at such an eps, rounds the
// same way in every row, which makes its iteration flat along the neutral mode. With the log weights carried to
// double precision the masses match, and the term's one rounding, relative to the largest weight, is at most
// half an ulp of a few log2 units.
__device__ __forceinline__ float loop_weight_offset(const void* pk) { return reinterpret_cast<const float*>(pk)[5]; }

// eps of the iteration that starts with `it` iterations done (sinkhorn.py:347-350).
__device__ inline double eps_for(const LoopCfg& c, int it, int stage) {
    if (c.n_stages > 0) return stage < c.n_stages ? c.stages[stage] : c.eps;
    return it < c.n_sched ? c.sched[it] : c.eps;
}

// The scalars of one eps, computed in double and rounded once, as consts() does (sinkhorn.py:323-334).
__device__ inline void set_scalars(sk_state* st, double e, double rho_x, double rho_y) {
    const double kx = rho_x > 0.0 ? rho_x / (rho_x + e) : 1.0;
    const double ky = rho_y > 0.0 ? rho_y / (rho_y + e) : 1.0;
    st->eps = e;
    st->sc_x[0] = (float)(2.0 / e);
    st->sc_x[1] = (float)(1.0 / e);
    st->sc_x[2] = (float)e;
    st->sc_x[3] = (float)kx;
    st->sc_y[0] = (float)(2.0 / e);
    st->sc_y[1] = (float)(1.0 / e);
    st->sc_y[2] = (float)e;
    st->sc_y[3] = (float)ky;
}

// Merge the slots of row i = 256 g + t (thread t of the workgroup, one row per thread) and apply the epilogue:
//     lse = (2 / eps) M + ln S  (half-step, accumulator units) or M + ln S  (plain row-LSE)
// When the partial kernel took its scores in log2 units (log2_ready, tested on the same header words), the
// slots hold M in log2 units: they merge without c, and M / c (correctly rounded, so that no constant factor
// enters the potentials) gives the accumulator units.
//     fh  = kappa ((|x|^2 + eps off) - eps lse) - |x|^2
// With meas, also the group's convergence partials {max_{i<n_real} |new - old|, sum_i |w (exp(min((old -
// new) / eps, 50)) - 1)|} (sinkhorn.py:360, 368-373), reduced in a fixed order into meas[g] (in the on-device
// loop only when the iteration's control will run: the callers drop meas otherwise).
// Returns false, storing nothing, when the loop is done (*skip != 0): the flag is loaded with the launch's other
// scalars and the row's first slots, and tested once they have arrived. COH: the slots were written in this
// launch by other workgroups, and the results (out, out2, meas) are read back in it (the loop control). NT: the
// workgroup's threads (kRowsPerGroup or more: threads past the group's rows take part in its barriers only).
template <bool COH, int NT>
__device__ inline bool merge_group(const PartialArgs& a, int g) {
    static_assert(NT >= kRowsPerGroup && NT % 64 == 0, "one thread per row of the group");
    const bool live = tid_x() < kRowsPerGroup;
    const int i = g * kRowsPerGroup + tid_x();
    const int* skip_p = a.skip != nullptr ? a.skip : &kNoSkip;
    const float sc0 = a.sc[0], sc1 = a.sc[1], sc2 = a.sc[2], sc3 = a.sc[3];   // valid in both modes
    const float* h1 = reinterpret_cast<const float*>(a.rows_role == 0 ? a.xr : a.yc);   // the first cloud
    const float* h2 = reinterpret_cast<const float*>(a.rows_role == 0 ? a.yc : a.xr);
    const float cb = h1[2], cb_s2 = h1[3], s2 = h2[1], cb_t = h1[4];
    const float L0 = loop_weight_offset(a.yc);                     // the column cloud's log2 weight offset (loop)
    const int ic = i < a.rows_pad ? i : a.rows_pad - 1;
    const float x2 = a.mode == kHalfStep ? a.xsq[ic] : 0.0f;
    const float o = a.off != nullptr ? a.off[ic] : 0.0f;
    const float old = a.meas != nullptr ? a.out[ic] : 0.0f;
    const float wi = a.meas != nullptr ? a.w[ic] : 0.0f;
    const float ll = a.rows_l2lo != nullptr ? a.rows_l2lo[ic] : 0.0f;   // the row's Ll (kept in its log2 potential)
    // The first kMergeBatch slots of the row (all there are up to that many workgroups per row group) come with
    // the scalars.
    const int p0 = first_wg(g, a.s), p1 = last_wg(g, a.s);
    const float2* pp = a.part + ic;
    float2 v0[kMergeBatch];
#pragma unroll
    for (int k = 0; k < kMergeBatch; ++k) v0[k] = p0 + k <= p1 ? ld<COH>(pp + (size_t)k * a.rows_pad) : make_float2(kEmpty, 0.0f);
    const int skip = *skip_p;
    asm volatile("" ::"s"(sc0), "s"(sc1), "s"(sc2), "s"(sc3), "s"(cb), "s"(cb_s2), "s"(s2), "s"(cb_t), "s"(L0),
                 "v"(x2), "v"(o), "v"(old), "v"(wi), "v"(ll), "v"(skip));
    if (skip != 0) return false;
    const float c_hs = sc0 * kLog2e;
    // log2_ready, on the header words loaded above
    const bool l2 = a.mode == kHalfStep && a.contraction == kF16x2 && cb != 0.0f && cb == c_hs && cb_s2 == s2;
    const float c = l2 ? 1.0f : a.mode == kHalfStep ? c_hs : kLog2e;
    float dmax = 0.0f;
    double derr = 0.0;
    if (live && i < a.rows_pad) {
        // One pass, online: (M, S) <- (max(M, m_k), S 2^(c (M - M')) + s_k 2^(c (m_k - M'))), slots loaded
        // kMergeBatch at a time so that their latencies overlap.
        float M = kEmpty, S = 0.0f;
        for (int q = p0; q <= p1; q += kMergeBatch) {
            float2 v[kMergeBatch];
#pragma unroll
            for (int k = 0; k < kMergeBatch; ++k)
                v[k] = q == p0 ? v0[k]
                               : q + k <= p1 ? ld<COH>(pp + (size_t)(q + k - p0) * a.rows_pad) : make_float2(kEmpty, 0.0f);
            float Mn = M;
#pragma unroll
            for (int k = 0; k < kMergeBatch; ++k) Mn = fmaxf(Mn, v[k].x);
            float Sn = S * ep_ex2(c * (M - Mn));
#pragma unroll
            for (int k = 0; k < kMergeBatch; ++k) Sn += v[k].y * ep_ex2(c * (v[k].x - Mn));
            M = Mn;
            S = Sn;
        }
        // the row maximum in the stored units (the slots store M / t with t = cb_t), with the loop's log2 weight
        // offset of the columns back on (loop_weight_offset)
        const double Md = (double)M + (l2 && a.u2 != nullptr ? (double)L0 : 0.0);
        // The row's log-sum-exp and the epilogue in double, rounded once: f may be far smaller than the max score
        // and the log of the sum it is the difference of (clouds far from unit scale under normalize=False), so
        // each float rounding of those would cost f relative precision.
        const Log2Split ls = lse_log2(S);
        const double l2s = (double)ls.e + (double)ls.lm;
        if (a.mode == kHalfStep) {
            const double kappa = sc3, x2d = x2, od = o;
            float val;
            // fh = kappa (|x|^2 + eps off - eps lse) - |x|^2 (src/trnopt/sinkhorn.py:119) is evaluated as
            //     fh = kappa (eps off - eps lse) + (kappa - 1) |x|^2,
            // the same number in the mathematics (kappa - 1 is exact), rounded at fh's own magnitude. Rounded the
            // reference's way, the state fh = f - |x|^2 is carried on the grid of f (|x|^2 - eps lse rounded at
            // |x|^2's magnitude, then |x|^2 subtracted exactly): a coarser quantisation that, iterated, pushes
            // the balanced potentials along their neutral mode (f + t, g - t) by a fraction of f's ulp per
            // iteration (2e-8 on the 10k x 10k d 64 mixture clouds at eps 0.05, whose f is near 0.4; the
            // reference's float32 sequence drifts the same way, less), which shows as a floor of the balanced
            // error (4.5e-7 there) and an offset of the cost. For kappa = 1 and no offset it is -eps lse, exact.
            if (l2 && a.out2 != nullptr) {
                // In log2 units, R = (c / 2) fh (the loop's state): (c / 2) eps lse = M + log2 S exactly in the
                // mathematics, so R = kappa (O - (M + log2 S)) + (kappa - 1) X2 with X2 = (c / 2) |x|^2 and
                // O = log2(e) off, and fh = R / (c / 2), each rounded once from the double; the state stored for
                // the other half-step's column terms is R + Ll (loop_weight_offset).
                const double k2 = 0.5 * (double)c_hs;
                const double R = kappa * (od * (double)kLog2eD - (Md + l2s)) + (kappa - 1.0) * (x2d * k2);
                val = (float)(R / k2);
                if (i < a.n_store) st<COH>(a.out2 + i, (float)(R + (double)ll));
            } else {
                // eps lse = 2 M + eps ln(S) in accumulator units (log2-unit slots: M / c), with the caller's eps
                // (float) as the reference's epilogue multiplies by it (src/trnopt/sinkhorn.py:119)
                const double eps_lse = 2.0 * (l2 ? Md / (double)c_hs : Md) + (double)sc2 * kLn2D * l2s;
                val = (float)(kappa * ((double)sc2 * od - eps_lse) + (kappa - 1.0) * x2d);
            }
            if (a.meas != nullptr) {
                if (i < a.n_real) dmax = fabsf(val - old);
                const float delta = fminf((old - val) * sc1, kDeltaCap);
                derr = (double)fabsf(wi * (expf(delta) - 1.0f));
            }
            if (i < a.n_store) st<COH>(a.out + i, val);
        } else if (i < a.n_store) {
            // natural log: ln S = ln(2) log2 S. (The exponentials used c = kLog2e, log2(e) rounded to float32,
            // 1 - 9e-9 of it, so S sums e^((1 - 9e-9)(a - M)) and ln(2) log2 S errs by 9e-9 |E_p[a - M]|; dividing
            // log2 S by kLog2e instead would add 9e-9 ln S, one-sided.)
            st<COH>(a.out + i, (float)(Md + kLn2D * l2s));
        }
    }
    if (a.meas != nullptr) {
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            dmax = fmaxf(dmax, __shfl_xor(dmax, o));
            derr += __shfl_xor(derr, o);
        }
        __shared__ float smax[NT / 64];
        __shared__ double ssum[NT / 64];
        const int wv = tid_x() >> 6;
        if ((tid_x() & 63) == 0) {
            smax[wv] = dmax;
            ssum[wv] = derr;
        }
        __syncthreads();
        if (tid_x() == 0) {
            float mx = smax[0];
            double sm = ssum[0];
            for (int k = 1; k < NT / 64; ++k) {
                mx = fmaxf(mx, smax[k]);
                sm += ssum[k];
            }
            st<COH>(a.meas + g, make_float2(mx, (float)sm));
        }
    }
    return true;
}

// Whether the g update of an iteration must run the loop control, given (it, stage, stage_it) as the f update's
// merge left them (already counting this iteration): a check at the reference's cadence, the last iteration,
// or an eps-schedule step. Otherwise the control would only write the state it finds (sinkhorn.py:347-378).
__device__ inline bool needs_control(int it, int stage, int stage_it, const LoopCfg& c) {
    if (it >= c.max_iters) return true;
    if (c.n_stages > 0) {
        if (stage < c.n_stages) return stage_it % c.check_every == 0;
        return c.fixed_iters == 0 && stage_it % c.check_every == 0;
    }
    if (it <= c.n_sched) return true;                 // the next iteration's eps comes from the schedule
    return c.fixed_iters == 0 && stage_it % c.check_every == 0;
}

// After the g update of one iteration, by one wave: the body of sinkhorn.py:356-378. With (it, stage_it)
// already advanced by the f update's merge, runs the balanced / unbalanced check at the reference's cadence,
// advances the stage, sets `done`, and writes the next iteration's eps and {2/eps, 1/eps, eps, kappa}.
template <bool COH>
__device__ inline void control_step(sk_state* st, const float2* meas, int nmeas, const LoopCfg& c) {
    float mx = 0.0f;
    double sm = 0.0;
    for (int k = tid_x(); k < nmeas; k += 64) {
        const float2 v = ld<COH>(meas + k);
        mx = fmaxf(mx, v.x);
        sm += (double)v.y;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        mx = fmaxf(mx, __shfl_xor(mx, o));
        sm += __shfl_xor(sm, o);
    }
    if (tid_x() != 0) return;
    const float inv_eps = st->sc_x[1];          // 1/eps of the iteration that just ran
    const int it = st->it;
    int stage = st->stage;
    int stage_it = st->stage_it;
    int conv = 0;
    if (c.n_stages > 0 && stage < c.n_stages) {
        // An intermediate stage: advance once the potentials settle or after stage_max_iters.
        if (stage_it % c.check_every == 0) {
            const double ch = (double)(mx * inv_eps);
            if (ch < c.stage_tol || stage_it >= c.stage_max_iters) {
                stage += 1;
                stage_it = 0;
            }
        }
    } else {
        const bool check = c.fixed_iters == 0 && (c.n_stages > 0 || it > c.n_sched) &&
                           (stage_it % c.check_every == 0 || it == c.max_iters);
        if (check) {
            const double err = c.balanced != 0 ? sm : (double)(mx * inv_eps);
            st->err = err;
            st->checks += 1;
            if (err < c.tol) conv = 1;
        }
    }
    const int done = (conv != 0 || it >= c.max_iters) ? 1 : 0;
    st->stage = stage;
    st->stage_it = stage_it;
    st->converged = conv;
    if (done == 0) set_scalars(st, eps_for(c, it, stage), c.rho_x, c.rho_y);
    st->done = done;
}

// The loop's state counters as a g update sees them on entry (before any workgroup can reach the control).
struct LoopCounters {
    int it, stage, stage_it;
};
__device__ inline LoopCounters loop_counters(const PartialArgs& a) {
    LoopCounters k = {0, 0, 0};
    if (a.state != nullptr) {
        k.it = a.state->it;
        k.stage = a.state->stage;
        k.stage_it = a.state->stage_it;
    }
    return k;
}

// After row group g is merged (all threads of the workgroup; the group's results are stored): the f update
// counts the iteration (once, by group 0's merge); a g update whose counters call for the loop control runs it in
// the last workgroup to arrive (counter: zero on entry, left zero), which on a new eps also derives the log2-unit
// potentials again and remakes the first cloud's log2-unit copy for the next f update. COH as in merge_group:
// the other groups' results were stored in this launch by other workgroups. NT: the workgroup's threads.
template <bool COH, int NT>
__device__ inline void loop_step(const PartialArgs& a, int g, const LoopCounters& lc, int* counter) {
    if (a.tick != nullptr) {                   // the f update: count the iteration (nobody reads these meanwhile)
        if (g == 0 && tid_x() == 0) {
            a.tick->it += 1;
            a.tick->stage_it += 1;
        }
        return;
    }
    if (a.state == nullptr || !needs_control(lc.it, lc.stage, lc.stage_it, a.cfg)) return;
    __shared__ int s_last;
    if constexpr (!COH) __threadfence();   // release: this group's outputs and meas[g]
    __syncthreads();                       // (COH: every wave's stores have completed)
    if (tid_x() == 0) s_last = (COH ? coh_add(counter, 1) : atomicAdd(counter, 1)) == a.ngroups - 1 ? 1 : 0;
    __syncthreads();
    if (s_last == 0) return;
    if constexpr (!COH) __threadfence();   // acquire: every group's meas
    // The loop control, by the first wave; thread 0 keeps the scalars of the iteration that ran and hands the next
    // iteration's over through LDS.
    __shared__ float s_sc[4];
    __shared__ float s_sc0_ran;
    __shared__ int s_done;
    if (tid_x() == 0) s_sc0_ran = a.state->sc_x[0];
    if (tid_x() < 64) control_step<COH>(a.state, a.meas, a.ngroups, a.cfg);
    if (tid_x() == 0) {
        st<COH>(counter, 0);
        s_done = a.state->done;
        for (int k = 0; k < 4; ++k) s_sc[k] = a.state->sc_x[k];
    }
    if (a.rebake == nullptr) return;
    __syncthreads();
    if (s_done != 0 || s_sc[0] == s_sc0_ran) return;     // same eps next: the copy and the log2 states stand
    // A new eps (a schedule or a stage): the log2-unit potentials R = (c / 2) fh of both clouds again from the
    // accumulator-unit ones (stored as R + Ll, loop_weight_offset), and the first cloud's log2-unit copy for the
    // new score scale, so that the next f update already finds them. (This is the g update: rows y, columns x.)
    const double k2 = 0.5 * (double)(s_sc[0] * kLog2e);
    const int nx = a.s.nt * SK_TILE;
    for (int i = tid_x(); i < a.rows_pad; i += NT)
        a.out2[i] = (float)((double)ld<COH>(a.out + i) * k2 + (double)a.rows_l2lo[i]);
    for (int i = tid_x(); i < nx; i += NT) a.u2[i] = (float)((double)a.u[i] * k2 + (double)a.cols_l2lo[i]);
    const void* second = a.xr;
    const BakeParams b = bake_params(a.rebake, second, s_sc);
    const float* h = reinterpret_cast<const float*>(a.rebake);
    if (b.valid ? h[2] == b.c && h[3] == packed_scale(second) : h[2] == 0.0f) return;
    if (b.valid) {
        const long long total = (long long)(nx / SK_TILE) * a.nc * 64;
        for (long long idx = tid_x(); idx < total; idx += NT) bake_unit(a.rebake, idx, nx, a.nc, b);
    }
    __syncthreads();
    if (tid_x() == 0) bake_header(a.rebake, second, b);
}

}  // namespace sk
