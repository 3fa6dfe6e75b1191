/*
 * trnopt_hip.h -- C ABI of the fused log-domain Sinkhorn half-step for AMD Instinct MI355X (gfx950).
 *
 * The library (libtrnopt_hip.so) replaces the device side of the reference package `trnopt`:
 *   - the fused NKI kernels of src/trnopt/nki_sinkhorn.py (make_row_lse_kernel :150-172,
 *     make_half_step_kernel :175-228), and
 *   - the host loop of src/trnopt/sinkhorn.py:346-378 (eps schedule, stages, convergence checks),
 *     which here runs on the device with no per-iteration host synchronisation.
 *
 * Conventions
 *   - Every pointer named as "device" is a device pointer on the current HIP device; the library never
 *     allocates or frees device memory. Scratch space is passed in as `ws` with its size in bytes.
 *   - All work is enqueued on the caller's `stream` (a hipStream_t passed as void*, NULL = default
 *     stream) and is asynchronous.
 *   - Every entry point returns 0 on success, a negative SK_E* code for a rejected argument, or a
 *     positive hipError_t for a runtime failure. sk_last_error() describes the last failure on the
 *     calling thread. Nothing aborts the process.
 *   - Point clouds are "packed": a header holding the cloud's power-of-two scale s (max |coordinate| * s
 *     in [2^4, 2^5)), then the points padded to a multiple of SK_TILE and the coordinates to
 *     SK_KP_ALIGN, every scaled coordinate s x split into two fp16 pieces (within 2^-23 of s x), in the
 *     tile-interleaved order that the fp16 MFMA kernels read with one coalesced 16-byte load per lane
 *     (sk_pack_cloud_f32 builds it from a row-major (n, d) fp32 array; sk_packed_bytes gives its size).
 *     The kernels form x.y from three products of the pieces (x0 y0, x0 y1, x1 y0), accumulated in
 *     fp32: at least as accurate as an fp32 dot product, and bit-identical in the two directions of a pair of half-steps (rows_role 0
 *     and 1) over the same two clouds. Coordinates must satisfy max |x| <= 7e13; every coordinate is held
 *     within 2^-23 of the cloud's largest for max |x| >= 2^-36, and the precision degrades gracefully below.
 *     The first cloud of a pair may also carry a log2-unit copy of its pieces (sk_bake_log2_f32), with
 *     which the scores come out of the matrix cores already scaled by (2 / eps) log2(e).
 *   - Shifted potentials follow the reference (src/trnopt/sinkhorn.py:28-33): fh = f - |x|^2.
 */
#ifndef TRNOPT_HIP_H
#define TRNOPT_HIP_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SK_TILE 32            /* points per packed tile (one 32x32 MFMA output block) */
#define SK_KP_ALIGN 16        /* coordinates are padded to a multiple of this (one fp16 MFMA K chunk) */
#define SK_PACKED_BYTES_PER_COORD 8   /* two fp16 pieces per padded coordinate, twice: own scale, log2 copy */
#define SK_PACKED_HEADER_BYTES 256    /* before the tiles: max |coordinate|, the scale, the log2 copy's tag */
#define SK_KP_MAX 128         /* largest padded dimension the kernels are built for */
#define SK_PAD_LOG_WEIGHT (-1e9)  /* log weight of a padding point (src/trnopt/sinkhorn.py:59) */

#define SK_OK 0
#define SK_E_ARG (-1)         /* null pointer, negative size, misaligned buffer */
#define SK_E_SHAPE (-2)       /* dimension beyond SK_KP_MAX, size not a multiple of SK_TILE */
#define SK_E_WORKSPACE (-3)   /* ws too small: ask the matching *_workspace_bytes() */
#define SK_E_DEVICE (-4)      /* no usable gfx950 device */

/* Library version: major * 10000 + minor * 100 + patch. */
int sk_version(void);

/* Message of the last failure on the calling thread ("" if none). */
const char* sk_last_error(void);

/* Padded sizes used by every other entry point. */
int sk_pad_points(int n);      /* n rounded up to a multiple of SK_TILE */
int sk_pad_dim(int d);         /* d rounded up to a multiple of SK_KP_ALIGN */

/*
 * Pack a row-major cloud pts (n, d), leading dimension ld >= d (device, fp32), into the tile layout
 * out (sk_packed_bytes(n, d) bytes, device, 16-byte aligned): a header, then npad = sk_pad_points(n)
 * points of kp = sk_pad_dim(d) coordinates, two fp16 pieces each. Padding is zero. Three launches on
 * `stream` (header, max |coordinate|, pieces).
 * Replaces the per-block [x^T ; 1] copies of _Cloud (src/trnopt/sinkhorn.py:159-165); the augmented
 * "1" is not stored, the column term enters the accumulator instead.
 */
size_t sk_packed_bytes(int n, int d);
int sk_pack_cloud_f32(const float* pts, int n, int d, int ld, void* out, void* stream);

/*
 * The log2-unit copy of the first cloud of a pair (the x of a solve, rows_role 0), stored in the second
 * half of its packed buffer: every coordinate x as two fp16 pieces of fl(c x) / s2, c = sc[0] log2(e) =
 * (2 / eps) log2(e) for sc = {2/eps, ...} on the device, s2 the second cloud's scale. Half-steps over this
 * pair with the same sc[0] then read the scores in log2 units straight from the matrix cores (one VALU
 * multiply less per score, same accuracy, the two directions still bit-identical); with any other sc[0],
 * or a copy made against another second cloud, they scale on the VALU as before. The copy is not made
 * (and the pair keeps scaling on the VALU) when max |fl(c x)| / s2 falls outside [2^-1, 2^15). One launch.
 * sk_loop_init_f32 makes it for the loop's first eps and the loop remakes it when eps changes; a caller of
 * sk_half_step_f32 may make it once per eps. No counterpart in the reference (an fp32-MFMA-free way to
 * apply its 1/eps scaling, src/trnopt/nki_sinkhorn.py:197-210).
 */
int sk_bake_log2_f32(void* first_pk, const void* second_pk, int n_first, int d, const float* sc, void* stream);

/*
 * Row-wise log-sum-exp of a matrix product (the core of the fused kernel):
 *     lse[i] = log sum_j exp( xa[i, :] . ya[j, :] ),   i < rows, j < m,
 * xa (rows, K) and ya (m, K) row-major fp32 device arrays, lse (rows,) fp32 device.
 * Replaces make_row_lse_kernel(K, rows, m)(xa_T, ya_T) (src/trnopt/nki_sinkhorn.py:150-172); unlike
 * the NKI kernel there is no constraint on rows or m and K may be up to SK_KP_MAX.
 */
/* ws: sk_row_lse_workspace_bytes() bytes, 256-byte aligned. */
size_t sk_row_lse_workspace_bytes(int rows, int m, int K);
int sk_row_lse_f32(const float* xa, const float* ya, float* lse, int rows, int m, int K,
                   void* ws, size_t ws_bytes, void* stream);

/*
 * One fused half-step (the f update; the g update is the same call with the clouds swapped):
 *     fh[i] = kappa * (xsq[i] + eps * off[i] - eps * lse_i) - xsq[i],
 *     lse_i = LSE_j( (2 x_i . y_j + gh[j]) / eps + log_b[j] ),
 * for i < rows_pad, without materialising the scores. Replaces make_half_step_kernel(d, rows, m)
 * (src/trnopt/nki_sinkhorn.py:175-228) and the PyTorch _half_step (src/trnopt/sinkhorn.py:108-119).
 *   x_pk   packed rows, y_pk packed columns (sk_pack_cloud_f32 layout, d coordinates)
 *   xsq, off  (rows_pad,)  |x|^2 and log(target/reference); off may be NULL (= 0)
 *   gh, log_b (m_pad,)     the other side's shifted potential and log weights (padding: PAD_LOG_WEIGHT)
 *   rows_role  0 if the rows are the first cloud of the pair (the f update of a solve), 1 if they are the
 *          second (the g update): fixes the order of the piece products so that both directions form
 *          bit-identical x_i . y_j
 *   sc     device float[4] = {2/eps, 1/eps, eps, kappa}, as the NKI kernel's sc (nki_sinkhorn.py:180)
 *   skip   device int or NULL: when *skip != 0 the call does nothing (the on-device loop's "done")
 *   fh     (rows_pad,) output; must not alias gh
 *   meas   NULL, or per-call convergence partials: then the previous contents of fh are the old
 *          potential, and meas receives, per group of 256 rows, {max_{i<n_real} |fh_new - fh_old|,
 *          sum_i |w_i (exp(min((fh_old - fh_new)/eps, 50)) - 1)|} (src/trnopt/sinkhorn.py:360, 368-373);
 *          w (rows_pad,) the row weights (padding 0) is then required. sk_half_step_meas_count()
 *          gives the number of float2 entries written.
 *   ws     workspace of sk_half_step_workspace_bytes() bytes, 256-byte aligned
 * rows_pad and m_pad must be multiples of SK_TILE. Two launches on `stream`: the MFMA partial pass, then
 * the merge of the partial (max, sum) slots with the kappa / offset epilogue.
 */
size_t sk_half_step_workspace_bytes(int rows_pad, int m_pad, int d);
int sk_half_step_meas_count(int rows_pad);
int sk_half_step_f32(const void* x_pk, const float* xsq, const float* off, int rows_pad,
                     const void* y_pk, const float* gh, const float* log_b, int m_pad, int d,
                     int rows_role, const float* sc, const int* skip, float* fh,
                     float* meas, const float* w, int n_real,
                     void* ws, size_t ws_bytes, void* stream);

/*
 * sk_half_step_f32 without a workspace argument, for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). No counterpart in the reference.
 * The partial (max, sum) slots live in a static device array of SK_NOALLOC_SCRATCH_BYTES that the library
 * holds on every GPU it runs on until the process ends; the call itself allocates nothing. Same arguments,
 * results and launches as sk_half_step_f32 (bit-identical output); a shape whose
 * sk_half_step_workspace_bytes() exceeds SK_NOALLOC_SCRATCH_BYTES is rejected with SK_E_WORKSPACE before
 * anything is enqueued. Every call on one GPU shares that GPU's array: calls that overlap on one GPU
 * (several host threads, or several streams running at once) race and must be serialised by the caller.
 * The first call on each device looks the array's device address up (hipGetSymbolAddress) and keeps it: make
 * that first call outside any stream capture; later calls enqueue only the two kernel launches, which a
 * capture records as kernel nodes (no allocation, no memset).
 */
#define SK_NOALLOC_SCRATCH_BYTES ((size_t)16 << 20)
int sk_half_step_noalloc_f32(const void* x_pk, const float* xsq, const float* off, int rows_pad,
                             const void* y_pk, const float* gh, const float* log_b, int m_pad, int d,
                             int rows_role, const float* sc, const int* skip, float* fh,
                             float* meas, const float* w, int n_real, void* stream);

/*
 * On-device Sinkhorn loop: the body of src/trnopt/sinkhorn.py:346-378 (eps schedule or stages, f then
 * g update, stage advance, balanced / unbalanced checks every check_every iterations, fp32 floors).
 */
typedef struct sk_cloud_f32 {
    const void* pk;       /* packed points (sk_pack_cloud_f32 layout); the loop rewrites x's log2-unit copy and
                             writes the cloud's log2 weight offset rint(log2(e) max log_w) into header word 5 at
                             init */
    const float* sq;      /* |p|^2 (npad), float64 sums cast to fp32 (src/trnopt/sinkhorn.py:149) */
    const float* log_w;   /* log weights (npad), padding SK_PAD_LOG_WEIGHT */
    const float* w;       /* exp(log_w) (npad), padding 0 */
    const float* off;     /* log(target / reference) (npad) or NULL */
    int n;                /* real points */
    int npad;             /* sk_pad_points(n) */
    const float* log_w_lo; /* or NULL (zeros): the low part of the log weights, fp32(log w - log_w) from the
                             caller's float64 log w (padding 0). The loop carries log_w + log_w_lo, so that the two
                             marginals' total masses agree to float64 rounding: a balanced iteration at an eps far
                             above the cost scale moves its potentials by eps times their log ratio every
                             iteration, and log weights rounded to fp32 leave it at a few 1e-8. */
} sk_cloud_f32;

/* Loop state, device resident, written by the loop's own kernels (layout is part of the ABI). */
typedef struct sk_state {
    double eps;           /* eps of the next iteration */
    double err;           /* last convergence measure; NaN until a check has run */
    int it;               /* iterations done */
    int stage;            /* index into stages (n_stages = the final eps) */
    int stage_it;         /* iterations in the current stage */
    int done;             /* 1: converged or max_iters reached; later loop kernels do nothing */
    int converged;
    int checks;           /* convergence checks run */
    float sc_x[4];        /* {2/eps, 1/eps, eps, kappa_x} of the next iteration (f update) */
    float sc_y[4];        /* same with kappa_y (g update) */
} sk_state;

typedef struct sk_loop_f32 {
    sk_cloud_f32 x, y;
    int d;
    float* fh;            /* (x.npad) shifted f, written by the f update */
    float* gh;            /* (y.npad) shifted g, zero-initialised by the caller (g0 = |y|^2) */
    sk_state* state;      /* device */
    const double* sched;  /* device, n_sched eps values (eps_start schedule), or NULL */
    int n_sched;
    const double* stages; /* device, n_stages eps values (wot-style stages), or NULL */
    int n_stages;
    double eps;           /* final eps */
    double rho_x, rho_y;  /* <= 0: that side balanced (kappa = 1) */
    double tol;           /* already floored as the reference floors it */
    double stage_tol;     /* already floored */
    int max_iters, check_every, stage_max_iters;
    int fixed_iters;      /* 1: never check */
    int balanced;         /* 1: balanced error measure, 0: max potential change / eps */
    void* ws;
    size_t ws_bytes;
} sk_loop_f32;

size_t sk_loop_workspace_bytes(int nx_pad, int ny_pad, int d);
/* Write the initial state (it = 0, first eps and its scalars); make x's log2-unit copy for that eps
 * (sk_bake_log2_f32), both clouds' log2 weights (log2(e) log w less an integer offset, as two floats) and the
 * loop's log2-unit potentials (c / 2) fh, (c / 2) gh in ws from fh and gh. */
int sk_loop_init_f32(const sk_loop_f32* L, void* stream);
/* Enqueue `iters` iterations (f update, g update with the loop control in its merge: a partial-kernel launch
 * each, which merges its own row groups from 40 row groups (10k rows) up, and a merge-kernel launch after it
 * below that);
 * iterations after `done` do nothing. ws (sk_loop_workspace_bytes) must be 256-byte aligned. */
int sk_loop_run_f32(const sk_loop_f32* L, int iters, void* stream);

/*
 * Several loops at once: `count` independent solves of the same d (each set up and initialised as above, on its
 * own workspace), such as the consecutive pairs of a wot pipeline (examples/singlecell_wot.py:84-89, which runs
 * them one after another through sinkhorn(); this is the batched form of sk_loop_run_f32 for them). Each
 * iteration is two launches, the f updates of all the loops and then their g updates, each loop's pass split over
 * its own share of the GPU's workgroups (in proportion to its work) and merged inside the launch, with each loop's
 * control as in sk_loop_run_f32: small solves fill the GPU together. A loop's splits differ from its own launches'
 * (fewer workgroups), so its potentials agree with sk_loop_run_f32's to float32 rounding, not bit for bit; with
 * count 1 the splits, and the results, are the same. A loop whose `done` is set does nothing; the others go on.
 *
 * sk_loop_batch_plan: the workgroups each loop's f and g pass gets (workgroups[2k], workgroups[2k + 1]) for loops
 * of nx_pad[k] x ny_pad[k] points (host arithmetic only).
 * sk_loop_batch_init_f32: writes the launches' argument blocks for loops[0 .. count) into ws
 * (sk_loop_batch_workspace_bytes(count) bytes, 256-byte aligned) and returns in launch[3] what
 * sk_loop_run_batch_f32 needs; synchronises the stream. Call it again whenever the loops change.
 * sk_loop_run_batch_f32: enqueues `iters` iterations of the loops last initialised into ws.
 * No counterpart in the reference (its pipeline solves one pair at a time).
 */
size_t sk_loop_batch_workspace_bytes(int count);
int sk_loop_batch_plan(const int* nx_pad, const int* ny_pad, int count, int d, int* workgroups);
int sk_loop_batch_init_f32(const sk_loop_f32* const* loops, int count, void* ws, size_t ws_bytes, int* launch,
                           void* stream);
int sk_loop_run_batch_f32(const void* ws, size_t ws_bytes, int count, const int* launch, int iters, void* stream);

/*
 * Median of the squared-Euclidean cost over all pairs, the normalisation cost / median(cost) of
 * normalization(how="median") (src/trnopt/sinkhorn.py:229-233), which the reference evaluates on the host
 * over the materialised n x m float64 matrix:
 *     median over i < n, j < m of max((|xc_i|^2 + |yc_j|^2) - 2 xc_i . yc_j, 0)   (float64),
 * np.median's definition (mean of the two middle values when n m is even). xc (n, d), yc (m, d): row-major
 * float64 device arrays, already centred; out: one device double. Six radix-select passes over the cost
 * keys: the first three recompute every cost, the third keeping the keys that can still hold the answer
 * (up to 2^22 of them, 8 bytes each, in ws) for the last three. ws (sk_cost_median_workspace_bytes) also
 * holds zero-padded copies of xc and yc. n m < 2^32, d <= SK_MEDIAN_D_MAX; ws 256-byte aligned.
 */
#define SK_MEDIAN_D_MAX 128
size_t sk_cost_median_workspace_bytes(int n, int m, int d);
int sk_cost_median_f64(const double* xc, const double* yc, int n, int m, int d, double* out,
                       void* ws, size_t ws_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TRNOPT_HIP_H */
