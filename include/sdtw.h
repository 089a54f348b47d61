/*
 * sdtw.h -- C ABI of the MI355X (gfx950) Soft-DTW engine.
 *
 * The engine replaces the device-side operator boundary of BGU-CS-VIL/sdtw-cuda-torch:
 * the six functions of softdtw_cuda/cuda/launcher.py that the autograd Functions call,
 * plus the torch-op distance of softdtw_cuda/distances.py.  Every entry point below names
 * the reference interface it stands in for.
 *
 * Conventions
 *   - All tensor arguments are raw device pointers to contiguous row-major fp32 data.
 *   - Shapes are int64: B pairs, N rows of x, M rows of y, K features.
 *   - gamma > 0 and finite.  bandwidth <= 0 disables the Sakoe-Chiba band (the reference
 *     maps None / <= 0 to -1.0, autograd.py:19-23); a positive band skips cells with
 *     |i - j| > bandwidth exactly as the reference CPU path does (launcher.py:315,345).
 *   - stream is a hipStream_t (torch's current stream); NULL is the null stream.  Every
 *     call only enqueues work: nothing synchronises the device, nothing allocates or
 *     frees device memory.  Scratch memory comes from the caller as `ws`/`ws_bytes`
 *     (size it with sdtw_workspace_bytes).
 *   - The return value is an sdtw_status; sdtw_strerror() describes it.
 *   - R (the forward table kept for the backward) is engine-internal: sdtw_table_elems()
 *     fp32 values in a band-skewed layout (64-row bands, one anti-diagonal step per 64
 *     contiguous floats).  Its cells are the reference's R[b,i+1,j+1] (launcher.py:177)
 *     rounded once from an fp64 recursion; out-of-band cells hold +inf.  Convert with
 *     sdtw_table_unpack_f32 / sdtw_table_pack_f32.
 *   - Re-entrant.  The only state: the process-wide settings (sdtw_set_numerics,
 *     sdtw_set_wait_limit, sdtw_set_deterministic), the no-allocation entry point's static
 *     scratch, and a once-only device-attribute query.
 */
#ifndef SDTW_H_
#define SDTW_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum sdtw_status {
    SDTW_OK = 0,
    SDTW_ERR_INVALID_VALUE = 1,  /* bad shape, gamma, pointer */
    SDTW_ERR_WORKSPACE = 2,      /* ws too small (see sdtw_workspace_bytes) */
    SDTW_ERR_LAUNCH = 3,         /* hipLaunchKernel / runtime error */
    SDTW_ERR_UNSUPPORTED = 4,    /* shape outside what the kernels support */
    SDTW_ERR_TIMEOUT = 5,        /* a bounded inter-band wait expired (results invalid) */
    SDTW_ERR_SCRATCH_LIMIT = 6   /* shape exceeds the no-allocation entry point's scratch */
} sdtw_status;

/* Operation selectors for sdtw_workspace_bytes. */
typedef enum sdtw_op {
    SDTW_OP_SQEUCLID_FWD = 0,
    SDTW_OP_SQEUCLID_BWD = 1,
    SDTW_OP_FWD = 2,
    SDTW_OP_BWD = 3,
    SDTW_OP_FUSED_FWD = 4,
    SDTW_OP_FUSED_BWD = 5
} sdtw_op;

/* Distance modes for sdtw_sqeuclid_fwd_f32 (one mode). */
typedef enum sdtw_dist_mode {
    /* Same fp32 bits as the reference's torch-CPU distance (distances.py:20-28) on an x86
     * host: row norms in ATen's 8-lane cascade order, x.y^T as a sequential FMA chain over
     * k (plain multiply-then-add when K*N*M < 400, ATen's small-matrix kernel).  For
     * K <= 64 the chain runs on the matrix cores: v_mfma_f32_16x16x4_f32 chained over k from
     * a zero accumulator gives the sequential chain's bits, so no faster inexact mode is
     * offered. */
    SDTW_DIST_EXACT = 0
} sdtw_dist_mode;

/* Cell arithmetic of the Soft-DTW recursions (sdtw_set_numerics). */
typedef enum sdtw_numerics {
    /* fp64 recursion state; the soft-min's correction term and the backward's transition
     * weights use the hardware fp32 exp2 / log2.  R is within ~1 fp32 ulp of the reference
     * CPU path's (forward rtol 1e-5 holds); gradients are as close to an fp64 evaluation
     * as the reference's own fp32 path is, but not within rtol 1e-4 of that path where R
     * differences cancel (E depends on R[succ] - R[i,j] - D[succ]). */
    SDTW_NUMERICS_FAST = 0,
    /* The reference CPU arithmetic (launcher.py:307-353) restated with fp64-accurate
     * exp / log in both recursions: R matches the CPU path bit for bit in every tested case
     * and E to within rare last-bit differences. */
    SDTW_NUMERICS_EXACT = 1,
    /* The default.  Forward as EXACT (R bit-identical to the CPU path's); the backward
     * takes the CPU path's own fp32 differences R[succ] - R[i,j] - D[succ] and evaluates
     * their transition weights with the hardware fp32 exp2, so E is within ~1e-6 relative
     * of the CPU path's and gradients meet rtol 1e-4 / atol 1e-5 against it. */
    SDTW_NUMERICS_MIXED = 2
} sdtw_numerics;

const char *sdtw_strerror(int status);
int sdtw_version(void);

/* Select the cell arithmetic of every later forward / backward launch in this process;
 * returns the previous mode, or -1 (nothing changed) for an unknown mode.  The default is
 * SDTW_NUMERICS_MIXED.  No counterpart in the reference (its CPU path is EXACT, its CUDA
 * kernels fp32). */
int sdtw_set_numerics(int mode);
int sdtw_get_numerics(void);

/* Diagnostic (synchronises the device): SDTW_ERR_TIMEOUT if the last wavefront launch of
 * `op` that used workspace `ws` hit its bounded inter-band wait, else SDTW_OK.  The kernels
 * never hang: a wait that expires raises this flag, the wave stops, and the pair's results
 * are marked invalid without any synchronisation -- out[p] = NaN (forward), NaN over the
 * band's rows of G or E (backward), and so NaN gradients through the distance backward; in
 * the fused backward's gradient mode, NaN over the band's rows of dL/dx and all of the
 * pair's dL/dy.
 * No counterpart in the reference (whose kernels have no inter-block waits). */
int sdtw_debug_status(int op, const void *ws, size_t ws_bytes, int64_t B, int64_t N, int64_t M,
                      int64_t K);

/* Polls a wavefront kernel's bounded wait makes before it gives up, for every later launch in
 * this process; returns the previous value.  The default, 2^22, is about 0.3 s without
 * progress.  A test hook: a tiny limit makes the waits that would have to poll give up at
 * once (every kernel still exits normally), so the give-up path can be exercised.  No
 * counterpart in the reference. */
unsigned sdtw_set_wait_limit(unsigned polls);

/* Bytes of the distance record sdtw_fused_fwd_d_f32 can write for sdtw_sqeuclid_bwd_f32
 * (per-pair clamp flags and row norms; device memory the caller owns). */
size_t sdtw_dist_record_bytes(int64_t B, int64_t N, int64_t M);

/* Process-wide: 1 makes sdtw_fused_bwd_f32 give run-to-run identical bits by taking its
 * E path (g*E in the workspace, reduced by the distance backward); 0 (the default) lets it
 * form the gradients inside the recursion kernel, whose dL/dy adds the bands' shares with
 * atomics in arrival order (last-bit differences between runs).  Takes effect for calls
 * (and sdtw_workspace_bytes queries) made after it.  Returns the previous setting.  No
 * counterpart in the reference; the torch layer sets it from
 * torch.are_deterministic_algorithms_enabled(). */
int sdtw_set_deterministic(int on);

/* Bands per workgroup the fused forward recursions (sdtw_fused_fwd_f32, sdtw_fused_fwd_d_f32)
 * take for an unbanded call at this shape on the current device under the current
 * arithmetic: 1 when the batch's one-band workgroups all fit on the GPU at once and the
 * arithmetic is mixed (the scaled linear-domain recursion, whose compute, producer,
 * helper and converter waves then have a SIMD each), else 2 when the 2-band workgroups all
 * fit (their matrix-core producer waves have SIMDs of their own), else 4; 0 for an invalid
 * shape.  (A banded call takes 2 where this is 1.)  The choice the launcher makes, exported
 * so a caller can choose between sdtw_fused_fwd_d_f32 and the two-call unfused forward.
 * (The fused backward, sdtw_fused_bwd_f32 and sdtw_fused_bwd_e_f32, takes 1 where the
 * batch's one-band workgroups all fit, else 2 or 4 as here.)  No counterpart in the
 * reference. */
int sdtw_fused_bands_per_workgroup(int64_t B, int64_t N, int64_t M, int64_t K);

/* Number of floats of the R table for B pairs of N x M cells. */
int64_t sdtw_table_elems(int64_t B, int64_t N, int64_t M);

/* R table -> dense (B, N, M) row-major, and back.  No counterpart in the reference, whose
 * R is already dense (launcher.py:177); these exist for inspection and tests. */
int sdtw_table_unpack_f32(const float *Rt, float *R, int64_t B, int64_t N, int64_t M,
                          void *stream);
int sdtw_table_pack_f32(const float *R, float *Rt, int64_t B, int64_t N, int64_t M,
                        void *stream);

/* Bytes of caller-provided scratch that `op` needs at this shape on the current device (0 if
 * none): the fused recursions' workgroup geometry, and with it their scratch, follows the
 * device's CU count.  A launch on a device that needs more reports SDTW_ERR_WORKSPACE. */
size_t sdtw_workspace_bytes(int op, int64_t B, int64_t N, int64_t M, int64_t K);

/* D[b,i,j] = max(0, (|x_bi|^2 + |y_bj|^2) - 2 x_bi . y_bj)  -> D (B,N,M).
 * Replaces softdtw_cuda/distances.py:6-28 (sqeuclidean / pairwise_distance). */
int sdtw_sqeuclid_fwd_f32(const float *x, const float *y, float *D, int64_t B, int64_t N,
                          int64_t M, int64_t K, int mode, void *ws, size_t ws_bytes,
                          void *stream);

/* Gradient of the distance above given G = dL/dD (B,N,M):
 *   G' = G where (x2 + y2 - 2xy) >= 0 else 0            (clamp_min backward)
 *   gx = 2 (x * rowsum(G') - G' y),  gy = 2 (y * colsum(G') - G'^T x)
 * D is the clamped forward output (used to find clamped cells).  mask = 0 skips the clamp
 * mask (the fused-mode chain rule of autograd_xy.py:45-49 has none).  record: NULL, or the
 * distance record sdtw_fused_fwd_d_f32 wrote with this D: the pairs it records as free of
 * clamped cells have the identity mask and their D is not read, and its row norms serve the
 * exact check of the others (no norms launch here).  gx or gy may be NULL: that gradient is
 * not formed (autograd's needs_input_grad); both NULL is a no-op.  Both gradients with no
 * mask, or with a record, take one launch for the two reductions.
 * Replaces the torch autograd backward of distances.py:20-28 (bmm/sum/clamp_min
 * backward) and, with mask = 0, autograd_xy.py:41-49. */
int sdtw_sqeuclid_bwd_f32(const float *x, const float *y, const float *D, const void *record,
                          const float *G, float *gx, float *gy, int64_t B, int64_t N, int64_t M,
                          int64_t K, int mask, void *ws, size_t ws_bytes, void *stream);

/* Soft-DTW forward over a materialised cost D (B,N,M): R table and out[b] = R[b,N-1,M-1].
 * Replaces softdtw_cuda/cuda/launcher.py:167-223 (softdtw_forward_cuda) with the
 * numerics of the reference CPU path launcher.py:307-324 (fp64 recursion, fp32 R). */
int sdtw_fwd_f32(const float *D, float *R, float *out, int64_t B, int64_t N, int64_t M,
                 double gamma, double bandwidth, void *ws, size_t ws_bytes, void *stream);

/* sdtw_fwd_f32 without a workspace argument and without any allocation.  No counterpart in
 * the reference: it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Its scratch (the
 * workgroup ticket, the error flag and the cross-workgroup rows) is a static device array
 * of sdtw_fwd_f32_noalloc_scratch_limit() bytes (16 MiB) per GPU, held until the process
 * ends; the first call on a device looks up that device's copy.  A shape whose scratch
 * (sdtw_workspace_bytes(SDTW_OP_FWD, B, N, M, 0)) exceeds the limit returns
 * SDTW_ERR_SCRATCH_LIMIT before any device call.  Each call resets the scratch in a kernel
 * launched ahead of the recursion (no memset node), so earlier contents never matter; but
 * every call on one GPU uses the same array, so calls that overlap on one GPU (different
 * streams, or threads) race and give wrong results: serialise them.  Results are bit-for-bit
 * those of sdtw_fwd_f32. */
int sdtw_fwd_f32_noalloc(const float *D, float *R, float *out, int64_t B, int64_t N, int64_t M,
                         double gamma, double bandwidth, void *stream);
size_t sdtw_fwd_f32_noalloc_scratch_limit(void);

/* Soft-DTW backward: G[b,i,j] = gout[b] * E[b,i,j], E = d out[b] / d D[b,i,j].
 * gout may be NULL (treated as 1, i.e. G = E, what launcher.py returns).  Its workspace
 * (sdtw_workspace_bytes(SDTW_OP_BWD, ...)) depends on the device's compute-unit count: it
 * holds one cross-workgroup row per band where the batch's one-band workgroups all fit.
 * Replaces softdtw_cuda/cuda/launcher.py:226-300 (softdtw_backward_cuda_log) together
 * with the `g * E` of autograd.py:46-47, with the numerics of launcher.py:327-353. */
int sdtw_bwd_f32(const float *D, const float *R, const float *gout, float *G, int64_t B,
                 int64_t N, int64_t M, double gamma, double bandwidth, void *ws,
                 size_t ws_bytes, void *stream);

/* Fused forward: cost recomputed per cell from x (B,N,K), y (B,M,K) with the same bits as
 * sdtw_sqeuclid_fwd_f32(EXACT); no (B,N,M) cost tensor exists.
 * Replaces softdtw_cuda/cuda/launcher.py:33-87 (softdtw_forward_cuda_fused_sqeuclid). */
int sdtw_fused_fwd_f32(const float *x, const float *y, float *R, float *out, int64_t B,
                       int64_t N, int64_t M, int64_t K, double gamma, double bandwidth,
                       void *ws, size_t ws_bytes, void *stream);

/* Unfused mode's forward in one launch: the fused forward whose matrix-core producer waves
 * also store every cost tile into D (B,N,M), with the bits sdtw_sqeuclid_fwd_f32(EXACT)
 * writes.  Replaces distances.py:6-28 followed by launcher.py:167-223 (the cost tensor,
 * then the recursion over it).  Workspace as SDTW_OP_FUSED_FWD.  SDTW_ERR_UNSUPPORTED
 * where the costs take scalar tiles (K > 64, or K*N*M < 400): use the two calls there.
 * record: NULL, or a distance record of sdtw_dist_record_bytes(B, N, M) bytes for
 * sdtw_sqeuclid_bwd_f32: per pair, whether a cost is not positive (0 or NaN), and the row
 * norms of x and y (no counterpart in the reference: it lets the distance backward skip
 * reading D and its norms launch). */
int sdtw_fused_fwd_d_f32(const float *x, const float *y, float *D, void *record, float *R,
                         float *out, int64_t B, int64_t N, int64_t M, int64_t K, double gamma,
                         double bandwidth, void *ws, size_t ws_bytes, void *stream);

/* Fused backward: E recomputed with per-cell costs from x, y, then
 *   gx = 2 (x * rowsum(gE) - gE y),  gy = 2 (y * colsum(gE) - gE^T x),  gE = gout[b] * E.
 * gout may be NULL (treated as 1).  gx or gy may be NULL: that gradient is not formed; both
 * NULL is a no-op.  With matrix-core cost tiles (K <= 64, K*N*M >= 400) in workgroups of at
 * most 2 bands, or 4 when K <= 16, the recursion kernel forms gx and gy from E tile by tile
 * and nothing of size (B,N,M) exists; gy then adds the bands' shares with atomics in
 * arrival order (see sdtw_set_deterministic).  Otherwise, and under the deterministic
 * setting, E lives in the workspace and the distance backward reduces it.
 * sdtw_workspace_bytes(SDTW_OP_FUSED_BWD, ...) sizes the path taken.
 * Replaces softdtw_cuda/cuda/launcher.py:90-162 (softdtw_backward_cuda_fused_sqeuclid)
 * together with the chain rule of autograd_xy.py:32-51. */
int sdtw_fused_bwd_f32(const float *x, const float *y, const float *R, const float *gout,
                       float *gx, float *gy, int64_t B, int64_t N, int64_t M, int64_t K,
                       double gamma, double bandwidth, void *ws, size_t ws_bytes,
                       void *stream);

/* Fused backward, E only: E (B,N,M) = d out / d D with per-cell costs from x, y.
 * Replaces softdtw_cuda/cuda/launcher.py:90-162 exactly (it returns E). */
int sdtw_fused_bwd_e_f32(const float *x, const float *y, const float *R, const float *gout,
                         float *E, int64_t B, int64_t N, int64_t M, int64_t K, double gamma,
                         double bandwidth, void *ws, size_t ws_bytes, void *stream);

/* ---- barycenter ----------------------------------------------------------------------------
 * softdtw_barycenter (barycenters.py:17-180) with its loop on the device: per iteration the
 * fused forward of the barycenter (N, K) broadcast to every pair against X (B, N, K), the
 * fused backward with upstream gradient w (so no gradient of X is formed), then one update
 * kernel: the gradient summed over pairs, clipped to norm 1 (clip_grad_norm_), torch's Adam
 * step (betas 0.9 / 0.999, eps 1e-8) with learning rate lrs[it] (the caller passes the
 * schedule's values, e.g. torch's CosineAnnealingLR), and the weighted loss sum_b w_b out_b of
 * the iterate before the step.  w are the normalised weights (device, B); bary holds the
 * initial barycenter and receives the result; losses (device, max_iter, or NULL) receives
 * the loss of each iteration run; *iters_run the number of iterations run.
 * early_stopping != 0 applies the reference's rule (stop once `patience` iterations in a row
 * improved the loss by no more than tol, after max_iter / 2): each iteration then copies its
 * loss to the host and synchronises the stream -- the only entry point besides
 * sdtw_debug_status that synchronises.  Workspace: sdtw_barycenter_workspace_bytes. */
size_t sdtw_barycenter_workspace_bytes(int64_t B, int64_t N, int64_t K, int max_iter);
int sdtw_barycenter_f32(const float *X, const float *w, float *bary, float *losses, int64_t B,
                        int64_t N, int64_t K, double gamma, int max_iter, const double *lrs,
                        int early_stopping, int patience, double tol, int *iters_run, void *ws,
                        size_t ws_bytes, void *stream);

/* ---- float64 path ------------------------------------------------------------------------
 * The reference keeps the caller's dtype: float64 inputs give a float64 cost
 * (distances.py:20-25) and float64 recursions (launcher.py:307-368, numba on float64 arrays),
 * which torch.autograd.gradcheck needs (test_softdtw_small.py:29-37).  These entry points
 * compute in double throughout.  R is the reference's dense (B, N+2, M+2) table
 * (launcher.py:177, :310).  No workspace; one workgroup per pair sweeps its anti-diagonals,
 * with no waits between workgroups.  B <= 65535. */

/* Doubles of the float64 R table: B * (N+2) * (M+2). */
int64_t sdtw_table_elems_f64(int64_t B, int64_t N, int64_t M);

/* As sdtw_sqeuclid_fwd_f32, in double.  Replaces distances.py:6-28 for float64 inputs. */
int sdtw_sqeuclid_fwd_f64(const double *x, const double *y, double *D, int64_t B, int64_t N,
                          int64_t M, int64_t K, void *stream);

/* As sdtw_sqeuclid_bwd_f32, in double (mask = 1: clamp_min mask from D; 0: none, the fused
 * chain rule).  Replaces the autograd backward of distances.py:20-28 and, with mask = 0,
 * autograd_xy.py:41-49, for float64 inputs. */
int sdtw_sqeuclid_bwd_f64(const double *x, const double *y, const double *D, const double *G,
                          double *gx, double *gy, int64_t B, int64_t N, int64_t M, int64_t K,
                          int mask, void *stream);

/* Forward over a float64 cost: R (B, N+2, M+2) and out[b] = R[b, N, M].  Replaces
 * launcher.py:167-223 / :356-361 for float64 inputs (the arithmetic of launcher.py:307-324). */
int sdtw_fwd_f64(const double *D, double *R, double *out, int64_t B, int64_t N, int64_t M,
                 double gamma, double bandwidth, void *stream);

/* Backward: G[b,i,j] = gout[b] * E[b,i,j] (gout NULL: G = E), R as sdtw_fwd_f64 wrote it
 * (read only).  Replaces launcher.py:226-300 / :364-368 with autograd.py:46-47 for float64
 * inputs (the arithmetic of launcher.py:327-353). */
int sdtw_bwd_f64(const double *D, const double *R, const double *gout, double *G, int64_t B,
                 int64_t N, int64_t M, double gamma, double bandwidth, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* SDTW_H_ */
