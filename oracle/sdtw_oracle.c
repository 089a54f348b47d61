/*
 * sdtw_oracle.c -- TEST INFRASTRUCTURE ONLY (the parity checker, never the product).
 *
 * A plain-C restatement of the reference's CPU Soft-DTW loops, used by tests/, by
 * __graft_entry__.smoke() and by bench.py's cpu_baseline leg.  Nothing in the shipped
 * package (sdtw-cuda-torch_amd/) may link or call this file.
 *
 * What it restates (reference = BGU-CS-VIL/sdtw-cuda-torch):
 *   - softdtw_cuda/cuda/launcher.py:307-324  _softdtw_forward_cpu_np   (forward DP)
 *   - softdtw_cuda/cuda/launcher.py:327-353  _softdtw_backward_cpu_np  (backward, linear space)
 *
 * Arithmetic model (why the types below are what they are):
 *   - launcher.py:310 builds R as `np.ones(..., dtype=D.dtype) * np.inf`.  Under numba the
 *     scalar np.inf is typed float64 and numba's ufunc loop selection has no value-based
 *     casting, so an fp32 D yields an fp64 R: the whole forward recursion runs in double and
 *     the caller rounds R to the input dtype once (launcher.py:359, `.type_as(D)`).
 *   - The backward receives that rounded R (fp32 for fp32 inputs) and pads D/E in the input
 *     dtype (launcher.py:330-334).  `R[b,i+1,j] - R[b,i,j] - D[b,i+1,j]` is evaluated in the
 *     input dtype (numba: float32 op float32 -> float32), then divided by the Python-float
 *     gamma in double; exp() and the three-term sum are double, and each E cell is stored
 *     (rounded) in the input dtype (launcher.py:347-351).
 *   - numba does not contract a*b+c into fma and does not reassociate; this file is
 *     compiled with -ffp-contract=off and without -ffast-math for the same reason.
 *   - exp/log are the C library's (numba lowers np.exp/np.log on scalars to libm calls).
 *
 * Parallelism mirrors `prange(B)`: independent pairs are spread over OpenMP threads; the
 * per-pair loops are sequential (j outer, i inner) exactly as in the reference.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define IDX3(b, i, j, H, W) (((int64_t)(b) * (H) + (i)) * (W) + (j))

/* 0 < bandwidth < |i - j|  (launcher.py:315, :345) */
static inline int out_of_band(double bandwidth, int64_t i, int64_t j) {
    int64_t d = i - j;
    if (d < 0) d = -d;
    return (0.0 < bandwidth) && (bandwidth < (double)d);
}

/* Forward DP for one pair, padded fp64 R of shape (N+2, M+2).  launcher.py:310-323 */
#define DEFINE_FWD(NAME, TD)                                                              \
    static void NAME##_pair(const TD *D, double *R, int64_t N, int64_t M, double gamma,   \
                            double bandwidth) {                                           \
        const int64_t W = M + 2;                                                          \
        for (int64_t t = 0; t < (N + 2) * W; ++t) R[t] = INFINITY;                        \
        R[0] = 0.0;                                                                       \
        for (int64_t j = 1; j <= M; ++j) {                                                \
            for (int64_t i = 1; i <= N; ++i) {                                            \
                if (out_of_band(bandwidth, i, j)) continue;                               \
                double r0 = -R[(i - 1) * W + (j - 1)] / gamma;                            \
                double r1 = -R[(i - 1) * W + j] / gamma;                                  \
                double r2 = -R[i * W + (j - 1)] / gamma;                                  \
                /* Python/numba max(a, b): b if b > a else a */                           \
                double rmax = (r1 > r0) ? r1 : r0;                                        \
                rmax = (r2 > rmax) ? r2 : rmax;                                           \
                double rsum = exp(r0 - rmax) + exp(r1 - rmax) + exp(r2 - rmax);           \
                double softmin = -gamma * (log(rsum) + rmax);                             \
                R[i * W + j] = (double)D[(i - 1) * M + (j - 1)] + softmin;                \
            }                                                                             \
        }                                                                                 \
    }

DEFINE_FWD(fwd_f32, float)
DEFINE_FWD(fwd_f64, double)

/* Backward for one pair.  R (N+2, M+2) in the input dtype is modified in place (the
 * reference works on a copy, launcher.py:366).  E_out is (N, M).  launcher.py:329-353 */
#define DEFINE_BWD(NAME, T)                                                               \
    static void NAME##_pair(const T *D_, T *R, T *E_out, T *Dp, T *E, int64_t N,          \
                            int64_t M, double gamma, double bandwidth) {                  \
        const int64_t W = M + 2;                                                          \
        memset(Dp, 0, sizeof(T) * (size_t)((N + 2) * W));                                 \
        memset(E, 0, sizeof(T) * (size_t)((N + 2) * W));                                  \
        for (int64_t i = 0; i < N; ++i)                                                   \
            for (int64_t j = 0; j < M; ++j) Dp[(i + 1) * W + (j + 1)] = D_[i * M + j];    \
        E[(N + 1) * W + (M + 1)] = (T)1.0;                                                \
        for (int64_t i = 0; i < N + 2; ++i) R[i * W + (M + 1)] = (T)(-INFINITY);          \
        for (int64_t j = 0; j < M + 2; ++j) R[(N + 1) * W + j] = (T)(-INFINITY);          \
        R[(N + 1) * W + (M + 1)] = R[N * W + M];                                          \
        for (int64_t j = M; j >= 1; --j) {                                                \
            for (int64_t i = N; i >= 1; --i) {                                            \
                if (isinf(R[i * W + j])) R[i * W + j] = (T)(-INFINITY);                   \
                if (out_of_band(bandwidth, i, j)) continue;                               \
                T rij = R[i * W + j];                                                     \
                T da = (T)((T)(R[(i + 1) * W + j] - rij) - Dp[(i + 1) * W + j]);          \
                T db = (T)((T)(R[i * W + (j + 1)] - rij) - Dp[i * W + (j + 1)]);          \
                T dc = (T)((T)(R[(i + 1) * W + (j + 1)] - rij) - Dp[(i + 1) * W + (j + 1)]); \
                double a = exp((double)da / gamma);                                       \
                double bb = exp((double)db / gamma);                                      \
                double c = exp((double)dc / gamma);                                       \
                double acc = (double)E[(i + 1) * W + j] * a;                              \
                acc = acc + (double)E[i * W + (j + 1)] * bb;                              \
                acc = acc + (double)E[(i + 1) * W + (j + 1)] * c;                         \
                E[i * W + j] = (T)acc;                                                    \
            }                                                                             \
        }                                                                                 \
        for (int64_t i = 0; i < N; ++i)                                                   \
            for (int64_t j = 0; j < M; ++j) E_out[i * M + j] = E[(i + 1) * W + (j + 1)];  \
    }

DEFINE_BWD(bwd_f32, float)
DEFINE_BWD(bwd_f64, double)

static int pick_threads(int nthreads) {
#ifdef _OPENMP
    return nthreads > 0 ? nthreads : omp_get_max_threads();
#else
    (void)nthreads;
    return 1;
#endif
}

/* R64: (B, N+2, M+2) fp64, the numba R before `.type_as(D)`. */
int sdtw_oracle_forward_f32(const float *D, double *R64, int64_t B, int64_t N, int64_t M,
                            double gamma, double bandwidth, int nthreads) {
    if (B < 0 || N <= 0 || M <= 0 || !(gamma > 0.0)) return 1;
    int nt = pick_threads(nthreads);
    (void)nt;
#pragma omp parallel for num_threads(nt) schedule(dynamic, 1)
    for (int64_t b = 0; b < B; ++b)
        fwd_f32_pair(D + b * N * M, R64 + b * (N + 2) * (M + 2), N, M, gamma, bandwidth);
    return 0;
}

int sdtw_oracle_forward_f64(const double *D, double *R64, int64_t B, int64_t N, int64_t M,
                            double gamma, double bandwidth, int nthreads) {
    if (B < 0 || N <= 0 || M <= 0 || !(gamma > 0.0)) return 1;
    int nt = pick_threads(nthreads);
    (void)nt;
#pragma omp parallel for num_threads(nt) schedule(dynamic, 1)
    for (int64_t b = 0; b < B; ++b)
        fwd_f64_pair(D + b * N * M, R64 + b * (N + 2) * (M + 2), N, M, gamma, bandwidth);
    return 0;
}

/* R: (B, N+2, M+2) in the input dtype, consumed (modified in place); E: (B, N, M). */
#define DEFINE_BWD_API(NAME, T)                                                           \
    int NAME(const T *D, T *R, T *E, int64_t B, int64_t N, int64_t M, double gamma,       \
             double bandwidth, int nthreads) {                                            \
        if (B < 0 || N <= 0 || M <= 0 || !(gamma > 0.0)) return 1;                        \
        int nt = pick_threads(nthreads);                                                  \
        (void)nt;                                                                         \
        int rc = 0;                                                                       \
        _Pragma("omp parallel for num_threads(nt) schedule(dynamic, 1)")                  \
        for (int64_t b = 0; b < B; ++b) {                                                 \
            size_t pad = (size_t)((N + 2) * (M + 2));                                     \
            T *Dp = (T *)malloc(sizeof(T) * pad);                                         \
            T *Ew = (T *)malloc(sizeof(T) * pad);                                         \
            if (!Dp || !Ew) {                                                             \
                rc = 2;                                                                   \
            } else {                                                                      \
                NAME##_pair_impl(D + b * N * M, R + b * (int64_t)pad, E + b * N * M, Dp,  \
                                 Ew, N, M, gamma, bandwidth);                             \
            }                                                                             \
            free(Dp);                                                                     \
            free(Ew);                                                                     \
        }                                                                                 \
        return rc;                                                                        \
    }

#define sdtw_oracle_backward_f32_pair_impl bwd_f32_pair
#define sdtw_oracle_backward_f64_pair_impl bwd_f64_pair
DEFINE_BWD_API(sdtw_oracle_backward_f32, float)
DEFINE_BWD_API(sdtw_oracle_backward_f64, double)
