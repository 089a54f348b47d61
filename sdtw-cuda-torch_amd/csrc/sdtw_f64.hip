// sdtw_f64.hip -- the float64 path: distance, recursions and distance backward in double.
//
// The reference keeps the caller's dtype end to end: for float64 inputs the cost is formed in
// float64 (distances.py:20-25) and the recursions run on float64 arrays (launcher.py:307-368:
// R is float64 and so are D, E and every difference), which is what torch.autograd.gradcheck
// relies on (the reference's test_softdtw_small.py:29-37).  These kernels restate that
// arithmetic in double, operation for operation:
//   forward   R[i,j] = D[i-1,j-1] - gamma (log(sum_k exp(r_k - rmax)) + rmax),
//             r_k = -R[nbr_k] / gamma, rmax the Python max (launcher.py:316-322);
//   backward  E[i,j] = sum over the three later neighbours of E[nbr] exp((R[nbr] - R[i,j] -
//             D[nbr]) / gamma), with R's +inf entries read as -inf and the padding of
//             launcher.py:330-345;
// with the Sakoe-Chiba test `0 < bandwidth < |i - j|` of launcher.py:315 and :345.
//
// Layout: R is the reference's own dense (B, N+2, M+2) table (row 0 / column 0 padding, row
// N+1 / column M+1 read by the backward).  One workgroup owns a pair and sweeps it by
// anti-diagonals: the cells of a diagonal are independent, so its threads compute them at
// once and a workgroup barrier separates consecutive diagonals.  There are no waits between
// workgroups.  The last diagonals live in LDS; where they do not fit, the same sweep reads
// its neighbours back from global memory (the workgroup's own writes, made visible by the
// barrier), so any N and M fit.  The distance kernels are LDS-tiled.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "../../include/sdtw.h"

namespace sdtw64 {

constexpr int kSweepThreads = 1024;

__device__ __forceinline__ bool out_of_band(double bw, int64_t i, int64_t j) {
    const int64_t d = i > j ? i - j : j - i;
    return 0.0 < bw && bw < (double)d;
}

// clamp_min's backward passes the gradient where the pre-clamp value is >= 0: every cell with
// D > 0, and the cells with D == 0 whose pre-clamp value is exactly zero (recomputed with the
// forward kernel's arithmetic, so with its bits).
__device__ __forceinline__ double masked(double g, double d, const double* xi, const double* yj,
                                         int K) {
    if (d > 0.0) return g;
    if (d != 0.0) return 0.0;  // NaN cost: torch's mask (NaN >= 0) is false
    double x2 = 0.0, y2 = 0.0, dot = 0.0;
    for (int k = 0; k < K; ++k) {
        const double a = xi[k], c = yj[k];
        x2 = fma(a, a, x2);
        y2 = fma(c, c, y2);
        dot = fma(a, c, dot);
    }
    return ((x2 + y2) - 2.0 * dot) >= 0.0 ? g : 0.0;
}

// The distance and its backward, tiled: a block of 256 threads owns a 64 x 64 output tile,
// each thread 4 x 4 outputs strided by 16 (conflict-free LDS reads), and the reduction runs
// in chunks of 16 staged through LDS.  Every output is one sequential sum over the reduction
// index (the operation order of distances.py:20-25: norms and dot accumulated over k, then
// (x2 + y2) - 2 dot, clamped at 0):
//   D[b,i,j]  = max(0, (|x_i|^2 + |y_j|^2) - 2 x_i.y_j)
//   gx[b,i,k] = 2 x[b,i,k] sum_j G'[b,i,j] - 2 sum_j G'[b,i,j] y[b,j,k]   (TRANS = false)
//   gy[b,j,k] = 2 y[b,j,k] sum_i G'[b,i,j] - 2 sum_i G'[b,i,j] x[b,i,k]   (TRANS = true)
constexpr int kT = 64, kKC = 16;

// D tile: rows i0 .. i0 + 63 of x, columns j0 .. j0 + 63 (rows of y); norms and dots
// accumulated over k in order.
__global__ void __launch_bounds__(256) dist_fwd_tiled_kernel(const double* __restrict__ x,
                                                             const double* __restrict__ y,
                                                             double* __restrict__ D, int N, int M,
                                                             int K) {
    __shared__ double xs[kKC][kT + 1], ys[kKC][kT + 1];
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    const int i0 = blockIdx.y * kT, j0 = blockIdx.x * kT;
    const int64_t b = blockIdx.z;
    const double* xb = x + b * N * K;
    const double* yb = y + b * M * K;
    double dot[4][4] = {}, x2[4] = {}, y2[4] = {};
    for (int k0 = 0; k0 < K; k0 += kKC) {
        // 64 rows x 16 features of x and of y: 4 of each per thread, zero past the edges
        for (int e = threadIdx.x; e < kT * kKC; e += 256) {
            const int r = e / kKC, kk = e % kKC, k = k0 + kk;
            xs[kk][r] = (i0 + r < N && k < K) ? xb[(int64_t)(i0 + r) * K + k] : 0.0;
            ys[kk][r] = (j0 + r < M && k < K) ? yb[(int64_t)(j0 + r) * K + k] : 0.0;
        }
        __syncthreads();
        const int kn = K - k0 < kKC ? K - k0 : kKC;
        for (int kk = 0; kk < kn; ++kk) {
            double a[4], c[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                a[u] = xs[kk][ty + 16 * u];
                c[u] = ys[kk][tx + 16 * u];
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                x2[u] = fma(a[u], a[u], x2[u]);
                y2[u] = fma(c[u], c[u], y2[u]);
#pragma unroll
                for (int v = 0; v < 4; ++v) dot[u][v] = fma(a[u], c[v], dot[u][v]);
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int i = i0 + ty + 16 * u;
        if (i >= N) continue;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int j = j0 + tx + 16 * v;
            if (j >= M) continue;
            const double pre = (x2[u] + y2[v]) - 2.0 * dot[u][v];
            D[(b * N + i) * M + j] = pre > 0.0 ? pre : (pre == pre ? 0.0 : pre);
        }
    }
}

// gx (TRANS = false): 64 output rows i x 64 features k, reduction over j; gy (TRANS = true):
// rows j, reduction over i.  The masked G tile (rows x 16 reduction indices) and the 16 x 64
// feature tile of the other operand are staged per chunk; every thread sums its rows' G'
// from LDS in order, as the simple kernel does.
template <bool TRANS>
__global__ void __launch_bounds__(256) dist_bwd_tiled_kernel(const double* __restrict__ x,
                                                             const double* __restrict__ y,
                                                             const double* __restrict__ D,
                                                             const double* __restrict__ G,
                                                             double* __restrict__ out, int N,
                                                             int M, int K, int mask) {
    __shared__ double gs[kKC][kT + 1], os[kKC][kT + 1];
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    const int r0 = blockIdx.y * kT, k0 = blockIdx.x * kT;
    const int64_t b = blockIdx.z;
    const int R = TRANS ? M : N, T = TRANS ? N : M;
    const double* selfb = TRANS ? y + b * M * K : x + b * N * K;
    const double* other = TRANS ? x + b * N * K : y + b * M * K;
    const double* Gb = G + b * N * M;
    const double* Db = mask ? D + b * N * M : nullptr;
    double acc[4][4] = {}, s[4] = {};
    for (int t0 = 0; t0 < T; t0 += kKC) {
        for (int e = threadIdx.x; e < kT * kKC; e += 256) {
            // G' tile: consecutive threads along G's rows (j for gy, the reduction index t
            // for gx), so that they read consecutive entries
            const int r = TRANS ? e % kT : e / kKC, tt = TRANS ? e / kT : e % kKC, t = t0 + tt;
            double g = 0.0;
            if (r0 + r < R && t < T) {
                const int64_t cell = TRANS ? (int64_t)t * M + (r0 + r) : (int64_t)(r0 + r) * M + t;
                const double* xi = TRANS ? other + (int64_t)t * K : selfb + (int64_t)(r0 + r) * K;
                const double* yj = TRANS ? selfb + (int64_t)(r0 + r) * K : other + (int64_t)t * K;
                g = Db ? masked(Gb[cell], Db[cell], xi, yj, K) : Gb[cell];
            }
            gs[tt][r] = g;
            const int ft = e / kT, kk = e % kT;  // feature tile: 16 reduction rows x 64 features
            os[ft][kk] = (t0 + ft < T && k0 + kk < K) ? other[(int64_t)(t0 + ft) * K + k0 + kk] : 0.0;
        }
        __syncthreads();
        const int tn = T - t0 < kKC ? T - t0 : kKC;
        for (int tt = 0; tt < tn; ++tt) {
            double g[4], o[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                g[u] = gs[tt][ty + 16 * u];
                o[u] = os[tt][tx + 16 * u];
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                s[u] += g[u];
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[u][v] = fma(g[u], o[v], acc[u][v]);
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int r = r0 + ty + 16 * u;
        if (r >= R) continue;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int k = k0 + tx + 16 * v;
            if (k >= K) continue;
            out[(b * R + r) * K + k] = 2.0 * s[u] * selfb[(int64_t)r * K + k] - 2.0 * acc[u][v];
        }
    }
}

// Forward recursion of pair blockIdx.x (launcher.py:307-324), R (N+2, M+2) dense.
__global__ void __launch_bounds__(kSweepThreads) dp_fwd_kernel(const double* __restrict__ Dall,
                                                               double* __restrict__ Rall,
                                                               double* __restrict__ out, int N,
                                                               int M, double gamma, double bw) {
    const int64_t b = blockIdx.x;
    const int64_t W = M + 2;
    double* R = Rall + b * (N + 2) * W;
    const double* D = Dall + b * N * M;
    const double INF = __builtin_inf();
    for (int64_t e = threadIdx.x; e < (N + 2) * W; e += blockDim.x) R[e] = e == 0 ? 0.0 : INF;
    __syncthreads();
    for (int d = 2; d <= N + M; ++d) {
        const int ilo = d - M > 1 ? d - M : 1;
        const int ihi = d - 1 < N ? d - 1 : N;
        for (int i = ilo + threadIdx.x; i <= ihi; i += blockDim.x) {
            const int j = d - i;
            if (out_of_band(bw, i, j)) continue;
            const double r0 = -R[(i - 1) * W + (j - 1)] / gamma;
            const double r1 = -R[(i - 1) * W + j] / gamma;
            const double r2 = -R[i * W + (j - 1)] / gamma;
            double rmax = (r1 > r0) ? r1 : r0;
            rmax = (r2 > rmax) ? r2 : rmax;
            const double rsum = exp(r0 - rmax) + exp(r1 - rmax) + exp(r2 - rmax);
            const double softmin = -gamma * (log(rsum) + rmax);
            R[i * W + j] = D[(int64_t)(i - 1) * M + (j - 1)] + softmin;
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) out[b] = R[N * W + M];
}

// Backward of pair blockIdx.x (launcher.py:327-353) into G (N, M): E is formed in G (its
// padding row and column are read as launcher.py:330-338 sets them: E 0 but E[N+1,M+1] = 1;
// R -inf but R[N+1,M+1] = R[N,M]; D 0), then scaled by gout[b].  R itself is not modified:
// its +inf entries are read as -inf, as the reference's in-place edit (launcher.py:343-344)
// leaves them for every later read.
__global__ void __launch_bounds__(kSweepThreads) dp_bwd_kernel(const double* __restrict__ Dall,
                                                               const double* __restrict__ Rall,
                                                               const double* __restrict__ gout,
                                                               double* __restrict__ Gall, int N,
                                                               int M, double gamma, double bw) {
    const int64_t b = blockIdx.x;
    const int64_t W = M + 2;
    const double* R = Rall + b * (N + 2) * W;
    const double* D = Dall + b * N * M;
    double* E = Gall + b * N * M;
    const double NINF = -__builtin_inf();
    const double corner = R[N * W + M];  // R[N+1, M+1], set before the sweep's edits
    auto Rat = [&](int i, int j) -> double {
        if (i > N || j > M) return (i > N && j > M) ? corner : NINF;
        const double v = R[i * W + j];
        return isinf(v) ? NINF : v;
    };
    auto Eat = [&](int i, int j) -> double {
        if (i > N || j > M) return (i > N && j > M) ? 1.0 : 0.0;
        return E[(int64_t)(i - 1) * M + (j - 1)];
    };
    auto Dat = [&](int i, int j) -> double {
        if (i > N || j > M) return 0.0;
        return D[(int64_t)(i - 1) * M + (j - 1)];
    };
    for (int64_t e = threadIdx.x; e < (int64_t)N * M; e += blockDim.x) E[e] = 0.0;
    __syncthreads();
    for (int d = N + M; d >= 2; --d) {
        const int ilo = d - M > 1 ? d - M : 1;
        const int ihi = d - 1 < N ? d - 1 : N;
        for (int i = ilo + threadIdx.x; i <= ihi; i += blockDim.x) {
            const int j = d - i;
            if (out_of_band(bw, i, j)) continue;
            const double rij = Rat(i, j);
            const double da = (Rat(i + 1, j) - rij) - Dat(i + 1, j);
            const double db = (Rat(i, j + 1) - rij) - Dat(i, j + 1);
            const double dc = (Rat(i + 1, j + 1) - rij) - Dat(i + 1, j + 1);
            const double a = exp(da / gamma);
            const double bb = exp(db / gamma);
            const double c = exp(dc / gamma);
            double acc = Eat(i + 1, j) * a;
            acc = acc + Eat(i, j + 1) * bb;
            acc = acc + Eat(i + 1, j + 1) * c;
            E[(int64_t)(i - 1) * M + (j - 1)] = acc;
        }
        __syncthreads();
    }
    if (gout) {
        const double g = gout[b];
        for (int64_t e = threadIdx.x; e < (int64_t)N * M; e += blockDim.x) E[e] = g * E[e];
    }
}

// The same recursions with the rolling anti-diagonals in LDS: the values of diagonals d - 1
// and d - 2 (forward) or d + 1 and d + 2 (backward), indexed by row over the padded table
// (row 0 .. N + 1), are read from LDS instead of global memory.  Each sweep visits every
// padded entry of its diagonals, so every neighbour read lands on an entry written one or
// two diagonals earlier.  The forward writes every entry of R, the backward every cell of G
// (gout * E, 0 out of the band), so neither needs an initialising or scaling pass.
constexpr int64_t kLdsBytes = 160 * 1024;
inline int64_t fwd_lds_bytes(int64_t N) { return 3 * (N + 2) * (int64_t)sizeof(double); }
inline int64_t bwd_lds_bytes(int64_t N) { return 9 * (N + 2) * (int64_t)sizeof(double); }

__global__ void __launch_bounds__(kSweepThreads) dp_fwd_lds_kernel(const double* __restrict__ Dall,
                                                                   double* __restrict__ Rall,
                                                                   double* __restrict__ out, int N,
                                                                   int M, double gamma, double bw) {
    extern __shared__ double sh[];
    const int64_t b = blockIdx.x;
    const int64_t W = M + 2;
    double* R = Rall + b * (N + 2) * W;
    const double* D = Dall + b * N * M;
    const double INF = __builtin_inf();
    const int L = N + 2;
    for (int d = 0; d <= N + M + 2; ++d) {
        double* cur = sh + (d % 3) * L;
        const double* p1 = sh + ((d + 2) % 3) * L;  // diagonal d - 1
        const double* p2 = sh + ((d + 1) % 3) * L;  // diagonal d - 2
        const int ilo = d - (M + 1) > 0 ? d - (M + 1) : 0;
        const int ihi = d < N + 1 ? d : N + 1;
        for (int i = ilo + threadIdx.x; i <= ihi; i += blockDim.x) {
            const int j = d - i;
            double v;
            if (i == 0 || j == 0) {
                v = (i == 0 && j == 0) ? 0.0 : INF;
            } else if (i > N || j > M || out_of_band(bw, i, j)) {
                v = INF;
            } else {
                const double r0 = -p2[i - 1] / gamma;  // (i-1, j-1)
                const double r1 = -p1[i - 1] / gamma;  // (i-1, j)
                const double r2 = -p1[i] / gamma;      // (i, j-1)
                double rmax = (r1 > r0) ? r1 : r0;
                rmax = (r2 > rmax) ? r2 : rmax;
                const double rsum = exp(r0 - rmax) + exp(r1 - rmax) + exp(r2 - rmax);
                const double softmin = -gamma * (log(rsum) + rmax);
                v = D[(int64_t)(i - 1) * M + (j - 1)] + softmin;
            }
            cur[i] = v;
            R[i * W + j] = v;
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) out[b] = R[N * W + M];
}

__global__ void __launch_bounds__(kSweepThreads) dp_bwd_lds_kernel(const double* __restrict__ Dall,
                                                                   const double* __restrict__ Rall,
                                                                   const double* __restrict__ gout,
                                                                   double* __restrict__ Gall, int N,
                                                                   int M, double gamma, double bw) {
    extern __shared__ double sh[];
    const int64_t b = blockIdx.x;
    const int64_t W = M + 2;
    const double* R = Rall + b * (N + 2) * W;
    const double* D = Dall + b * N * M;
    double* G = Gall + b * N * M;
    const double NINF = -__builtin_inf();
    const double corner = R[N * W + M];
    const double g = gout ? gout[b] : 1.0;
    const int L = N + 2;
    // buffers k = 0, 1, 2 of E, R (its +inf read as -inf) and D, by row
    auto Eb = [&](int k) { return sh + k * L; };
    auto Rb = [&](int k) { return sh + (3 + k) * L; };
    auto Db = [&](int k) { return sh + (6 + k) * L; };
    for (int d = N + M + 2; d >= 2; --d) {
        const int k0 = d % 3, k1 = (d + 1) % 3, k2 = (d + 2) % 3;  // diagonals d, d+1, d+2
        double *Ec = Eb(k0), *Rc = Rb(k0), *Dc = Db(k0);
        const double *E1 = Eb(k1), *R1 = Rb(k1), *D1 = Db(k1);
        const double *E2 = Eb(k2), *R2 = Rb(k2), *D2 = Db(k2);
        const int ilo = d - (M + 1) > 1 ? d - (M + 1) : 1;
        const int ihi = d - 1 < N + 1 ? d - 1 : N + 1;
        for (int i = ilo + threadIdx.x; i <= ihi; i += blockDim.x) {
            const int j = d - i;
            double e, r, dv;
            if (i == N + 1 || j == M + 1) {
                const bool c = (i == N + 1 && j == M + 1);
                e = c ? 1.0 : 0.0;
                r = c ? corner : NINF;
                dv = 0.0;
            } else {
                const double rv = R[i * W + j];
                r = isinf(rv) ? NINF : rv;
                dv = D[(int64_t)(i - 1) * M + (j - 1)];
                e = 0.0;
                if (!out_of_band(bw, i, j)) {
                    const double da = (R1[i + 1] - r) - D1[i + 1];  // (i+1, j)
                    const double db = (R1[i] - r) - D1[i];          // (i, j+1)
                    const double dc = (R2[i + 1] - r) - D2[i + 1];  // (i+1, j+1)
                    const double a = exp(da / gamma);
                    const double bb = exp(db / gamma);
                    const double cc = exp(dc / gamma);
                    double acc = E1[i + 1] * a;
                    acc = acc + E1[i] * bb;
                    acc = acc + E2[i + 1] * cc;
                    e = acc;
                }
                G[(int64_t)(i - 1) * M + (j - 1)] = g * e;
            }
            Ec[i] = e;
            Rc[i] = r;
            Dc[i] = dv;
        }
        __syncthreads();
    }
}

bool shape_ok(int64_t B, int64_t N, int64_t M, int64_t K, bool need_k) {
    if (B < 0 || N <= 0 || M <= 0 || B > 65535) return false;
    if (need_k && (K <= 0 || K > INT32_MAX)) return false;
    // int row / diagonal indices; the grids put rows / 4 on grid.y
    if (N > INT32_MAX / 2 - 2 || M > INT32_MAX / 2 - 2) return false;
    if ((N + 3) / 4 > 65535 || (M + 3) / 4 > 65535) return false;
    return true;
}

int status_of(hipError_t e) { return e == hipSuccess ? SDTW_OK : SDTW_ERR_LAUNCH; }

}  // namespace sdtw64

using namespace sdtw64;

extern "C" {

int64_t sdtw_table_elems_f64(int64_t B, int64_t N, int64_t M) {
    if (B < 0 || N <= 0 || M <= 0) return 0;
    return B * (N + 2) * (M + 2);
}

int sdtw_sqeuclid_fwd_f64(const double* x, const double* y, double* D, int64_t B, int64_t N,
                          int64_t M, int64_t K, void* stream) {
    if (!shape_ok(B, N, M, K, true)) return SDTW_ERR_INVALID_VALUE;
    if (B == 0) return SDTW_OK;
    if (!x || !y || !D) return SDTW_ERR_INVALID_VALUE;
    hipLaunchKernelGGL(dist_fwd_tiled_kernel,
                       dim3((unsigned)((M + kT - 1) / kT), (unsigned)((N + kT - 1) / kT), (unsigned)B),
                       dim3(256), 0, (hipStream_t)stream, x, y, D, (int)N, (int)M, (int)K);
    return status_of(hipGetLastError());
}

int sdtw_sqeuclid_bwd_f64(const double* x, const double* y, const double* D, const double* G,
                          double* gx, double* gy, int64_t B, int64_t N, int64_t M, int64_t K,
                          int mask, void* stream) {
    if (!shape_ok(B, N, M, K, true)) return SDTW_ERR_INVALID_VALUE;
    if (B == 0) return SDTW_OK;
    if (!x || !y || !G || !gx || !gy || (mask && !D)) return SDTW_ERR_INVALID_VALUE;
    if ((K + 63) / 64 > INT32_MAX) return SDTW_ERR_UNSUPPORTED;
    const hipStream_t st = (hipStream_t)stream;
    const unsigned kb = (unsigned)((K + kT - 1) / kT);
    hipLaunchKernelGGL(dist_bwd_tiled_kernel<false>, dim3(kb, (unsigned)((N + kT - 1) / kT), (unsigned)B),
                       dim3(256), 0, st, x, y, D, G, gx, (int)N, (int)M, (int)K, mask);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return SDTW_ERR_LAUNCH;
    hipLaunchKernelGGL(dist_bwd_tiled_kernel<true>, dim3(kb, (unsigned)((M + kT - 1) / kT), (unsigned)B),
                       dim3(256), 0, st, x, y, D, G, gy, (int)N, (int)M, (int)K, mask);
    return status_of(hipGetLastError());
}

int sdtw_fwd_f64(const double* D, double* R, double* out, int64_t B, int64_t N, int64_t M,
                 double gamma, double bandwidth, void* stream) {
    if (!shape_ok(B, N, M, 1, false)) return SDTW_ERR_INVALID_VALUE;
    if (!(gamma > 0.0) || !isfinite(gamma)) return SDTW_ERR_INVALID_VALUE;
    if (B == 0) return SDTW_OK;
    if (!D || !R || !out) return SDTW_ERR_INVALID_VALUE;
    const int64_t lds = fwd_lds_bytes(N);
    if (lds <= kLdsBytes) {
        if (lds > 64 * 1024 &&
            hipFuncSetAttribute(reinterpret_cast<const void*>(dp_fwd_lds_kernel),
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
            return SDTW_ERR_LAUNCH;
        hipLaunchKernelGGL(dp_fwd_lds_kernel, dim3((unsigned)B), dim3(kSweepThreads), (size_t)lds,
                           (hipStream_t)stream, D, R, out, (int)N, (int)M, gamma, bandwidth);
    } else {
        hipLaunchKernelGGL(dp_fwd_kernel, dim3((unsigned)B), dim3(kSweepThreads), 0,
                           (hipStream_t)stream, D, R, out, (int)N, (int)M, gamma, bandwidth);
    }
    return status_of(hipGetLastError());
}

int sdtw_bwd_f64(const double* D, const double* R, const double* gout, double* G, int64_t B,
                 int64_t N, int64_t M, double gamma, double bandwidth, void* stream) {
    if (!shape_ok(B, N, M, 1, false)) return SDTW_ERR_INVALID_VALUE;
    if (!(gamma > 0.0) || !isfinite(gamma)) return SDTW_ERR_INVALID_VALUE;
    if (B == 0) return SDTW_OK;
    if (!D || !R || !G) return SDTW_ERR_INVALID_VALUE;
    const int64_t lds = bwd_lds_bytes(N);
    if (lds <= kLdsBytes) {
        if (lds > 64 * 1024 &&
            hipFuncSetAttribute(reinterpret_cast<const void*>(dp_bwd_lds_kernel),
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
            return SDTW_ERR_LAUNCH;
        hipLaunchKernelGGL(dp_bwd_lds_kernel, dim3((unsigned)B), dim3(kSweepThreads), (size_t)lds,
                           (hipStream_t)stream, D, R, gout, G, (int)N, (int)M, gamma, bandwidth);
    } else {
        hipLaunchKernelGGL(dp_bwd_kernel, dim3((unsigned)B), dim3(kSweepThreads), 0,
                           (hipStream_t)stream, D, R, gout, G, (int)N, (int)M, gamma, bandwidth);
    }
    return status_of(hipGetLastError());
}

}  // extern "C"
