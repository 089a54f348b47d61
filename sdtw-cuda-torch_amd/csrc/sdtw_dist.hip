// sdtw_dist.hip -- squared-Euclidean cost and its gradient for gfx950.
//
//   norms_kernel      x2[r] = sum_k x[r,k]^2 in ATen's CPU order (one lane per row).
//   dist_kernel       D = clamp_min(x2 + y2 - 2 x.y^T, 0): 64x64 output tiles, x/y k-slices
//                     staged in LDS, every output's dot product a sequential FMA chain over k
//                     (the order of the host GEMM), so D has the reference's bits.
//   dist_bwd_kernel   gx = 2 (x * rowsum(G') - G' y) and gy = 2 (y * colsum(G') - G'^T x)
//                     with G' = G masked by the clamp (clamp_min backward passes where
//                     x2 + y2 - 2xy >= 0).
#include "sdtw_device.hpp"
#include "sdtw_internal.hpp"

namespace sdtw {

__global__ void __launch_bounds__(256) norms_kernel(const float* __restrict__ v,
                                                    float* __restrict__ out, int64_t rows,
                                                    int K) {
    const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (r < rows) out[r] = aten_sumsq(v + r * K, K);
}

hipError_t launch_norms(const float* v, float* out, int64_t rows, int K, hipStream_t st) {
    if (rows <= 0) return hipSuccess;
    const int64_t blocks = (rows + 255) / 256;
    hipLaunchKernelGGL(norms_kernel, dim3((unsigned)blocks), dim3(256), 0, st, v, out, rows,
                       K);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------
// Exact distance: WG = 16x16 threads, tile 64 (rows of x) x 64 (rows of y); thread (ty,tx)
// owns outputs (ty + 16m, tx + 16n), m,n in [0,4).  k advances in slices of KC through LDS;
// each accumulator sees k = 0, 1, ..., K-1 in order.
// ---------------------------------------------------------------------------------------
constexpr int DT = 64;
constexpr int KC = 16;

template <bool MULADD>
__global__ void __launch_bounds__(256) dist_kernel(DistParams p) {
    __shared__ float xs[KC][DT + 1];
    __shared__ float ys[KC][DT + 1];
    const int b = blockIdx.z;
    const int i0 = blockIdx.y * DT;
    const int j0 = blockIdx.x * DT;
    const int tx = threadIdx.x & 15;
    const int ty = threadIdx.x >> 4;
    const int N = p.N, M = p.M, K = p.K;
    const float* xb = p.x + (int64_t)b * N * K;
    const float* yb = p.y + (int64_t)b * M * K;
    float acc[4][4];
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int n = 0; n < 4; ++n) acc[m][n] = 0.0f;
    for (int k0 = 0; k0 < K; k0 += KC) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int e = threadIdx.x + 256 * u;
            const int r = e / KC, kk = e % KC;
            const int k = k0 + kk;
            xs[kk][r] = (i0 + r < N && k < K) ? xb[(int64_t)(i0 + r) * K + k] : 0.0f;
            ys[kk][r] = (j0 + r < M && k < K) ? yb[(int64_t)(j0 + r) * K + k] : 0.0f;
        }
        __syncthreads();
        const int kn = min(KC, K - k0);
        for (int kk = 0; kk < kn; ++kk) {
            float a[4], bb[4];
#pragma unroll
            for (int m = 0; m < 4; ++m) a[m] = xs[kk][ty + 16 * m];
#pragma unroll
            for (int n = 0; n < 4; ++n) bb[n] = ys[kk][tx + 16 * n];
#pragma unroll
            for (int m = 0; m < 4; ++m)
#pragma unroll
                for (int n = 0; n < 4; ++n) {
                    if (MULADD)
                        acc[m][n] = __fadd_rn(acc[m][n], __fmul_rn(a[m], bb[n]));
                    else
                        acc[m][n] = __fmaf_rn(a[m], bb[n], acc[m][n]);
                }
        }
        __syncthreads();
    }
    const float* x2 = p.x2 + (int64_t)b * N;
    const float* y2 = p.y2 + (int64_t)b * M;
    float* Db = p.D + (int64_t)b * N * M;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const int i = i0 + ty + 16 * m;
        if (i >= N) continue;
        const float xi = x2[i];
#pragma unroll
        for (int n = 0; n < 4; ++n) {
            const int j = j0 + tx + 16 * n;
            if (j < M) Db[(int64_t)i * M + j] = clamp0(exact_cost_pre(xi, y2[j], acc[m][n]));
        }
    }
}

hipError_t launch_dist(const DistParams& p, bool muladd, bool mfma, hipStream_t st) {
    hipError_t e = launch_norms(p.x, p.x2, (int64_t)p.B * p.N, p.K, st);
    if (e != hipSuccess) return e;
    e = launch_norms(p.y, p.y2, (int64_t)p.B * p.M, p.K, st);
    if (e != hipSuccess) return e;
    (void)mfma;
    dim3 grid((p.M + DT - 1) / DT, (p.N + DT - 1) / DT, p.B);
    if (muladd)
        hipLaunchKernelGGL(dist_kernel<true>, grid, dim3(256), 0, st, p);
    else
        hipLaunchKernelGGL(dist_kernel<false>, grid, dim3(256), 0, st, p);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------
// Distance backward.  Output rows r (x rows for gx, y rows for gy), reduction index t.
//   grad[r,k] = 2 * (W[r,k] * rs[r] - sum_t G'(r,t) Z[t,k]),   rs[r] = sum_t G'(r,t)
// TRANS = false: gx (W = x, Z = y, G'(r,t) = G[r,t]);  TRANS = true: gy (W = y, Z = x,
// G'(r,t) = G[t,r]).  Tile TR rows x TK features, 256 threads each owning 4 x 4 outputs.
// ---------------------------------------------------------------------------------------
constexpr int TT = 16;  // reduction slice

template <bool MULADD>
SDTW_DEV bool pass_mask(const DistBwdParams& p, int b, int i, int j, float d) {
    if (d > 0.0f) return true;
    if (!(d == 0.0f)) return false;  // NaN: clamp_min backward gives 0
    // clamped (or exactly zero) cell: recompute the pre-clamp value
    const float* xi = p.x + ((int64_t)b * p.N + i) * p.K;
    const float* yj = p.y + ((int64_t)b * p.M + j) * p.K;
    const float dot = exact_dot<MULADD>(xi, yj, p.K);
    return exact_cost_pre(p.x2[(int64_t)b * p.N + i], p.y2[(int64_t)b * p.M + j], dot) >= 0.0f;
}

template <bool TRANS, int TR, int TK, bool MULADD>
__global__ void __launch_bounds__(256) dist_bwd_kernel(DistBwdParams p) {
    constexpr int TX = TK / 4;  // threads along k
    static_assert((TR / 4) * TX == 256, "tile must map to 256 threads");
    __shared__ float gs[TT][TR + 1];
    __shared__ float zs[TT][TK + 1];
    const int b = blockIdx.z;
    const int r0 = blockIdx.y * TR;
    const int k0 = blockIdx.x * TK;
    const int tx = threadIdx.x % TX;
    const int ty = threadIdx.x / TX;
    const int N = p.N, M = p.M, K = p.K;
    const int R_ = TRANS ? M : N;  // output rows
    const int T_ = TRANS ? N : M;  // reduction length
    const float* Gb = p.G + (int64_t)b * N * M;
    const float* Db = p.D ? p.D + (int64_t)b * N * M : nullptr;
    const float* Z = TRANS ? p.x + (int64_t)b * N * K : p.y + (int64_t)b * M * K;
    const float* W = TRANS ? p.y + (int64_t)b * M * K : p.x + (int64_t)b * N * K;
    float* out = TRANS ? p.gy + (int64_t)b * M * K : p.gx + (int64_t)b * N * K;
    float acc[4][4], rs[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        rs[m] = 0.0f;
#pragma unroll
        for (int n = 0; n < 4; ++n) acc[m][n] = 0.0f;
    }
    for (int t0 = 0; t0 < T_; t0 += TT) {
        // G' slice: TR rows x TT reduction entries
        for (int e = threadIdx.x; e < TR * TT; e += 256) {
            int r, tt;
            if (TRANS) {  // contiguous along r in memory
                r = e % TR;
                tt = e / TR;
            } else {  // contiguous along t
                r = e / TT;
                tt = e % TT;
            }
            const int rr = r0 + r, t = t0 + tt;
            float v = 0.0f;
            if (rr < R_ && t < T_) {
                const int i = TRANS ? t : rr;
                const int j = TRANS ? rr : t;
                const int64_t idx = (int64_t)i * M + j;
                v = Gb[idx];
                if (p.mask && !pass_mask<MULADD>(p, b, i, j, Db[idx])) v = 0.0f;
            }
            gs[tt][r] = v;
        }
        for (int e = threadIdx.x; e < TT * TK; e += 256) {
            const int tt = e / TK, kk = e % TK;
            const int t = t0 + tt, k = k0 + kk;
            zs[tt][kk] = (t < T_ && k < K) ? Z[(int64_t)t * K + k] : 0.0f;
        }
        __syncthreads();
#pragma unroll 4
        for (int tt = 0; tt < TT; ++tt) {
            float gv[4], zv[4];
#pragma unroll
            for (int m = 0; m < 4; ++m) gv[m] = gs[tt][ty + (TR / 4) * m];
#pragma unroll
            for (int n = 0; n < 4; ++n) zv[n] = zs[tt][tx + TX * n];
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                rs[m] += gv[m];
#pragma unroll
                for (int n = 0; n < 4; ++n) acc[m][n] = fmaf(gv[m], zv[n], acc[m][n]);
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const int r = r0 + ty + (TR / 4) * m;
        if (r >= R_) continue;
#pragma unroll
        for (int n = 0; n < 4; ++n) {
            const int k = k0 + tx + TX * n;
            if (k < K) {
                const int64_t o = (int64_t)r * K + k;
                out[o] = 2.0f * (W[o] * rs[m] - acc[m][n]);
            }
        }
    }
}

template <bool TRANS, bool MULADD>
static void launch_dist_bwd_one(const DistBwdParams& p, hipStream_t st) {
    const int R_ = TRANS ? p.M : p.N;
    if (p.K <= 16) {
        dim3 grid((p.K + 15) / 16, (R_ + 255) / 256, p.B);
        hipLaunchKernelGGL((dist_bwd_kernel<TRANS, 256, 16, MULADD>), grid, dim3(256), 0, st, p);
    } else {
        dim3 grid((p.K + 63) / 64, (R_ + 63) / 64, p.B);
        hipLaunchKernelGGL((dist_bwd_kernel<TRANS, 64, 64, MULADD>), grid, dim3(256), 0, st, p);
    }
}

hipError_t launch_dist_bwd(const DistBwdParams& p, hipStream_t st) {
    if (p.muladd) {
        launch_dist_bwd_one<false, true>(p, st);
        launch_dist_bwd_one<true, true>(p, st);
    } else {
        launch_dist_bwd_one<false, false>(p, st);
        launch_dist_bwd_one<true, false>(p, st);
    }
    return hipGetLastError();
}

}  // namespace sdtw
