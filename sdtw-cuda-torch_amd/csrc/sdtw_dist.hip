// sdtw_dist.hip -- squared-Euclidean cost and its gradient for gfx950.
//
//   norms_kernel      x2[r] = sum_k x[r,k]^2 in ATen's CPU order (eight lanes per row), for
//                     the fused recursions and the clamp mask of the backward.
//   dist_xs_kernel    D = clamp_min(x2 + y2 - 2 x.y^T, 0) for K <= 64: 64x64 output tiles,
//                     64 rows of x stationary in LDS and y tiles streamed through two LDS
//                     buffers; every output's dot product a sequential FMA chain over k (the
//                     order of the host GEMM) on the matrix cores, so D has the reference's
//                     bits; row norms computed from the staged tiles (norms_kernel's bits).
//   dist_kernel       the same on the VALU with k chunks through LDS, for K > 64 and for the
//                     tiny problems whose reference dot is ATen's multiply-then-add kernel.
//   dist_bwd_mfma_kernel
//                     gx = 2 (x * rowsum(G') - G' y) and gy = 2 (y * colsum(G') - G'^T x)
//                     on the matrix cores, with G' = G masked by the clamp (clamp_min
//                     backward passes where x2 + y2 - 2xy >= 0).
#include <type_traits>

#include "sdtw_device.hpp"
#include "sdtw_internal.hpp"

namespace sdtw {

// Row norm with eight threads per row (threads 8g .. 8g + 7 of a wave share a row): for
// K >= 8 thread t computes ATen's vector lane t (the scalar row_sum over v[8c + t]); the
// row's first thread adds the tail and the eight lane sums in ATen's order (aten_sumsq), so
// the result has the same bits with 8x the parallelism.  Every thread of the wave must
// call it (the lane sums are exchanged with shuffles); the value is returned in thread t = 0.
SDTW_DEV float row_norm8(const float* row, int K, int t, bool ok) {
    if (K >= 8) {
        const int nvec = K / 8;
        const float part = ok ? aten_row_sum_sq(row + t, 8, nvec) : 0.0f;
        const int base = (int)(threadIdx.x & 63) & ~7;
        float lane[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) lane[j] = __shfl(part, base + j);
        float fa = 0.0f;
        if (ok && t == 0) {
            for (int e = nvec * 8; e < K; ++e) fa = __fadd_rn(fa, sq(row[e]));
#pragma unroll
            for (int j = 0; j < 8; ++j) fa = __fadd_rn(fa, lane[j]);
        }
        return fa;
    }
    return (ok && t == 0) ? __fadd_rn(0.0f, aten_row_sum_sq(row, 1, K)) : 0.0f;
}

// Norms of two row sets, eight threads per row, thread gid of the grid: rows [0, rows0) of
// v0 into out0, then rows1 more of v1 into out1.
SDTW_DEV void norms_at(int64_t gid, const float* __restrict__ v0, float* __restrict__ out0,
                       int64_t rows0, const float* __restrict__ v1, float* __restrict__ out1,
                       int64_t rows1, int K) {
    const int64_t r = gid >> 3;
    const int t = (int)(gid & 7);
    const bool first = r < rows0;
    const int64_t rr = first ? r : r - rows0;
    const bool ok = first || rr < rows1;
    const float* row = (first ? v0 : v1) + (ok ? rr : 0) * K;
    const float v = row_norm8(row, K, t, ok);
    if (ok && t == 0) (first ? out0 : out1)[rr] = v;
}

__global__ void __launch_bounds__(256) norms_kernel(const float* __restrict__ v0,
                                                    float* __restrict__ out0, int64_t rows0,
                                                    const float* __restrict__ v1,
                                                    float* __restrict__ out1, int64_t rows1,
                                                    int K) {
    norms_at((int64_t)blockIdx.x * blockDim.x + threadIdx.x, v0, out0, rows0, v1, out1, rows1, K);
}

// Blocks [0, prep_blocks) do the wavefront launch's prep work, the next zero_blocks zero the
// word ranges z0 and z1, the rest form the norms (each block takes one job whole, so the
// norms' shuffles stay within full waves).
__global__ void __launch_bounds__(256) prep_norms_kernel(
    int* ticket, int* err, unsigned long long* rows, int64_t nwords, unsigned long long lo,
    unsigned long long hi, int prep_blocks, int zero_blocks, unsigned* __restrict__ z0,
    int64_t n0, unsigned* __restrict__ z1, int64_t n1, const float* __restrict__ v0,
    float* __restrict__ out0, int64_t rows0, const float* __restrict__ v1,
    float* __restrict__ out1, int64_t rows1, int K) {
    const int b = (int)blockIdx.x;
    if (b < prep_blocks) {
        prep_rows((int64_t)b * blockDim.x + threadIdx.x, (int64_t)prep_blocks * blockDim.x,
                  ticket, err, rows, nwords, lo, hi);
        return;
    }
    if (b < prep_blocks + zero_blocks) {
        const int64_t stride = (int64_t)zero_blocks * blockDim.x;
        const int64_t idx = (int64_t)(b - prep_blocks) * blockDim.x + threadIdx.x;
        for (int64_t k = idx; k < n0; k += stride) z0[k] = 0u;
        for (int64_t k = idx; k < n1; k += stride) z1[k] = 0u;
        return;
    }
    norms_at((int64_t)(b - prep_blocks - zero_blocks) * blockDim.x + threadIdx.x, v0, out0, rows0,
             v1, out1, rows1, K);
}

hipError_t launch_prep_norms(int* ticket, int* err, unsigned long long* rows, int64_t nwords,
                             unsigned long long lo, unsigned long long hi, const float* x,
                             float* x2, int64_t rows_x, const float* y, float* y2,
                             int64_t rows_y, int K, unsigned* z0, int64_t n0, unsigned* z1,
                             int64_t n1, hipStream_t st) {
    int64_t prep = (nwords + 255) / 256;
    prep = prep < 1 ? 1 : (prep > 1024 ? 1024 : prep);
    if (!z0) n0 = 0;
    if (!z1) n1 = 0;
    const int64_t nz = n0 > n1 ? n0 : n1;
    int64_t zero = (nz + 255) / 256;
    zero = zero > 1024 ? 1024 : zero;
    const int64_t norm_blocks = ((rows_x + rows_y) * 8 + 255) / 256;
    hipLaunchKernelGGL(prep_norms_kernel, dim3((unsigned)(prep + zero + norm_blocks)), dim3(256), 0,
                       st, ticket, err, rows, nwords, lo, hi, (int)prep, (int)zero, z0, n0, z1, n1,
                       x, x2, rows_x, y, y2, rows_y, K);
    return hipGetLastError();
}

hipError_t launch_norms(const float* x, float* x2, int64_t rows_x, const float* y, float* y2,
                        int64_t rows_y, int K, hipStream_t st) {
    const int64_t rows = rows_x + rows_y;
    if (rows <= 0) return hipSuccess;
    const int64_t blocks = (rows * 8 + 255) / 256;
    hipLaunchKernelGGL(norms_kernel, dim3((unsigned)blocks), dim3(256), 0, st, x, x2, rows_x,
                       y, y2, rows_y, K);
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
    __shared__ float xn[DT], yn[DT];  // norms of the tile's rows of x and y
    // XCD-aware tile order (workgroups go to the 8 XCDs round-robin by linear id): the
    // tiles of one pair, which read the same rows of x and y, run on one XCD's L2
    const int gx = gridDim.x, gy = gridDim.y;
    const int nwg = gx * gy * gridDim.z;
    const int id = blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z);
    const int v = (nwg & 7) == 0 ? (id & 7) * (nwg >> 3) + (id >> 3) : id;
    const int b = v / (gx * gy);
    const int i0 = ((v / gx) % gy) * DT;
    const int j0 = (v % gx) * DT;
    const int tx = threadIdx.x & 15;
    const int ty = threadIdx.x >> 4;
    const int N = p.N, M = p.M, K = p.K;
    const float* xb = p.x + (int64_t)b * N * K;
    const float* yb = p.y + (int64_t)b * M * K;
    // the 128 row norms the tile needs, eight threads per row (visible after the first
    // barrier of the k loop)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int task = threadIdx.x + 256 * q;
        const int rr = task >> 3, t = task & 7;
        const bool isx = rr < DT;
        const int row = isx ? i0 + rr : j0 + (rr - DT);
        const bool ok = row < (isx ? N : M);
        const float v = row_norm8((isx ? xb : yb) + (int64_t)(ok ? row : 0) * K, K, t, ok);
        if (t == 0) (isx ? xn : yn)[rr & (DT - 1)] = v;
    }
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
    float* Db = p.D + (int64_t)b * N * M;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const int i = i0 + ty + 16 * m;
        if (i >= N) continue;
        const float xi = xn[ty + 16 * m];
#pragma unroll
        for (int n = 0; n < 4; ++n) {
            const int j = j0 + tx + 16 * n;
            if (j < M) Db[(int64_t)i * M + j] = clamp0(exact_cost_pre(xi, yn[tx + 16 * n], acc[m][n]));
        }
    }
}

typedef float floatx4_t __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------------------
// Exact distance on the matrix cores, for K <= 64.  A chain of v_mfma_f32_16x16x4_f32 over
// k = 0, 4, 8, ... from a zero accumulator computes each output as one sequential fp32 FMA
// chain over k (measured bit-identical on gfx950; the fused cost tiles rely on the same
// property), which is the order of the host GEMM, so D keeps the reference's bits.  Tiles
// 64 (rows of x) x 64 (rows of y); wave w owns rows 16w .. 16w + 15 against the four
// 16-column blocks (A operand x[16w + (l & 15)][k], B operand y[16nb + (l & 15)][k],
// k = 4s + (l >> 4)).  x and y tiles sit in LDS row-major with a row stride of XS = 68
// floats: the staging writes (consecutive k of a row) and the operand reads (16 rows at 4
// consecutive k: banks 4 (row mod 16) + k mod 4) each cover 64 distinct banks.  Padding rows,
// columns and features load as 0: fma(0, 0, acc) leaves a chain unchanged, and padding
// outputs are not stored.  The row norms are computed from the staged tiles (norms_kernel's
// arithmetic, so the same bits).
// ---------------------------------------------------------------------------------------
constexpr int KM = 64;
constexpr int XS = 68;

// ---------------------------------------------------------------------------------------
// A workgroup owns 64 rows of x of one pair (x stationary) and walks a run of the pair's
// 64-column tiles of y: the tiles are split into p.ysplit runs so that enough workgroups are
// in flight to hide each other's latency.  The x tile and its norms are staged once; the
// next y tile is loaded into registers while the matrix cores work on the current one, then
// stored into the other of two LDS buffers and its norms computed from LDS.  VEC: K % 4 == 0,
// rows are loaded as 16-byte vectors.
// ---------------------------------------------------------------------------------------
template <bool VEC>
__global__ void __launch_bounds__(256) dist_xs_kernel(DistParams p) {
    __shared__ __align__(16) float xs[DT * XS];
    __shared__ __align__(16) float ys[2][DT * XS];
    __shared__ float xn[DT], yn[2][DT];
    // workgroup = (pair, row block); XCD-aware order: the row blocks of a pair, which read
    // the same y, run on one XCD's L2
    const int nrb = (p.N + DT - 1) / DT;
    const int nwg = gridDim.x;
    const int id = blockIdx.x;
    const int v = (nwg & 7) == 0 ? (id & 7) * (nwg >> 3) + (id >> 3) : id;
    const int ys_ = p.ysplit;
    const int b = __builtin_amdgcn_readfirstlane(v / (nrb * ys_));
    const int i0 = __builtin_amdgcn_readfirstlane(((v / ys_) % nrb) * DT);
    const int part = __builtin_amdgcn_readfirstlane(v % ys_);
    const int l = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int N = p.N, M = p.M, K = p.K;
    const float* xb = p.x + (int64_t)b * N * K;
    const float* ybase = p.y + (int64_t)b * M * K;
    float* Db = p.D + (int64_t)b * N * M;
    // staging of 64 rows x 64 features: VEC, thread t takes row 4q + (t >> 4), features
    // 4 (t & 15) .. + 3 for q = 0..3; else element e = t + 256 q: row e / 64, feature e % 64
    float4 pre[4];
    auto load_tile = [&](const float* src, int r0, int rows) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            if (VEC) {
                const int r = 16 * q + (threadIdx.x >> 4), k = 4 * (threadIdx.x & 15);
                pre[q] = (r0 + r < rows && k < K)
                             ? *reinterpret_cast<const float4*>(src + (int64_t)(r0 + r) * K + k)
                             : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            } else {
                float e4[4];
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const int e = threadIdx.x + 256 * (4 * q + c);
                    const int r = e / KM, k = e % KM;
                    e4[c] = (r0 + r < rows && k < K) ? src[(int64_t)(r0 + r) * K + k] : 0.0f;
                }
                pre[q] = make_float4(e4[0], e4[1], e4[2], e4[3]);
            }
        }
    };
    auto store_tile = [&](float* dst) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            if (VEC) {
                const int r = 16 * q + (threadIdx.x >> 4), k = 4 * (threadIdx.x & 15);
                *reinterpret_cast<float4*>(dst + r * XS + k) = pre[q];
            } else {
                const float e4[4] = {pre[q].x, pre[q].y, pre[q].z, pre[q].w};
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const int e = threadIdx.x + 256 * (4 * q + c);
                    dst[(e / KM) * XS + e % KM] = e4[c];
                }
            }
        }
    };
    // norms of the 64 staged rows (eight threads per row, ATen's order; padding rows give 0)
    auto tile_norms = [&](const float* src, float* out) {
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int task = threadIdx.x + 256 * q;
            const int r = task >> 3, t = task & 7;
            const float nv = row_norm8(src + r * XS, K, t, true);
            if (t == 0) out[r] = nv;
        }
    };
    const int ntiles = (p.M + DT - 1) / DT;
    const int per = (ntiles + ys_ - 1) / ys_;
    const int jt0 = part * per, jt1 = min(ntiles, jt0 + per);
    load_tile(xb, i0, N);
    store_tile(xs);
    load_tile(ybase, jt0 * DT, M);
    store_tile(ys[0]);
    __syncthreads();
    tile_norms(xs, xn);
    tile_norms(ys[0], yn[0]);
    __syncthreads();
    const float* xa = xs + (16 * w + (l & 15)) * XS + (l >> 4);
    const int steps = (K + 3) / 4;
    for (int jt = jt0; jt < jt1; ++jt) {
        const int cur = (jt - jt0) & 1;
        if (jt + 1 < jt1) load_tile(ybase, (jt + 1) * DT, M);
        floatx4_t acc[4];
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) acc[nb] = floatx4_t{0.0f, 0.0f, 0.0f, 0.0f};
        const float* yb0 = ys[cur] + (l & 15) * XS + (l >> 4);
        auto kstep = [&](int s) {
            const float a = xa[4 * s];
            float bv[4];
#pragma unroll
            for (int nb = 0; nb < 4; ++nb) bv[nb] = yb0[16 * nb * XS + 4 * s];
#pragma unroll
            for (int nb = 0; nb < 4; ++nb)
                acc[nb] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, bv[nb], acc[nb], 0, 0, 0);
        };
        if (steps == KM / 4) {
#pragma unroll
            for (int s = 0; s < KM / 4; ++s) kstep(s);
        } else {
            for (int s = 0; s < steps; ++s) kstep(s);
        }
        // lane l holds rows 16w + 4 (l >> 4) + r of column 16nb + (l & 15)
        const int j0 = jt * DT;
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) {
            const int jl = 16 * nb + (l & 15);
            const int j = j0 + jl;
            const float y2 = yn[cur][jl];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int il = 16 * w + 4 * (l >> 4) + r;
                const int i = i0 + il;
                if (i < N && j < M) Db[(int64_t)i * M + j] = clamp0(exact_cost_pre(xn[il], y2, acc[nb][r]));
            }
        }
        if (jt + 1 < jt1) {
            store_tile(ys[cur ^ 1]);
            __syncthreads();
            tile_norms(ys[cur ^ 1], yn[cur ^ 1]);
            __syncthreads();
        }
    }
}

hipError_t launch_dist(const DistParams& p, bool muladd, bool mfma, hipStream_t st) {
    (void)mfma;
    if (muladd) {  // ATen's multiply-then-add kernel: not an FMA chain, so on the VALU
        dim3 grid((p.M + DT - 1) / DT, (p.N + DT - 1) / DT, p.B);
        hipLaunchKernelGGL(dist_kernel<true>, grid, dim3(256), 0, st, p);
    } else if (p.K <= KM) {
        DistParams q = p;
        const int64_t rows = (int64_t)p.B * ((p.N + DT - 1) / DT);
        const int64_t ntiles = (p.M + DT - 1) / DT;
        // about 2048 workgroups (at 3 resident per CU, latency is hidden; measured at the
        // headline: 27 us against 33 us with one workgroup per row block), runs of at least
        // one tile
        int64_t split = (2048 + rows - 1) / rows;
        split = split < 1 ? 1 : (split > ntiles ? ntiles : split);
        q.ysplit = (int)split;
        const int64_t wgs = rows * split;
        if (p.K % 4 == 0)
            hipLaunchKernelGGL(dist_xs_kernel<true>, dim3((unsigned)wgs), dim3(256), 0, st, q);
        else
            hipLaunchKernelGGL(dist_xs_kernel<false>, dim3((unsigned)wgs), dim3(256), 0, st, q);
    } else {  // K > 64: chunks of k through LDS on the VALU
        dim3 grid((p.M + DT - 1) / DT, (p.N + DT - 1) / DT, p.B);
        hipLaunchKernelGGL(dist_kernel<false>, grid, dim3(256), 0, st, p);
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------
// Distance backward.  Output rows r (x rows for gx, y rows for gy), reduction index t.
//   grad[r,k] = 2 * (W[r,k] * rs[r] - sum_t G'(r,t) Z[t,k]),   rs[r] = sum_t G'(r,t)
// TRANS = false: gx (W = x, Z = y, G'(r,t) = G[r,t]);  TRANS = true: gy (W = y, Z = x,
// G'(r,t) = G[t,r]).  G' is G with the clamp_min mask of the forward applied (cells whose
// pre-clamp value was negative get 0).
// ---------------------------------------------------------------------------------------
// Whether the clamp_min mask passes a cell whose clamped cost is 0: its pre-clamp value
// x2 + y2 - 2 x.y (recomputed with the forward's bits) is >= 0.  Rare (x_i ~ y_j).
template <bool MULADD>
SDTW_DEV bool clamp_passes(const DistBwdParams& p, int b, int i, int j) {
    const float dot = exact_dot<MULADD>(p.x + ((int64_t)b * p.N + i) * p.K, p.y + ((int64_t)b * p.M + j) * p.K, p.K);
    return exact_cost_pre(p.x2[(int64_t)b * p.N + i], p.y2[(int64_t)b * p.M + j], dot) >= 0.0f;
}

// Matrix-core version of the same product.  A workgroup (4 waves) owns 64 output rows x KT
// features (KT = 16, 32 or 64); wave w computes rows 16w..16w+15 with
// v_mfma_f32_16x16x4_f32.  The reduction index t advances in chunks of BT = 64.  A chunk
// is a 64 x 64 block of the (N, M) matrices G (and D, for the clamp mask) plus 64 rows of Z;
// each thread loads its part with 16-byte loads into registers, two chunks ahead of the one
// being multiplied, then stores it (masked) into one of two LDS buffers:
//   gx: G'(r, t) = G[r0 + r][t0 + t] stored gT[r][t], row stride 68 floats
//   gy: G'(r, t) = G[t0 + t][r0 + r] stored g[t][r],  row stride 80 floats
//   Z:  zs[t][k] = Z[t0 + t][k0 + k],                 row stride 80 floats
// With these strides the operand reads of a k-step (A: row 16w + (l & 15), t = 4kk +
// (l >> 4); B: t = 4kk + (l >> 4), feature 16kb + (l & 15)) touch 64 distinct banks.
// Row sums rs[r] are accumulated from the A operands.  The reduction order differs from the
// reference's matmul; gradients are compared within rtol 1e-4 / atol 1e-5.
constexpr int BT = 64;      // reduction chunk
constexpr int GS_X = 68;    // gx: LDS row stride of gT (floats)
constexpr int GS_Y = 80;    // gy: LDS row stride of g
constexpr int ZS = 80;      // LDS row stride of zs
constexpr int GBUF = 64 * 80;  // floats per G' buffer (the larger layout)
constexpr int ZBUF = 64 * ZS;  // floats per Z buffer

// Split reduction: z = b * ST + st (z after the XCD remap below); piece st takes chunks
// [st*cps, (st+1)*cps).
// With ST > 1 every piece stores W*rs - acc of its chunks as a partial (device-coherent
// stores), waits for them to complete and counts itself in the tile's counter; the last
// piece to arrive adds the ST partials in order 0..ST-1 (deterministic), writes the
// gradient and resets the counter to zero for the next launch.
struct DistBwdSmem {
    float gbuf[2][GBUF];
    float zbuf[2][ZBUF];
    int last_piece;
};

// One output tile: pair b, row strip by (64 rows of gx, or of gy when TRANS), feature tile
// bx (KT features), reduction piece st of ST.  ntx / nty: feature tiles / row strips of the
// pass (the tile's index among the pass's tiles).  flag_id: this workgroup's slot in
// p.flags (the gx pass of a masked two-launch call), or -1.
template <bool TRANS, int KT, bool MULADD, bool MASK>
SDTW_DEV void dist_bwd_tile(const DistBwdParams& p, int ST, int bx, int by, int b, int st,
                            int ntx, int nty, int flag_id, DistBwdSmem& sm) {
    constexpr int KB = KT / 16;          // 16-wide feature blocks per wave
    constexpr int ZQ = BT * KT / 1024;   // 16-byte Z loads per thread per chunk
    static_assert(ZQ >= 1, "feature tile must feed 256 threads");
    auto& gbuf = sm.gbuf;
    auto& zbuf = sm.zbuf;
    const int r0 = by * 64;
    const int k0 = bx * KT;
    const int tid = threadIdx.x, l = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int N = p.N, M = p.M, K = p.K;
    const int R_ = TRANS ? M : N;  // output rows
    const int T_ = TRANS ? N : M;  // reduction length
    const float* Gb = p.G + (int64_t)b * N * M;
    const float* Db = p.D ? p.D + (int64_t)b * N * M : nullptr;
    const float* Z = TRANS ? p.x + (int64_t)b * N * K : p.y + (int64_t)b * M * K;
    const float* W = TRANS ? p.y + (int64_t)b * M * K : p.x + (int64_t)b * N * K;
    float* out = TRANS ? p.gy + (int64_t)b * M * K : p.gx + (int64_t)b * N * K;
    const bool vec_g = (M & 3) == 0;  // 16-byte loads of G / D rows are aligned
    const bool vec_z = (K & 3) == 0;

    // this thread's elements of a chunk: block row e4 >> 4 (of 64), columns 4 (e4 & 15) ..+3,
    // e4 = tid + 256 q; Z: row e4 / (KT/4), features 4 (e4 % (KT/4)) ..+3
    struct Regs {
        float4 g[4], d[4], z[ZQ];
    };
    // Two load paths, chosen per workgroup at compile time (a loop mixing them would make
    // the compiler wait for every load in flight): FG, every chunk a full 64 x 64 block of
    // rows of length M % 4 == 0, loaded as 16-byte vectors; else element by element with
    // bounds.  ZF likewise for Z (K % 4 == 0 and K % KT == 0).  D is read only on the masked
    // path (MK).
    auto load_chunk = [&](int t0, Regs& R, auto fg_tag, auto zf_tag, auto mk_tag) {
        constexpr bool FG = decltype(fg_tag)::value, ZF = decltype(zf_tag)::value;
        constexpr bool MK = MASK && decltype(mk_tag)::value;
        const int a0 = TRANS ? t0 : r0, b0 = TRANS ? r0 : t0;  // block origin in (N, M)
        if (FG) {
            const int64_t base = (int64_t)(a0 + (tid >> 4)) * M + b0 + 4 * (tid & 15);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                R.g[q] = *reinterpret_cast<const float4*>(Gb + base + (int64_t)16 * q * M);
                R.d[q] = MK ? *reinterpret_cast<const float4*>(Db + base + (int64_t)16 * q * M)
                            : make_float4(1.f, 1.f, 1.f, 1.f);
            }
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int e4 = tid + 256 * q;
                const int ia = a0 + (e4 >> 4), jb = b0 + 4 * (e4 & 15);
                const int64_t row = (int64_t)min(ia, N - 1) * M;
                float gv[4], dv[4];
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    // unconditional load from a clamped index, then a select: a fixed number
                    // of loads per chunk keeps the compiler's load accounting exact
                    const bool ok = ia < N && jb + v < M;
                    const int64_t idx = row + min(jb + v, M - 1);
                    const float gl = Gb[idx];
                    gv[v] = ok ? gl : 0.0f;
                    if (MK) {
                        const float dl = Db[idx];
                        dv[v] = ok ? dl : 1.0f;
                    } else {
                        dv[v] = 1.0f;
                    }
                }
                R.g[q] = make_float4(gv[0], gv[1], gv[2], gv[3]);
                R.d[q] = make_float4(dv[0], dv[1], dv[2], dv[3]);
            }
        }
        if (ZF) {
#pragma unroll
            for (int q = 0; q < ZQ; ++q) {
                const int e4 = tid + 256 * q;
                R.z[q] = *reinterpret_cast<const float4*>(Z + (int64_t)(t0 + e4 / (KT / 4)) * K + k0 + 4 * (e4 % (KT / 4)));
            }
        } else {
#pragma unroll
            for (int q = 0; q < ZQ; ++q) {
                const int e4 = tid + 256 * q;
                const int zt = t0 + e4 / (KT / 4), zk = k0 + 4 * (e4 % (KT / 4));
                const int64_t row = (int64_t)min(zt, T_ - 1) * K;
                float zv[4];
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const float z = Z[row + min(zk + v, K - 1)];
                    zv[v] = (zt < T_ && zk + v < K) ? z : 0.0f;
                }
                R.z[q] = make_float4(zv[0], zv[1], zv[2], zv[3]);
            }
        }
    };
    // Masked G' and Z into LDS buffer `buf`.  Cells whose clamped cost is positive pass the
    // clamp_min mask, NaN ones do not.  A cost of exactly 0 passes only where the pre-clamp
    // value was >= 0: the first run (EXACT false) masks every cost that is not positive and
    // records that it saw one, and a workgroup that saw one reruns with the exact per-cell
    // check (loads of x and y rows inside the pipeline, hence slower).  Keeping loads out of
    // the first run lets the compiler wait on each chunk's loads alone.  The gx pass also
    // publishes that record per workgroup (p.flags): where no cost was non-positive, the mask
    // is the identity and the gy pass skips D.
    bool nonpos_seen = false;
    auto store_chunk = [&](int t0, const Regs& R, int buf, auto exact_tag, auto mk_tag) {
        constexpr bool MK = MASK && decltype(mk_tag)::value;
        constexpr bool EXACT = MK && decltype(exact_tag)::value;
        const int a0 = TRANS ? t0 : r0, b0 = TRANS ? r0 : t0;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int e4 = tid + 256 * q;
            const int br = e4 >> 4, bc = 4 * (e4 & 15);
            float g4[4] = {R.g[q].x, R.g[q].y, R.g[q].z, R.g[q].w};
            const float d4[4] = {R.d[q].x, R.d[q].y, R.d[q].z, R.d[q].w};
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int i = a0 + br, j = b0 + bc + v;
                if (EXACT) {
                    if (!(d4[v] > 0.0f) &&  // positive passes (also the padding, d = 1)
                        !(d4[v] == 0.0f && i < N && j < M && clamp_passes<MULADD>(p, b, i, j)))
                        g4[v] = 0.0f;
                } else if (MK) {  // selects only: no branch, no load
                    nonpos_seen |= !(d4[v] > 0.0f) && i < N && j < M;
                    g4[v] = d4[v] > 0.0f ? g4[v] : 0.0f;
                }
            }
            if (TRANS) {  // block row = t, columns = r: g[t][r..r+3]
                *reinterpret_cast<float4*>(&gbuf[buf][br * GS_Y + bc]) = make_float4(g4[0], g4[1], g4[2], g4[3]);
            } else {      // block row = r, columns = t: gT[r][t..t+3]
                *reinterpret_cast<float4*>(&gbuf[buf][br * GS_X + bc]) = make_float4(g4[0], g4[1], g4[2], g4[3]);
            }
        }
#pragma unroll
        for (int q = 0; q < ZQ; ++q) {
            const int e4 = tid + 256 * q;
            *reinterpret_cast<float4*>(&zbuf[buf][(e4 / (KT / 4)) * ZS + 4 * (e4 % (KT / 4))]) = R.z[q];
        }
    };

    floatx4_t acc[KB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) acc[kb] = floatx4_t{0.0f, 0.0f, 0.0f, 0.0f};
    float rs_part = 0.0f;  // row 16w + (l & 15), t = 4kk + (l >> 4) of every k-step
    // operands of k-step kk + 1 are read before the products of k-step kk are issued, so the
    // LDS latency overlaps the matrix pipe (the scheduling barriers keep that order)
    auto multiply = [&](int buf) {
        const float* gb = gbuf[buf];
        const float* zb = zbuf[buf];
        auto read_ops = [&](int kk, float& a, float* bv) {
            const int t = 4 * kk + (l >> 4), r = 16 * w + (l & 15);
            a = TRANS ? gb[t * GS_Y + r] : gb[r * GS_X + t];
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) bv[kb] = zb[t * ZS + 16 * kb + (l & 15)];
        };
        float a_c, b_c[KB];
        read_ops(0, a_c, b_c);
#pragma unroll
        for (int kk = 0; kk < BT / 4; ++kk) {
            float a_n = 0.0f, b_n[KB];
            if (kk + 1 < BT / 4) read_ops(kk + 1, a_n, b_n);
            __builtin_amdgcn_sched_barrier(0);
            rs_part += a_c;
#pragma unroll
            for (int kb = 0; kb < KB; ++kb)
                acc[kb] = __builtin_amdgcn_mfma_f32_16x16x4f32(a_c, b_c[kb], acc[kb], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            a_c = a_n;
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) b_c[kb] = b_n[kb];
        }
    };

    const int total = (T_ + BT - 1) / BT;
    const int cps = __builtin_amdgcn_readfirstlane((total + ST - 1) / ST);
    const int cbeg = __builtin_amdgcn_readfirstlane(min(st * cps, total));
    const int nchunks = __builtin_amdgcn_readfirstlane(min(cbeg + cps, total) - cbeg);
    // Pipeline: chunk c is stored from register set c & 1, whose loads for chunk c + 2 are
    // issued right after; the products of chunk c run from LDS buffer c & 1.  The steady
    // state loads unconditionally (a register set conditionally reloaded inside the loop
    // would be copied between iterations, and a copy waits for every load in flight); the
    // last two to three chunks are an explicit epilogue.
    auto run = [&](auto exact_tag, auto fg, auto zf, auto mk) {
        Regs ra, rb;
        if (nchunks > 0) load_chunk(cbeg * BT, ra, fg, zf, mk);
        if (nchunks > 1) load_chunk((cbeg + 1) * BT, rb, fg, zf, mk);
        int c = 0;
        for (; c + 3 < nchunks; c += 2) {
            store_chunk((cbeg + c) * BT, ra, 0, exact_tag, mk);
            load_chunk((cbeg + c + 2) * BT, ra, fg, zf, mk);
            __syncthreads();
            multiply(0);
            store_chunk((cbeg + c + 1) * BT, rb, 1, exact_tag, mk);
            load_chunk((cbeg + c + 3) * BT, rb, fg, zf, mk);
            __syncthreads();
            multiply(1);
        }
        const int rem = nchunks - c;  // 0 .. 3
        if (rem >= 1) {
            store_chunk((cbeg + c) * BT, ra, 0, exact_tag, mk);
            if (rem == 3) load_chunk((cbeg + c + 2) * BT, ra, fg, zf, mk);
            __syncthreads();
            multiply(0);
        }
        if (rem >= 2) {
            store_chunk((cbeg + c + 1) * BT, rb, 1, exact_tag, mk);
            __syncthreads();
            multiply(1);
        }
        if (rem == 3) {
            store_chunk((cbeg + c + 2) * BT, ra, 0, exact_tag, mk);
            __syncthreads();
            multiply(0);
        }
    };
    const bool fg = vec_g && r0 + 64 <= R_ && T_ % BT == 0;
    const bool zf = vec_z && K % KT == 0 && T_ % BT == 0;
    auto run_any = [&](auto exact_tag, auto mk) {
        if (fg && zf) run(exact_tag, std::true_type{}, std::true_type{}, mk);
        else if (fg) run(exact_tag, std::true_type{}, std::false_type{}, mk);
        else run(exact_tag, std::false_type{}, std::false_type{}, mk);
    };
    // the mask is needed only for a pair whose forward saw a cost that was not positive (where
    // the forward recorded it), else, in the gy pass, only if the gx pass saw one
    bool use_mask = MASK;
    if (MASK && p.clamped) {
        use_mask = __builtin_amdgcn_readfirstlane(p.clamped[b]) != 0;
    } else if (MASK && TRANS && p.flags) {
        int any = 0;
        for (int f = tid; f < p.nflags; f += 256) any |= p.flags[f];
        use_mask = __syncthreads_or(any);
    }
    int nonpos = 0;
    if (use_mask) {
        run_any(std::false_type{}, std::true_type{});
        nonpos = __syncthreads_or(nonpos_seen);
        if (nonpos) {  // rare: rerun the tile with the exact mask
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) acc[kb] = floatx4_t{0.0f, 0.0f, 0.0f, 0.0f};
            rs_part = 0.0f;
            run_any(std::true_type{}, std::true_type{});
        }
    } else {
        run_any(std::false_type{}, std::false_type{});
    }
    if (MASK && !TRANS && p.flags && flag_id >= 0 && tid == 0) p.flags[flag_id] = nonpos;

    // rs of row 16w + x: sum of the four lanes with (l & 15) == x
    float rs = rs_part + __shfl_xor(rs_part, 16);
    rs = rs + __shfl_xor(rs, 32);
    // lane l holds outputs (row 16w + 4(l >> 4) + v, feature k0 + 16kb + (l & 15))
    float val[4][KB];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const int rl = 4 * (l >> 4) + v;
        const float rsv = __shfl(rs, rl);
        const int r = min(r0 + 16 * w + rl, R_ - 1);
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
            const int k = min(k0 + 16 * kb + (l & 15), K - 1);
            val[v][kb] = W[(int64_t)r * K + k] * rsv - acc[kb][v];
        }
    }
    if (ST > 1) {
        // the passes' scratch regions are disjoint: gx first, then gy
        const int64_t tile = ((int64_t)b * nty + by) * ntx + bx;
        float* part = p.part + (TRANS ? dist_bwd_split_floats_x(p.B, p.N, p.M, p.K) : 0) + tile * ST * 64 * KT;
        int* cnt = p.cnt + (TRANS ? dist_bwd_tiles(p.B, p.N, p.K) : 0);
        // partial of piece st: element (row 16w + 4(l>>4) + v, feature 16kb + (l&15))
        auto pidx = [&](int q, int v, int kb) {
            return ((int64_t)q * 64 + 16 * w + 4 * (l >> 4) + v) * KT + 16 * kb + (l & 15);
        };
#pragma unroll
        for (int v = 0; v < 4; ++v)
#pragma unroll
            for (int kb = 0; kb < KB; ++kb)
                __hip_atomic_store(part + pidx(st, v, kb), val[v][kb], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): this thread's partials are stored
        __syncthreads();
        if (tid == 0)
            sm.last_piece = __hip_atomic_fetch_add(cnt + tile, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == ST - 1;
        __syncthreads();
        if (!sm.last_piece) return;
#pragma unroll
        for (int v = 0; v < 4; ++v)
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) {
                float sum = 0.0f;
                for (int q = 0; q < ST; ++q)
                    sum += __hip_atomic_load(part + pidx(q, v, kb), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                val[v][kb] = sum;
            }
        if (tid == 0) __hip_atomic_store(cnt + tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const int r = r0 + 16 * w + 4 * (l >> 4) + v;
        if (r >= R_) continue;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
            const int k = k0 + 16 * kb + (l & 15);
            if (k < K) out[(int64_t)r * K + k] = 2.0f * val[v][kb];
        }
    }
}

// One pass, grid (feature tiles, row strips, B * ST).  Workgroups are dispatched to the 8
// XCDs round-robin by linear id; the id is remapped so that consecutive tiles (the row strips
// of one pair, which read the same Z) run on the same XCD and share its L2.
template <bool TRANS, int KT, bool MULADD, bool MASK>
__global__ void __launch_bounds__(256) dist_bwd_mfma_kernel(DistBwdParams p, int ST) {
    __shared__ __align__(16) DistBwdSmem sm;
    const int ntx = gridDim.x, nty = gridDim.y;
    const int nwg = ntx * nty * gridDim.z;
    const int id = blockIdx.x + ntx * (blockIdx.y + nty * blockIdx.z);
    const int v = (nwg & 7) == 0 ? (id & 7) * (nwg >> 3) + (id >> 3) : id;
    // integer divisions expand to vector code: pin the (uniform) results to scalar registers
    // so that the pipeline loop is a uniform loop
    const int bx = __builtin_amdgcn_readfirstlane(v % ntx);
    const int by = __builtin_amdgcn_readfirstlane((v / ntx) % nty);
    const int bz = __builtin_amdgcn_readfirstlane(v / (ntx * nty));
    const int b = __builtin_amdgcn_readfirstlane(bz / ST), st = bz - b * ST;
    dist_bwd_tile<TRANS, KT, MULADD, MASK>(p, ST, bx, by, b, st, ntx, nty, id, sm);
}

// Both passes in one launch, tiles in pair-major order: pair b's gx tiles (STX pieces each),
// then its gy tiles (STY pieces).  With the XCD remap of linear ids, a pair's tiles of both
// passes run together on one XCD, so the pass that reads a G block second finds it in that
// XCD's L2 (a pair's G, N*M*4 bytes, against 4 MiB of L2) rather than in HBM.  Used where the
// gy pass does not wait on the gx pass's mask record: no mask, or per-pair clamp records
// from the forward.
template <int KT, bool MULADD, bool MASK>
__global__ void __launch_bounds__(256) dist_bwd_merged_kernel(DistBwdParams p, int STX, int STY) {
    __shared__ __align__(16) DistBwdSmem sm;
    const int ntx = (p.K + KT - 1) / KT;
    const int rx = (p.N + 63) / 64, ry = (p.M + 63) / 64;
    const int tx = ntx * rx * STX, ty = ntx * ry * STY;  // tiles per pair of each pass
    const int nwg = gridDim.x;
    const int id = blockIdx.x;
    const int v = (nwg & 7) == 0 ? (id & 7) * (nwg >> 3) + (id >> 3) : id;
    const int b = __builtin_amdgcn_readfirstlane(v / (tx + ty));
    const int k = __builtin_amdgcn_readfirstlane(v - b * (tx + ty));
    if (k < tx) {
        const int bx = __builtin_amdgcn_readfirstlane(k % ntx);
        const int by = __builtin_amdgcn_readfirstlane((k / ntx) % rx);
        const int st = __builtin_amdgcn_readfirstlane(k / (ntx * rx));
        dist_bwd_tile<false, KT, MULADD, MASK>(p, STX, bx, by, b, st, ntx, rx, -1, sm);
    } else {
        const int kk = k - tx;
        const int bx = __builtin_amdgcn_readfirstlane(kk % ntx);
        const int by = __builtin_amdgcn_readfirstlane((kk / ntx) % ry);
        const int st = __builtin_amdgcn_readfirstlane(kk / (ntx * ry));
        dist_bwd_tile<true, KT, MULADD, MASK>(p, STY, bx, by, b, st, ntx, ry, -1, sm);
    }
}

__global__ void zero_ints_kernel(int* p, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        p[i] = 0;
}

template <bool TRANS, bool MULADD>
static void launch_dist_bwd_one(const DistBwdParams& p, hipStream_t st) {
    const int R_ = TRANS ? p.M : p.N, T_ = TRANS ? p.N : p.M;
    const int KT = dist_bwd_kt(p.K);
    const int ST = p.part ? dist_bwd_splits(p.B, R_, T_, p.K) : 1;
    dim3 grid((p.K + KT - 1) / KT, (R_ + 63) / 64, p.B * ST);
    if (p.mask) {
        if (KT == 16)
            hipLaunchKernelGGL((dist_bwd_mfma_kernel<TRANS, 16, MULADD, true>), grid, dim3(256), 0, st, p, ST);
        else if (KT == 32)
            hipLaunchKernelGGL((dist_bwd_mfma_kernel<TRANS, 32, MULADD, true>), grid, dim3(256), 0, st, p, ST);
        else
            hipLaunchKernelGGL((dist_bwd_mfma_kernel<TRANS, 64, MULADD, true>), grid, dim3(256), 0, st, p, ST);
    } else {
        if (KT == 16)
            hipLaunchKernelGGL((dist_bwd_mfma_kernel<TRANS, 16, MULADD, false>), grid, dim3(256), 0, st, p, ST);
        else if (KT == 32)
            hipLaunchKernelGGL((dist_bwd_mfma_kernel<TRANS, 32, MULADD, false>), grid, dim3(256), 0, st, p, ST);
        else
            hipLaunchKernelGGL((dist_bwd_mfma_kernel<TRANS, 64, MULADD, false>), grid, dim3(256), 0, st, p, ST);
    }
}

template <bool MULADD>
static void launch_dist_bwd_merged(const DistBwdParams& p, hipStream_t st) {
    const int KT = dist_bwd_kt(p.K);
    const int STX = p.part ? dist_bwd_splits(p.B, p.N, p.M, p.K) : 1;
    const int STY = p.part ? dist_bwd_splits(p.B, p.M, p.N, p.K) : 1;
    const int64_t ntx = (p.K + KT - 1) / KT;
    const int64_t tiles = (int64_t)p.B * ntx * (((p.N + 63) / 64) * STX + ((p.M + 63) / 64) * STY);
    const dim3 grid((unsigned)tiles);
    if (p.mask) {
        if (KT == 16)
            hipLaunchKernelGGL((dist_bwd_merged_kernel<16, MULADD, true>), grid, dim3(256), 0, st, p, STX, STY);
        else if (KT == 32)
            hipLaunchKernelGGL((dist_bwd_merged_kernel<32, MULADD, true>), grid, dim3(256), 0, st, p, STX, STY);
        else
            hipLaunchKernelGGL((dist_bwd_merged_kernel<64, MULADD, true>), grid, dim3(256), 0, st, p, STX, STY);
    } else {
        if (KT == 16)
            hipLaunchKernelGGL((dist_bwd_merged_kernel<16, MULADD, false>), grid, dim3(256), 0, st, p, STX, STY);
        else if (KT == 32)
            hipLaunchKernelGGL((dist_bwd_merged_kernel<32, MULADD, false>), grid, dim3(256), 0, st, p, STX, STY);
        else
            hipLaunchKernelGGL((dist_bwd_merged_kernel<64, MULADD, false>), grid, dim3(256), 0, st, p, STX, STY);
    }
}

hipError_t launch_dist_bwd(const DistBwdParams& p, hipStream_t st) {
    const bool split = p.part && (dist_bwd_splits(p.B, p.N, p.M, p.K) > 1 || dist_bwd_splits(p.B, p.M, p.N, p.K) > 1);
    if (split) {  // counters start at zero; every pass leaves them at zero
        const int64_t n = dist_bwd_counters(p.B, p.N, p.M, p.K);
        const int blocks = (int)((n + 255) / 256 < 1024 ? (n + 255) / 256 : 1024);
        hipLaunchKernelGGL(zero_ints_kernel, dim3(blocks > 0 ? blocks : 1), dim3(256), 0, st, p.cnt, n);
    }
    // both gradients, and no mask record to pass from the gx pass to the gy pass: one launch
    if (p.gx && p.gy && (!p.mask || p.clamped)) {
        DistBwdParams q = p;
        q.flags = nullptr;
        if (q.muladd) launch_dist_bwd_merged<true>(q, st);
        else launch_dist_bwd_merged<false>(q, st);
        return hipGetLastError();
    }
    // with the mask, the gx pass writes one flag per workgroup, which the gy pass reads; a
    // null gx or gy skips that pass (a gy pass without a gx pass applies the full mask)
    DistBwdParams q = p;
    if (!q.mask || !q.gx) q.flags = nullptr;
    q.nflags = (int)(dist_bwd_tiles(p.B, p.N, p.K) * (p.part ? dist_bwd_splits(p.B, p.N, p.M, p.K) : 1));
    if (q.muladd) {
        if (q.gx) launch_dist_bwd_one<false, true>(q, st);
        if (q.gy) launch_dist_bwd_one<true, true>(q, st);
    } else {
        if (q.gx) launch_dist_bwd_one<false, false>(q, st);
        if (q.gy) launch_dist_bwd_one<true, false>(q, st);
    }
    return hipGetLastError();
}

}  // namespace sdtw
