// sdtw_dp.hip -- Soft-DTW forward / backward wavefront kernels for gfx950.
//
// Layout and schedule
//   * One workgroup per pair b.  The workgroup's T lanes (T = 64 * waves) own T consecutive
//     rows of the DP table (a "row block"); lane l owns row i = i0 + l.  Row blocks are
//     swept top to bottom (forward) or bottom to top (backward).
//   * Inside a row block the lanes walk the anti-diagonals: at step s lane l updates cell
//     (i0 + l, s - l).  A cell's upper neighbours were produced by lane l-1 one and two
//     steps earlier; they arrive through a two-slot LDS ring, one barrier per step.  The
//     left neighbour is the lane's own previous value (a register).
//   * Between row blocks the last lane's fp64 values (forward) or (E, R, D) triples
//     (backward) are handed over through a small per-pair "edge" array in the workspace.
//   * R is written as fp32 (B, N, M); the recursion itself runs in fp64, so R is rounded
//     exactly once per cell, as in the reference CPU path (launcher.py:310, :359).
//
// The cost of a cell comes from a materialised D (unfused) or is recomputed from x, y with
// the exact-distance arithmetic (fused); see sdtw_device.hpp.
#include "sdtw_device.hpp"
#include "sdtw_internal.hpp"

namespace sdtw {

struct CostD {
    const float* D;  // (N, M) of this pair
    int M;
    SDTW_DEV float operator()(int i, int j) const { return D[(int64_t)i * M + j]; }
};

template <bool MULADD>
struct CostXY {
    const float* x;   // (N, K) of this pair
    const float* y;   // (M, K)
    const float* x2;  // (N)
    const float* y2;  // (M)
    int K;
    SDTW_DEV float operator()(int i, int j) const {
        const float dot = exact_dot<MULADD>(x + (int64_t)i * K, y + (int64_t)j * K, K);
        return clamp0(exact_cost_pre(x2[i], y2[j], dot));
    }
};

// ---------------------------------------------------------------------------------------
// Forward
// ---------------------------------------------------------------------------------------
template <class Cost>
SDTW_DEV void fwd_pair(const Cost& cost, float* __restrict__ Rb, float* __restrict__ outb,
                       double* __restrict__ edge, int N, int M, double gamma, double bw) {
    extern __shared__ double xch[];  // [2][T]
    const int T = blockDim.x;
    const int l = threadIdx.x;
    const double INF = dinf();
    for (int i0 = 0; i0 < N; i0 += T) {
        const int rows = min(T, N - i0);
        const int i = i0 + l;
        const bool has_row = l < rows;
        const bool more_rows = i0 + rows < N;
        xch[T + l] = INF;  // slot read at step 0
        __syncthreads();
        double left = INF;                                // R[i, j-1]; column -1 is +inf
        double diag = (l == 0 && i0 == 0) ? 0.0 : INF;    // R[i-1, j-1] at the first step
        const int nsteps = rows + M - 1;
        for (int s = 0; s < nsteps; ++s) {
            const int j = s - l;
            double up;
            if (l == 0)
                up = (i0 > 0 && j < M) ? edge[j] : INF;   // row -1 is +inf except R[-1,-1]=0
            else
                up = xch[((s + 1) & 1) * T + (l - 1)];
            double r = INF;
            const bool act = has_row && j >= 0 && j < M;
            if (act) {
                if (!out_of_band(bw, i, j)) r = (double)cost(i, j) + softmin3(diag, up, left, gamma);
                Rb[(int64_t)i * M + j] = (float)r;
                left = r;
                if (more_rows && l == rows - 1) edge[j] = r;
                if (i == N - 1 && j == M - 1) *outb = (float)r;
            }
            diag = up;
            xch[(s & 1) * T + l] = r;
            __syncthreads();
        }
    }
}

__global__ void __launch_bounds__(1024) fwd_kernel(FwdParams p) {
    const int b = blockIdx.x;
    CostD cost{p.D + (int64_t)b * p.N * p.M, p.M};
    fwd_pair(cost, p.R + (int64_t)b * p.N * p.M, p.out + b, p.edge + (int64_t)b * p.M, p.N,
             p.M, p.gamma, p.bw);
}

template <bool MULADD>
__global__ void __launch_bounds__(1024) fused_fwd_kernel(FwdParams p) {
    const int b = blockIdx.x;
    CostXY<MULADD> cost{p.x + (int64_t)b * p.N * p.K, p.y + (int64_t)b * p.M * p.K,
                        p.x2 + (int64_t)b * p.N, p.y2 + (int64_t)b * p.M, p.K};
    fwd_pair(cost, p.R + (int64_t)b * p.N * p.M, p.out + b, p.edge + (int64_t)b * p.M, p.N,
             p.M, p.gamma, p.bw);
}

// ---------------------------------------------------------------------------------------
// Backward
//
// Reverse step q, lane l (row i = i0 + l of a block of `rows` rows) visits column
//   j = (M - 1) - q + (rows - 1 - l).
// Neighbours of (i, j): down (i+1, j) from lane l+1 one step ago, right (i, j+1) is the
// lane's own previous cell, diag (i+1, j+1) from lane l+1 two steps ago.  Cells outside the
// table carry the reference's padding: R = -inf, D = 0, E = 0, except the corner
// (N, M) which carries (E=1, R=R[N-1,M-1] as stored, D=0)  (launcher.py:330-338).
// Every visited cell first maps R=+inf to -inf (launcher.py:343-344), also outside the band.
// ---------------------------------------------------------------------------------------
template <class Cost, bool WRITE_G>
SDTW_DEV void bwd_pair(const Cost& cost, const float* __restrict__ Rb, float g,
                       float* __restrict__ Gb, float* __restrict__ edge, int N, int M,
                       double gamma, double bw) {
    extern __shared__ float xchf[];  // [2][3][T]
    const int T = blockDim.x;
    const int l = threadIdx.x;
    const float NINF = -finf();
    const Nbr pad{0.0f, NINF, 0.0f};
    float* eE = edge;          // [M+1]
    float* eR = edge + (M + 1);
    float* eD = edge + 2 * (M + 1);
    const float corner_R = Rb[(int64_t)(N - 1) * M + (M - 1)];
    // Walk row blocks from the bottom.
    const int nblocks = (N + T - 1) / T;
    for (int blk = nblocks - 1; blk >= 0; --blk) {
        const int i0 = blk * T;
        const int rows = min(T, N - i0);
        const int i = i0 + l;
        const bool has_row = l < rows;
        const bool last_block = (i0 + rows == N);
        // edge value below this block at column jj (jj in [0, M])
        auto below = [&](int jj) -> Nbr {
            if (last_block) {
                if (jj == M) return Nbr{1.0f, corner_R, 0.0f};
                return pad;
            }
            return Nbr{eE[jj], eR[jj], eD[jj]};
        };
        xchf[(1 * 3 + 0) * T + l] = pad.E;
        xchf[(1 * 3 + 1) * T + l] = pad.R;
        xchf[(1 * 3 + 2) * T + l] = pad.D;
        __syncthreads();
        Nbr right = pad;
        Nbr diag = (l == rows - 1) ? below(M) : pad;
        const int nsteps = rows + M - 1;
        for (int q = 0; q < nsteps; ++q) {
            const int j = (M - 1) - q + (rows - 1 - l);
            Nbr down;
            if (l == rows - 1) {
                down = (j >= 0 && j < M) ? below(j) : pad;
            } else if (l < rows - 1) {
                const int sl = ((q + 1) & 1) * 3;
                down = Nbr{xchf[(sl + 0) * T + l + 1], xchf[(sl + 1) * T + l + 1],
                           xchf[(sl + 2) * T + l + 1]};
            } else {
                down = pad;
            }
            Nbr me = pad;
            const bool act = has_row && j >= 0 && j < M;
            if (act) {
                float rij = Rb[(int64_t)i * M + j];
                if (__builtin_isinf(rij)) rij = NINF;
                const float dij = cost(i, j);
                float e = 0.0f;
                if (!out_of_band(bw, i, j)) e = bwd_cell(rij, down, right, diag, gamma);
                if (WRITE_G) Gb[(int64_t)i * M + j] = __fmul_rn(g, e);
                me = Nbr{e, rij, dij};
                right = me;
                if (l == 0 && i0 > 0) {  // hand the block's first row to the block above
                    eE[j] = me.E;
                    eR[j] = me.R;
                    eD[j] = me.D;
                }
            }
            diag = down;
            const int so = (q & 1) * 3;
            xchf[(so + 0) * T + l] = me.E;
            xchf[(so + 1) * T + l] = me.R;
            xchf[(so + 2) * T + l] = me.D;
            __syncthreads();
        }
        // the block above reads the pad value at column M of the edge
        if (l == 0 && i0 > 0) {
            eE[M] = pad.E;
            eR[M] = pad.R;
            eD[M] = pad.D;
        }
        __syncthreads();
    }
}

__global__ void __launch_bounds__(1024) bwd_kernel(BwdParams p) {
    const int b = blockIdx.x;
    const float g = p.gout ? p.gout[b] : 1.0f;
    CostD cost{p.D + (int64_t)b * p.N * p.M, p.M};
    bwd_pair<CostD, true>(cost, p.R + (int64_t)b * p.N * p.M, g, p.G + (int64_t)b * p.N * p.M,
                          p.edge + (int64_t)b * 3 * (p.M + 1), p.N, p.M, p.gamma, p.bw);
}

template <bool MULADD>
__global__ void __launch_bounds__(1024) fused_bwd_kernel(BwdParams p) {
    const int b = blockIdx.x;
    const float g = p.gout ? p.gout[b] : 1.0f;
    CostXY<MULADD> cost{p.x + (int64_t)b * p.N * p.K, p.y + (int64_t)b * p.M * p.K,
                        p.x2 + (int64_t)b * p.N, p.y2 + (int64_t)b * p.M, p.K};
    bwd_pair<CostXY<MULADD>, true>(cost, p.R + (int64_t)b * p.N * p.M, g,
                                   p.G + (int64_t)b * p.N * p.M,
                                   p.edge + (int64_t)b * 3 * (p.M + 1), p.N, p.M, p.gamma,
                                   p.bw);
}

// ---------------------------------------------------------------------------------------
// Launchers
// ---------------------------------------------------------------------------------------
static int block_threads(int64_t N) {
    int64_t t = ((N + 63) / 64) * 64;
    if (t > 1024) t = 1024;
    if (t < 64) t = 64;
    return (int)t;
}

hipError_t launch_fwd(const FwdParams& p, bool fused, bool muladd, hipStream_t st) {
    const int T = block_threads(p.N);
    const size_t lds = sizeof(double) * 2 * T;
    if (!fused)
        hipLaunchKernelGGL(fwd_kernel, dim3(p.B), dim3(T), lds, st, p);
    else if (muladd)
        hipLaunchKernelGGL(fused_fwd_kernel<true>, dim3(p.B), dim3(T), lds, st, p);
    else
        hipLaunchKernelGGL(fused_fwd_kernel<false>, dim3(p.B), dim3(T), lds, st, p);
    return hipGetLastError();
}

hipError_t launch_bwd(const BwdParams& p, bool fused, bool muladd, hipStream_t st) {
    const int T = block_threads(p.N);
    const size_t lds = sizeof(float) * 6 * T;
    if (!fused)
        hipLaunchKernelGGL(bwd_kernel, dim3(p.B), dim3(T), lds, st, p);
    else if (muladd)
        hipLaunchKernelGGL(fused_bwd_kernel<true>, dim3(p.B), dim3(T), lds, st, p);
    else
        hipLaunchKernelGGL(fused_bwd_kernel<false>, dim3(p.B), dim3(T), lds, st, p);
    return hipGetLastError();
}

}  // namespace sdtw
