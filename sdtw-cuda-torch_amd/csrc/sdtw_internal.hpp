// sdtw_internal.hpp -- parameter blocks and launcher declarations shared by the .hip files.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sdtw {

// Polls a bounded inter-wave wait makes before it gives up (about 0.3 s of no progress).
constexpr unsigned kDefaultSpinLimit = 1u << 22;

// Parameters of the wavefront kernels (forward and backward share one block).
struct DPParams {
    const float* D;     // unfused cost (B,N,M) or nullptr
    const float* x;     // fused: (B,N,K)
    const float* y;     // fused: (B,M,K)
    const float* x2;    // fused: row norms (B,N)
    const float* y2;    // fused: row norms (B,M)
    float* R;           // band-skewed table: forward writes, backward reads
    float* out;         // (B) forward result
    float* G_out;       // backward: (B,N,M) = gout * E, or nullptr (gradient mode)
    // Fused backward, gradient mode (G_out null): the gradients formed in the kernel from the
    // E tiles, never materialising (B,N,M).  gx_out: dL/dx (B,N,K); gy_out: dL/dy (B,M,K),
    // zeroed by the prep launch and accumulated band by band.  Null = not wanted.
    float* gx_out;
    float* gy_out;
    const float* gout;  // backward: (B) upstream gradient or nullptr (= 1)
    float* D_out;       // fused forward: the cost tiles also stored here (B,N,M), or nullptr
    int* clamped;       // with D_out: per pair, set to 1 if a stored cost is not positive
                        // (0 or NaN: the distance backward's clamp mask is then not the
                        // identity); zeroed by the prep launch.  Or nullptr.
    float* x2_fill;     // fused: x2 / y2 (writable) for the prep launch to form, or nullptr
    float* y2_fill;
    int* ticket;        // workgroup ticket counter (zeroed by the prep kernel)
    double* gring;      // forward: (B*G, RW) fp64 last rows of each workgroup's bands
    float4* gring4;     // backward: (B*G, RW) (E, R, D, tag) first rows
    int RW;             // entries per cross-workgroup row: M plus 64 of padding each side
    int* err;           // spin-timeout flag
    unsigned spin_limit;  // polls a bounded wait makes before it gives up (kDefaultSpinLimit)
    int B, N, M, K;
    int lin;            // forward under mixed arithmetic, matrix-core costs, no band, W <= 2:
                        // pairs whose costs allow it run the scaled linear-domain recursion
                        // (fwd_band_lin)
    int ww;             // backward with costs read from D, W == 1: two weight waves per band
                        // form each cell's three weights ahead of the compute wave
                        // (bwd_weight_wave); 1 under hardware exp2, 2 under exact arithmetic
                        // (the stage's planes, set by the launch)
    int nb, W, G;       // 64-row bands per pair, waves per workgroup, workgroups per pair
    int S;              // steps per band in the R table (dp_band_steps(M))
    double gamma, inv_gamma, bw;
};

struct DistParams {
    const float* x;  // (B,N,K)
    const float* y;  // (B,M,K)
    float* D;        // (B,N,M)
    int B, N, M, K;
    int ysplit;      // runs of y tiles per row block (x-stationary kernel)
};

struct DistBwdParams {
    const float* x;
    const float* y;
    const float* x2;  // norms (for the clamp mask)
    const float* y2;
    const float* D;   // clamped forward cost (mask) or nullptr
    const float* G;   // (B,N,M)
    float* gx;        // (B,N,K)
    float* gy;        // (B,M,K)
    int B, N, M, K;
    int mask;
    int muladd;
    float* part;      // split-reduction partials (dist_bwd_split_floats) or nullptr
    int* cnt;         // per-tile arrival counters (dist_bwd_counters ints), or nullptr
    int* flags;       // mask: per gx-pass workgroup "a cost was not positive" (dist_bwd_flags)
    int nflags;
    const int* clamped;  // mask: per pair "a cost was not positive" from the forward, or
                         // nullptr (unknown: the mask reads D)
};

// Split reduction of the distance backward: the reduction of a 64-row x KT-feature output
// tile is cut into dist_bwd_splits() pieces (of whole 64-wide chunks) so that about 256
// workgroups, one per CU, are in flight.
__host__ __device__ inline int dist_bwd_kt(int64_t K) { return K <= 16 ? 16 : (K <= 32 ? 32 : 64); }
__host__ __device__ inline int64_t dist_bwd_tiles(int64_t B, int64_t R, int64_t K) {
    return B * ((R + 63) / 64) * ((K + dist_bwd_kt(K) - 1) / dist_bwd_kt(K));
}
__host__ __device__ inline int dist_bwd_splits(int64_t B, int64_t R, int64_t T, int64_t K) {
    const int64_t tiles = dist_bwd_tiles(B, R, K);
    const int64_t chunks = (T + 63) / 64;
    int64_t st = (256 + tiles - 1) / tiles;
    st = st > 8 ? 8 : st;
    st = st > chunks ? chunks : st;
    return (int)(st < 1 ? 1 : st);
}
// scratch floats / counters of the two passes (gx over N rows first, then gy over M rows:
// disjoint, since the passes may run in one launch)
__host__ __device__ inline int64_t dist_bwd_split_floats_x(int64_t B, int64_t N, int64_t M, int64_t K) {
    const int st = dist_bwd_splits(B, N, M, K);
    return st > 1 ? dist_bwd_tiles(B, N, K) * st * 64 * dist_bwd_kt(K) : 0;  // unsplit: none
}
__host__ __device__ inline int64_t dist_bwd_split_floats(int64_t B, int64_t N, int64_t M, int64_t K) {
    return dist_bwd_split_floats_x(B, N, M, K) + dist_bwd_split_floats_x(B, M, N, K);
}
__host__ __device__ inline int64_t dist_bwd_counters(int64_t B, int64_t N, int64_t M, int64_t K) {
    return dist_bwd_tiles(B, N, K) + dist_bwd_tiles(B, M, K);
}
// workgroups of the gx pass (tiles times reduction pieces), one flag each
inline int64_t dist_bwd_flags(int64_t B, int64_t N, int64_t M, int64_t K) {
    return dist_bwd_tiles(B, N, K) * dist_bwd_splits(B, N, M, K);
}

// The prep work of one thread of a grid of `stride` threads: thread 0 zeroes the workgroup
// ticket and the error flag; every thread marks its share of the cross-workgroup rows empty
// (forward rows: one 64-bit word per entry, lo == hi; backward rows: the words (E,R) and
// (D,tag) of each entry, lo and hi).
__device__ inline void prep_rows(int64_t idx, int64_t stride, int* ticket, int* err,
                                 unsigned long long* rows, int64_t nwords,
                                 unsigned long long lo, unsigned long long hi) {
    if (idx == 0) {
        *ticket = 0;
        *err = 0;
    }
    for (int64_t k = idx; k < nwords; k += stride) rows[k] = (k & 1) ? hi : lo;
}
// The prep work, the row norms of x and y, and the zeroing of up to two ranges of 32-bit
// words (z0: n0 words, z1: n1 words; null or 0 = none) in one launch (the fused recursions
// need all of it before they start).
hipError_t launch_prep_norms(int* ticket, int* err, unsigned long long* rows, int64_t nwords,
                             unsigned long long lo, unsigned long long hi, const float* x,
                             float* x2, int64_t rows_x, const float* y, float* y2,
                             int64_t rows_y, int K, unsigned* z0, int64_t n0, unsigned* z1,
                             int64_t n1, hipStream_t st);
hipError_t launch_norms(const float* x, float* x2, int64_t rows_x, const float* y, float* y2,
                        int64_t rows_y, int K, hipStream_t st);
hipError_t launch_dist(const DistParams& p, bool muladd, bool mfma, hipStream_t st);
hipError_t launch_dist_bwd(const DistBwdParams& p, hipStream_t st);
// exact = the reference CPU arithmetic restated bit for bit; else hardware fp32 exp2/log2
// for the soft-min terms and backward weights (fp64 recursion state either way)
hipError_t launch_fwd(const DPParams& p, bool fused, bool muladd, bool exact, hipStream_t st);
hipError_t launch_bwd(const DPParams& p, bool fused, bool muladd, bool exact, hipStream_t st);
hipError_t launch_table_unpack(const float* Rt, float* Rd, int B, int N, int M, hipStream_t st);

// One barycenter update (sdtw_bary.hip): scalars of the Adam step and the clip, fp32 as the
// element-wise optimiser arithmetic uses them.
struct BaryStep {
    float one_m_b1;  // 1 - beta1
    float b2;        // beta2
    float one_m_b2;  // 1 - beta2
    float bc2_sqrt;  // sqrt(1 - beta2^t)
    float eps;
    float neg_step;  // -lr / (1 - beta1^t)
    float max_norm;  // gradient-norm clip
};
hipError_t launch_fill_zero(float* p, int64_t n, hipStream_t st);
hipError_t launch_bary_broadcast(const float* bary, float* xb, int64_t B, int64_t NK,
                                 hipStream_t st);
// Workgroups of the gradient reduction (the number of partial sums it leaves in `part`).
int bary_parts(int64_t NK);
// The clipped Adam step of the barycenter from the per-pair gradients gx (B, NK); also
// writes the new barycenter into every pair's copy xb (B, NK) and the weighted loss.
hipError_t launch_bary_update(const float* gx, const float* out, const float* w, float* bary,
                              float* xb, float* m, float* v, float* gbuf, float* part,
                              float* loss, int B, int NK, const BaryStep& s, hipStream_t st);
hipError_t launch_table_pack(const float* Rd, float* Rt, int B, int N, int M, hipStream_t st);

// Geometry of the band decomposition used by the wavefront kernels.
struct DPGeom {
    int nb, W, G;
};
// wmax: bands per workgroup (4, one compute wave per SIMD; 2 with producer waves, which take
// the other two SIMDs)
inline DPGeom dp_geom(int64_t N, int wmax = 4) {
    DPGeom g;
    g.nb = (int)((N + 63) / 64);
    g.W = g.nb < wmax ? g.nb : wmax;
    g.G = (g.nb + g.W - 1) / g.W;
    return g;
}
// Steps of one band in the R table: the M + 63 diagonal steps rounded up to the kernels'
// 16-step groups (the padding steps hold +inf).
inline int dp_band_steps(int64_t M) { return (int)(((M + 63) + 15) / 16 * 16); }
// entries of one cross-workgroup row (M columns plus 64 entries of padding on each side)
inline int64_t dp_row_entries(int64_t M) { return M + 128; }
// floats in the band-skewed R table
inline int64_t dp_table_elems(int64_t B, int64_t N, int64_t M) {
    return B * ((N + 63) / 64) * (int64_t)dp_band_steps(M) * 64;
}

}  // namespace sdtw
