// sdtw_dp.hpp -- Soft-DTW forward / backward wavefront kernels for gfx950 (device code,
// included by the sdtw_dp_*.hip translation units that instantiate the variants).
//
// Decomposition
//   * The rows of a pair are cut into 64-row bands; one wave owns one band, lane l owns
//     row 64*b + l.  A wave walks its band's anti-diagonals: at step s lane l updates cell
//     (64b + l, s - l); a band takes M + 63 steps, padded to S (a multiple of U).
//   * Up-neighbours inside a band arrive from lane l-1 by a DPP wave shift (wave_shr:1);
//     lane 0 receives the last row of the band above through a ring:
//       - band above in the same workgroup: an LDS ring with produced/consumed counters;
//       - band above in another workgroup: a per-boundary row in global memory, moved with
//         device-coherent atomics and published every U columns (no back-pressure, so a
//         producer never waits on a consumer).
//   * A workgroup holds W <= 4 consecutive bands (one wave per SIMD); a pair spans
//     G = ceil(nb / W) workgroups.  Workgroups draw tickets from an atomic counter and the
//     ticket decides (pair, group), so every cross-workgroup wait is on a workgroup that
//     started earlier: no deadlock whatever the residency.  Every wait is bounded; on
//     timeout the kernel records an error flag and exits.
//   * The backward runs the same machinery mirrored (bands bottom-up, columns right to left,
//     neighbours from lane l+1 by wave_shl:1).
//   * Steps run in groups of U: the next group's inputs (costs, R, ring values) are fetched
//     while the current group computes, the per-step bodies are branch-free, and the lane
//     feeding the next band hands its U values over once per group.
//   * The recursion state is fp64; R is stored once as fp32 in a band-skewed table
//     R[(pair*nb + band)*S + step][lane] (each step writes 256 contiguous bytes), which is
//     what the backward reads back.
//   * Two cell arithmetics (template flag EXACT):
//       - exact (default): the reference CPU arithmetic restated with fp64-accurate exp / log
//         written out as polynomials; R rounds to the CPU path's fp32 bits;
//       - fast: the same fp64 state, but the soft-min's correction term and the backward's
//         transition weights use the hardware fp32 exp2 / log2.  The correction is at most
//         gamma*log(3) per cell, so R stays within ~1 fp32 ulp of the exact recursion.
#pragma once

#include "sdtw_device.hpp"
#include "sdtw_internal.hpp"
#include "sdtw_math.hpp"

namespace sdtw {

constexpr int WAVE = 64;
constexpr int U = 8;      // steps per group (also the global publish granularity)
constexpr int RS = 128;   // LDS ring slots per band boundary (power of two, multiple of U)
constexpr unsigned kSpinLimit = 1u << 22;

// ---------------------------------------------------------------------------------------
// wave-level helpers
// ---------------------------------------------------------------------------------------
SDTW_DEV int dpp_shr1(int old, int v) { return __builtin_amdgcn_update_dpp(old, v, 0x138, 0xF, 0xF, false); }
SDTW_DEV int dpp_shl1(int old, int v) { return __builtin_amdgcn_update_dpp(old, v, 0x130, 0xF, 0xF, false); }

// lane l receives lane l-1's v; lane 0 receives `old`
SDTW_DEV double shr1(double old, double v) {
    const int lo = dpp_shr1(__double2loint(old), __double2loint(v));
    const int hi = dpp_shr1(__double2hiint(old), __double2hiint(v));
    return __hiloint2double(hi, lo);
}

// LDS flags: relaxed accesses; LDS operations of a wave complete in order, and the explicit
// lgkmcnt wait before a publish makes the ring data visible first.
SDTW_DEV int lds_load(const int* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP); }
SDTW_DEV void lds_publish(int* p, int v) {
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): prior LDS writes done
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
// Cross-workgroup rows: every access -- data and counter -- is an agent-scope (device
// coherent, sc1) atomic, so no access ever hits a stale non-coherent cache line (another
// XCD's L2, or an earlier launch that used the same workspace).  Ordering data before its
// counter needs only the producer's own stores to have completed: publish() waits for
// vmcnt(0) and then stores the counter.  No cache-wide writeback/invalidate is involved.
SDTW_DEV int glb_load(const int* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
SDTW_DEV void glb_publish(int* p, int v) {
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): the row's data stores have completed
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Data of the cross-workgroup rows moves with agent-scope (device-coherent) accesses, so a
// consumer on another XCD never reads a stale cached copy, e.g. of an earlier launch that
// used the same workspace.
SDTW_DEV void glb_put(double* p, double v) {
    __hip_atomic_store(reinterpret_cast<unsigned long long*>(p), (unsigned long long)__double_as_longlong(v),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
SDTW_DEV double glb_get(const double* p) {
    return __longlong_as_double((long long)__hip_atomic_load(reinterpret_cast<const unsigned long long*>(p),
                                                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}
SDTW_DEV void glb_put4(float4* p, float4 v) {
    unsigned long long* q = reinterpret_cast<unsigned long long*>(p);
    const unsigned long long lo = ((unsigned long long)__float_as_uint(v.y) << 32) | __float_as_uint(v.x);
    const unsigned long long hi = ((unsigned long long)__float_as_uint(v.w) << 32) | __float_as_uint(v.z);
    __hip_atomic_store(q, lo, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(q + 1, hi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
SDTW_DEV float4 glb_get4(const float4* p) {
    const unsigned long long* q = reinterpret_cast<const unsigned long long*>(p);
    const unsigned long long lo = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const unsigned long long hi = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return make_float4(__uint_as_float((unsigned)lo), __uint_as_float((unsigned)(lo >> 32)),
                       __uint_as_float((unsigned)hi), __uint_as_float((unsigned)(hi >> 32)));
}

// Spin until *flag >= need.  Returns false (and raises the error flag) on timeout.
template <bool GLOBAL>
SDTW_DEV bool wait_at_least(const int* flag, int need, int& known, int* err) {
    unsigned spins = 0;
    while (known < need) {
        known = GLOBAL ? glb_load(flag) : lds_load(flag);
        if (known >= need) break;
        __builtin_amdgcn_s_sleep(1);
        if (++spins > kSpinLimit) {
            __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return false;
        }
    }
    return true;
}

// Soft-min of the three predecessors (diag R0, up R1, left R2) in fp64: the reference CPU
// formula (launcher.py:317-322) restated around the minimum m as
//   m - gamma * log(sum_k exp(-(R_k - m) / gamma)),
// summed in the reference's index order ((t0 + t1) + t2; the minimum's term is exactly 1).
// The value path has no compare-and-select: the minimum is a min instruction and the
// exponential's lower clamp a max.  Those drop NaN operands, so NaN is put back
// explicitly: `nanfix` is NaN when an input is NaN or all three are +inf (where the
// reference's expression evaluates inf - inf), else 0.
SDTW_DEV double softmin_exact(double R0, double R1, double R2, double gamma, double inv_gamma,
                             double& nanfix) {
    const double m = fmin(fmin(R0, R1), R2);
    const bool nan_in = (R0 != R0) || (R1 != R1) || (R2 != R2);
    nanfix = (m - m) + (nan_in ? __builtin_nan("") : 0.0);
    const double e0 = fm::exp_neg<10>((m - R0) * inv_gamma);
    const double e1 = fm::exp_neg<10>((m - R1) * inv_gamma);
    const double e2 = fm::exp_neg<10>((m - R2) * inv_gamma);
    const double rsum = (e0 + e1) + e2;
    return fma(-gamma, fm::log_1to3(rsum), m);
}

// One backward cell (launcher.py:347-351): fp32 differences, fp64 exp/products/sum (in the
// reference's order), E rounded to fp32.  The exponential's clamp drops NaN, which is put
// back explicitly.
SDTW_DEV float bwd_cell_exact(float rij, float En, float Rn, float Dn, float Er, float Rr,
                             float Dr, float Eg, float Rg, float Dg, double inv_gamma) {
    const float da = __fsub_rn(__fsub_rn(Rn, rij), Dn);
    const float db = __fsub_rn(__fsub_rn(Rr, rij), Dr);
    const float dc = __fsub_rn(__fsub_rn(Rg, rij), Dg);
    const bool nan_in = (da != da) || (db != db) || (dc != dc);
    const double a = fm::exp_neg<9>((double)da * inv_gamma);
    const double b = fm::exp_neg<9>((double)db * inv_gamma);
    const double c = fm::exp_neg<9>((double)dc * inv_gamma);
    double acc = __dmul_rn((double)En, a);
    acc = __dadd_rn(acc, __dmul_rn((double)Er, b));
    acc = __dadd_rn(acc, __dmul_rn((double)Eg, c));
    return (float)(nan_in ? __builtin_nan("") : acc);
}

// Fast forward cell: D + softmin with the soft-min written around the minimum m,
//   m - gamma ln2 * log2(sum_k 2^((m - R_k) * log2(e) / gamma)),
// the exponents formed in fp64 and rounded once to fp32 for v_exp_f32 / v_log_f32.
// `c` = log2(e) / gamma, `ngl` = -gamma ln2.  Special values need no extra code: a NaN
// predecessor or cost makes its exponent (or m + d) NaN; three +inf predecessors make
// every exponent inf - inf = NaN, as the reference's expression does (launcher.py:317-322).
SDTW_DEV double fwd_cell_hw(double R0, double R1, double R2, float d, double c, double ngl) {
    const double m = fmin(fmin(R0, R1), R2);
    const double mc = m * c;
    const float t0 = (float)fma(-R0, c, mc);
    const float t1 = (float)fma(-R1, c, mc);
    const float t2 = (float)fma(-R2, c, mc);
    const float s = __fadd_rn(__fadd_rn(__builtin_amdgcn_exp2f(t0), __builtin_amdgcn_exp2f(t1)),
                              __builtin_amdgcn_exp2f(t2));
    return fma(ngl, (double)__builtin_amdgcn_logf(s), m + (double)d);
}

// Fast backward cell: the reference's fp32 differences (launcher.py:347-349), scaled by
// c = log2(e) / gamma into v_exp_f32, weights summed with fp32 fmas.  NaN propagates
// through exp2 and the products as in the reference's fp64 expression.
SDTW_DEV float bwd_cell_hw(float rij, float En, float Rn, float Dn, float Er, float Rr, float Dr,
                           float Eg, float Rg, float Dg, float c) {
    const float a = __builtin_amdgcn_exp2f(__fmul_rn(__fsub_rn(__fsub_rn(Rn, rij), Dn), c));
    const float b = __builtin_amdgcn_exp2f(__fmul_rn(__fsub_rn(__fsub_rn(Rr, rij), Dr), c));
    const float g = __builtin_amdgcn_exp2f(__fmul_rn(__fsub_rn(__fsub_rn(Rg, rij), Dg), c));
    return __fmaf_rn(Eg, g, __fmaf_rn(Er, b, __fmul_rn(En, a)));
}

// ---------------------------------------------------------------------------------------
// Cost providers.  load(j) returns the cost of the lane's row at column j one group before
// it is used.  It never faults: outside the table it reads a clamped cell, whose value the
// step then ignores (the cell is inactive).
// ---------------------------------------------------------------------------------------
struct CostD {
    const float* Drow;  // row min(i, N-1) of this pair's (N, M) cost
    int M;
    SDTW_DEV void init(const DPParams& P, int p) {
        M = P.M;
        Drow = P.D + (int64_t)p * P.N * P.M;
    }
    SDTW_DEV void stage(const DPParams&, int, unsigned char*) {}
    SDTW_DEV void set_row(int i, int N) { Drow += (int64_t)(i < N ? i : N - 1) * M; }
    SDTW_DEV float load(int j) const {
        const int jc = min(max(j, 0), M - 1);
        return Drow[jc];
    }
};

// Fused cost: the exact squared-Euclidean formula recomputed per cell.  y of the pair is
// staged in LDS when it fits (rows padded to an odd stride, so lanes reading consecutive
// rows hit distinct banks); x of the lane's row stays in registers when K <= KX.
template <bool MULADD, int KX>
struct CostXY {
    const float* x;
    const float* y;
    const float* y2;
    const float* x2;
    const float* ys;  // LDS copy of y or nullptr
    int M, K, ystride;
    float xr[KX > 0 ? KX : 1];
    float x2i;
    SDTW_DEV void init(const DPParams& P, int p) {
        M = P.M;
        K = P.K;
        x = P.x + (int64_t)p * P.N * P.K;
        y = P.y + (int64_t)p * P.M * P.K;
        x2 = P.x2 + (int64_t)p * P.N;
        y2 = P.y2 + (int64_t)p * P.M;
        x2i = 0.0f;
        ystride = P.ystride;
        ys = nullptr;
    }
    // cooperative copy of y into LDS (all threads of the workgroup)
    SDTW_DEV void stage(const DPParams& P, int p, unsigned char* smem) {
        if (P.ystride == 0) return;
        float* dst = reinterpret_cast<float*>(smem);
        const float* src = P.y + (int64_t)p * P.M * P.K;
        const int total = P.M * P.K;
        for (int e = threadIdx.x; e < total; e += blockDim.x) {
            const int r = e / P.K, k = e - r * P.K;
            dst[r * P.ystride + k] = src[e];
        }
        ys = dst;
    }
    SDTW_DEV void set_row(int i, int N) {
        const int ii = i < N ? i : N - 1;
        x2i = x2[ii];
        x += (int64_t)ii * K;
        if (KX > 0) {
#pragma unroll
            for (int k = 0; k < KX; ++k) xr[k] = (k < K) ? x[k] : 0.0f;
        }
    }
    SDTW_DEV float load(int j) const {
        const int jc = min(max(j, 0), M - 1);
        const float* yj = ys ? ys + jc * ystride : y + (int64_t)jc * K;
        float acc = 0.0f;
        if (KX > 0) {
#pragma unroll
            for (int k = 0; k < KX; ++k) {
                if (k < K) {
                    if (MULADD)
                        acc = __fadd_rn(acc, __fmul_rn(xr[k], yj[k]));
                    else
                        acc = __fmaf_rn(xr[k], yj[k], acc);
                }
            }
        } else {
            for (int k = 0; k < K; ++k) {
                if (MULADD)
                    acc = __fadd_rn(acc, __fmul_rn(x[k], yj[k]));
                else
                    acc = __fmaf_rn(x[k], yj[k], acc);
            }
        }
        return clamp0(exact_cost_pre(x2i, y2[jc], acc));
    }
};

// shared-memory layout of the DP kernels
struct Smem {
    unsigned char* base;
    int W;
    SDTW_DEV int* ticket() const { return reinterpret_cast<int*>(base); }
    SDTW_DEV int* prod() const { return reinterpret_cast<int*>(base) + 4; }
    SDTW_DEV int* cons() const { return reinterpret_cast<int*>(base) + 4 + W; }
    SDTW_DEV unsigned char* ring() const { return base + 256; }
};

SDTW_DEV size_t ring_bytes_fwd(int W) { return (size_t)W * RS * sizeof(double); }
SDTW_DEV size_t ring_bytes_bwd(int W) { return (size_t)W * RS * sizeof(float4); }

// ---------------------------------------------------------------------------------------
// Forward
// ---------------------------------------------------------------------------------------
template <class Cost, bool BAND, bool EXACT>
SDTW_DEV void fwd_band(const DPParams& P, Cost& cost, const Smem& sm, int p, int g, int w) {
    const int l = threadIdx.x & (WAVE - 1);
    const int W = P.W, G = P.G, nb = P.nb, N = P.N, M = P.M, S = P.S;
    const int b = g * W + w;
    const int i = b * WAVE + l;
    const bool row_ok = i < N;
    const double gamma = P.gamma, inv_gamma = P.inv_gamma, bw = P.bw;
    const double c2 = inv_gamma * 1.4426950408889634074;  // log2(e) / gamma
    const double ngl = -gamma * 0.69314718055994530942;   // -gamma ln2
    const double INF = dinf();
    cost.set_row(i, N);

    double* lring = reinterpret_cast<double*>(sm.ring());
    const bool in_glb = (b > 0) && (w == 0);  // band above in workgroup g-1 (else LDS)
    const bool out_lds = (b + 1 < nb) && (w + 1 < W);
    const bool out_glb = (b + 1 < nb) && (w + 1 == W);
    const double* gin = P.gring + ((int64_t)p * G + (g - 1)) * M;
    const int* gin_flag = P.gflag + p * G + (g - 1);
    double* gout = P.gring + ((int64_t)p * G + g) * M;
    int* gout_flag = P.gflag + p * G + g;
    const double* lin = lring + (w - 1) * RS;
    double* lout = lring + w * RS;
    const int* lin_flag = sm.prod() + (w - 1);

    float* Rt = P.R + ((int64_t)p * nb + b) * S * WAVE + l;

    int known_in = 0;    // columns of the band above known to be available
    int known_free = 0;  // columns of my ring known to be consumed (LDS producer)
    double left = INF;
    double diag = (b == 0 && l == 0) ? 0.0 : INF;
    double prev = INF;   // this lane's value one step ago (sent to lane l+1 by DPP)

    double up_cur[U], up_nxt[U], hold[U];
    float d_cur[U], d_nxt[U];
    // ring values of columns [c0, c0 + U) for lane 0 (INF past M or for band 0)
    auto fetch_up = [&](int c0, double* dst) -> bool {
#pragma unroll
        for (int u = 0; u < U; ++u) dst[u] = INF;
        if (b == 0 || c0 >= M) return true;
        const int need = min(c0 + U, M);
        if (in_glb) {
            if (!wait_at_least<true>(gin_flag, need, known_in, P.err)) return false;
#pragma unroll
            for (int u = 0; u < U; ++u)
                if (c0 + u < M) dst[u] = glb_get(gin + c0 + u);
        } else {
            if (!wait_at_least<false>(lin_flag, need, known_in, P.err)) return false;
            const double2* src = reinterpret_cast<const double2*>(lin + (c0 & (RS - 1)));
#pragma unroll
            for (int u = 0; u < U / 2; ++u) {
                const double2 v = src[u];
                dst[2 * u] = v.x;
                dst[2 * u + 1] = v.y;
            }
            if (l == 0) lds_publish(sm.cons() + (w - 1), need);
        }
        return true;
    };
    // hand the last row's columns written by the group at s0 (lane 63 computed column
    // s0 + u - 63 at step s0 + u) to the band below
    auto handover = [&](int s0) {
        if (l != WAVE - 1) return;
        const int c0 = s0 - (WAVE - 1);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int c = c0 + u;
            if (c >= 0 && c < M) {
                if (out_lds)
                    lout[c & (RS - 1)] = hold[u];
                else
                    glb_put(gout + c, hold[u]);
            }
        }
        const int done = min(max(s0 + U - (WAVE - 1), 0), M);
        if (out_lds)
            lds_publish(sm.prod() + w, done);
        else if (done > 0)
            glb_publish(gout_flag, done);
    };

    // Costs are fetched one group ahead.  Ring values from the LDS are fetched for the
    // current group at its start; from global memory one group ahead, and a global producer
    // publishes a group's values at the start of the next group, when everything it has
    // in flight is old, so the publish wait is short.
#pragma unroll
    for (int u = 0; u < U; ++u) d_nxt[u] = cost.load(u - l);
    if (in_glb && !fetch_up(0, up_nxt)) return;

    for (int s0 = 0; s0 < S; s0 += U) {
        if (out_glb && s0 > 0) handover(s0 - U);
#pragma unroll
        for (int u = 0; u < U; ++u) d_cur[u] = d_nxt[u];
        if (in_glb) {
#pragma unroll
            for (int u = 0; u < U; ++u) up_cur[u] = up_nxt[u];
        } else if (!fetch_up(s0, up_cur)) {
            return;
        }
        const int n0 = s0 + U;
        if (n0 < S) {
#pragma unroll
            for (int u = 0; u < U; ++u) d_nxt[u] = cost.load(n0 + u - l);
            if (in_glb && !fetch_up(n0, up_nxt)) return;
        }
        // this group writes columns up to s0 + U - 64 of my last row; writing column c
        // reuses the slot of column c - RS, which the consumer must have taken
        if (out_lds) {
            const int need_free = s0 + U - WAVE + 1 - RS;
            if (need_free > 0 && !wait_at_least<false>(sm.cons() + w, need_free, known_free, P.err)) return;
        }
        float* Rg = Rt + (int64_t)s0 * WAVE;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int j = s0 + u - l;
            const bool act = row_ok && (unsigned)j < (unsigned)M;
            bool keep = act;
            if (BAND) keep = keep && !out_of_band(bw, i, j);
            const double up = shr1(up_cur[u], prev);
            double cand;
            if (EXACT) {
                double nanfix;
                const double sm_ = softmin_exact(diag, up, left, gamma, inv_gamma, nanfix);
                cand = ((double)d_cur[u] + sm_) + nanfix;
            } else {
                cand = fwd_cell_hw(diag, up, left, d_cur[u], c2, ngl);
            }
            // inactive lanes publish +inf: before its first column a lane's left/up are the
            // +inf padding, out-of-band cells stay +inf (launcher.py:310, :315)
            const double r = keep ? cand : INF;
            left = r;
            diag = up;
            prev = r;
            hold[u] = r;
            Rg[u * WAVE] = (float)r;
        }
        if (out_lds) handover(s0);
    }
    if (out_glb) handover(S - U);
    // out[p] = R[N-1, M-1] as stored (step M-1+l of this lane, written by this lane)
    if (i == N - 1) P.out[p] = Rt[(int64_t)(M - 1 + l) * WAVE];
}

template <class Cost, bool BAND, bool EXACT>
__global__ void __launch_bounds__(256) fwd_kernel(DPParams P) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    Smem sm{smem_raw, P.W};
    const int w = threadIdx.x / WAVE;
    if (threadIdx.x == 0) *sm.ticket() = atomicAdd(P.ticket, 1);
    if (threadIdx.x < 2 * P.W) sm.prod()[threadIdx.x] = 0;  // prod and cons are contiguous
    __syncthreads();
    const int t = *sm.ticket();
    const int p = t / P.G, g = t - p * P.G;
    Cost cost;
    cost.init(P, p);
    cost.stage(P, p, sm.ring() + ring_bytes_fwd(P.W));
    __syncthreads();
    if (g * P.W + w >= P.nb) return;
    fwd_band<Cost, BAND, EXACT>(P, cost, sm, p, g, w);
}

// ---------------------------------------------------------------------------------------
// Backward
//
// Reverse step q, lane l visits column j = (M-1) - q + (63 - l), whose forward step is
// s = M + 62 - q.  Neighbours of (i, j): down (i+1, j) from lane l+1 one step ago
// (wave_shl:1; lane 63 from the band below), right (i, j+1) = the lane's own previous cell,
// diag (i+1, j+1) = down one step ago.  Outside the table the reference pads R = -inf,
// D = 0, E = 0, except the corner (N, M) = (E 1, R R[N-1,M-1] as stored, D 0)
// (launcher.py:330-338); row N-1 takes its down/diag from that padding directly.  Each
// visited cell maps R = +inf to -inf first (launcher.py:343-344).
// ---------------------------------------------------------------------------------------
template <class Cost, bool BAND, bool EXACT>
SDTW_DEV void bwd_band(const DPParams& P, Cost& cost, const Smem& sm, int p, int g, int w) {
    const int l = threadIdx.x & (WAVE - 1);
    const int W = P.W, G = P.G, nb = P.nb, N = P.N, M = P.M, S = P.S;
    const int b = g * W + w;
    const int i = b * WAVE + l;
    const bool row_ok = i < N;
    const bool last_row = (i == N - 1);
    const double inv_gamma = P.inv_gamma, bw = P.bw;
    const float c2 = (float)(inv_gamma * 1.4426950408889634074);  // log2(e) / gamma
    const float NINF = -finf();
    const float gsc = P.gout ? P.gout[p] : 1.0f;
    cost.set_row(i, N);

    // corner R (as stored by the forward) of this pair
    const int lb = nb - 1, ll = (N - 1) - lb * WAVE;
    const float corner_R = P.R[(((int64_t)p * nb + lb) * S + (M - 1 + ll)) * WAVE + ll];

    // rings carry (E, R, D) of a band's first row to the band above
    float4* lring = reinterpret_cast<float4*>(sm.ring());
    const bool in_glb = (b + 1 < nb) && (w + 1 == W);  // band below in workgroup g+1 (else LDS)
    const bool out_lds = (b > 0) && (w > 0);
    const bool out_glb = (b > 0) && (w == 0);
    // global rows indexed by the producing group; WG g consumes what group g+1 produced
    const float4* gin = P.gring4 + ((int64_t)p * G + (g + 1)) * M;
    const int* gin_flag = P.gflag + p * G + (g + 1);
    float4* gout = P.gring4 + ((int64_t)p * G + g) * M;
    int* gout_flag = P.gflag + p * G + g;
    const float4* lin = lring + (w + 1) * RS;
    float4* lout = lring + w * RS;
    const int* lin_flag = sm.prod() + (w + 1);

    const float* Rt = P.R + ((int64_t)p * nb + b) * S * WAVE + l;
    float* Grow = P.G_out + ((int64_t)p * N + (row_ok ? i : N - 1)) * M;

    int known_in = 0, known_free = 0;
    float rE = 0.0f, rR = NINF, rD = 0.0f;  // right neighbour
    float gE = last_row ? 1.0f : 0.0f;      // diag neighbour
    float gR = last_row ? corner_R : NINF;
    float gD = 0.0f;
    float pE = 0.0f, pR = NINF, pD = 0.0f;  // published one step ago

    float4 dn_cur[U], dn_nxt[U], hold[U];
    float r_cur[U], r_nxt[U], d_cur[U], d_nxt[U];
    const float4 pad4 = make_float4(0.0f, NINF, 0.0f, 0.0f);
    auto fetch_dn = [&](int q0, float4* dst) -> bool {
#pragma unroll
        for (int u = 0; u < U; ++u) dst[u] = pad4;
        if (b + 1 >= nb || q0 >= M) return true;
        const int need = min(q0 + U, M);
        if (in_glb) {
            if (!wait_at_least<true>(gin_flag, need, known_in, P.err)) return false;
#pragma unroll
            for (int u = 0; u < U; ++u)
                if (q0 + u < M) dst[u] = glb_get4(gin + q0 + u);
        } else {
            if (!wait_at_least<false>(lin_flag, need, known_in, P.err)) return false;
#pragma unroll
            for (int u = 0; u < U; ++u) dst[u] = lin[(q0 + u) & (RS - 1)];
            if (l == 0) lds_publish(sm.cons() + (w + 1), need);
        }
        return true;
    };
    // hand the band's first row to the band above: lane 0 produced sequence numbers
    // q - 63 (= M - 1 - j) during the group at q0
    auto handover = [&](int q0) {
        if (l != 0) return;
        const int c0 = q0 - (WAVE - 1);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int c = c0 + u;
            if (c >= 0 && c < M) {
                if (out_lds)
                    lout[c & (RS - 1)] = hold[u];
                else
                    glb_put4(gout + c, hold[u]);
            }
        }
        const int done = min(max(q0 + U - (WAVE - 1), 0), M);
        if (out_lds)
            lds_publish(sm.prod() + w, done);
        else if (done > 0)
            glb_publish(gout_flag, done);
    };
    // forward step of reverse step q, clamped into the band (padding steps are inactive)
    auto fstep = [&](int q) { return max(M + 62 - q, 0); };

#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int sf = fstep(u);
        r_nxt[u] = Rt[(int64_t)sf * WAVE];
        d_nxt[u] = cost.load(sf - l);
    }
    if (in_glb && !fetch_dn(0, dn_nxt)) return;

    for (int q0 = 0; q0 < S; q0 += U) {
        if (out_glb && q0 > 0) handover(q0 - U);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            r_cur[u] = r_nxt[u];
            d_cur[u] = d_nxt[u];
        }
        if (in_glb) {
#pragma unroll
            for (int u = 0; u < U; ++u) dn_cur[u] = dn_nxt[u];
        } else if (!fetch_dn(q0, dn_cur)) {
            return;
        }
        const int n0 = q0 + U;
        if (n0 < S) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int sf = fstep(n0 + u);
                r_nxt[u] = Rt[(int64_t)sf * WAVE];
                d_nxt[u] = cost.load(sf - l);
            }
            if (in_glb && !fetch_dn(n0, dn_nxt)) return;
        }
        if (out_lds) {  // as in the forward: sequence numbers up to q0 + U - 64 this group
            const int need_free = q0 + U - WAVE + 1 - RS;
            if (need_free > 0 && !wait_at_least<false>(sm.cons() + w, need_free, known_free, P.err)) return;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int q = q0 + u;
            const int j = (M - 1) - q + (WAVE - 1 - l);
            float dE = __int_as_float(dpp_shl1(__float_as_int(dn_cur[u].x), __float_as_int(pE)));
            float dR = __int_as_float(dpp_shl1(__float_as_int(dn_cur[u].y), __float_as_int(pR)));
            float dD = __int_as_float(dpp_shl1(__float_as_int(dn_cur[u].z), __float_as_int(pD)));
            if (last_row) {  // the padded row below the table
                const bool corner = (j == M);
                dE = corner ? 1.0f : 0.0f;
                dR = corner ? corner_R : NINF;
                dD = 0.0f;
            }
            const bool act = row_ok && (unsigned)j < (unsigned)M;
            float rij = r_cur[u];
            rij = __builtin_isinf(rij) ? NINF : rij;
            const float cand = EXACT ? bwd_cell_exact(rij, dE, dR, dD, rE, rR, rD, gE, gR, gD, inv_gamma)
                                     : bwd_cell_hw(rij, dE, dR, dD, rE, rR, rD, gE, gR, gD, c2);
            bool keep = true;
            if (BAND) keep = !out_of_band(bw, i, j);
            const float e = keep ? cand : 0.0f;
            if (act) Grow[j] = __fmul_rn(gsc, e);
            // inactive steps carry the reference's padding (E 0, R -inf, D 0): before a
            // lane's first column that is exactly its right neighbour (column M)
            const float mE = act ? e : 0.0f;
            const float mR = act ? rij : NINF;
            const float mD = act ? d_cur[u] : 0.0f;
            rE = mE;
            rR = mR;
            rD = mD;
            gE = dE;
            gR = dR;
            gD = dD;
            pE = mE;
            pR = mR;
            pD = mD;
            hold[u] = make_float4(mE, mR, mD, 0.0f);
        }
        if (out_lds) handover(q0);
    }
    if (out_glb) handover(S - U);
}

template <class Cost, bool BAND, bool EXACT>
__global__ void __launch_bounds__(256) bwd_kernel(DPParams P) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    Smem sm{smem_raw, P.W};
    const int w = threadIdx.x / WAVE;
    if (threadIdx.x == 0) *sm.ticket() = atomicAdd(P.ticket, 1);
    if (threadIdx.x < 2 * P.W) sm.prod()[threadIdx.x] = 0;
    __syncthreads();
    const int t = *sm.ticket();
    const int p = t / P.G;
    const int g = (P.G - 1) - (t - p * P.G);  // lowest ticket of a pair takes the bottom group
    Cost cost;
    cost.init(P, p);
    cost.stage(P, p, sm.ring() + ring_bytes_bwd(P.W));
    __syncthreads();
    if (g * P.W + w >= P.nb) return;
    bwd_band<Cost, BAND, EXACT>(P, cost, sm, p, g, w);
}

// ---------------------------------------------------------------------------------------
// Launch helpers (the prep kernel that zeroes the ticket, error flag and ring counters is
// launched by launch_dp_prep, defined once in sdtw_dp.hip)
// ---------------------------------------------------------------------------------------
hipError_t launch_dp_prep(const DPParams& P, hipStream_t st);

inline size_t dp_smem_bytes(const DPParams& P, bool bwd) {
    const size_t ring = (size_t)P.W * RS * (bwd ? sizeof(float4) : sizeof(double));
    const size_t ys = P.ystride ? (size_t)P.M * P.ystride * sizeof(float) : 0;
    return 256 + ring + ys;
}

template <class K>
hipError_t launch_dp(K kernel, const DPParams& P, bool bwd, hipStream_t st) {
    const size_t lds = dp_smem_bytes(P, bwd);
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    hipError_t e = launch_dp_prep(P, st);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kernel, dim3(P.B * P.G), dim3(P.W * WAVE), lds, st, P);
    return hipGetLastError();
}

template <class Cost, bool BWD, bool EXACT>
hipError_t launch_cost(const DPParams& P, hipStream_t st) {
    if constexpr (BWD) {
        if (P.bw > 0.0) return launch_dp(bwd_kernel<Cost, true, EXACT>, P, true, st);
        return launch_dp(bwd_kernel<Cost, false, EXACT>, P, true, st);
    } else {
        if (P.bw > 0.0) return launch_dp(fwd_kernel<Cost, true, EXACT>, P, false, st);
        return launch_dp(fwd_kernel<Cost, false, EXACT>, P, false, st);
    }
}

// One (direction, arithmetic, cost source) family of kernels.  Fused kernels keep x of the
// lane's row in registers, sized to the smallest power of two >= K (up to 64); wider
// features, and the tiny problems that take the multiply-then-add dot, read x from memory.
template <bool BWD, bool EXACT, bool FUSED>
hipError_t launch_dp_variant(const DPParams& P, bool muladd, hipStream_t st) {
    if constexpr (!FUSED) {
        (void)muladd;
        return launch_cost<CostD, BWD, EXACT>(P, st);
    } else {
        if (muladd) return launch_cost<CostXY<true, 0>, BWD, EXACT>(P, st);
        if (P.K <= 4) return launch_cost<CostXY<false, 4>, BWD, EXACT>(P, st);
        if (P.K <= 8) return launch_cost<CostXY<false, 8>, BWD, EXACT>(P, st);
        if (P.K <= 16) return launch_cost<CostXY<false, 16>, BWD, EXACT>(P, st);
        if (P.K <= 32) return launch_cost<CostXY<false, 32>, BWD, EXACT>(P, st);
        if (P.K <= 64) return launch_cost<CostXY<false, 64>, BWD, EXACT>(P, st);
        return launch_cost<CostXY<false, 0>, BWD, EXACT>(P, st);
    }
}

#define SDTW_DP_VARIANTS(X)        \
    X(false, false, false)         \
    X(false, false, true)          \
    X(false, true, false)          \
    X(false, true, true)           \
    X(true, false, false)          \
    X(true, false, true)           \
    X(true, true, false)           \
    X(true, true, true)

#define SDTW_DP_EXTERN(B, E, F) \
    extern template hipError_t launch_dp_variant<B, E, F>(const DPParams&, bool, hipStream_t);
SDTW_DP_VARIANTS(SDTW_DP_EXTERN)
#undef SDTW_DP_EXTERN

}  // namespace sdtw
