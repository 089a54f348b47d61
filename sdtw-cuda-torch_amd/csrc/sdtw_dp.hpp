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
//       - band above in another workgroup: a per-boundary row in global memory holding one
//         entry per column, reset to an "empty" signalling-NaN pattern before the launch.
//         The producer stores each value with a device-coherent atomic and nothing else; the
//         consumer loads a group's entries one group ahead and accepts them once none is
//         empty.  No counter, no fence, no wait on the producer side, and no back-pressure.
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
//         (table-driven, tables staged in LDS); R rounds to the CPU path's fp32 bits;
//       - fast: the same fp64 state, but the soft-min's correction term and the backward's
//         transition weights use the hardware fp32 exp2 / log2.  The correction is at most
//         gamma*log(3) per cell, so R stays within ~1 fp32 ulp of the exact recursion.
#pragma once

#include <type_traits>

#include "sdtw_device.hpp"
#include "sdtw_internal.hpp"
#include "sdtw_math.hpp"

namespace sdtw {

constexpr int WAVE = 64;
constexpr int U = 16;     // steps per group (the unit of prefetch and of band handover)
constexpr int RS = 128;   // LDS ring slots per band boundary (power of two, multiple of U)
constexpr int RPAD = 64;  // padding entries on each side of a cross-workgroup row

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

// LDS counters: relaxed accesses.  All LDS operations of a CU are performed as wave-wide
// operations in one global order, a wave's in issue order, so a counter stored after ring
// writes (or after ring reads) is seen by another wave only after those are performed.  The
// compiler fence keeps the program order; no wait on the hardware counters is needed.
SDTW_DEV int lds_load(const int* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP); }
SDTW_DEV void lds_publish(int* p, int v) {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
// Cross-workgroup rows.  Every access is an agent-scope (device-coherent, sc1) atomic, so
// no access hits a stale non-coherent cache line (another XCD's L2, or an earlier launch
// that used the same workspace).  An entry not yet written holds an "empty" pattern: a
// signalling NaN, which no arithmetic result can be (arithmetic produces quiet NaNs).  A
// consumer therefore needs no counter: it accepts an entry once it is not empty.  64-bit
// atomic accesses are single-copy atomic, so an entry is seen either empty or whole.
constexpr unsigned long long kEmpty64 = 0x7FF4000000005D7Full;  // forward rows (fp64)
constexpr unsigned kEmpty32 = 0x7FA05D7Fu;                      // backward rows: E slot
SDTW_DEV bool row_empty(double v) { return (unsigned long long)__double_as_longlong(v) == kEmpty64; }
// a backward entry (E, R, D, tag) is written as two 64-bit halves; the first is whole when
// E is not empty, the second when tag (reset to 0) is not 0
SDTW_DEV bool row_empty4(float4 v) { return __float_as_uint(v.x) == kEmpty32 || v.w == 0.0f; }

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
SDTW_DEV double glb_get_entry(const double* p) { return glb_get(p); }
SDTW_DEV float4 glb_get_entry(const float4* p) { return glb_get4(p); }
SDTW_DEV bool entry_empty(double v) { return row_empty(v); }
SDTW_DEV bool entry_empty(float4 v) { return row_empty4(v); }

SDTW_DEV void raise_timeout(int* err) { __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

// Spin until the LDS counter *flag >= need.  Returns false (and raises the error flag) after
// `limit` polls that found it short.  `known` caches the last value read; every lane reads
// the same counter, so it is kept wave-uniform (a scalar register) and the loop branches on
// scalar compares.
SDTW_DEV bool wait_at_least(const int* flag, int need, int& known, int* err, unsigned limit) {
    unsigned spins = 0;
    while (known < need) {
        known = __builtin_amdgcn_readfirstlane(lds_load(flag));
        if (known >= need) break;
        if (spins++ >= limit) {
            raise_timeout(err);
            return false;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    // the ring accesses the wait guards must not be moved above the counter read; the
    // hardware performs a wave's LDS operations in order, so a compiler fence suffices
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    return true;
}

// A wave whose bounded wait expired stops, and marks its pair's results invalid where a
// caller reads them without a synchronisation: the forward sets out[p] to NaN, the backward
// fills its band's rows of G with NaN.  Every wave that depends on the stopped one (bands
// further along the pair, the band's own compute or producer wave) then also gives up, since
// the entries it waits for never arrive; so the last band of the pair never stores a value
// over the NaN.  The flag (sdtw_debug_status) is raised too.
SDTW_DEV void give_up_fwd(const DPParams& P, int p) {
    raise_timeout(P.err);
    if ((threadIdx.x & 63) == 0) P.out[p] = __builtin_nanf("");
}
SDTW_DEV void give_up_bwd(const DPParams& P, int p, int b) {
    raise_timeout(P.err);
    const int r0 = b * 64;
    const int nrows = min(P.N - r0, 64);
    if (nrows <= 0) return;
    const float qnan = __builtin_nanf("");
    if (P.G_out) {
        float* base = P.G_out + ((int64_t)p * P.N + r0) * P.M;
        const int64_t cells = (int64_t)nrows * P.M;
        for (int64_t e = threadIdx.x & 63; e < cells; e += 64) base[e] = qnan;
    }
    // gradient mode: the band's rows of dL/dx, and all of the pair's dL/dy (added, since the
    // other bands add their tiles to it: NaN + v stays NaN whatever the order)
    if (P.gx_out) {
        float* base = P.gx_out + ((int64_t)p * P.N + r0) * P.K;
        const int64_t n = (int64_t)nrows * P.K;
        for (int64_t e = threadIdx.x & 63; e < n; e += 64) base[e] = qnan;
    }
    if (P.gy_out) {
        float* base = P.gy_out + (int64_t)p * P.M * P.K;
        const int64_t n = (int64_t)P.M * P.K;
        for (int64_t e = threadIdx.x & 63; e < n; e += 64) unsafeAtomicAdd(base + e, qnan);
    }
}
template <bool BWD>
SDTW_DEV void give_up(const DPParams& P, int p, int b) {
    if constexpr (BWD) give_up_bwd(P, p, b);
    else give_up_fwd(P, p);
}

// Slot of entry c (a column, or a backward sequence number) in an LDS handoff ring.  The
// rotation by 63 puts the U entries a band hands over per group (c = s0 - 63 .. s0 - 48, for
// a group starting at step s0, a multiple of U) in one aligned block of slots, so they are
// written with immediate offsets; a consumer's group (c = c0 .. c0 + U - 1, c0 a multiple
// of U) then reads one entry and a block of U - 1.
SDTW_DEV int hslot(int c) { return (c + WAVE - 1) & (RS - 1); }

// One forward cell: d + soft-min of the three predecessors (diag R0, up R1, left R2) in fp64,
// the reference CPU formula (launcher.py:317-322) restated around the minimum m as
//   m - gamma * log(sum_k exp(-(R_k - m) / gamma)).
// The minimum's term is exactly 1, so only the exponentials of the other two predecessors
// (R_a, R_b, in index order) are evaluated, and the sum is (e_a + e_b) + 1.  exp / log are
// the table-driven fp64 ones (T, L in LDS); every intermediate is fp64-accurate and R is
// rounded once to fp32 by the caller, which is what makes R equal the CPU path's bits.
// Min and maxNum drop NaN operands, so NaN is put back explicitly: `nanfix` is NaN when an
// input is NaN (R0 + R1 + R2 is then NaN: R is never -inf from a cost >= 0) or all three are
// +inf (where the reference's expression evaluates inf - inf), else 0.  d + m + nanfix is
// formed off the exponential chain.
SDTW_DEV double fwd_cell_exact(double R0, double R1, double R2, float d, double gamma, double inv_gamma,
                               const double* T, const double* L) {
    const double m = fmin(fmin(R0, R1), R2);
    const double sum3 = (R0 + R1) + R2;
    const double nanfix = (m - m) + (sum3 != sum3 ? __builtin_nan("") : 0.0);
    const bool a0 = (R0 == m);
    const bool a2 = !a0 && !(R1 == m);
    const double Ra = a0 ? R1 : R0;
    const double Rb = a2 ? R1 : R2;
    const double ea = fm::exp_tab_abs((m - Ra) * inv_gamma, T);
    const double eb = fm::exp_tab_abs((m - Rb) * inv_gamma, T);
    const double rsum = (ea + eb) + 1.0;
    return fma(-gamma, fm::log_tab_1to3(rsum, L), ((double)d + m) + nanfix);
}

// fwd_cell_exact for finite inputs with a finite minimum, in fewer instructions: the minimum
// and the two other predecessors come from a four-operation min/max network (lo, hi of the
// diagonal and left ones; the minimum is min(lo, up), the others hi and max(lo, up); the sum
// of the two non-minimum terms does not depend on their order), and no NaN is restored.  Where those
// conditions hold it returns fwd_cell_exact's bits.  The forward takes it only while every
// cost the band uses and every value the band above hands over is finite; then each active
// cell has a finite predecessor (the diagonal one, or the left one in row 0, or R[0,0]).
SDTW_DEV double fwd_cell_exact_finite(double R0, double R1, double R2, float d, double gamma,
                                      double inv_gamma, const double* T, const double* L) {
    const double lo = fmin(R0, R2), hi = fmax(R0, R2);
    const double m = fmin(lo, R1), o = fmax(lo, R1);
    const double xa = fm::exp_tab_abs_arg((m - o) * inv_gamma);
    const double xb = fm::exp_tab_abs_arg((m - hi) * inv_gamma);
    const double tca = fm::exp_tab_abs_tc(xa), tcb = fm::exp_tab_abs_tc(xb);
    // (table reads written first; the compiler's own schedule measured faster than one
    // pinned with scheduling barriers that waits for both after the polynomials)
    const double fa = T[fm::lo_word(tca) & (fm::kExpTabN - 1)];
    const double fb = T[fm::lo_word(tcb) & (fm::kExpTabN - 1)];
    const double pa = fm::exp_tab_abs_em1(xa, tca), pb = fm::exp_tab_abs_em1(xb, tcb);
    const double rsum = (fm::exp_tab_abs_join(fa, pa, tca) + fm::exp_tab_abs_join(fb, pb, tcb)) + 1.0;
    return fma(-gamma, fm::log_tab_1to3(rsum, L), (double)d + m);
}

// One backward cell (launcher.py:347-351): fp32 differences, fp64 exp/products/sum (in the
// reference's order), E rounded to fp32.  The exponential's clamp drops NaN, which is put
// back explicitly.
SDTW_DEV float bwd_cell_exact(float rij, float En, float Rn, float Dn, float Er, float Rr,
                              float Dr, float Eg, float Rg, float Dg, double inv_gamma,
                              const double* T) {
    const float da = __fsub_rn(__fsub_rn(Rn, rij), Dn);
    const float db = __fsub_rn(__fsub_rn(Rr, rij), Dr);
    const float dc = __fsub_rn(__fsub_rn(Rg, rij), Dg);
    const bool nan_in = (da != da) || (db != db) || (dc != dc);
    const double a = fm::exp_tab((double)da * inv_gamma, T);
    const double b = fm::exp_tab((double)db * inv_gamma, T);
    const double c = fm::exp_tab((double)dc * inv_gamma, T);
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
// Cost ring.  Every band stages the costs of its 64 rows in LDS: a ring of CR columns per
// row (slot = column mod CR), row stride CS floats.  A provider fills one tile of TC
// columns x 64 rows per group, one group ahead, with coalesced loads (unfused) or matrix-
// core products (fused); lane l then reads its diagonal cell (row l, column s - l) with a
// conflict-free ds_read (CS - 1 is odd).  The live window of a group is 64 + 2*TC columns,
// inside CR.  Ring slots of columns outside [0, M) hold values that are never used.
//
// Provider interface (all lanes call each function, wave-uniform arguments).  Per group,
// with c the tile completed this group and cn the tile after it:
//   begin(ring, c)     at the group start
//   step(u, c, cn)     inside recursion step u (matrix-core products, loads), u = 0..U-1
//   end(ring, c, cn)   after the last step; tile c is in the ring afterwards
// prologue(ring, c) stages tile c synchronously; preload(c) starts the first pipelined one.
// ---------------------------------------------------------------------------------------
constexpr int CR = 128;  // ring columns (power of two)
constexpr int CS = 144;  // row stride in floats: CS mod 64 = 16 (tile writes by 4-row
                         // groups hit disjoint banks), CS - 1 odd (diagonal reads)
// Slots CR .. CR + U - 1 of every row mirror slots 0 .. U - 1 (every tile store writes both),
// so a lane reads U consecutive columns from slot c & (CR - 1) on with immediate offsets,
// without wrapping the index per column.
constexpr int TC = U;    // tile columns per group

// Unfused: the tile is read from the (B, N, M) cost.  Lane l loads column c0 + (l & 15)
// of rows 4k + (l >> 4), k = 0..15: each load covers 4 rows x 64 contiguous bytes.
// Indices are clamped into the table, so no load leaves it.
struct CostD {
    const float* base;  // this pair's cost
    int M, row0, N;
    int badc;           // first column of a stored tile holding a non-finite cost (or INT_MAX)
    float v[16];
    SDTW_DEV void init(const DPParams& P, int p, int b) {
        M = P.M;
        N = P.N;
        base = P.D + (int64_t)p * P.N * P.M;
        row0 = b * WAVE;
        badc = INT_MAX;
    }
    SDTW_DEV int first_bad_col() const { return badc; }
    SDTW_DEV int bad_col_raw() const { return badc; }
    SDTW_DEV void issue(int c0) {
        const int l = threadIdx.x & (WAVE - 1);
        const int col = min(max(c0 + (l & 15), 0), M - 1);
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const int row = min(row0 + 4 * k + (l >> 4), N - 1);
            v[k] = base[(int64_t)row * M + col];
        }
    }
    // write the loaded tile c0 into the ring
    SDTW_DEV void store(float* ring, int c0) {
        const int l = threadIdx.x & (WAVE - 1);
        const int sl = (c0 + (l & 15)) & (CR - 1);
        float* dst = ring + (l >> 4) * CS + sl;
        float sum = 0.0f;  // NaN or infinite if a cost is
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            dst[4 * k * CS] = v[k];
            sum += v[k];
        }
        if (sl < U) {  // the mirror slots
#pragma unroll
            for (int k = 0; k < 16; ++k) dst[4 * k * CS + CR] = v[k];
        }
        if (__builtin_amdgcn_ballot_w64(!(fabsf(sum) < __builtin_inff()))) badc = min(badc, c0);
    }
    SDTW_DEV bool prologue(float* ring, int c) {
        issue(c);
        store(ring, c);
        return true;
    }
    SDTW_DEV void preload(int) {}
    // the tile is loaded at the first step and lands in the ring after the last one
    SDTW_DEV bool begin(float*, int) { return true; }
    SDTW_DEV void step(int u, int c, int) {
        if (u == 0) {
            issue(c);
            // keep the loads here: under register pressure the scheduler would otherwise
            // sink them next to their stores at the group end, exposing their latency
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    SDTW_DEV void end(float* ring, int c, int) { store(ring, c); }
};

// Fused: cost = max(0, (|x_i|^2 + |y_j|^2) - 2 x_i.y_j) with the dot on the matrix cores.
// v_mfma_f32_16x16x4_f32 chained over k = 0, 4, 8, ... accumulates each output as one
// sequential fp32 FMA chain over k (measured bit-identical on gfx950), which is the order
// of the reference's CPU matmul, so the cost has the same bits as the materialised one.
// The band's x rows stay in registers (A operands, 16 rows per block, 4 blocks); the tile's
// 16 columns of y are the B operand.  KX >= K is padded with zeros (fma(0, 0, acc) = acc).
typedef float floatx4 __attribute__((ext_vector_type(4)));

template <int KX>
struct CostMfma {
    static constexpr int KXV = KX;
    static constexpr int NKK = KX / 4;
    const float* y;
    const float* y2;
    int M, K;
    float xa[4][NKK];  // A: x[row0 + 16 rb + (l & 15)][4 kk + (l >> 4)]
    float x2o[4][4];   // norms of the output rows row0 + 16 rb + 4 (l >> 4) + r
    float yb[2][NKK];  // B: y[c0 + (l & 15)][4 kk + (l >> 4)], two tiles in flight
    float y2n[2], y2c; // norm of the issued / the begun tile's column
    bool tile_bad;     // the last finished tile holds a non-finite cost (wave-uniform)
    bool tile_nonpos;  // ... a cost that is not positive (0 or NaN; wave-uniform)
    floatx4 acc[4];
    SDTW_DEV void init(const DPParams& P, int p, int b) {
        const int l = threadIdx.x & (WAVE - 1);
        M = P.M;
        K = P.K;
        const int N = P.N, row0 = b * WAVE;
        const float* x = P.x + (int64_t)p * N * K;
        const float* x2 = P.x2 + (int64_t)p * N;
        y = P.y + (int64_t)p * M * K;
        y2 = P.y2 + (int64_t)p * M;
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
            const int row = min(row0 + 16 * rb + (l & 15), N - 1);
#pragma unroll
            for (int kk = 0; kk < NKK; ++kk) {
                const int k = 4 * kk + (l >> 4);
                xa[rb][kk] = (k < K) ? x[(int64_t)row * K + k] : 0.0f;
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) x2o[rb][r] = x2[min(row0 + 16 * rb + 4 * (l >> 4) + r, N - 1)];
        }
    }
    // operands of the tile at column c0 into slot S (a producer wave keeps two tiles of
    // loads in flight, so a tile's y rows arrive while the tile before it is multiplied)
    // (FULL: K == KX, every load inside the row, issued unconditionally: a fixed count of
    // memory operations per tile; else only the loads inside K)
    template <int S = 0, bool FULL = false>
    SDTW_DEV void issue(int c0) {
        const int l = threadIdx.x & (WAVE - 1);
        const int col = min(max(c0 + (l & 15), 0), M - 1);
        const float* yc = y + (int64_t)col * K;
#pragma unroll
        for (int kk = 0; kk < NKK; ++kk) {
            const int k = 4 * kk + (l >> 4);
            if constexpr (FULL) yb[S][kk] = yc[k];
            else yb[S][kk] = (k < K) ? yc[k] : 0.0f;
        }
        y2n[S] = y2[col];
    }
    // k-step kk of the tile's products (four independent accumulation chains)
    template <int S = 0>
    SDTW_DEV void mma(int kk) {
#pragma unroll
        for (int rb = 0; rb < 4; ++rb)
            acc[rb] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[rb][kk], yb[S][kk], acc[rb], 0, 0, 0);
    }
    template <int S = 0>
    SDTW_DEV void zero() {
        y2c = y2n[S];
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) acc[rb] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    SDTW_DEV bool prologue(float* ring, int c) {
        issue(c);
        zero();
#pragma unroll
        for (int kk = 0; kk < NKK; ++kk) mma(kk);
        finish(ring, c);
        return true;
    }
    SDTW_DEV void preload(int c) { issue(c); }
    // one k-step per recursion step, so the matrix pipe never holds up the wave's in-order
    // issue; the next tile's B operand is loaded after the last product has read it
    SDTW_DEV bool begin(float*, int) {
        zero();
        return true;
    }
    SDTW_DEV void step(int u, int, int) {
        if (u < NKK) mma(u);
    }
    SDTW_DEV void end(float* ring, int c, int cn) {
        if (U < NKK) {  // more k-steps than recursion steps
#pragma unroll
            for (int kk = U; kk < NKK; ++kk) mma(kk);
        }
        finish(ring, c);
        issue(cn);
    }
    SDTW_DEV void finish(float* ring, int c0) {
        const int l = threadIdx.x & (WAVE - 1);
        const int sl = (c0 + (l & 15)) & (CR - 1);
        float* dst = ring + 4 * (l >> 4) * CS + sl;
        // the mirror slots (sl < U) take a second copy; the other lanes store their value
        // to the same slot again, so the stores need no branch
        float* dst2 = sl < U ? dst + CR : dst;
        float sum = 0.0f;
        float mn = __builtin_inff();
#pragma unroll
        for (int rb = 0; rb < 4; ++rb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float v = clamp0(exact_cost_pre(x2o[rb][r], y2c, acc[rb][r]));
                dst[(16 * rb + r) * CS] = v;
                dst2[(16 * rb + r) * CS] = v;
                sum += v;
                mn = (v > 0.0f) ? fminf(mn, v) : 0.0f;  // NaN or 0 -> 0
            }
        tile_bad = __builtin_amdgcn_ballot_w64(!(fabsf(sum) < __builtin_inff())) != 0;
        // entries of rows >= N or columns >= M repeat the last row / column (clamped
        // indices), so the tile holds a non-positive cost iff a cell of the table does
        tile_nonpos = __builtin_amdgcn_ballot_w64(!(mn > 0.0f)) != 0;
    }
    // the same tile into the pair's cost tensor Dp (N, M): lane l's column c0 + (l & 15) of
    // rows row0 + 16 rb + 4 (l >> 4) + r, 16 lanes per 64-byte row segment.  UNIF: entries of
    // rows >= N or columns >= M were formed from the last row's / column's operands (clamped
    // indices), so they are stored to that row / column, which then receives its own bits
    // again: every lane stores every entry, with no branch (a fixed count of memory
    // operations per tile); else those entries are skipped.
    template <bool UNIF = false>
    SDTW_DEV void store_d(float* Dp, int c0, int row0, int N) const {
        const int l = threadIdx.x & (WAVE - 1);
        if constexpr (UNIF) {
            const int col = min(max(c0 + (l & 15), 0), M - 1);
#pragma unroll
            for (int rb = 0; rb < 4; ++rb)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int row = min(row0 + 16 * rb + 4 * (l >> 4) + r, N - 1);
                    Dp[(int64_t)row * M + col] = clamp0(exact_cost_pre(x2o[rb][r], y2c, acc[rb][r]));
                }
        } else {
            const int col = c0 + (l & 15);
            if ((unsigned)col >= (unsigned)M) return;
#pragma unroll
            for (int rb = 0; rb < 4; ++rb)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int row = row0 + 16 * rb + 4 * (l >> 4) + r;
                    if (row < N) Dp[(int64_t)row * M + col] = clamp0(exact_cost_pre(x2o[rb][r], y2c, acc[rb][r]));
                }
        }
    }
};

// the matrix-core width of a cost source (0: not matrix-core tiles)
template <class C>
struct KXOf : std::integral_constant<int, 0> {};
template <int KX>
struct KXOf<CostMfma<KX>> : std::integral_constant<int, KX> {};

// Fused fallback (features beyond the register-resident width, and the tiny problems whose
// reference dot is ATen's multiply-then-add kernel): each lane computes its 16 tile entries
// (the CostD entry mapping) with a scalar chain over k from memory.
template <bool MULADD>
struct CostScalar {
    const float* x;
    const float* y;
    const float* x2;
    const float* y2;
    int M, N, K, row0;
    int badc;  // first column of a finished tile holding a non-finite cost (or INT_MAX)
    SDTW_DEV int first_bad_col() const { return badc; }
    SDTW_DEV int bad_col_raw() const { return badc; }
    SDTW_DEV void init(const DPParams& P, int p, int b) {
        M = P.M;
        N = P.N;
        K = P.K;
        row0 = b * WAVE;
        badc = INT_MAX;
        x = P.x + (int64_t)p * N * K;
        y = P.y + (int64_t)p * M * K;
        x2 = P.x2 + (int64_t)p * N;
        y2 = P.y2 + (int64_t)p * M;
    }
    SDTW_DEV bool prologue(float* ring, int c) {
        finish(ring, c);
        return true;
    }
    SDTW_DEV void preload(int) {}
    SDTW_DEV bool begin(float*, int) { return true; }
    SDTW_DEV void step(int, int, int) {}
    SDTW_DEV void end(float* ring, int c, int) { finish(ring, c); }
    SDTW_DEV void finish(float* ring, int c0) {
        const int l = threadIdx.x & (WAVE - 1);
        const int col = min(max(c0 + (l & 15), 0), M - 1);
        const float* yj = y + (int64_t)col * K;
        const int sl = (c0 + (l & 15)) & (CR - 1);
        float* dst = ring + (l >> 4) * CS + sl;
        float sum = 0.0f;
        for (int k4 = 0; k4 < 16; ++k4) {
            const int row = min(row0 + 4 * k4 + (l >> 4), N - 1);
            const float* xi = x + (int64_t)row * K;
            float acc = 0.0f;
            for (int k = 0; k < K; ++k)
                acc = MULADD ? __fadd_rn(acc, __fmul_rn(xi[k], yj[k])) : __fmaf_rn(xi[k], yj[k], acc);
            const float v = clamp0(exact_cost_pre(x2[row], y2[col], acc));
            dst[4 * k4 * CS] = v;
            if (sl < U) dst[4 * k4 * CS + CR] = v;  // the mirror slots
            sum += v;
        }
        if (__builtin_amdgcn_ballot_w64(!(fabsf(sum) < __builtin_inff()))) badc = min(badc, c0);
    }
};

// Costs staged by a producer wave, one per band: matrix-core tiles (CostMfma; the producer
// then needs a SIMD of its own, since the fp32 matrix instructions take the cycles of the
// SIMD they run on) or, in the backward, tiles loaded from D (CostD; light enough to share
// the compute wave's SIMD).  The producer writes the tiles into the band's cost ring in reading order (tile t:
// columns 16t.. in the forward, M - 16 (t + 1).. in the backward, in the provider's layout)
// and counts them in ready[w]; the compute wave counts its finished groups in done[w].  The
// compute wave starts group g once tiles 0 .. g + 1 are in (its cost reads during group g
// reach tile g + 1).  The producer stores tile t once the slots it reuses (those of the
// columns 128 further on in reading order) are dead: in the forward they are last read in
// group t - 5, so done >= t - 4; in the backward they also carry g*E until group t - 4 has
// finished, whose G tile the producer itself then reads (GTile) before reusing the
// slots, so done >= t - 3.  Both leave the producer at least two groups of slack, and
// neither wait can close a cycle.  Waits are bounded like every other (timeout flag).
struct Smem;

// whether the costs of a recursion come from producer waves: matrix-core tiles in both
// directions; D tiles in the backward only (in the forward the compute wave's own loads cost
// less than the ring handshake)
template <class C, bool BWD>
struct Produced : std::false_type {};
template <int KX, bool BWD>
struct Produced<CostMfma<KX>, BWD> : std::true_type {};
template <>
struct Produced<CostD, true> : std::true_type {};

struct CostRing {
    const int* ready;
    int* done;
    int* err;
    const int* badc;  // first column of a produced tile holding a non-finite cost (LDS)
    unsigned limit;
    int known, groups, pro;
    // read after the wait for the tiles a group uses: their producer stores it first
    SDTW_DEV int first_bad_col() const { return __builtin_amdgcn_readfirstlane(lds_load(badc)); }
    SDTW_DEV int bad_col_raw() const { return lds_load(badc); }  // the load only
    SDTW_DEV void bind(const Smem& sm, int w, const DPParams& P);
    SDTW_DEV void init(const DPParams&, int, int) {}
    // false: the wait expired (flag raised); the compute wave then stops
    SDTW_DEV bool wait(int n) { return wait_at_least(ready, n, known, err, limit); }
    // the two prologue tiles
    SDTW_DEV bool prologue(float*, int) { return wait(++pro); }
    SDTW_DEV void preload(int) {}
    SDTW_DEV bool begin(float*, int) { return wait(groups + 2); }
    SDTW_DEV void step(int, int, int) {}
    SDTW_DEV void end(float*, int, int) {
        ++groups;
        if ((threadIdx.x & (WAVE - 1)) == 0) lds_publish(done, groups);
    }
};

// shared-memory layout of the DP kernels: static, the exp (/ log) tables at LDS address 0
// (the exp table, fm::kExpTabN doubles, 2 KiB: kExp2Tab for the backward's exp_tab, its
// folded form for the forward's exp_tab_abs; then, in the forward only, the log table,
// 2 fm::kLogTabN doubles, 8 KiB), so the cells' table reads fold the base into their
// immediate offset; dynamic, [ticket, counters 256 B][handoff rings][cost rings], with
// W + 1 produced/consumed counter pairs, one per handoff ring
constexpr int kTabBytesFwd = (fm::kExpTabN + 2 * fm::kLogTabN) * 8;
constexpr int kTabBytesBwd = fm::kExpTabN * 8;
struct Smem {
    unsigned char* base;  // dynamic LDS
    int W;
    size_t ring_bytes;  // handoff rings of all bands
    int tab_bytes;      // kTabBytesFwd or kTabBytesBwd
    double* tab;        // the kernel's static table array
    SDTW_DEV int* ticket() const { return reinterpret_cast<int*>(base); }
    SDTW_DEV int* prod() const { return reinterpret_cast<int*>(base) + 4; }
    SDTW_DEV int* cons() const { return reinterpret_cast<int*>(base) + 4 + (W + 1); }
    // matrix-core costs from producer waves: tiles finished per band, groups finished by the
    // band's compute wave (8 + 8 ints from int 16 of the header)
    SDTW_DEV int* ready() const { return reinterpret_cast<int*>(base) + 16; }
    SDTW_DEV int* done() const { return reinterpret_cast<int*>(base) + 24; }
    // forward, finite-input cell: ring k's producer (band k - 1, or the helper wave for
    // ring 0) no longer hands over values of the finite-input cell (ints 32 .. 36); the first
    // column of a produced cost tile holding a non-finite cost, per band (ints 40 .. 43)
    SDTW_DEV int* poison_in() const { return reinterpret_cast<int*>(base) + 32; }
    SDTW_DEV int* bad_col() const { return reinterpret_cast<int*>(base) + 40; }
    // backward, gradient mode: G tiles copied out of the band's cost ring by its gradient
    // waves, for dL/dx (ints 48 .. 51) and for dL/dy (ints 52 .. 55)
    SDTW_DEV int* gdone() const { return reinterpret_cast<int*>(base) + 48; }
    // forward, linear domain: groups staged by band w's compute wave (ints 56, 57) and
    // converted by its converter wave (58, 59); the pair's norm maxima and bad flag (60 .. 62)
    SDTW_DEV int* lin_staged() const { return reinterpret_cast<int*>(base) + 56; }
    SDTW_DEV int* lin_done() const { return reinterpret_cast<int*>(base) + 58; }
    SDTW_DEV unsigned* lin_red() const { return reinterpret_cast<unsigned*>(base) + 60; }
    // groups whose cost exponentials the exponential wave has staged (W = 1; int 63)
    SDTW_DEV int* lin_pdready() const { return reinterpret_cast<int*>(base) + 63; }
    // backward with weight waves: groups whose weights weight wave k has staged (ints 56,
    // 57, which the backward does not otherwise use)
    SDTW_DEV int* bwd_wready() const { return reinterpret_cast<int*>(base) + 56; }
    SDTW_DEV double* tables() const { return tab; }
    SDTW_DEV unsigned char* ring() const { return base + 256; }
    SDTW_DEV float* cost_ring(int w) const {
        return reinterpret_cast<float*>(base + 256 + ring_bytes) + (size_t)w * WAVE * CS;
    }
    // every thread of the workgroup, before the first barrier
    SDTW_DEV void load_tables() const {
        double* t = tables();
        for (int e = threadIdx.x; e < tab_bytes / 8; e += blockDim.x)
            t[e] = e >= fm::kExpTabN  ? fm::kLogTab[e - fm::kExpTabN]
                   : tab_bytes == kTabBytesFwd ? fm::exp2tab_folded(e)  // the forward's exp_tab_abs
                                               : fm::kExp2Tab[e];
    }
};

SDTW_DEV void CostRing::bind(const Smem& sm, int w, const DPParams& P) {
    ready = sm.ready() + w;
    done = sm.done() + w;
    badc = sm.bad_col() + w;
    err = P.err;
    limit = P.spin_limit;
    known = 0;
    groups = 0;
    pro = 0;
}

// The G tile completed by the backward group at q0 of band b: columns [M + 47 - q0,
// M + 63 - q0) of every row (each step writes g*E into the cost-ring slot of the cost it has
// just consumed).  read() takes it from the band's cost ring (lane l: column c0 + (l & 15),
// rows 4k + (l >> 4)), write() stores it as 16 coalesced 4-row blocks; a producer wave puts
// its next loads between the two, so they do not queue behind the stores.
struct GTile {
    float v[16];
    int col;  // this lane's column, or -1
    SDTW_DEV void read(const DPParams& P, const float* cring, int q0) {
        const int l = threadIdx.x & (WAVE - 1);
        col = P.M + 47 - q0 + (l & 15);
        if ((unsigned)col >= (unsigned)P.M) {
            col = -1;
            return;
        }
        const float* src = cring + (l >> 4) * CS + (col & (CR - 1));
#pragma unroll
        for (int k = 0; k < 16; ++k) v[k] = src[4 * k * CS];
    }
    SDTW_DEV void write(const DPParams& P, int p, int b) const {
        if (col < 0) return;
        const int l = threadIdx.x & (WAVE - 1);
        const int M = P.M;
        const int nrows = min(P.N - b * WAVE, WAVE);
        float* dst = P.G_out + ((int64_t)p * P.N + b * WAVE + (l >> 4)) * M + col;
        if (nrows == WAVE) {
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                *dst = v[k];
                dst += 4 * M;
            }
        } else {
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                if (4 * k + (l >> 4) < nrows) *dst = v[k];
                dst += 4 * M;
            }
        }
    }
};

// The producer wave of band b (compute wave w): tile t of the pair's cost in reading order;
// matrix-core products are issued before the wait for the ring slots, the next tile's loads
// (its B operand, or its D values) right after the store.  In the backward the G tile of
// group t - 4 is read from the slots before they are reused and stored after those loads;
// the last groups' tiles are stored after the loop.
//
// Gradient mode (GRAD, backward only): the band's gradient waves copy each G tile out of the
// slots instead, counting the tiles in gdone (one count per gradient part); the producer
// then waits for both counts >= t - 3 (which implies done >= t - 3) and stores no G tile.
// REC: set the pair's clamp record (P.clamped) where a tile holds a cost that is not
// positive; with DB only where asked for (a wave other than the producer may store D).
template <class Src, bool BWD, bool GRAD = false, bool DST = false, bool DB = false, bool REC = DST>
SDTW_DEV void producer_wave(const DPParams& P, const Smem& sm, int p, int b, int w) {
    constexpr bool MMA = !std::is_same<Src, CostD>::value;
    static_assert(!GRAD || (BWD && MMA), "gradient mode: fused backward only");
    Src c;
    c.init(P, p, b);
    float* ring = sm.cost_ring(w);
    const int* done = GRAD ? sm.gdone() + w : sm.done() + w;
    const int* done_y = sm.gdone() + 4 + w;  // gradient mode: the second part's count
    int known_y = 0;
    int* ready = sm.ready() + w;
    int known = 0;
    bool marked = false;  // the band's first non-finite cost tile has been published
    bool clamp_marked = false;  // the pair's clamp record has been set by this wave
    const int groups = P.S / U;  // groups of the compute wave
    const int T = groups + 1;    // tiles it reads
    auto col = [&](int t) { return BWD ? P.M - TC * (t + 1) : TC * t; };
    // matrix-core tiles: the operands of the next tile are loaded once this one has been
    // multiplied.  With DB (K == KX, and a kernel whose register budget holds it) there are
    // two operand slots and the loads of tile t + 2 go to slot t & 1, so each has a whole
    // tile's time to arrive; every tile then issues the same memory operations (the loads
    // at clamped columns past the table, and the stores of D in full, DST: P.D_out set), so
    // the wait before a tile's products covers only the loads it needs.
    static_assert(!DST || (MMA && !BWD), "D stores: forward matrix-core tiles only");
    static_assert(!DB || MMA, "two operand slots: matrix-core tiles only");
    if constexpr (DB) {
        // (scheduling barriers keep each slot's loads together and in slot order, which the
        // waits count on)
        c.template issue<0, true>(col(0));
        __builtin_amdgcn_sched_barrier(0);
        c.template issue<1, true>(col(1));
        __builtin_amdgcn_sched_barrier(0);
    } else if constexpr (MMA) {
        c.template issue<0>(col(0));
    } else {
        c.issue(col(0));
    }
    auto tile = [&](int t, auto slot_tag) -> bool {
        constexpr int SL = DB ? decltype(slot_tag)::value : 0;
        if constexpr (MMA) {
            c.template zero<SL>();
#pragma unroll
            for (int kk = 0; kk < Src::NKK; ++kk) c.template mma<SL>(kk);
        }
        const int need = BWD ? t - 3 : t - 4;
        if (need > 0 && (!wait_at_least(done, need, known, P.err, P.spin_limit) ||
                         (GRAD && !wait_at_least(done_y, need, known_y, P.err, P.spin_limit)))) {
            give_up<BWD>(P, p, b);
            return false;
        }
        GTile gt;
        const bool flush = BWD && !GRAD && t >= 4;
        if (flush) gt.read(P, ring, (t - 4) * U);
        if constexpr (MMA) c.finish(ring, col(t));
        else c.store(ring, col(t));
        if constexpr (MMA && !BWD) {
            // the compute wave reads this after waiting for the tile: published first
            if (c.tile_bad && !marked) {
                marked = true;
                if ((threadIdx.x & (WAVE - 1)) == 0) lds_publish(sm.bad_col() + w, col(t));
            }
        }
        if ((threadIdx.x & (WAVE - 1)) == 0) lds_publish(ready, t + 1);
        if constexpr (DB) {
            __builtin_amdgcn_sched_barrier(0);
            c.template issue<SL, true>(col(t + 2));
            __builtin_amdgcn_sched_barrier(0);
        } else if constexpr (MMA) {
            if (t + 1 < T) c.template issue<0>(col(t + 1));
        } else {
            if (t + 1 < T) c.issue(col(t + 1));
        }
        // unfused mode's cost tensor, from the same tile (forward; after the next loads, so
        // that they do not queue behind these stores), and the pair's clamp record
        // (DST: the stores are compiled in; without DB they follow P.D_out at run time; with DB,
        // REC and not DST another wave stores D, lin_exp_wave, and only the record is set here)
        if constexpr (MMA && !BWD) {
            if (DST || (!DB && P.D_out)) c.template store_d<DB>(P.D_out + (int64_t)p * P.N * P.M, col(t), b * WAVE, P.N);
            if (REC || (!DB && P.D_out)) {
                if (P.clamped && c.tile_nonpos && !clamp_marked) {
                    clamp_marked = true;
                    if ((threadIdx.x & (WAVE - 1)) == 0) P.clamped[p] = 1;
                }
            }
        }
        if (flush) gt.write(P, p, b);
        return true;
    };
    using S0_ = std::integral_constant<int, 0>;
    using S1_ = std::integral_constant<int, 1>;
    if constexpr (DB) {
        for (int t = 0; t < T; t += 2) {
            if (!tile(t, S0_{})) return;
            if (t + 1 < T && !tile(t + 1, S1_{})) return;
        }
    } else {
        for (int t = 0; t < T; ++t)
            if (!tile(t, S0_{})) return;
    }
    if (BWD && !GRAD) {
        for (int g = max(T - 4, 0); g < groups; ++g) {
            if (!wait_at_least(done, g + 1, known, P.err, P.spin_limit)) {
                give_up<BWD>(P, p, b);
                return;
            }
            GTile gt;
            gt.read(P, ring, g * U);
            gt.write(P, p, b);
        }
    }
}

// Gradient waves of band b (fused backward, gradient mode).  The gradients of the
// squared-Euclidean cost follow from E (here g*E, the upstream gradient applied) as in the
// reference's autograd (autograd_xy.py:41-49):
//   dL/dx_i = 2 (x_i sum_j E_ij - sum_j E_ij y_j),   dL/dy_j = 2 (y_j sum_i E_ij - sum_i E_ij x_i),
// formed here from the G tiles without materialising E.  The G tile of group g (the band's
// 64 rows, columns c0 = M + 47 - 16 g .. c0 + 15) is copied out of the band's cost ring as
// soon as the compute wave has finished the group, and counted (gdone), after which the
// producer may reuse the slots.  On the matrix cores,
//   * part X accumulates E Y for the band's rows over all tiles (A = E[16 rb + (l & 15)]
//     [c0 + 4 kk + (l >> 4)], B = y[c0 + 4 kk + (l >> 4)][16 fb + (l & 15)]) with the row
//     sums, and writes dL/dx once at the end;
//   * part Y forms the tile's E^T X (A = E[4 kk + (l >> 4)][c0 + (l & 15)], the G tile's own
//     layout; B = x[row0 + 4 kk + (l >> 4)][16 fb + (l & 15)], kept in registers) and column
//     sums, and adds the band's share 2 (y cs - E^T X) to dL/dy (zeroed by the prep launch)
//     with fire-and-forget atomics.  The bands' shares of an entry therefore meet in the
//     order they arrive: dL/dy can differ in the last bits between runs (dL/dx cannot).
//     Ordering the bands (each waiting for the band below to flag a tile once its additions
//     have returned) costs more than the whole recursion at wide features: the returns and
//     the flag polls sit in every tile of the chain.  Callers that need run-to-run identical
//     bits take the E path (sdtw_set_deterministic).
// One wave does both parts (PART 3), or two waves one each (PART 1, 2), each with its own
// count (gdone x / y).  The next tile's y operands are loaded before the wait for the
// compute wave, so no memory latency sits between two tiles.  Entries of a tile outside
// the table (rows >= N, columns outside [0, M)) are zeroed.  Waits are bounded; a wave that
// gives up marks the pair's results NaN.
constexpr int kGradPartX = 1, kGradPartY = 2;
constexpr int kGdoneIdle = 1 << 30;  // count of a part with nothing to do

template <int KX, int PART>
SDTW_DEV void grad_wave(const DPParams& P, const Smem& sm, int p, int b, int w) {
    constexpr int FB = KX >= 16 ? KX / 16 : 1;  // 16-feature blocks of the outputs
    constexpr bool HAS_X = (PART & kGradPartX) != 0, HAS_Y = (PART & kGradPartY) != 0;
    const int l = threadIdx.x & (WAVE - 1);
    const int li = l & 15, lq = l >> 4;
    int* gdx = sm.gdone() + w;
    int* gdy = sm.gdone() + 4 + w;
    const bool want_gx = HAS_X && P.gx_out != nullptr;
    const bool want_gy = HAS_Y && P.gy_out != nullptr;
    if (!want_gx && !want_gy) {  // nothing to form: the producer need not wait for this wave
        if (l == 0) {
            if (HAS_X) lds_publish(gdx, kGdoneIdle);
            if (HAS_Y) lds_publish(gdy, kGdoneIdle);
        }
        return;
    }
    if (l == 0) {  // a part this wave owns but does not form
        if (HAS_X && !want_gx) lds_publish(gdx, kGdoneIdle);
        if (HAS_Y && !want_gy) lds_publish(gdy, kGdoneIdle);
    }
    const int N = P.N, M = P.M, K = P.K;
    const int row0 = b * WAVE;
    const int groups = P.S / U;
    const float* x = P.x + (int64_t)p * N * K;
    const float* y = P.y + (int64_t)p * M * K;
    const float* cring = sm.cost_ring(w);
    const int* done = sm.done() + w;
    float* gy = want_gy ? P.gy_out + (int64_t)p * M * K : nullptr;

    float xB[HAS_Y ? 16 : 1][FB];
    if constexpr (HAS_Y) {
#pragma unroll
        for (int kk = 0; kk < 16; ++kk)
#pragma unroll
            for (int fb = 0; fb < FB; ++fb) {
                const int row = row0 + 4 * kk + lq, f = 16 * fb + li;
                xB[kk][fb] = (want_gy && row < N && f < K) ? x[(int64_t)row * K + f] : 0.0f;
            }
    }
    floatx4 gacc[HAS_X ? 4 : 1][FB];
    float rsp[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (HAS_X) {
#pragma unroll
        for (int rb = 0; rb < 4; ++rb)
#pragma unroll
            for (int fb = 0; fb < FB; ++fb) gacc[rb][fb] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    // the y operands of tile g: B of E Y (yb) and the y of 2 (y cs - E^T X) (yc)
    auto live_tile = [&](int g) { const int c0 = M + 47 - g * U; return c0 < M && c0 + 15 >= 0; };
    auto load_y = [&](int g, float (&yb)[4][FB], float (&yc)[4][FB]) {
        const int c0 = M + 47 - g * U;
        const bool live = g < groups && live_tile(g);
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int fb = 0; fb < FB; ++fb) {
                const int f = 16 * fb + li;
                const int cb = c0 + 4 * q + lq, cc = c0 + 4 * lq + q;
                const bool okb = HAS_X && live && want_gx && (unsigned)cb < (unsigned)M && f < K;
                const bool okc = HAS_Y && live && want_gy && (unsigned)cc < (unsigned)M && f < K;
                yb[q][fb] = okb ? y[(int64_t)cb * K + f] : 0.0f;
                yc[q][fb] = okc ? y[(int64_t)cc * K + f] : 0.0f;
            }
    };
    float yBn[4][FB], yCn[4][FB];
    load_y(0, yBn, yCn);
    int known = 0;
    for (int g = 0; g < groups; ++g) {
        const int c0 = M + 47 - g * U;
        const bool live = live_tile(g);
        float yB[4][FB], yC[4][FB];
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int fb = 0; fb < FB; ++fb) {
                yB[q][fb] = yBn[q][fb];
                yC[q][fb] = yCn[q][fb];
            }
        load_y(g + 1, yBn, yCn);
        if (!wait_at_least(done, g + 1, known, P.err, P.spin_limit)) {
            give_up_bwd(P, p, b);
            return;
        }
        float eT[HAS_Y ? 16 : 1], eA[HAS_X ? 4 : 1][4];
        if constexpr (HAS_Y) {
            const int ct = c0 + li;
            const bool ct_ok = live && (unsigned)ct < (unsigned)M;
            const float* src = cring + lq * CS + (ct & (CR - 1));
#pragma unroll
            for (int k = 0; k < 16; ++k) eT[k] = (ct_ok && row0 + 4 * k + lq < N) ? src[4 * k * CS] : 0.0f;
        }
        if constexpr (HAS_X) {
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                const int ca = c0 + 4 * kk + lq;
                const bool ca_ok = live && (unsigned)ca < (unsigned)M;
                const float* srcA = cring + li * CS + (ca & (CR - 1));
#pragma unroll
                for (int rb = 0; rb < 4; ++rb)
                    eA[rb][kk] = (ca_ok && row0 + 16 * rb + li < N) ? srcA[16 * rb * CS] : 0.0f;
            }
        }
        // the slots may be reused once these reads are performed (LDS operations of a wave
        // are performed in order, the count after them)
        if (l == 0) {
            if (want_gx) lds_publish(gdx, g + 1);
            if (want_gy) lds_publish(gdy, g + 1);
        }
        if (!live) continue;
        if constexpr (HAS_X) {
            if (want_gx) {
#pragma unroll
                for (int kk = 0; kk < 4; ++kk)
#pragma unroll
                    for (int rb = 0; rb < 4; ++rb)
#pragma unroll
                        for (int fb = 0; fb < FB; ++fb)
                            gacc[rb][fb] = __builtin_amdgcn_mfma_f32_16x16x4f32(eA[rb][kk], yB[kk][fb], gacc[rb][fb], 0, 0, 0);
#pragma unroll
                for (int rb = 0; rb < 4; ++rb) rsp[rb] += (eA[rb][0] + eA[rb][1]) + (eA[rb][2] + eA[rb][3]);
            }
        }
        if constexpr (HAS_Y) {
            if (want_gy) {
                floatx4 pg[FB];
#pragma unroll
                for (int fb = 0; fb < FB; ++fb) pg[fb] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int kk = 0; kk < 16; ++kk)
#pragma unroll
                    for (int fb = 0; fb < FB; ++fb)
                        pg[fb] = __builtin_amdgcn_mfma_f32_16x16x4f32(eT[kk], xB[kk][fb], pg[fb], 0, 0, 0);
                // column sums: lane l holds rows 4 k + (l >> 4) of column c0 + (l & 15)
                float cs = 0.0f;
#pragma unroll
                for (int k = 0; k < 16; ++k) cs += eT[k];
                cs += __shfl_xor(cs, 16);
                cs += __shfl_xor(cs, 32);
                float csr[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) csr[r] = __shfl(cs, 4 * lq + r);
#pragma unroll
                for (int r = 0; r < 4; ++r)
#pragma unroll
                    for (int fb = 0; fb < FB; ++fb) {
                        const int col = c0 + 4 * lq + r, f = 16 * fb + li;
                        if ((unsigned)col < (unsigned)M && f < K)
                            (void)unsafeAtomicAdd(gy + (int64_t)col * K + f,
                                                  2.0f * (yC[r][fb] * csr[r] - pg[fb][r]));
                    }
            }
        }
    }
    if constexpr (HAS_X) {
        if (want_gx) {
            float* gx = P.gx_out + (int64_t)p * N * K;
#pragma unroll
            for (int rb = 0; rb < 4; ++rb) {
                // lanes l, l ^ 16, l ^ 32, l ^ 48 hold the four column quarters of row
                // 16 rb + (l & 15)
                float rs = rsp[rb];
                rs += __shfl_xor(rs, 16);
                rs += __shfl_xor(rs, 32);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float rsr = __shfl(rs, 4 * lq + r);
                    const int row = row0 + 16 * rb + 4 * lq + r;
#pragma unroll
                    for (int fb = 0; fb < FB; ++fb) {
                        const int f = 16 * fb + li;
                        if (row < N && f < K) {
                            const int64_t e = (int64_t)row * K + f;
                            gx[e] = 2.0f * (x[e] * rsr - gacc[rb][fb][r]);
                        }
                    }
                }
            }
        }
    }
}

// W + 1 handoff rings: one per band plus the helper wave's
// (forward: then the workgroup's staging block of kStageFwd doubles, see fwd_band; at W = 4
// it fills the 160 KiB of LDS exactly)
constexpr int kStageFwd = WAVE + 2 * U;
SDTW_HD size_t ring_bytes_fwd(int W) { return ((size_t)(W + 1) * RS + kStageFwd) * sizeof(double); }
// (backward: then the workgroup's staging block of kStageBwd bytes, see bwd_band)
constexpr int kStageBwd = 12 * WAVE + 16 * U + 16 * U;
SDTW_HD size_t ring_bytes_bwd(int W) { return (size_t)(W + 1) * RS * sizeof(float4) + kStageBwd; }
// Backward with weight waves (W = 1): after the handoff rings and the staging block, the
// weight stage, kWBufs groups of U steps x 64 lanes of float4 (a, b, c, unused), so that
// each lane's per-step read and write is one 16-byte access, conflict-free.  Under exact
// arithmetic the weights are doubles: two such planes, double2 (a, b) then (c, NaN flag).
constexpr int kWBufs = 3;
constexpr size_t kWStageBytes = (size_t)kWBufs * U * WAVE * sizeof(float4);  // per plane

// Forward in the scaled linear domain (fwd_band_lin): LDS after the staging block.  The
// handoff rings keep their p values in the slots of the log-domain rings; their exponents
// follow the staging block as W + 1 rings of RS ints; then each band's converter stage: two
// buffers (groups alternate) of 64 lane rows of kLinRow entries (p as doubles, then e as
// ints; the row pitch of 17 keeps a wave's accesses to one column conflict-free).
constexpr int kLinNeg = -(1 << 30);  // exponent of a zero value (R = +inf)
constexpr int kLinRow = U + 1;
constexpr int kLinBuf = WAVE * kLinRow;
// (W = 1 adds the cost-exponential stage: kPdBufs buffers of 64 lane rows of kLinRow (pD,
// eD), filled by the workgroup's exponential wave, lin_exp_wave)
constexpr int kPdBufs = 3;
SDTW_HD size_t lin_extra_bytes(int W) {
    return (size_t)(W + 1) * RS * 4 + (size_t)W * 2 * kLinBuf * 12 + (W == 1 ? (size_t)kPdBufs * kLinBuf * 12 : 0);
}
SDTW_DEV int* lin_ering(const Smem& sm) { return reinterpret_cast<int*>(sm.ring() + ring_bytes_fwd(sm.W)); }
SDTW_DEV float4* bwd_wstage(const Smem& sm) { return reinterpret_cast<float4*>(sm.ring() + ring_bytes_bwd(sm.W)); }
SDTW_DEV double* lin_stage_p(const Smem& sm, int w, int k) {
    return reinterpret_cast<double*>(lin_ering(sm) + (sm.W + 1) * RS) + (w * 2 + k) * kLinBuf;
}
SDTW_DEV int* lin_stage_e(const Smem& sm, int w, int k) {
    return reinterpret_cast<int*>(lin_stage_p(sm, sm.W, 0)) + (w * 2 + k) * kLinBuf;
}
SDTW_DEV double* lin_pd_p(const Smem& sm, int k) {
    return reinterpret_cast<double*>(lin_stage_e(sm, sm.W, 0)) + k * kLinBuf;
}
SDTW_DEV int* lin_pd_e(const Smem& sm, int k) { return reinterpret_cast<int*>(lin_pd_p(sm, kPdBufs)) + k * kLinBuf; }
// Cross-workgroup rows of the forward: 8-byte entries (R), or in a launch that can take the
// linear domain 16-byte ones, (p, then e and the tag 1), written and read as two 64-bit
// halves, each whole or empty.  All rows of such a launch are 16-byte pitched, so the rows
// of its log-domain pairs (8-byte entries, first half) and linear-domain pairs do not overlap.
SDTW_HD int64_t fwd_row_pitch(const DPParams& P) { return P.lin ? 2 * (int64_t)P.RW : P.RW; }
SDTW_DEV void glb_put_lin(double2* q, double pv, int ev) {
    unsigned long long* a = reinterpret_cast<unsigned long long*>(q);
    __hip_atomic_store(a, (unsigned long long)__double_as_longlong(pv), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(a + 1, (1ull << 32) | (unsigned)ev, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

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

    double* lring = reinterpret_cast<double*>(sm.ring());
    const double* tabE = sm.tables();     // exp / log tables in LDS
    const double* tabL = tabE + fm::kExpTabN;
    float* cring = sm.cost_ring(w);
    const float* crow = cring + l * CS;  // my row of the cost ring
    // LDS ring k carries the input of band k of this workgroup: ring 0 is filled by the
    // workgroup's helper wave from the previous workgroup, ring k > 0 by band k - 1.
    const bool out_lds = (b + 1 < nb) && (w + 1 < W);
    const bool out_glb = (b + 1 < nb) && (w + 1 == W);
    // cross-workgroup row of this workgroup: RW = M + 2*RPAD entries, column c at RPAD + c
    double* gout = P.gring + ((int64_t)p * G + g) * fwd_row_pitch(P) + RPAD;
    const double* lin = lring + w * RS;
    double* lout = lring + (w + 1) * RS;
    const int* lin_flag = sm.prod() + w;
    // Last row to the band below: at every step each lane stores its value with one wide LDS
    // write, so no cross-lane moves collect lane 63's values.  Lane 63's store (column
    // s0 + u - 63 at step s0 + u) goes to the handoff ring, or, for the band that hands over
    // through global memory (the workgroup's last, w = W - 1), to entries WAVE + U ..
    // WAVE + 2U - 1 of the workgroup's staging block.  Every other store (lane l < 63, and
    // lane 63 of a pair's last band) goes to entry l + u of the block's first WAVE + U
    // entries, which all waves share and nothing reads.
    double* stage = lring + (W + 1) * RS;

    float* Rt = P.R + ((int64_t)p * nb + b) * S * WAVE + l;

    int known_in = 0;    // columns of the band above known to be in the LDS ring
    int known_free = 0;  // columns of my LDS ring known to be consumed
    double left = INF;
    double diag = (b == 0 && l == 0) ? 0.0 : INF;
    double prev = INF;   // this lane's value one step ago (sent to lane l+1 by DPP)

    double up_cur[U];
    float d_cur[U], d_nxt[U];

    // Band above: columns [c0, c0 + U) of its last row from the LDS ring, for lane 0.  The
    // ring is read whether or not it waits: band 0's ring holds +inf throughout (set at
    // kernel start, never written), and past column M - 1 lane 0 is inactive.
    // The finite-input flags are read in the same LDS round trip as the count (each is stored
    // before the count it guards): pz, the band above no longer hands over finite-cell values;
    // bc, the first column of a cost tile with a non-finite cost (read after the cost wait).
    auto fetch_lds = [&](int c0, double* dst, int& pz, int& bc) -> bool {
        const bool live = b > 0 && c0 < M;
        const int need = min(c0 + U, M);
        int cnt = lds_load(lin_flag);
        pz = lds_load(sm.poison_in() + w);
        bc = cost.bad_col_raw();
        cnt = __builtin_amdgcn_readfirstlane(cnt);
        pz = __builtin_amdgcn_readfirstlane(pz);
        bc = __builtin_amdgcn_readfirstlane(bc);
        known_in = max(known_in, cnt);
        if (live && known_in < need) {
            if (!wait_at_least(lin_flag, need, known_in, P.err, P.spin_limit)) return false;
            pz = __builtin_amdgcn_readfirstlane(lds_load(sm.poison_in() + w));
        }
        __atomic_signal_fence(__ATOMIC_SEQ_CST);  // the ring reads stay after the count
        const double* blk = lin + hslot(c0 + 1);  // entries c0 + 1 .. c0 + U - 1
        dst[0] = lin[hslot(c0)];
        const double2* src = reinterpret_cast<const double2*>(blk);
#pragma unroll
        for (int k = 0; k < U / 2 - 1; ++k) {
            const double2 v = src[k];
            dst[1 + 2 * k] = v.x;
            dst[2 + 2 * k] = v.y;
        }
        dst[U - 1] = blk[U - 2];
        if (live && l == 0) lds_publish(sm.cons() + w, need);
        return true;
    };
    // Where this lane's per-step store of the group at s0 goes (entry u for step u).  Lane
    // 63's ring stores are unconditional: slots of columns < 0 or >= M are never read before
    // being rewritten or at all.
    // (the edge lane's address is wave-uniform, so one per-lane select picks it)
    auto step_dst = [&](int s0) -> double* {
        double* edge = out_lds ? lout + hslot(s0 - (WAVE - 1)) : (out_glb ? stage + (WAVE + U) : stage + l);
        return l == WAVE - 1 ? edge : stage + l;
    };
    // Hand the last row's columns computed by the group at s0 (lane 63 computed column
    // s0 + u - 63 at step s0 + u) to the band below: publish the ring entries lane 63 stored,
    // or copy the staged ones to the cross-workgroup row.
    auto handover = [&](int s0) {
        const int c0 = s0 - (WAVE - 1);
        if (out_lds) {
            if (l == WAVE - 1) lds_publish(sm.prod() + (w + 1), min(max(s0 + U - (WAVE - 1), 0), M));
        } else if (l >= WAVE - U) {
            const int u = l - (WAVE - U);
            // columns in [-63, M + 15]: inside the row's padding, no test needed
            glb_put(gout + c0 + u, stage[WAVE + U + u]);
        }
    };

    // Pipeline of one group (all of it straight-line code between the waits):
    //   - costs of this group were read from the ring during the previous group;
    //   - the tile two groups ahead takes its operands (begin), the one three groups ahead
    //     starts loading (issue, after step 3), and the tile two ahead lands in the ring
    //     (finish, after the last step), so the ring holds tiles up to s0 + 2*TC;
    //   - the band above's row is read from the LDS ring at the group start (reading it
    //     a group ahead would add a group of lag per band boundary).
    // Tiles past the table are harmless: loads are clamped and their slots are not live.
    if (!cost.prologue(cring, 0) || !cost.prologue(cring, TC)) {
        give_up_fwd(P, p);
        return;
    }
    cost.preload(2 * TC);
    {
        const float* dn = crow + ((-l) & (CR - 1));  // U consecutive slots (mirrored past CR)
#pragma unroll
        for (int u = 0; u < U; ++u) d_nxt[u] = dn[u];
    }

    // One group of U steps from s0.  Returns 0, -1 if a wait expired, or 1 (FINITE bodies
    // only) if the group's inputs are not all finite: nothing has been computed then, and
    // the caller runs the group again, and the rest of the band, with the general cell.
    // Every step of the group start is idempotent (copies, waits, counter publications of
    // the same values), so running it twice is harmless.
    //   FINITE: fwd_cell_exact_finite, valid while every cost the band uses and every entry
    //     of the band above that lane 0 uses is finite (checked here per group through flags
    //     that the cost providers, the band above and the helper wave keep);
    //   INTERIOR: every lane is inside the table for all U steps (a full band, columns
    //     s0 - 63 .. s0 + U - 1 within [0, M)), so no step needs the inactive masking.
    // Separate loops run the bodies (a branch per group between two unrolled bodies would
    // join their loop-carried registers).
    auto group = [&](int s0, auto finite_tag, auto interior_tag) -> int {
        constexpr bool FINITE = decltype(finite_tag)::value;
        constexpr bool INTERIOR = decltype(interior_tag)::value;
#pragma unroll
        for (int u = 0; u < U; ++u) d_cur[u] = d_nxt[u];
        int pz, bc;
        if (!cost.begin(cring, s0 + 2 * TC) || !fetch_lds(s0, up_cur, pz, bc)) return -1;
        if constexpr (FINITE) {
            // the group's costs reach column s0 + U - 1; the band above's entries come from a
            // band that has left the finite-input cell, or (across workgroups) were seen
            // non-finite by the helper wave
            if (bc <= s0 + U - 1 || (b > 0 && pz != 0)) return 1;
        }
        // this group writes columns up to s0 + U - 64 of my last row; writing column c
        // reuses the slot of column c - RS, which the consumer must have taken
        if (out_lds) {
            const int need_free = s0 + U - WAVE + 1 - RS;
            if (need_free > 0 && !wait_at_least(sm.cons() + (w + 1), need_free, known_free, P.err, P.spin_limit))
                return -1;
        }
        float* Rg = Rt + (int64_t)s0 * WAVE;
        double* dst = step_dst(s0);
        const float* dn = crow + ((s0 + TC - l) & (CR - 1));  // next group's costs
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const double up = shr1(up_cur[u], prev);
            double r;
            if constexpr (INTERIOR) {
                r = fwd_cell_exact_finite(diag, up, left, d_cur[u], gamma, inv_gamma, tabE, tabL);
            } else {
                const int j = s0 + u - l;
                const bool act = row_ok && (unsigned)j < (unsigned)M;
                bool keep = act;
                if (BAND) keep = keep && !out_of_band(bw, i, j);
                double cand;
                if constexpr (FINITE) {
                    cand = fwd_cell_exact_finite(diag, up, left, d_cur[u], gamma, inv_gamma, tabE, tabL);
                } else if (EXACT) {
                    cand = fwd_cell_exact(diag, up, left, d_cur[u], gamma, inv_gamma, tabE, tabL);
                } else {
                    cand = fwd_cell_hw(diag, up, left, d_cur[u], c2, ngl);
                }
                // inactive lanes publish +inf: before its first column a lane's left/up are
                // the +inf padding, out-of-band cells stay +inf (launcher.py:310, :315)
                r = keep ? cand : INF;
            }
            left = r;
            diag = up;
            prev = r;
            dst[u] = r;
            Rg[u * WAVE] = (float)r;
            // next group's costs, and the tile work, between the steps
            d_nxt[u] = dn[u];
            cost.step(u, s0 + 2 * TC, s0 + 3 * TC);
        }
        cost.end(cring, s0 + 2 * TC, s0 + 3 * TC);
        if (out_lds || out_glb) handover(s0);
        return 0;
    };
    using T_ = std::true_type;
    using F_ = std::false_type;
    int s0 = 0;
    int rc = 0;
    if constexpr (EXACT && !BAND) {
        // interior groups: s0 >= 64 (column s0 - 63 > 0 for lane 63) and s0 + U <= M, in a
        // full band
        const bool full = (b + 1) * WAVE <= N;
        const int q_in = min(full ? WAVE : S, S);
        const int q_out = full ? max((M - U) / U * U + U, WAVE) : S;
        for (; s0 < q_in; s0 += U)
            if ((rc = group(s0, T_{}, F_{})) != 0) break;
        if (rc == 0)
            for (; s0 < min(q_out, S); s0 += U)
                if ((rc = group(s0, T_{}, T_{})) != 0) break;
        if (rc == 0)
            for (; s0 < S; s0 += U)
                if ((rc = group(s0, T_{}, F_{})) != 0) break;
        if (rc < 0) return give_up_fwd(P, p);
        // the band below (same workgroup) leaves the finite-input cell before it reads a
        // value of this band's general cell
        if (rc == 1 && out_lds && l == 0) lds_publish(sm.poison_in() + (w + 1), 1);
    }
    // the general cell: the band, the fast arithmetic, and a band whose inputs are not all
    // finite (from the group that found it, s0, onwards)
    for (; s0 < S; s0 += U)
        if (group(s0, F_{}, F_{}) < 0) return give_up_fwd(P, p);
    // out[p] = R[N-1, M-1] as stored (step M-1+l of this lane, written by this lane)
    if (i == N - 1) P.out[p] = Rt[(int64_t)(M - 1 + l) * WAVE];
}

// Helper wave of a workgroup with a band boundary above (forward) or below (backward) it
// in another workgroup.  It polls that workgroup's cross-workgroup row, 64 entries per load,
// copies the leading entries already written into LDS ring `k` and publishes them through
// the ring's counter, exactly like an in-workgroup producer band.  The compute waves thus
// never wait on global memory they did not load themselves.  Back-pressure as for a band:
// entry e reuses the slot of e - RS, which the consumer must have taken.  Bounded: a poll
// that finds nothing new sleeps, and too many in a row raise the timeout flag.
template <class T>
SDTW_DEV void helper_wave(const DPParams& P, const Smem& sm, const T* gin, int k) {
    const int l = threadIdx.x & (WAVE - 1);
    const int M = P.M;
    T* ring = reinterpret_cast<T*>(sm.ring()) + k * RS;
    int known_free = 0;
    unsigned spins = 0;
    for (int c = 0; c < M;) {
        const int need_free = c + WAVE - RS;
        if (need_free > 0 && !wait_at_least(sm.cons() + k, need_free, known_free, P.err, P.spin_limit)) return;
        const int e = c + l;
        T v;
        bool empty = false;
        if (e < M) {
            v = glb_get_entry(gin + e);
            empty = entry_empty(v);
        }
        const unsigned long long miss = __ballot(empty);
        const int n = miss ? (int)__builtin_ctzll(miss) : WAVE;  // leading written entries
        if (l < n && e < M) ring[hslot(e)] = v;
        if constexpr (std::is_same<T, double>::value) {
            // a non-finite entry: the consumer band must leave the finite-input cell before
            // it reads this one (flag stored before the count that covers it)
            const bool nf = l < n && e < M && !(fabs(v) < dinf());
            if (__builtin_amdgcn_ballot_w64(nf) && l == 0) lds_publish(sm.poison_in() + k, 1);
        }
        if (n > 0) {
            c = min(c + n, M);
            if (l == 0) lds_publish(sm.prod() + k, c);
            spins = 0;
        } else {
            if (spins++ >= P.spin_limit) {
                raise_timeout(P.err);  // the compute wave it feeds then gives up
                return;
            }
            __builtin_amdgcn_s_sleep(2);
        }
    }
}

// Waves of a workgroup: compute waves 0 .. W-1 (one band each) and the helper wave W; with
// staged costs, the producer waves W .. 2W-1 (of bands 0 .. W-1) and the helper wave 2W.
// With W = 2, matrix-core producers take the SIMDs the compute waves leave free under
// round-robin wave placement; with W = 4 (large batches, see the launcher) every producer
// shares its compute wave's SIMD, as D producers (backward) always do.
// ---------------------------------------------------------------------------------------
// Forward in the scaled linear domain.
//
// The recursion R = d + softmin(R_diag, R_up, R_left) (launcher.py:317-322) is the log of a
// linear one: with P = exp(-R / gamma),  P(i,j) = exp(-d(i,j) / gamma) (P_diag + P_up +
// P_left).  Each P is held as p 2^e (p a double, e an int), so nothing underflows: a step
// aligns the three predecessors to their largest exponent (ldexp, exact), adds them and
// multiplies by the cost's exponential pD 2^eD.  No exp or log is on the dependency chain:
// pD depends on the cost alone, and a converter wave per band turns p 2^e back into
// R = -gamma log(p 2^e) for the R table, on a SIMD of its own.  p is renormalised (frexp)
// once per group and stays within [0.48, 2^42) in between; a zero (R = +inf: the padding,
// inactive lanes) is (0, kLinNeg), which no maximum of exponents picks over a live value.
// Rounding: P carries a relative error of a few units in the last place per cell, that is R
// an absolute one of a few gamma 2^-53, below the ulp(R) per cell of the log-domain form;
// R is rounded once to fp32 by the converter.  A pair takes this path when its row norms
// are finite and bound every cost so that no exponent nears 2^29 (lin_pair_ok); the others
// run fwd_band in the same launch.
// ---------------------------------------------------------------------------------------

// exp(-d / gamma) = pD 2^eD, pD in [0.998, 2.003): exp_tab_abs's reduction with the power
// of two kept apart (T is the folded table: entry j << 12 is put back into its high word).
SDTW_DEV void lin_cost(float d, double ninv_gamma, const double* T, double& pD, int& eD) {
    const double xc = (double)d * ninv_gamma;
    const double tc = fm::exp_tab_abs_tc(xc);
    const int k = fm::lo_word(tc);
    const int j = k & (fm::kExpTabN - 1);
    const double tf = T[j];
    const double em1 = fm::exp_tab_abs_em1(xc, tc);
    const double t = fm::from_words(fm::hi_word(tf) + (j << 12), fm::lo_word(tf));
    pD = ::fma(t, em1, t);
    eD = k >> 8;  // floor(k / 256)
}

// R = -gamma log(p 2^e): p = m 2^k with m in [1, 2), log m by log_tab_1to3, (e + k - 1) ln2
// in two parts (each fma forms its product exactly), then one rounding for the product with
// -gamma.  p = 0 gives +inf.
SDTW_DEV double lin_to_R(double pv, int ev, double ngamma, const double* L) {
    const int k = __builtin_amdgcn_frexp_exp(pv);
    const double m = 2.0 * __builtin_amdgcn_frexp_mant(pv);
    const double ef = (double)(ev + k - 1);
    const double t = ::fma(ef, fm::kLn2Hi, ::fma(ef, fm::kLn2Lo, fm::log_tab_1to3(m, L)));
    return pv == 0.0 ? dinf() : ngamma * t;
}

// Whether pair p takes the linear domain: every row norm finite, and the cost bound
// d <= 2 (|x_i|^2 + |y_j|^2) (2.01 for the fp32 evaluation) keeps each cost's k = 256 n + j
// below 2^30 and every exponent along a path of N + M + 1 cells below 2^29 in magnitude.
// Called by every thread of the workgroup (it holds a barrier); the workgroups of a pair
// read the same norms and take the same decision.
SDTW_DEV bool lin_pair_ok(const DPParams& P, const Smem& sm, int p) {
    unsigned* red = sm.lin_red();  // zeroed before the kernel's first barrier
    float mx = 0.0f, my = 0.0f;
    bool bad = false;
    for (int e = threadIdx.x; e < P.N; e += blockDim.x) {
        const float v = P.x2[(int64_t)p * P.N + e];
        bad = bad || !(v <= 1e30f);
        mx = fmaxf(mx, v);
    }
    for (int e = threadIdx.x; e < P.M; e += blockDim.x) {
        const float v = P.y2[(int64_t)p * P.M + e];
        bad = bad || !(v <= 1e30f);
        my = fmaxf(my, v);
    }
    if (bad) atomicOr(red + 2, 1u);
    atomicMax(red, __float_as_uint(mx));  // non-negative floats order as their bits
    atomicMax(red + 1, __float_as_uint(my));
    __syncthreads();
    if (red[2] != 0u) return false;
    const double xmax = 2.01 * ((double)__uint_as_float(red[0]) + (double)__uint_as_float(red[1])) * P.inv_gamma;
    return xmax * fm::kInvLn2x256 < 1073741824.0 &&
           (double)(P.N + P.M + 2) * (xmax * 1.4426950408889634 + 4.0) < 536870912.0;
}

// PD: the cost exponentials come staged from the workgroup's exponential wave (W = 1)
// rather than from the compute wave's own evaluation of the cost ring.
template <bool PD, class Cost>
SDTW_DEV void fwd_band_lin(const DPParams& P, Cost& cost, const Smem& sm, int p, int g, int w) {
    const int l = threadIdx.x & (WAVE - 1);
    const int W = P.W, G = P.G, nb = P.nb, N = P.N, M = P.M, S = P.S;
    const int b = g * W + w;
    const bool row_ok = b * WAVE + l < N;
    const double ninv_gamma = -P.inv_gamma;
    const double* tabE = sm.tables();
    float* cring = sm.cost_ring(w);
    const float* crow = cring + l * CS;
    const bool out_lds = (b + 1 < nb) && (w + 1 < W);
    const bool out_glb = (b + 1 < nb) && (w + 1 == W);
    double* pring = reinterpret_cast<double*>(sm.ring());
    int* ering = lin_ering(sm);
    const double* in_p = pring + w * RS;
    const int* in_e = ering + w * RS;
    double* out_p = pring + (w + 1) * RS;
    int* out_e = ering + (w + 1) * RS;
    const int* in_flag = sm.prod() + w;
    int* staged = sm.lin_staged() + w;
    const int* conv = sm.lin_done() + w;
    const int* pdready = sm.lin_pdready();
    const int groups = S / U;

    int known_in = 0, known_free = 0, known_conv = 0, known_pd = 0;
    double lp = 0.0;  // this lane's value one step ago (its left; lane l+1's up by DPP)
    int le = kLinNeg;
    double dp = (b == 0 && l == 0) ? 1.0 : 0.0;  // diagonal: R[0,0] = 0 above-left of cell (0, 0)
    int de = (b == 0 && l == 0) ? 0 : kLinNeg;
    double up_p[U];
    int up_e[U];
    float d_cur[U], d_nxt[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {  // band 0: the +inf row above the table
        up_p[u] = 0.0;
        up_e[u] = kLinNeg;
    }

    // Band above: entries c0 .. c0 + U - 1 of its last row (lane 0's up values) from the LDS
    // ring, as fwd_band's fetch_lds.  Past column M - 1 lane 0 is inactive.
    auto fetch = [&](int c0) -> bool {
        if (b == 0) return true;
        const bool live = c0 < M;
        const int need = min(c0 + U, M);
        if (live && known_in < need && !wait_at_least(in_flag, need, known_in, P.err, P.spin_limit))
            return false;
        __atomic_signal_fence(__ATOMIC_SEQ_CST);  // the ring reads stay after the count
        const double* blk = in_p + hslot(c0 + 1);  // entries c0 + 1 .. c0 + U - 1
        up_p[0] = in_p[hslot(c0)];
        const double2* src = reinterpret_cast<const double2*>(blk);
#pragma unroll
        for (int k = 0; k < U / 2 - 1; ++k) {
            const double2 v = src[k];
            up_p[1 + 2 * k] = v.x;
            up_p[2 + 2 * k] = v.y;
        }
        up_p[U - 1] = blk[U - 2];
        const int* eblk = in_e + hslot(c0 + 1);  // a multiple of 16 slots: 16-byte aligned
        up_e[0] = in_e[hslot(c0)];
        const int4* esrc = reinterpret_cast<const int4*>(eblk);
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            const int4 v = esrc[k];
            up_e[1 + 4 * k] = v.x;
            up_e[2 + 4 * k] = v.y;
            up_e[3 + 4 * k] = v.z;
            up_e[4 + 4 * k] = v.w;
        }
        up_e[13] = eblk[12];
        up_e[14] = eblk[13];
        up_e[15] = eblk[14];
        if (live && l == 0) lds_publish(sm.cons() + w, need);
        return true;
    };

    // One group of U steps from s0 (pipeline as fwd_band's).  Each step's values go to the
    // lane's row of the converter stage (buffer (s0 / U) & 1), except lane 63's when a band
    // of this workgroup is below: those go to the handoff ring, where the converter reads
    // them too.  A band below in the next workgroup gets them from the converter.
    // INTERIOR: every lane inside the table for all U steps (no masking).
    auto group = [&](int s0, auto interior_tag) -> int {
        constexpr bool INTERIOR = decltype(interior_tag)::value;
#pragma unroll
        for (int u = 0; u < U; ++u) d_cur[u] = d_nxt[u];
        // the counters this group start checks, loaded together (one LDS round trip; each
        // wait below then polls only if its cached count falls short)
        {
            const int v_ready = lds_load(cost.ready);
            const int v_in = lds_load(in_flag);
            const int v_conv = lds_load(conv);
            const int v_free = lds_load(sm.cons() + (w + 1));
            const int v_pd = PD ? lds_load(pdready) : 0;
            known_pd = max(known_pd, __builtin_amdgcn_readfirstlane(v_pd));
            cost.known = max(cost.known, __builtin_amdgcn_readfirstlane(v_ready));
            known_in = max(known_in, __builtin_amdgcn_readfirstlane(v_in));
            known_conv = max(known_conv, __builtin_amdgcn_readfirstlane(v_conv));
            known_free = max(known_free, __builtin_amdgcn_readfirstlane(v_free));
        }
        if (!cost.begin(cring, s0 + 2 * TC) || !fetch(s0)) return -1;
        if (out_lds) {
            const int need_free = s0 + U - WAVE + 1 - RS;
            if (need_free > 0 && !wait_at_least(sm.cons() + (w + 1), need_free, known_free, P.err, P.spin_limit))
                return -1;
        }
        // the stage buffer of this group was last read by the converter for group gi - 2
        const int gi = s0 / U;
        if (gi >= 2 && !wait_at_least(conv, gi - 1, known_conv, P.err, P.spin_limit)) return -1;
        // the exponentials of this group and the next are staged (the next ones before this
        // group can finish: the producer may then reuse the cost slots they were read from)
        if (PD && !wait_at_least(pdready, min(gi + 2, groups), known_pd, P.err, P.spin_limit)) return -1;
        const int k = gi & 1;
        const double* pdp = lin_pd_p(sm, gi % kPdBufs) + l * kLinRow;
        const int* pde = lin_pd_e(sm, gi % kPdBufs) + l * kLinRow;
        const bool edge = out_lds && l == WAVE - 1;
        double* sp = edge ? out_p + hslot(s0 - (WAVE - 1)) : lin_stage_p(sm, w, k) + l * kLinRow;
        int* se = edge ? out_e + hslot(s0 - (WAVE - 1)) : lin_stage_e(sm, w, k) + l * kLinRow;
        const float* dn = crow + ((s0 + TC - l) & (CR - 1));  // next group's costs
#pragma unroll
        for (int u = 0; u < U; ++u) {
            double pD;
            int eD;
            if constexpr (PD) {
                pD = pdp[u];
                eD = pde[u];
            } else {
                lin_cost(d_cur[u], ninv_gamma, tabE, pD, eD);
            }
            const double upp = shr1(up_p[u], lp);
            const int upe = dpp_shr1(up_e[u], le);
            const int em = max(max(upe, le), de);
            const double sum = (::ldexp(upp, upe - em) + ::ldexp(lp, le - em)) + ::ldexp(dp, de - em);
            double q = sum * pD;
            int en = em + eD;
            if (u == U - 1) {
                en += __builtin_amdgcn_frexp_exp(q);
                q = __builtin_amdgcn_frexp_mant(q);
            }
            if constexpr (!INTERIOR) {
                const int j = s0 + u - l;
                const bool act = row_ok && (unsigned)j < (unsigned)M;
                q = act ? q : 0.0;
                en = act ? en : kLinNeg;
            }
            dp = upp;
            de = upe;
            lp = q;
            le = en;
            sp[u] = q;
            se[u] = en;
            if constexpr (!PD) d_nxt[u] = dn[u];
            cost.step(u, s0 + 2 * TC, s0 + 3 * TC);
        }
        cost.end(cring, s0 + 2 * TC, s0 + 3 * TC);
        if (l == 0) lds_publish(staged, gi + 1);
        // (a band below in the next workgroup takes lane 63's values from the converter wave,
        // which reads this stage anyway: lin_convert_wave)
        if (out_lds && l == WAVE - 1) lds_publish(sm.prod() + (w + 1), min(max(s0 + U - (WAVE - 1), 0), M));
        return 0;
    };

    if (!cost.prologue(cring, 0) || !cost.prologue(cring, TC)) return give_up_fwd(P, p);
    cost.preload(2 * TC);
    if constexpr (!PD) {
        const float* dn = crow + ((-l) & (CR - 1));
#pragma unroll
        for (int u = 0; u < U; ++u) d_nxt[u] = dn[u];
    }
    using T_ = std::true_type;
    using F_ = std::false_type;
    const bool full = (b + 1) * WAVE <= N;
    const int q_in = full ? min(WAVE, S) : S;
    const int q_out = full ? max((M - U) / U * U + U, WAVE) : S;
    int s0 = 0;
    for (; s0 < q_in; s0 += U)
        if (group(s0, F_{}) != 0) return give_up_fwd(P, p);
    for (; s0 < min(q_out, S); s0 += U)
        if (group(s0, T_{}) != 0) return give_up_fwd(P, p);
    for (; s0 < S; s0 += U)
        if (group(s0, F_{}) != 0) return give_up_fwd(P, p);
}

// The exponential wave of a one-band workgroup (W = 1): for each group h of the band, the
// cost exponentials exp(-d / gamma) = pD 2^eD of its cells (lane l's row of the cost ring,
// as the compute wave would read them) into stage buffer h mod 3, counted in lin_pdready.
// Group h's costs are in the ring once tiles 0 .. h are (ready >= h + 1); buffer h mod 3 is
// free once the compute wave has finished group h - 3 (done >= h - 2), so the wave works up
// to two groups ahead.  The compute wave waits for group g + 1's exponentials before it
// starts group g, so they are read before it finishes group g, after which the producer
// may reuse the oldest of their slots.
// With STORE_D (the unfused one-launch forward) it also stores each cost tile h to D from
// the ring, in the producer's coalesced layout (store_d's, entries past the table stored to
// the last row / column, which receive their own bits again), taking the stores off the
// producer.
template <bool STORE_D>
SDTW_DEV void lin_exp_wave(const DPParams& P, const Smem& sm, int p, int b, int w) {
    const int l = threadIdx.x & (WAVE - 1);
    const int groups = P.S / U;
    const int N = P.N, M = P.M;
    const double ninv_gamma = -P.inv_gamma;
    const double* tabE = sm.tables();
    const float* ring = sm.cost_ring(w);
    const float* crow = ring + l * CS;
    float* Dp = STORE_D ? P.D_out + (int64_t)p * N * M : nullptr;
    const int* ready = sm.ready() + w;
    const int* done = sm.done() + w;
    int* pdready = sm.lin_pdready();
    int known_r = 0, known_d = 0;
    for (int h = 0; h < groups; ++h) {
        if (!wait_at_least(ready, h + 1, known_r, P.err, P.spin_limit)) return;
        if (h >= kPdBufs && !wait_at_least(done, h - (kPdBufs - 1), known_d, P.err, P.spin_limit)) return;
        double* pp = lin_pd_p(sm, h % kPdBufs) + l * kLinRow;
        int* pe = lin_pd_e(sm, h % kPdBufs) + l * kLinRow;
        const float* dn = crow + ((h * U - l) & (CR - 1));  // U consecutive slots (mirrored)
        float d[U];
#pragma unroll
        for (int u = 0; u < U; ++u) d[u] = dn[u];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            double pD;
            int eD;
            lin_cost(d[u], ninv_gamma, tabE, pD, eD);
            pp[u] = pD;
            pe[u] = eD;
        }
        if (l == 0) lds_publish(pdready, h + 1);
        if constexpr (STORE_D) {
            // tile h: lane l's column 16 h + (l & 15), rows 4 (l >> 4) + 16 rb + r
            const int c = h * U + (l & 15);
            const float* src = ring + 4 * (l >> 4) * CS + (c & (CR - 1));
            const int col = min(c, M - 1);
            const int row0 = b * WAVE + 4 * (l >> 4);
#pragma unroll
            for (int rb = 0; rb < 4; ++rb)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int row = min(row0 + 16 * rb + r, N - 1);
                    Dp[(int64_t)row * M + col] = src[(16 * rb + r) * CS];
                }
        }
    }
}

// The helper wave of a linear-domain pair: helper_wave for 16-byte (p, e) entries.
SDTW_DEV void helper_wave_lin(const DPParams& P, const Smem& sm, const double2* gin) {
    const int l = threadIdx.x & (WAVE - 1);
    const int M = P.M;
    double* ring_p = reinterpret_cast<double*>(sm.ring());
    int* ring_e = lin_ering(sm);
    int known_free = 0;
    unsigned spins = 0;
    for (int c = 0; c < M;) {
        const int need_free = c + WAVE - RS;
        if (need_free > 0 && !wait_at_least(sm.cons(), need_free, known_free, P.err, P.spin_limit)) return;
        const int e = c + l;
        double pv = 0.0;
        int ev = 0;
        bool empty = false;
        if (e < M) {
            const unsigned long long* a = reinterpret_cast<const unsigned long long*>(gin + e);
            const unsigned long long lo = __hip_atomic_load(a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const unsigned long long hi = __hip_atomic_load(a + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            pv = __longlong_as_double((long long)lo);
            ev = (int)(unsigned)hi;
            empty = lo == kEmpty64 || (unsigned)(hi >> 32) != 1u;
        }
        const unsigned long long miss = __ballot(empty);
        const int n = miss ? (int)__builtin_ctzll(miss) : WAVE;  // leading written entries
        if (l < n && e < M) {
            ring_p[hslot(e)] = pv;
            ring_e[hslot(e)] = ev;
        }
        if (n > 0) {
            c = min(c + n, M);
            if (l == 0) lds_publish(sm.prod(), c);
            spins = 0;
        } else {
            if (spins++ >= P.spin_limit) {
                raise_timeout(P.err);  // the compute wave it feeds then gives up
                return;
            }
            __builtin_amdgcn_s_sleep(2);
        }
    }
}

// The converter wave of band w: per group, once its compute wave has staged it, p 2^e of
// every cell to R (fp32) in the R table, and out[p] = R[N-1, M-1] as stored.  For a band
// with a band below in the next workgroup it also copies lane 63's staged values of the
// group (columns s0 - 63 .. s0 - 48, inside the row's padding) to the workgroup's
// cross-workgroup row, off the compute wave.
SDTW_DEV void lin_convert_wave(const DPParams& P, const Smem& sm, int p, int g, int w) {
    const int l = threadIdx.x & (WAVE - 1);
    const int W = P.W, G = P.G, nb = P.nb, N = P.N, M = P.M, S = P.S;
    const int b = g * W + w;
    const int i = b * WAVE + l;
    const double ngamma = -P.gamma;
    const double* tabL = sm.tables() + fm::kExpTabN;
    const bool out_lds = (b + 1 < nb) && (w + 1 < W);
    const bool out_glb = (b + 1 < nb) && (w + 1 == W);
    double2* gout = reinterpret_cast<double2*>(P.gring) + ((int64_t)p * G + g) * P.RW + RPAD;
    const double* ring_p = reinterpret_cast<const double*>(sm.ring()) + (w + 1) * RS;
    const int* ring_e = lin_ering(sm) + (w + 1) * RS;
    const int* staged = sm.lin_staged() + w;
    int* done = sm.lin_done() + w;
    float* Rt = P.R + ((int64_t)p * nb + b) * S * WAVE + l;
    const int s_out = i == N - 1 ? M - 1 + l : -1;  // this lane's step of cell (N-1, M-1)
    int known = 0;
    for (int s0 = 0; s0 < S; s0 += U) {
        const int gi = s0 / U;
        if (!wait_at_least(staged, gi + 1, known, P.err, P.spin_limit)) return;
        const int k = gi & 1;
        const bool edge = out_lds && l == WAVE - 1;
        const double* sp = edge ? ring_p + hslot(s0 - (WAVE - 1)) : lin_stage_p(sm, w, k) + l * kLinRow;
        const int* se = edge ? ring_e + hslot(s0 - (WAVE - 1)) : lin_stage_e(sm, w, k) + l * kLinRow;
        double pv[U];
        int ev[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            pv[u] = sp[u];
            ev[u] = se[u];
        }
        // lanes 48 .. 63: lane 63's value of step s0 + l - 48, for the cross-workgroup row
        const int hu = l - (WAVE - U);
        const bool ho = out_glb && hu >= 0;
        const double hp = lin_stage_p(sm, w, k)[(WAVE - 1) * kLinRow + (hu & (U - 1))];
        const int he = lin_stage_e(sm, w, k)[(WAVE - 1) * kLinRow + (hu & (U - 1))];
        // the reads are performed before this store (one LDS order per CU, a wave's in
        // issue order), so the compute wave may then reuse the buffer
        if (l == 0) lds_publish(done, gi + 1);
        if (ho) glb_put_lin(gout + (s0 - (WAVE - 1)) + hu, hp, he);
        // all U conversions as one straight-line block (their table reads and chains
        // interleave), then the stores, and out[p] by the one lane that holds it
        float rv[U];
#pragma unroll
        for (int u = 0; u < U; ++u) rv[u] = (float)lin_to_R(pv[u], ev[u], ngamma, tabL);
        float* Rg = Rt + (int64_t)s0 * WAVE;
#pragma unroll
        for (int u = 0; u < U; ++u) Rg[u * WAVE] = rv[u];
        if ((unsigned)(s_out - s0) < (unsigned)U) {
            float ro = rv[0];
#pragma unroll
            for (int u = 1; u < U; ++u) ro = s_out - s0 == u ? rv[u] : ro;
            P.out[p] = ro;
        }
    }
}

// Wave roles of a launch that can take the linear domain (W <= 2): compute waves 0 .. W-1,
// producers W .. 2W-1, the helper 2W, converters 3 (W = 1) or 6, 7 (W = 2; wave 5 idle),
// and with W = 1 the exponential wave 6 (waves 4, 5 idle), so that each compute wave keeps
// a SIMD to itself under round-robin placement.  Every wave calls lin_pair_ok first.
template <class Cost>
SDTW_DEV void fwd_lin_roles(const DPParams& P, const Smem& sm, int p, int g, int w) {
    const bool lin = lin_pair_ok(P, sm, p);
    const int W = P.W;
    if (w == 2 * W) {
        if (g > 0) {
            const int64_t row = (int64_t)p * P.G + (g - 1);
            if (lin) helper_wave_lin(P, sm, reinterpret_cast<const double2*>(P.gring) + row * P.RW + RPAD);
            else helper_wave(P, sm, P.gring + row * fwd_row_pitch(P) + RPAD, 0);
        }
        return;
    }
    if (W == 1 && w >= 4) {
        // (D stores here where the producer leaves them out: K == KX, see below)
        if (w == 6 && lin && g < P.nb) {
            if (P.D_out && P.K == KXOf<Cost>::value) lin_exp_wave<true>(P, sm, p, g, 0);
            else lin_exp_wave<false>(P, sm, p, g, 0);
        }
        return;
    }
    const int conv0 = W == 1 ? 3 : 6;
    if (w >= conv0) {
        const int wb = w - conv0;
        if (lin && g * W + wb < P.nb) lin_convert_wave(P, sm, p, g, wb);
        return;
    }
    if (w > 2 * W) return;
    const int wb = w >= W ? w - W : w;
    if (g * W + wb >= P.nb) return;
    if (w >= W) {
        // (W = 1, linear domain: the exponential wave stores D, so the producer does not)
        if (P.K != KXOf<Cost>::value) producer_wave<Cost, false>(P, sm, p, g * W + wb, wb);
        else if (P.D_out && !(lin && W == 1)) producer_wave<Cost, false, false, true, true>(P, sm, p, g * W + wb, wb);
        else if (P.D_out) producer_wave<Cost, false, false, false, true, true>(P, sm, p, g * W + wb, wb);
        else producer_wave<Cost, false, false, false, true>(P, sm, p, g * W + wb, wb);
        return;
    }
    CostRing cost;
    cost.bind(sm, w, P);
    if (lin && W == 1) fwd_band_lin<true>(P, cost, sm, p, g, w);
    else if (lin) fwd_band_lin<false>(P, cost, sm, p, g, w);
    else fwd_band<CostRing, false, true>(P, cost, sm, p, g, w);
}

template <class Cost, bool BWD>
constexpr int dp_threads() { return Produced<Cost, BWD>::value ? 9 * WAVE : 5 * WAVE; }

// The forward kernels' body.  LIN: a launch that can take the scaled linear domain (exact
// cell arithmetic, matrix-core costs, no band, P.lin set by the host for mixed arithmetic,
// W <= 2; fwd_lin_roles).
template <class Cost, bool BAND, bool EXACT, bool LIN>
SDTW_DEV void fwd_body(const DPParams& P, unsigned char* smem_raw, double* tab) {
    static_assert(!LIN || (Produced<Cost, false>::value && !BAND && EXACT), "linear domain");
    Smem sm{smem_raw, P.W, ring_bytes_fwd(P.W) + (LIN ? lin_extra_bytes(P.W) : 0), kTabBytesFwd, tab};
    // wave-uniform values are moved to scalar registers so that the branches on band,
    // group and pair compile to scalar branches, not exec-masked regions
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
    if (threadIdx.x == 0) *sm.ticket() = atomicAdd(P.ticket, 1);
    if (threadIdx.x < 2 * (P.W + 1)) sm.prod()[threadIdx.x] = 0;  // prod and cons are contiguous
    if (threadIdx.x < 16) sm.ready()[threadIdx.x] = 0;            // ready and done likewise
    if (threadIdx.x < 8) {
        sm.poison_in()[threadIdx.x] = 0;
        sm.bad_col()[threadIdx.x] = INT_MAX;
        if (LIN) sm.lin_staged()[threadIdx.x] = 0;  // with lin_done and lin_red
    }
    sm.load_tables();
    // ring 0 starts at +inf: the padding row above band 0 (the helper wave overwrites it
    // in workgroups that have a band above them)
    for (int e = threadIdx.x; e < RS; e += blockDim.x) reinterpret_cast<double*>(sm.ring())[e] = dinf();
    __syncthreads();
    const int t = __builtin_amdgcn_readfirstlane(*sm.ticket());
    const int p = t / P.G, g = t - p * P.G;
    if constexpr (LIN) {
        fwd_lin_roles<Cost>(P, sm, p, g, w);
    } else {
        if (w == (Produced<Cost, false>::value ? 2 * P.W : P.W)) {
            // helper wave: the previous workgroup's last row into ring 0
            if (g > 0) helper_wave(P, sm, P.gring + ((int64_t)p * P.G + (g - 1)) * fwd_row_pitch(P) + RPAD, 0);
            return;
        }
        if constexpr (Produced<Cost, false>::value) {
            const int wb = w >= P.W ? w - P.W : w;  // band of this compute or producer wave
            if (g * P.W + wb >= P.nb) return;
            if (w >= P.W) {
                producer_wave<Cost, false>(P, sm, p, g * P.W + wb, wb);
            } else {
                CostRing cost;
                cost.bind(sm, w, P);
                fwd_band<CostRing, BAND, EXACT>(P, cost, sm, p, g, w);
            }
        } else {
            if (g * P.W + w >= P.nb) return;
            Cost cost;
            cost.init(P, p, g * P.W + w);
            fwd_band<Cost, BAND, EXACT>(P, cost, sm, p, g, w);
        }
    }
}

template <class Cost, bool BAND, bool EXACT>
__global__ void __launch_bounds__((dp_threads<Cost, false>())) fwd_kernel(DPParams P) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    __shared__ __align__(16) double tab[kTabBytesFwd / 8];
    fwd_body<Cost, BAND, EXACT, false>(P, smem_raw, tab);
}

// The linear-domain launch: at most 8 waves (fwd_lin_roles), so each may hold 256 VGPRs
// (the producer's two tiles of operands in flight and the store addresses then fit without
// reusing the registers of outstanding loads).
template <class Cost>
__global__ void __launch_bounds__(8 * WAVE) fwd_lin_kernel(DPParams P) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    __shared__ __align__(16) double tab[kTabBytesFwd / 8];
    fwd_body<Cost, false, true, true>(P, smem_raw, tab);
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
// WW: the weight waves of the band (bwd_weight_wave) stage each cell's three weights, and
// this wave's step is the E recurrence on them (the same operations as bwd_cell_hw's or
// bwd_cell_exact's, so the same bits); the bands hand over E alone (the R and D slots of the
// handoff entries are not written).
template <class Cost, bool BAND, bool EXACT, bool WW = false>
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
    const double* tabE = sm.tables();  // exp table in LDS
    float* cring = sm.cost_ring(w);
    float* crow = cring + l * CS;  // my row of the cost ring

    // corner R (as stored by the forward) of this pair
    const int lb = nb - 1, ll = (N - 1) - lb * WAVE;
    const float corner_R = P.R[(((int64_t)p * nb + lb) * S + (M - 1 + ll)) * WAVE + ll];

    // rings carry (E, R, D) of a band's first row to the band above
    float4* lring = reinterpret_cast<float4*>(sm.ring());
    // LDS ring k carries the output of band k (the input of band k - 1); ring W is filled
    // by the workgroup's helper wave from the next workgroup.
    const bool out_lds = (b > 0) && (w > 0);
    const bool out_glb = (b > 0) && (w == 0);
    // cross-workgroup row produced by this workgroup (consumed by workgroup g - 1)
    float4* gout = P.gring4 + ((int64_t)p * G + g) * P.RW + RPAD;
    const float4* lin = lring + (w + 1) * RS;
    float4* lout = lring + w * RS;
    const int* lin_flag = sm.prod() + (w + 1);
    // First row to the band above: at every step each lane stores its (E, R, D) with two LDS
    // writes (E and R by one two-address write, D), so no cross-lane moves collect lane 0's
    // values.  Lane 0's stores (sequence number q - 63 at reverse step q) go to the x, y, z
    // of the handoff ring's entries (w is not read), or, for the band that hands over
    // through global memory (the workgroup's first, w = 0), to the last U float4 entries of
    // the workgroup's staging block.  Every other store (lanes 1 .. 63, and lane 0 of a
    // pair's first band) goes to bytes 12 l + 16 u .. + 11 of the block's first part, which
    // all waves share and nothing reads (a stride of three words between lanes keeps each
    // write free of bank conflicts).
    unsigned char* stage = sm.ring() + (size_t)(W + 1) * RS * sizeof(float4);
    float4* stage_glb = reinterpret_cast<float4*>(stage + 12 * WAVE + 16 * U);

    const float* Rt = P.R + ((int64_t)p * nb + b) * S * WAVE + l;
    const float4* wst = bwd_wstage(sm) + l;  // WW: this lane's entries of the weight stage
    const int* wready = sm.bwd_wready();  // [group parity]
    int known_w0 = 0, known_w1 = 0;

    int known_in = 0, known_free = 0;
    float rE = 0.0f, rR = NINF, rD = 0.0f;  // right neighbour
    float gE = last_row ? 1.0f : 0.0f;      // diag neighbour
    float gR = last_row ? corner_R : NINF;
    float gD = 0.0f;
    float pE = 0.0f, pR = NINF, pD = 0.0f;  // published one step ago

    float4 dn_cur[U];
    float r_cur[U], r_nxt[U], d_cur[U], d_nxt[U];
    // Band below: sequence numbers [q0, q0 + U) of its first row from the LDS ring, for
    // lane 63.  Where no band lies below, the values are the padding row below the table
    // (E 0, R -inf, D 0): lane 63 then holds row N - 1 (or is beyond the table), and only the
    // unmasked interior body takes them from here rather than from the padding directly.
    // Past sequence number M - 1 lane 63 is inactive and the values are unused; they are
    // set to the padding too, which compiles to fewer live registers than leaving them stale.
    auto fetch_lds = [&](int q0, float4* dst) -> bool {
#pragma unroll
        for (int u = 0; u < U; ++u) dst[u] = make_float4(0.0f, NINF, 0.0f, 1.0f);
        if (b + 1 >= nb || q0 >= M) return true;
        const int need = min(q0 + U, M);
        if (!wait_at_least(lin_flag, need, known_in, P.err, P.spin_limit)) return false;
#pragma unroll
        for (int u = 0; u < U; ++u) dst[u] = u == 0 ? lin[hslot(q0)] : lin[hslot(q0 + 1) + u - 1];
        if (l == 0) lds_publish(sm.cons() + (w + 1), need);
        return true;
    };
    // where this lane's per-step stores of the group at q0 go (float4 entry u for step u,
    // x y z written); lane 0's ring stores are unconditional, as in the forward
    auto step_dst = [&](int q0) -> float* {
        float* own = reinterpret_cast<float*>(stage + 12 * l);
        float* edge = out_lds ? reinterpret_cast<float*>(lout + hslot(q0 - (WAVE - 1)))
                              : (out_glb ? reinterpret_cast<float*>(stage_glb) : own);
        return l == 0 ? edge : own;
    };
    // hand the band's first row to the band above: lane 0 produced sequence numbers
    // q - 63 (= M - 1 - j) during the group at q0; publish the ring entries it stored (the
    // count after them), or copy the staged ones to the cross-workgroup row
    auto handover = [&](int q0) {
        const int c0 = q0 - (WAVE - 1);
        if (out_lds) {
            if (l == 0) lds_publish(sm.prod() + w, min(max(q0 + U - (WAVE - 1), 0), M));
        } else if (l < U) {
            const float4 v = stage_glb[l];
            glb_put4(gout + c0 + l, make_float4(v.x, v.y, v.z, 1.0f));
        }
    };
    // Each step writes g*E of the lane's cell into the cost-ring slot whose cost it has just
    // consumed (its own row, column j), whether or not the cell is in the table.  The group
    // at q0 completes columns [M + 47 - q0, M + 63 - q0) of every row (lane 0 visits column
    // M + 62 - q), which are stored here as 16 coalesced tile rows.  No slot is reused while
    // still live: at the end of group q0 the ring holds columns from the newest cost tile,
    // M - 48 - q0, up to M + 62 - q0, 111 < CR columns; writes of cells outside the table
    // land on slots of columns that are rewritten before use or already stored.
    // (with costs from a producer wave, the producer stores the tiles)
    auto flush = [&](int q0) {
        if constexpr (!std::is_same<Cost, CostRing>::value) {
            GTile gt;
            gt.read(P, cring, q0);
            gt.write(P, p, b);
        }
    };
    // forward step of reverse step q, clamped into the band (padding steps are inactive)
    auto fstep = [&](int q) { return max(M + 62 - q, 0); };

    // cost tile of reverse group q0: columns [M - TC - q0, M - q0) (lane 63's newest); the
    // pipeline is the forward's, mirrored
    auto tile_col = [&](int q0) { return M - TC - q0; };
    auto ring_col = [&](int q) { return ((M - 1) - q + (WAVE - 1 - l)) & (CR - 1); };
    if (!cost.prologue(cring, tile_col(0)) || !cost.prologue(cring, tile_col(TC))) {
        give_up_bwd(P, p, b);
        return;
    }
    cost.preload(tile_col(2 * TC));
    if constexpr (!WW) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            r_nxt[u] = Rt[(int64_t)fstep(u) * WAVE];
            d_nxt[u] = crow[ring_col(u)];
        }
    }

    // One group: 16 reverse steps from q0.  INTERIOR: every lane is inside the table for all
    // of them (a full band, columns M + 62 - q0 .. M - 16 - q0 within [0, M), no Sakoe-Chiba
    // band), so no cell needs the inactive masking, and the padding row below the table (E 0,
    // R -inf, D 0; lane 63 of a full last band) arrives as the ring padding that fetch_lds
    // supplies where no band lies below: the corner (j = M) is outside such a group.  The
    // interior groups form one run of q0, walked by a loop of its own (three loops in
    // sequence rather than a branch per group, which would join the loop-carried registers
    // of two bodies).  Only with costs from the distance matrix: with a tile-computing cost
    // provider the extra body costs more registers than it saves.
    auto group = [&](int q0, auto interior_tag) -> bool {
        constexpr bool INTERIOR = decltype(interior_tag)::value;
        if constexpr (!WW) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                r_cur[u] = r_nxt[u];
                d_cur[u] = d_nxt[u];
            }
        }
        // the counters this group start checks, loaded together (one LDS round trip; each
        // wait below then polls only if its cached count falls short)
        {
            const int v_in = lds_load(lin_flag);
            const int v_free = lds_load(sm.cons() + w);
            if constexpr (std::is_same<Cost, CostRing>::value)
                cost.known = max(cost.known, __builtin_amdgcn_readfirstlane(lds_load(cost.ready)));
            if constexpr (WW) {
                known_w0 = max(known_w0, __builtin_amdgcn_readfirstlane(lds_load(wready)));
                known_w1 = max(known_w1, __builtin_amdgcn_readfirstlane(lds_load(wready + 1)));
            }
            known_in = max(known_in, __builtin_amdgcn_readfirstlane(v_in));
            known_free = max(known_free, __builtin_amdgcn_readfirstlane(v_free));
        }
        const int gi = q0 / U;
        if (WW && !((gi & 1) ? wait_at_least(wready + 1, gi / 2 + 1, known_w1, P.err, P.spin_limit)
                             : wait_at_least(wready, gi / 2 + 1, known_w0, P.err, P.spin_limit)))
            return false;
        if (!cost.begin(cring, tile_col(q0 + 2 * TC)) || !fetch_lds(q0, dn_cur)) return false;
        const float4* wbuf = wst + (gi % kWBufs) * (U * WAVE);
        // (exact: plane 0 holds (a, b), plane 1 (c, NaN flag), as double2)
        const double2* wq0 = reinterpret_cast<const double2*>(wbuf);
        const double2* wq1 = wq0 + kWBufs * U * WAVE;
        const int n0 = q0 + U;
        if (out_lds) {  // as in the forward: sequence numbers up to q0 + U - 64 this group
            const int need_free = q0 + U - WAVE + 1 - RS;
            if (need_free > 0 && !wait_at_least(sm.cons() + w, need_free, known_free, P.err, P.spin_limit))
                return false;
        }
        float* dst = step_dst(q0);
        // next group's costs: columns (M + 62 - l) - n0 - u, U consecutive slots from the
        // lowest one (mirrored past CR), read downwards; next group's R: in an interior group
        // every forward step M + 62 - n0 - u is >= 0, so no clamp
        const float* dnx = crow + ((M + 62 - l - n0 - (U - 1)) & (CR - 1));
        const float* rnx = Rt + (int64_t)(M + 62 - n0) * WAVE;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int q = q0 + u;
            const int j = (M - 1) - q + (WAVE - 1 - l);
            if constexpr (WW) {
                float dE = __int_as_float(dpp_shl1(__float_as_int(dn_cur[u].x), __float_as_int(pE)));
                if (!INTERIOR && last_row) dE = (j == M) ? 1.0f : 0.0f;
                const bool act = INTERIOR || (row_ok && (unsigned)j < (unsigned)M);
                float cand;
                if constexpr (EXACT) {  // bwd_cell_exact's sum on the staged weights
                    const double2 ab = wq0[u * WAVE], cf = wq1[u * WAVE];
                    double acc = __dmul_rn((double)dE, ab.x);
                    acc = __dadd_rn(acc, __dmul_rn((double)rE, ab.y));
                    acc = __dadd_rn(acc, __dmul_rn((double)gE, cf.x));
                    cand = (float)(cf.y != 0.0 ? __builtin_nan("") : acc);
                } else {  // (down, right, diag) weights
                    const float4 wt = wbuf[u * WAVE];
                    cand = __fmaf_rn(gE, wt.z, __fmaf_rn(rE, wt.y, __fmul_rn(dE, wt.x)));
                }
                bool keep = true;
                if (BAND && !INTERIOR) keep = !out_of_band(bw, i, j);
                const float e = keep ? cand : 0.0f;
                crow[j & (CR - 1)] = __fmul_rn(gsc, e);
                const float mE = act ? e : 0.0f;
                rE = mE;
                gE = dE;
                pE = mE;
                dst[4 * u] = mE;
                cost.step(u, tile_col(q0 + 2 * TC), tile_col(q0 + 3 * TC));
                continue;
            }
            float dE = __int_as_float(dpp_shl1(__float_as_int(dn_cur[u].x), __float_as_int(pE)));
            float dR = __int_as_float(dpp_shl1(__float_as_int(dn_cur[u].y), __float_as_int(pR)));
            float dD = __int_as_float(dpp_shl1(__float_as_int(dn_cur[u].z), __float_as_int(pD)));
            if (!INTERIOR && last_row) {  // the padded row below the table
                const bool corner = (j == M);
                dE = corner ? 1.0f : 0.0f;
                dR = corner ? corner_R : NINF;
                dD = 0.0f;
            }
            const bool act = INTERIOR || (row_ok && (unsigned)j < (unsigned)M);
            float rij = r_cur[u];
            rij = __builtin_isinf(rij) ? NINF : rij;
            const float cand = EXACT ? bwd_cell_exact(rij, dE, dR, dD, rE, rR, rD, gE, gR, gD, inv_gamma, tabE)
                                     : bwd_cell_hw(rij, dE, dR, dD, rE, rR, rD, gE, gR, gD, c2);
            bool keep = true;
            if (BAND && !INTERIOR) keep = !out_of_band(bw, i, j);
            const float e = keep ? cand : 0.0f;
            crow[j & (CR - 1)] = __fmul_rn(gsc, e);
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
            dst[4 * u] = mE;
            dst[4 * u + 1] = mR;
            dst[4 * u + 2] = mD;
            // next group's R and costs, and the tile work, between the steps (fstep clamps
            // reads past the band's first step)
            r_nxt[u] = INTERIOR ? rnx[-(int64_t)u * WAVE] : Rt[(int64_t)fstep(n0 + u) * WAVE];
            d_nxt[u] = dnx[U - 1 - u];
            cost.step(u, tile_col(q0 + 2 * TC), tile_col(q0 + 3 * TC));
        }
        cost.end(cring, tile_col(q0 + 2 * TC), tile_col(q0 + 3 * TC));
        if (out_lds || out_glb) handover(q0);
        flush(q0);
        return true;
    };
    int q0 = 0;
    if constexpr (!BAND && (std::is_same<Cost, CostD>::value || std::is_same<Cost, CostRing>::value)) {
        const bool has_interior = (b + 1) * WAVE <= N;
        const int q_in = has_interior ? WAVE : S;
        const int q_out = has_interior ? max(((M - U) / U + 1) * U, WAVE) : S;
        for (; q0 < q_in; q0 += U)
            if (!group(q0, std::false_type{})) return give_up_bwd(P, p, b);
        for (; q0 < q_out; q0 += U)
            if (!group(q0, std::true_type{})) return give_up_bwd(P, p, b);
    }
    for (; q0 < S; q0 += U)
        if (!group(q0, std::false_type{})) return give_up_bwd(P, p, b);
}

// Weight waves of band b (the backward with costs read from D, hardware exp2, one band per
// workgroup).  The cell's weights (launcher.py:347-351)
//   a = exp((R(i+1,j) - R(i,j) - D(i+1,j)) / gamma)    (down)
//   b = exp((R(i,j+1) - R(i,j) - D(i,j+1)) / gamma)    (right)
//   c = exp((R(i+1,j+1) - R(i,j) - D(i+1,j+1)) / gamma) (diagonal)
// depend only on the forward's R and on D, both in memory before the launch, including the
// row below the band (the band below's first row, which lane 63 reads from its R table and
// from D).  Two waves form them, wave k for the groups h = k mod 2, with bwd_cell_hw's
// operations on the values the compute wave would use (the same masking of inactive cells,
// +inf mapped to -inf, the padding row and corner below the table), ahead of the compute
// wave, into a three-buffer LDS stage (group h in buffer h % kWBufs; wave k counts its
// groups in bwd_wready()[k]).  A wave's state at the start of group h (its cell and the cell
// below one step earlier, whose weights the other wave formed) is read from memory again.
// It reads a group's costs from the band's cost ring once the producer has published the
// tile after them (the compute wave's own rule), and writes buffer h % kWBufs once the
// compute wave has finished group h - kWBufs.  Its waits are bounded; on expiry it stops,
// and the compute wave's bounded wait for its count then gives up for the band.
template <bool EXACT>
SDTW_DEV void bwd_weight_wave(const DPParams& P, const Smem& sm, int p, int b, int k) {
    const int l = threadIdx.x & (WAVE - 1);
    const int nb = P.nb, N = P.N, M = P.M, S = P.S;
    const int i = b * WAVE + l;
    const bool row_ok = i < N;
    const bool last_row = (i == N - 1);
    const float c2 = (float)(P.inv_gamma * 1.4426950408889634074);  // log2(e) / gamma
    const double inv_gamma = P.inv_gamma;
    const double* tabE = sm.tables();  // exp table in LDS (exact)
    const float NINF = -finf();
    const int lb = nb - 1, ll = (N - 1) - lb * WAVE;
    const float corner_R = P.R[(((int64_t)p * nb + lb) * S + (M - 1 + ll)) * WAVE + ll];
    const float* crow = sm.cost_ring(0) + l * CS;
    const float* Rt = P.R + ((int64_t)p * nb + b) * S * WAVE + l;
    const float* Dp = P.D + (int64_t)p * N * M;
    // the row below: lane 0 of band b + 1 (its entry of forward step j is column j) and
    // row (b + 1) * 64 of D; none below the last band (the padding row: R -inf, D 0)
    const bool below = b + 1 < nb;
    const float* Rb = P.R + ((int64_t)p * nb + (below ? b + 1 : b)) * S * WAVE;
    const float* Db = Dp + (int64_t)(below ? b + 1 : b) * WAVE * M;
    // the cell below this lane's, (i + 1, j): band and lane of row i + 1 (clamped)
    const int rdn = min(i + 1, N - 1), bdn = rdn / WAVE, ldn = rdn - bdn * WAVE;
    const float* Rdn = P.R + ((int64_t)p * nb + bdn) * S * WAVE + ldn;
    float4* stage = bwd_wstage(sm) + l;
    int* wready = sm.bwd_wready() + k;
    const int* ready = sm.ready();
    const int* done = sm.done();
    int known_ready = 0, known_done = 0;
    const int groups = S / U;
    auto fstep = [&](int q) { return max(M + 62 - q, 0); };
    // for the group at q0: this lane's R; (lanes u < U) the row below at lane 63's column of
    // step q0 + u, M - 1 - q0 - u; and the R and D of this lane's cell and of the cell below
    // it at step q0 - 1 (column jp), from which the group's starting state is formed
    float r_nxt[U];
    float bR_nxt = NINF, bD_nxt = 0.0f, oR_nxt = NINF, oD_nxt = 0.0f, uR_nxt = NINF, uD_nxt = 0.0f;
    auto fetch = [&](int q0) {
#pragma unroll
        for (int u = 0; u < U; ++u) r_nxt[u] = Rt[(int64_t)fstep(q0 + u) * WAVE];
        const int jb = M - 1 - q0 - l;
        const bool ok = below && l < U && jb >= 0;
        const float rb = Rb[(int64_t)max(jb, 0) * WAVE];
        const float db = Db[max(jb, 0)];
        bR_nxt = ok ? (__builtin_isinf(rb) ? NINF : rb) : NINF;
        bD_nxt = ok ? db : 0.0f;
        const int jp = min(max((M - 1) - (q0 - 1) + (WAVE - 1 - l), 0), M - 1);
        oR_nxt = Rt[(int64_t)min(fstep(q0 - 1), S - 1) * WAVE];
        oD_nxt = Dp[(int64_t)min(i, N - 1) * M + jp];
        uR_nxt = Rdn[(int64_t)min(jp + ldn, S - 1) * WAVE];
        uD_nxt = Dp[(int64_t)rdn * M + jp];
    };
    float rR = NINF, rD = 0.0f;                       // right neighbour
    float gR = last_row ? corner_R : NINF, gD = 0.0f;  // diagonal neighbour
    float pR = NINF, pD = 0.0f;                       // this lane's cell one step ago
    fetch(k * U);
    for (int h = k; h < groups; h += 2) {
        const int q0 = h * U;
        float r_cur[U];
#pragma unroll
        for (int u = 0; u < U; ++u) r_cur[u] = r_nxt[u];
        const float bR = bR_nxt, bD = bD_nxt;
        if (h > 0) {  // the state after step q0 - 1
            const int jp = (M - 1) - (q0 - 1) + (WAVE - 1 - l);
            const bool act_p = row_ok && (unsigned)jp < (unsigned)M;
            pR = act_p ? (__builtin_isinf(oR_nxt) ? NINF : oR_nxt) : NINF;
            pD = act_p ? oD_nxt : 0.0f;
            rR = pR;
            rD = pD;
            const bool act_dn = (i + 1 < N) && (unsigned)jp < (unsigned)M;
            gR = act_dn ? (__builtin_isinf(uR_nxt) ? NINF : uR_nxt) : NINF;
            gD = act_dn ? uD_nxt : 0.0f;
            if (last_row) {
                gR = (jp == M) ? corner_R : NINF;
                gD = 0.0f;
            }
        }
        if (h + 2 < groups) fetch(q0 + 2 * U);
        if (!wait_at_least(ready, h + 2, known_ready, P.err, P.spin_limit)) return;
        if (h >= kWBufs && !wait_at_least(done, h - kWBufs + 1, known_done, P.err, P.spin_limit)) return;
        float4* buf = stage + (h % kWBufs) * (U * WAVE);
        double2* q0p = reinterpret_cast<double2*>(buf);
        double2* q1p = q0p + kWBufs * U * WAVE;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int q = q0 + u;
            const int j = (M - 1) - q + (WAVE - 1 - l);
            const float sR = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bR), u));
            const float sD = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bD), u));
            float dR = __int_as_float(dpp_shl1(__float_as_int(sR), __float_as_int(pR)));
            float dD = __int_as_float(dpp_shl1(__float_as_int(sD), __float_as_int(pD)));
            if (last_row) {  // the padded row below the table
                dR = (j == M) ? corner_R : NINF;
                dD = 0.0f;
            }
            const bool act = row_ok && (unsigned)j < (unsigned)M;
            float rij = r_cur[u];
            rij = __builtin_isinf(rij) ? NINF : rij;
            const float d = crow[j & (CR - 1)];
            if constexpr (EXACT) {  // bwd_cell_exact's weights
                const float da = __fsub_rn(__fsub_rn(dR, rij), dD);
                const float db = __fsub_rn(__fsub_rn(rR, rij), rD);
                const float dc = __fsub_rn(__fsub_rn(gR, rij), gD);
                const bool nan_in = (da != da) || (db != db) || (dc != dc);
                const double wa = fm::exp_tab((double)da * inv_gamma, tabE);
                const double wb = fm::exp_tab((double)db * inv_gamma, tabE);
                const double wg = fm::exp_tab((double)dc * inv_gamma, tabE);
                q0p[u * WAVE] = make_double2(wa, wb);
                q1p[u * WAVE] = make_double2(wg, nan_in ? 1.0 : 0.0);
            } else {
                const float wa = __builtin_amdgcn_exp2f(__fmul_rn(__fsub_rn(__fsub_rn(dR, rij), dD), c2));
                const float wb = __builtin_amdgcn_exp2f(__fmul_rn(__fsub_rn(__fsub_rn(rR, rij), rD), c2));
                const float wg = __builtin_amdgcn_exp2f(__fmul_rn(__fsub_rn(__fsub_rn(gR, rij), gD), c2));
                buf[u * WAVE] = make_float4(wa, wb, wg, 0.0f);
            }
            const float mR = act ? rij : NINF;
            const float mD = act ? d : 0.0f;
            rR = mR;
            rD = mD;
            gR = dR;
            gD = dD;
            pR = mR;
            pD = mD;
        }
        if (l == 0) lds_publish(wready, h / 2 + 1);
    }
}

// GW > 0: gradient mode for workgroups of up to GW bands.  GW = 2: waves compute 0 .. W-1,
// producers W .. 2W-1, dL/dy waves 2W .. 3W-1, dL/dx waves 3W .. 4W-1, helper 4W (under
// round-robin placement with W = 2 the dL/dy waves share the compute waves' SIMDs and the
// dL/dx waves the producers'; measured faster than the other way round, whose dL/dx
// products then sit beside the recursion).  GW = 4 (widths <= 16, whose gradient work is
// light): one gradient wave per band, 2W .. 3W-1, helper 3W.
template <int GW>
constexpr int grad_waves_per_band() { return GW == 2 ? 4 : 3; }
template <class Cost, bool BAND, bool EXACT, int GW = 0>
__global__ void __launch_bounds__((GW ? (grad_waves_per_band<GW>() * GW + 1) * WAVE : dp_threads<Cost, true>()))
bwd_kernel(DPParams P) {
    static_assert(GW == 0 || KXOf<Cost>::value > 0, "gradient mode needs matrix-core cost tiles");
    extern __shared__ __align__(16) unsigned char smem_raw[];
    __shared__ __align__(16) double tab[kTabBytesBwd / 8];
    // with weight waves (P.ww: costs from D, W = 1; waves compute 0, producer 1, helper 2,
    // weights 3 and 5, 4 idle, so that each weight wave shares its SIMD with a light wave)
    // their stage (P.ww planes) follows the handoff rings
    constexpr bool WW_OK = std::is_same<Cost, CostD>::value && GW == 0;
    const bool ww = WW_OK && P.ww;
    Smem sm{smem_raw, P.W, ring_bytes_bwd(P.W) + (ww ? P.ww * kWStageBytes : 0), kTabBytesBwd, tab};
    // wave-uniform values are moved to scalar registers so that the branches on band,
    // group and pair compile to scalar branches, not exec-masked regions
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
    if (threadIdx.x == 0) *sm.ticket() = atomicAdd(P.ticket, 1);
    if (threadIdx.x < 2 * (P.W + 1)) sm.prod()[threadIdx.x] = 0;
    if (threadIdx.x < 16) sm.ready()[threadIdx.x] = 0;
    if (threadIdx.x < 8) sm.gdone()[threadIdx.x] = 0;
    if (threadIdx.x < 2) sm.bwd_wready()[threadIdx.x] = 0;
    sm.load_tables();
    __syncthreads();
    const int t = __builtin_amdgcn_readfirstlane(*sm.ticket());
    const int p = t / P.G;
    const int g = (P.G - 1) - (t - p * P.G);  // lowest ticket of a pair takes the bottom group
    const int helper = GW ? grad_waves_per_band<GW>() * P.W : (Produced<Cost, true>::value ? 2 * P.W : P.W);
    if (w == helper) {
        // helper wave: the next workgroup's first row into ring W
        if (g + 1 < P.G) helper_wave(P, sm, P.gring4 + ((int64_t)p * P.G + (g + 1)) * P.RW + RPAD, P.W);
        return;
    }
    if constexpr (GW > 0) {
        const int role = w >= 3 * P.W ? 3 : (w >= 2 * P.W ? 2 : (w >= P.W ? 1 : 0));
        const int wb = w - role * P.W;
        if (g * P.W + wb >= P.nb) return;
        if (role == 3) {
            grad_wave<KXOf<Cost>::value, kGradPartX>(P, sm, p, g * P.W + wb, wb);
        } else if (role == 2) {
            if constexpr (GW == 2) grad_wave<KXOf<Cost>::value, kGradPartY>(P, sm, p, g * P.W + wb, wb);
            else grad_wave<KXOf<Cost>::value, kGradPartX | kGradPartY>(P, sm, p, g * P.W + wb, wb);
        } else if (role == 1) {
            producer_wave<Cost, true, true>(P, sm, p, g * P.W + wb, wb);
        } else {
            CostRing cost;
            cost.bind(sm, w, P);
            bwd_band<CostRing, BAND, EXACT>(P, cost, sm, p, g, w);
        }
    } else if constexpr (Produced<Cost, true>::value) {
        if constexpr (WW_OK) {
            if (ww) {  // one band per workgroup (g is the band)
                if (w == 3 || w == 5) {
                    bwd_weight_wave<EXACT>(P, sm, p, g, w == 3 ? 0 : 1);
                } else if (w == 1) {
                    producer_wave<Cost, true>(P, sm, p, g, 0);
                } else if (w == 0) {
                    CostRing cost;
                    cost.bind(sm, 0, P);
                    bwd_band<CostRing, BAND, EXACT, true>(P, cost, sm, p, g, 0);
                }
                return;
            }
        }
        const int wb = w >= P.W ? w - P.W : w;
        if (g * P.W + wb >= P.nb) return;
        if (w >= P.W) {
            producer_wave<Cost, true>(P, sm, p, g * P.W + wb, wb);
        } else {
            CostRing cost;
            cost.bind(sm, w, P);
            bwd_band<CostRing, BAND, EXACT>(P, cost, sm, p, g, w);
        }
    } else {
        if (g * P.W + w >= P.nb) return;
        Cost cost;
        cost.init(P, p, g * P.W + w);
        bwd_band<Cost, BAND, EXACT>(P, cost, sm, p, g, w);
    }
}

// ---------------------------------------------------------------------------------------
// Launch helpers (the prep kernel that zeroes the ticket and error flag and empties the
// cross-workgroup rows is launched by launch_dp_prep, defined once in sdtw_dp.hip)
// ---------------------------------------------------------------------------------------
hipError_t launch_dp_prep(const DPParams& P, bool bwd, hipStream_t st);

inline size_t dp_smem_bytes(const DPParams& P, bool bwd) {
    const size_t ring = bwd ? ring_bytes_bwd(P.W) + P.ww * kWStageBytes
                            : ring_bytes_fwd(P.W) + (P.lin ? lin_extra_bytes(P.W) : 0);
    return 256 + ring + (size_t)P.W * WAVE * CS * sizeof(float);  // the tables are static
}

template <class K>
hipError_t launch_dp(K kernel, const DPParams& P, bool bwd, bool produced, hipStream_t st,
                     bool grad = false) {
    const size_t lds = dp_smem_bytes(P, bwd);
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    hipError_t e = launch_dp_prep(P, bwd, st);
    if (e != hipSuccess) return e;
    // one wave per band, plus a helper wave when a pair spans several workgroups; with
    // matrix-core costs, the helper slot and one producer wave per band
    // (a launch that can take the linear domain: a converter wave per band, fwd_lin_roles)
    const int waves = grad ? (P.W <= 2 ? 4 : 3) * P.W + 1
                      : !bwd && P.lin ? (P.W == 1 ? 7 : 8)
                      : bwd && P.ww ? 6
                      : (produced ? 2 * P.W + 1 : P.W + (P.G > 1 ? 1 : 0));
    hipLaunchKernelGGL(kernel, dim3(P.B * P.G), dim3(waves * WAVE), lds, st, P);
    return hipGetLastError();
}

template <class Cost, bool BWD, bool EXACT>
hipError_t launch_cost(const DPParams& P, hipStream_t st) {
    if constexpr (BWD) {
        // weight waves only where the kernel has them (costs from D, W = 1); their stage
        // has one plane under hardware exp2, two under exact arithmetic (double weights)
        DPParams Q = P;
        if (!std::is_same<Cost, CostD>::value || P.W != 1) Q.ww = 0;
        else if (Q.ww) Q.ww = EXACT ? 2 : 1;
        if (Q.bw > 0.0) return launch_dp(bwd_kernel<Cost, true, EXACT>, Q, true, Produced<Cost, true>::value, st);
        return launch_dp(bwd_kernel<Cost, false, EXACT>, Q, true, Produced<Cost, true>::value, st);
    } else {
        // the linear domain only where the kernel can take it
        DPParams Q = P;
        if (P.bw > 0.0 || !EXACT || !Produced<Cost, false>::value || P.W > 2) Q.lin = 0;
        if constexpr (EXACT && Produced<Cost, false>::value) {
            if (Q.lin) return launch_dp(fwd_lin_kernel<Cost>, Q, false, true, st);
        }
        if (Q.bw > 0.0) return launch_dp(fwd_kernel<Cost, true, EXACT>, Q, false, Produced<Cost, false>::value, st);
        return launch_dp(fwd_kernel<Cost, false, EXACT>, Q, false, Produced<Cost, false>::value, st);
    }
}

// Fused backward in gradient mode (P.gx_out or P.gy_out set, P.G_out null): workgroups of up
// to 2 bands for any matrix-core width, up to 4 for widths <= 16 (their waves fit 128
// registers).  Instantiated in sdtw_dp_bwd_grad_*.hip.
template <bool EXACT>
hipError_t launch_dp_grad(const DPParams& P, hipStream_t st);

template <class Cost, bool EXACT>
hipError_t launch_grad_cost(const DPParams& P, hipStream_t st) {
    if (P.W <= 2) {
        if (P.bw > 0.0) return launch_dp(bwd_kernel<Cost, true, EXACT, 2>, P, true, true, st, true);
        return launch_dp(bwd_kernel<Cost, false, EXACT, 2>, P, true, true, st, true);
    }
    if constexpr (KXOf<Cost>::value <= 16) {
        if (P.W <= 4) {
            if (P.bw > 0.0) return launch_dp(bwd_kernel<Cost, true, EXACT, 4>, P, true, true, st, true);
            return launch_dp(bwd_kernel<Cost, false, EXACT, 4>, P, true, true, st, true);
        }
    }
    return hipErrorInvalidValue;
}

// One (direction, arithmetic, cost source) family of kernels.  Fused kernels take the
// matrix-core cost tiles, with x rows in registers padded to the smallest of 4, 8, 16, 32,
// 64 >= K; wider features, and the tiny problems whose reference dot is a multiply-then-add,
// take the scalar tiles.
template <bool BWD, bool EXACT, bool FUSED>
hipError_t launch_dp_variant(const DPParams& P, bool muladd, hipStream_t st) {
    if constexpr (!FUSED) {
        (void)muladd;
        return launch_cost<CostD, BWD, EXACT>(P, st);
    } else {
        if (BWD && (P.gx_out || P.gy_out)) {
            if (muladd || P.K > 64) return hipErrorInvalidValue;
            return launch_dp_grad<EXACT>(P, st);
        }
        if (muladd) return launch_cost<CostScalar<true>, BWD, EXACT>(P, st);
        if (P.K <= 4) return launch_cost<CostMfma<4>, BWD, EXACT>(P, st);
        if (P.K <= 8) return launch_cost<CostMfma<8>, BWD, EXACT>(P, st);
        if (P.K <= 16) return launch_cost<CostMfma<16>, BWD, EXACT>(P, st);
        if (P.K <= 32) return launch_cost<CostMfma<32>, BWD, EXACT>(P, st);
        if (P.K <= 64) return launch_cost<CostMfma<64>, BWD, EXACT>(P, st);
        return launch_cost<CostScalar<false>, BWD, EXACT>(P, st);
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
extern template hipError_t launch_dp_grad<false>(const DPParams&, hipStream_t);
extern template hipError_t launch_dp_grad<true>(const DPParams&, hipStream_t);

// the gradient-mode dispatch over the matrix-core widths (defined where instantiated)
template <bool EXACT>
hipError_t launch_dp_grad(const DPParams& P, hipStream_t st) {
    if (P.K <= 4) return launch_grad_cost<CostMfma<4>, EXACT>(P, st);
    if (P.K <= 8) return launch_grad_cost<CostMfma<8>, EXACT>(P, st);
    if (P.K <= 16) return launch_grad_cost<CostMfma<16>, EXACT>(P, st);
    if (P.K <= 32) return launch_grad_cost<CostMfma<32>, EXACT>(P, st);
    return launch_grad_cost<CostMfma<64>, EXACT>(P, st);
}

}  // namespace sdtw
