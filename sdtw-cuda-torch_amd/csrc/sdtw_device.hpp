// sdtw_device.hpp -- device-side arithmetic shared by the gfx950 Soft-DTW kernels.
//
// Two families of helpers live here:
//   * exact squared-Euclidean cost: the fp32 bits torch-CPU produces for
//     clamp_min(x2 + y2 - 2 * bmm(x, y^T), 0) (reference distances.py:20-28) on an x86 host;
//   * the Soft-DTW cell updates in the arithmetic of the reference CPU path
//     (launcher.py:317-323 forward, launcher.py:343-351 backward).
// Everything here is compiled with -ffp-contract=off: the orders below are the contract.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define SDTW_DEV __device__ __forceinline__

namespace sdtw {

SDTW_DEV double dinf() { return __builtin_inf(); }
SDTW_DEV float finf() { return __builtin_inff(); }

// ---------------------------------------------------------------------------------------
// Row norms in ATen's CPU order.
//
// torch's (x*x).sum(-1) on a contiguous innermost dim of length K runs ATen's cascade sum
// (aten/src/ATen/native/cpu/SumKernel.cpp) with 8-wide fp32 vectors (the AVX2 kernel, which
// the AVX512 dispatch also uses for sum):
//   K >= 8 : the K/8 full vectors are reduced by row_sum (4 interleaved accumulators, a
//            16-row cascade), then the K%8 tail scalars are summed first and the 8 vector
//            lanes are added to that, lane 0..7 in order;
//   K <  8 : the scalar row_sum over the K elements (same 4-accumulator scheme).
// The 8 vector lanes are independent, so lane t is computed as a scalar row_sum over the
// strided sequence v[8c + t].
// ---------------------------------------------------------------------------------------
SDTW_DEV float sq(float v) { return __fmul_rn(v, v); }

// row_sum<ilp=4> over `size` scalars w(e) = sq(v[e * stride]).
SDTW_DEV float aten_row_sum_sq(const float* v, int stride, int size) {
    const int size_ilp = size / 4;
    float acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int k = 0; k < 4; ++k) acc[a][k] = 0.0f;
    // multi_row_sum: level_power = max(4, CeilLog2(size_ilp) / 4) is 4 for every
    // size_ilp < 2^20, i.e. for any realistic feature count.
    const int level_power = 4;
    const int level_step = 1 << level_power;
    const int level_mask = level_step - 1;
    int i = 0;
    while (i + level_step <= size_ilp) {
        for (int jj = 0; jj < level_step; ++jj, ++i) {
#pragma unroll
            for (int k = 0; k < 4; ++k)
                acc[0][k] = __fadd_rn(acc[0][k], sq(v[(int64_t)(i * 4 + k) * stride]));
        }
#pragma unroll
        for (int j = 1; j < 4; ++j) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                acc[j][k] = __fadd_rn(acc[j][k], acc[j - 1][k]);
                acc[j - 1][k] = 0.0f;
            }
            const int mask = level_mask << (j * level_power);
            if ((i & mask) != 0) break;
        }
    }
    for (; i < size_ilp; ++i) {
#pragma unroll
        for (int k = 0; k < 4; ++k)
            acc[0][k] = __fadd_rn(acc[0][k], sq(v[(int64_t)(i * 4 + k) * stride]));
    }
#pragma unroll
    for (int j = 1; j < 4; ++j)
#pragma unroll
        for (int k = 0; k < 4; ++k) acc[0][k] = __fadd_rn(acc[0][k], acc[j][k]);
    float p0 = acc[0][0];
    for (int e = size_ilp * 4; e < size; ++e) p0 = __fadd_rn(p0, sq(v[(int64_t)e * stride]));
    p0 = __fadd_rn(p0, acc[0][1]);
    p0 = __fadd_rn(p0, acc[0][2]);
    p0 = __fadd_rn(p0, acc[0][3]);
    return p0;
}

// (x*x).sum(-1) for one contiguous row of length K, bit-exact with ATen CPU.
SDTW_DEV float aten_sumsq(const float* v, int K) {
    if (K >= 8) {
        const int nvec = K / 8;
        float fa = 0.0f;
        for (int e = nvec * 8; e < K; ++e) fa = __fadd_rn(fa, sq(v[e]));
#pragma unroll
        for (int t = 0; t < 8; ++t) fa = __fadd_rn(fa, aten_row_sum_sq(v + t, 8, nvec));
        return fa;
    }
    return __fadd_rn(0.0f, aten_row_sum_sq(v, 1, K));
}

// x . y over K in the order the host GEMM uses: a sequential fp32 FMA chain from 0 (MKL
// sgemm), or multiply-then-add (ATen's naive bmm kernel, used when K*N*M < 400).
template <bool MULADD>
SDTW_DEV float exact_dot(const float* __restrict__ a, const float* __restrict__ b, int K) {
    float acc = 0.0f;
    for (int k = 0; k < K; ++k) {
        if (MULADD)
            acc = __fadd_rn(acc, __fmul_rn(a[k], b[k]));
        else
            acc = __fmaf_rn(a[k], b[k], acc);
    }
    return acc;
}

// clamp_min(fl(fl(x2 + y2) - 2*dot), 0): 2*dot is exact; NaN passes through like torch.
SDTW_DEV float exact_cost_pre(float x2, float y2, float dot) {
    return __fsub_rn(__fadd_rn(x2, y2), 2.0f * dot);
}
SDTW_DEV float clamp0(float d) { return d < 0.0f ? 0.0f : d; }

// ---------------------------------------------------------------------------------------
// Soft-DTW cell updates in the reference CPU arithmetic.
// ---------------------------------------------------------------------------------------

// 0 < bandwidth < |i - j|   (launcher.py:315, :345)
SDTW_DEV bool out_of_band(double bandwidth, int i, int j) {
    const int d = i > j ? i - j : j - i;
    return (0.0 < bandwidth) && (bandwidth < (double)d);
}

// softmin of the three predecessors, fp64 throughout (launcher.py:317-322):
//   r_k = -R_k / gamma, rmax = max(max(r0, r1), r2),
//   -gamma * (log(sum_k exp(r_k - rmax)) + rmax)
SDTW_DEV double softmin3(double R0, double R1, double R2, double gamma) {
    const double r0 = -R0 / gamma;
    const double r1 = -R1 / gamma;
    const double r2 = -R2 / gamma;
    double rmax = (r1 > r0) ? r1 : r0;  // Python max(a, b): b if b > a else a
    rmax = (r2 > rmax) ? r2 : rmax;
    const double rsum = exp(r0 - rmax) + exp(r1 - rmax) + exp(r2 - rmax);
    return -gamma * (log(rsum) + rmax);
}

// One backward cell (launcher.py:347-351): fp32 differences, fp64 exp / products / sum,
// E stored in fp32.  Inputs are the neighbours' (E, R, D) with the reference's padding.
struct Nbr {
    float E, R, D;
};

SDTW_DEV float bwd_cell(float rij, const Nbr& dn, const Nbr& rt, const Nbr& dg, double gamma) {
    const float da = __fsub_rn(__fsub_rn(dn.R, rij), dn.D);
    const float db = __fsub_rn(__fsub_rn(rt.R, rij), rt.D);
    const float dc = __fsub_rn(__fsub_rn(dg.R, rij), dg.D);
    const double a = exp((double)da / gamma);
    const double b = exp((double)db / gamma);
    const double c = exp((double)dc / gamma);
    double acc = __dmul_rn((double)dn.E, a);
    acc = __dadd_rn(acc, __dmul_rn((double)rt.E, b));
    acc = __dadd_rn(acc, __dmul_rn((double)dg.E, c));
    return (float)acc;
}

}  // namespace sdtw
