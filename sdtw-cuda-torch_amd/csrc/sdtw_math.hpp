// sdtw_math.hpp -- fp64 exp / log for the Soft-DTW recursions, usable on host and device.
//
// Both follow textbook methods (no library code reproduced):
//   exp: Cody-Waite range reduction x = k ln2 + r with ln2 split into a 32-bit head and a
//        tail (so k*ln2_hi is exact for |k| < 2^20), |r| <= ln2/2, Taylor polynomial of
//        degree 11 in Horner form, scaling by 2^k with ldexp.
//        Truncation error r^12/12! < 6.5e-15 relative on the reduced range.
//   log: s = m 2^e with m in [sqrt(1/2), sqrt(2)), u = (m-1)/(m+1) (|u| <= 0.1716, the
//        division by Newton-Raphson reciprocal plus one residual correction),
//        log m = 2 atanh(u) = 2u (1 + u^2/3 + u^4/5 + ... + u^20/21),
//        log s = e ln2 + log m.   Truncation error < 3e-17 relative.
// Accuracy is checked against the C library over the ranges the kernels use
// (tests/test_fast_math.py); ~1e-15 relative is far below what moves an fp32-rounded R.
#pragma once

#ifdef __HIPCC__
#include <hip/hip_runtime.h>
#define SDTW_HD __host__ __device__ __forceinline__
#else
#include <cmath>
#define SDTW_HD inline
#endif

namespace sdtw {
namespace fm {

constexpr double kLog2e = 1.4426950408889634074;     // log2(e)
constexpr double kLn2Hi = 6.93147180369123816490e-01;  // ln2 rounded to 32 significant bits
constexpr double kLn2Lo = 1.90821492927058770002e-10;  // ln2 - kLn2Hi
constexpr double kSqrtHalf = 0.70710678118654752440;

// 1/d for d in [1.7, 2.5] (log64's m + 1): hardware reciprocal seed on the device, two
// Newton-Raphson steps q <- q + q (1 - d q), each doubling the correct bits.
SDTW_HD double recip(double d) {
#if defined(__HIP_DEVICE_COMPILE__)
    double q = __builtin_amdgcn_rcp(d);
#else
    double q = 1.0 / d;
#endif
    double e = ::fma(-d, q, 1.0);
    q = ::fma(q, e, q);
    e = ::fma(-d, q, 1.0);
    q = ::fma(q, e, q);
    return q;
}

// exp(x) for x <= ~709 (the kernels only pass x <= 0).  -inf -> 0, NaN -> NaN.
// The degree-12 polynomial is evaluated with Estrin's scheme (dependency depth 5 instead
// of 12 for Horner).
SDTW_HD double exp64(double x) {
    // clamp far below the fp64 underflow threshold (comparison keeps NaN)
    const double xc = (x < -1080.0) ? -1080.0 : x;
    const double k = ::rint(xc * kLog2e);
    double r = ::fma(-k, kLn2Hi, xc);
    r = ::fma(-k, kLn2Lo, r);
    // c_n = 1/n!
    const double r2 = r * r;
    const double r4 = r2 * r2;
    const double r8 = r4 * r4;
    const double q0 = ::fma(r, 1.0, 1.0);
    const double q1 = ::fma(r, 1.666666666666666666667e-01, 0.5);
    const double q2 = ::fma(r, 8.333333333333333333333e-03, 4.166666666666666666667e-02);
    const double q3 = ::fma(r, 1.984126984126984126984e-04, 1.388888888888888888889e-03);
    const double q4 = ::fma(r, 2.755731922398589065256e-06, 2.480158730158730158730e-05);
    const double q5 = ::fma(r, 2.505210838544171877505e-08, 2.755731922398589065256e-07);
    const double c12 = 2.087675698786809897921e-09;
    const double s0 = ::fma(q1, r2, q0);
    const double s1 = ::fma(q3, r2, q2);
    const double s2 = ::fma(q5, r2, q4);
    const double t0 = ::fma(s1, r4, s0);
    const double t1 = ::fma(c12, r4, s2);
    const double p = ::fma(t1, r8, t0);
    return ::ldexp(p, (int)k);
}

// log(s) for finite s > 0 (the kernels pass s in [1, 3]).  +inf -> +inf, NaN -> NaN.
SDTW_HD double log64(double s) {
    int e;
    double m = ::frexp(s, &e);  // m in [0.5, 1)
    if (m < kSqrtHalf) {
        m = m + m;
        e -= 1;
    }
    const double num = m - 1.0;  // exact (Sterbenz)
    const double den = m + 1.0;
    const double q = recip(den);
    double u = num * q;
    u = ::fma(::fma(-u, den, num), q, u);  // one correction: u = num/den to ~1 ulp
    const double v = u * u;
    const double v2 = v * v;
    const double v4 = v2 * v2;
    const double v8 = v4 * v4;
    // sum_{n=0}^{10} v^n / (2n+1)
    const double a0 = ::fma(v, 1.0 / 3.0, 1.0);
    const double a1 = ::fma(v, 1.0 / 7.0, 1.0 / 5.0);
    const double a2 = ::fma(v, 1.0 / 11.0, 1.0 / 9.0);
    const double a3 = ::fma(v, 1.0 / 15.0, 1.0 / 13.0);
    const double a4 = ::fma(v, 1.0 / 19.0, 1.0 / 17.0);
    const double b0 = ::fma(a1, v2, a0);
    const double b1 = ::fma(a3, v2, a2);
    const double b2 = ::fma(1.0 / 21.0, v2, a4);
    const double c0 = ::fma(b1, v4, b0);
    const double p = ::fma(b2, v8, c0);
    const double lm = 2.0 * u * p;
    const double de = (double)e;
    const double r = ::fma(de, kLn2Hi, ::fma(de, kLn2Lo, lm));
    return (s < __builtin_inf()) ? r : s;  // +inf -> +inf, NaN -> NaN (select, no branch)
}

// ---------------------------------------------------------------------------------------
// Variants for the recursions' argument ranges, built for short dependency chains: no
// compare-and-select on the value path (those cost ~4x an fp64 FMA in latency on gfx950).
// ---------------------------------------------------------------------------------------

// exp(x) for x <= 0 with a Taylor polynomial of degree DEG on |r| <= ln2/2 (Estrin):
// DEG 10: truncation < 2.2e-13 relative; DEG 9: < 7e-12.  -inf -> 0.  The clamp is a
// maxNum, so NaN -> 0: callers that must propagate NaN do so separately.
template <int DEG>
SDTW_HD double exp_neg(double x) {
    static_assert(DEG == 9 || DEG == 10 || DEG == 12, "supported degrees: 9, 10, 12");
    const double xc = ::fmax(x, -1080.0);
    const double k = ::rint(xc * kLog2e);
    double r = ::fma(-k, kLn2Hi, xc);
    r = ::fma(-k, kLn2Lo, r);
    const double r2 = r * r;
    const double r4 = r2 * r2;
    const double r8 = r4 * r4;
    const double q0 = ::fma(r, 1.0, 1.0);
    const double q1 = ::fma(r, 1.666666666666666666667e-01, 0.5);
    const double q2 = ::fma(r, 8.333333333333333333333e-03, 4.166666666666666666667e-02);
    const double q3 = ::fma(r, 1.984126984126984126984e-04, 1.388888888888888888889e-03);
    const double s0 = ::fma(q1, r2, q0);
    const double s1 = ::fma(q3, r2, q2);
    const double t0 = ::fma(s1, r4, s0);
    double p;
    if (DEG == 9) {
        const double q4 = ::fma(r, 2.755731922398589065256e-06, 2.480158730158730158730e-05);
        p = ::fma(q4, r8, t0);
    } else if (DEG == 10) {
        const double q4 = ::fma(r, 2.755731922398589065256e-06, 2.480158730158730158730e-05);
        const double s2 = ::fma(2.755731922398589065256e-07, r2, q4);
        p = ::fma(s2, r8, t0);
    } else {
        const double q4 = ::fma(r, 2.755731922398589065256e-06, 2.480158730158730158730e-05);
        const double q5 = ::fma(r, 2.505210838544171877505e-08, 2.755731922398589065256e-07);
        const double s2 = ::fma(q5, r2, q4);
        const double t1 = ::fma(2.087675698786809897921e-09, r4, s2);
        p = ::fma(t1, r8, t0);
    }
    return ::ldexp(p, (int)k);
}

constexpr double kInvSqrt3 = 0.57735026918962576451;   // 1/sqrt(3)
constexpr double kLogSqrt3 = 0.54930614433405484570;   // log(sqrt(3))

// log(s) for s in [1, 3] (a soft-min's sum of exponentials, one of which is 1).
// z = s / sqrt(3) lies in [0.577, 1.732]; u = (z-1)/(z+1) (|u| <= 0.268) by a hardware
// reciprocal, one Newton-Raphson step and one residual correction;
// log s = log(sqrt 3) + 2u sum_{n=0}^{12} u^(2n)/(2n+1)  (truncation < 1e-15).
// No frexp, no compare: NaN propagates.
SDTW_HD double log_1to3(double s) {
    const double z = s * kInvSqrt3;
    const double num = z - 1.0;  // exact (Sterbenz, z in [0.5, 2])
    const double den = z + 1.0;
#if defined(__HIP_DEVICE_COMPILE__)
    double q = __builtin_amdgcn_rcp(den);
    q = ::fma(q, ::fma(-den, q, 1.0), q);
#else
    double q = 1.0 / den;
#endif
    double u = num * q;
    u = ::fma(::fma(-u, den, num), q, u);
    const double v = u * u;
    const double v2 = v * v;
    const double v4 = v2 * v2;
    const double v8 = v4 * v4;
    const double a0 = ::fma(v, 1.0 / 3.0, 1.0);
    const double a1 = ::fma(v, 1.0 / 7.0, 1.0 / 5.0);
    const double a2 = ::fma(v, 1.0 / 11.0, 1.0 / 9.0);
    const double a3 = ::fma(v, 1.0 / 15.0, 1.0 / 13.0);
    const double a4 = ::fma(v, 1.0 / 19.0, 1.0 / 17.0);
    const double a5 = ::fma(v, 1.0 / 23.0, 1.0 / 21.0);
    const double b0 = ::fma(a1, v2, a0);
    const double b1 = ::fma(a3, v2, a2);
    const double b2 = ::fma(a5, v2, a4);
    const double c0 = ::fma(b1, v4, b0);
    const double c1 = ::fma(1.0 / 25.0, v4, b2);
    const double p = ::fma(c1, v8, c0);
    return ::fma(2.0 * u, p, kLogSqrt3);
}

}  // namespace fm
}  // namespace sdtw
