// sdtw_internal.hpp -- parameter blocks and launcher declarations shared by the .hip files.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sdtw {

struct FwdParams {
    const float* D;   // unfused cost (B,N,M) or nullptr
    const float* x;   // fused: (B,N,K)
    const float* y;   // fused: (B,M,K)
    const float* x2;  // fused: row norms (B,N)
    const float* y2;  // fused: row norms (B,M)
    float* R;         // (B,N,M)
    float* out;       // (B)
    double* edge;     // (B,M) fp64 hand-over between row blocks
    int B, N, M, K;
    double gamma, bw;
};

struct BwdParams {
    const float* D;
    const float* x;
    const float* y;
    const float* x2;
    const float* y2;
    const float* R;     // (B,N,M)
    const float* gout;  // (B) or nullptr
    float* G;           // (B,N,M): gout * E
    float* edge;        // (B,3,M+1) hand-over between row blocks
    int B, N, M, K;
    double gamma, bw;
};

struct DistParams {
    const float* x;  // (B,N,K)
    const float* y;  // (B,M,K)
    float* x2;       // (B,N)
    float* y2;       // (B,M)
    float* D;        // (B,N,M)
    int B, N, M, K;
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
};

hipError_t launch_norms(const float* v, float* out, int64_t rows, int K, hipStream_t st);
hipError_t launch_dist(const DistParams& p, bool muladd, bool mfma, hipStream_t st);
hipError_t launch_dist_bwd(const DistBwdParams& p, hipStream_t st);
hipError_t launch_fwd(const FwdParams& p, bool fused, bool muladd, hipStream_t st);
hipError_t launch_bwd(const BwdParams& p, bool fused, bool muladd, hipStream_t st);

}  // namespace sdtw
