// sdtw_dp.hip -- wavefront-kernel dispatch, the scratch-reset kernel, and the R table
// pack / unpack kernels.  The wavefront kernels themselves live in sdtw_dp.hpp and are
// instantiated per (direction, arithmetic, cost source) in sdtw_dp_{fwd,bwd}_*.hip.
#include "sdtw_dp.hpp"

namespace sdtw {

__global__ void prep_kernel(int* ticket, int* gflag, int nflags, int* err) {
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx == 0) {
        *ticket = 0;
        *err = 0;
    }
    for (int k = idx; k < nflags; k += gridDim.x * blockDim.x) gflag[k] = 0;
}

hipError_t launch_dp_prep(const DPParams& P, hipStream_t st) {
    const int nflags = P.B * P.G;
    const int pblocks = min(max((nflags + 255) / 256, 1), 1024);
    hipLaunchKernelGGL(prep_kernel, dim3(pblocks), dim3(256), 0, st, P.ticket, P.gflag, nflags, P.err);
    return hipGetLastError();
}

hipError_t launch_fwd(const DPParams& P, bool fused, bool muladd, bool exact, hipStream_t st) {
    if (exact)
        return fused ? launch_dp_variant<false, true, true>(P, muladd, st)
                     : launch_dp_variant<false, true, false>(P, muladd, st);
    return fused ? launch_dp_variant<false, false, true>(P, muladd, st)
                 : launch_dp_variant<false, false, false>(P, muladd, st);
}

hipError_t launch_bwd(const DPParams& P, bool fused, bool muladd, bool exact, hipStream_t st) {
    if (exact)
        return fused ? launch_dp_variant<true, true, true>(P, muladd, st)
                     : launch_dp_variant<true, true, false>(P, muladd, st);
    return fused ? launch_dp_variant<true, false, true>(P, muladd, st)
                 : launch_dp_variant<true, false, false>(P, muladd, st);
}

// ---------------------------------------------------------------------------------------
// R table (band-skewed) <-> dense (B, N, M)
// ---------------------------------------------------------------------------------------
__global__ void table_unpack_kernel(const float* __restrict__ Rt, float* __restrict__ Rd, int B,
                                    int N, int M, int nb, int S) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t total = (int64_t)B * N * M;
    if (idx >= total) return;
    const int j = (int)(idx % M);
    const int64_t pi = idx / M;
    const int i = (int)(pi % N);
    const int p = (int)(pi / N);
    const int b = i / WAVE, l = i - b * WAVE;
    Rd[idx] = Rt[(((int64_t)p * nb + b) * S + (j + l)) * WAVE + l];
}

__global__ void table_pack_kernel(const float* __restrict__ Rd, float* __restrict__ Rt, int B, int N,
                                  int M, int nb, int S) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t total = (int64_t)B * N * M;
    if (idx >= total) return;
    const int j = (int)(idx % M);
    const int64_t pi = idx / M;
    const int i = (int)(pi % N);
    const int p = (int)(pi / N);
    const int b = i / WAVE, l = i - b * WAVE;
    Rt[(((int64_t)p * nb + b) * S + (j + l)) * WAVE + l] = Rd[idx];
}

hipError_t launch_table_unpack(const float* Rt, float* Rd, int B, int N, int M, hipStream_t st) {
    const int64_t total = (int64_t)B * N * M;
    if (total == 0) return hipSuccess;
    const int nb = (N + WAVE - 1) / WAVE;
    hipLaunchKernelGGL(table_unpack_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st,
                       Rt, Rd, B, N, M, nb, dp_band_steps(M));
    return hipGetLastError();
}

hipError_t launch_table_pack(const float* Rd, float* Rt, int B, int N, int M, hipStream_t st) {
    const int64_t total = (int64_t)B * N * M;
    if (total == 0) return hipSuccess;
    const int nb = (N + WAVE - 1) / WAVE;
    hipLaunchKernelGGL(table_pack_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, Rd,
                       Rt, B, N, M, nb, dp_band_steps(M));
    return hipGetLastError();
}

}  // namespace sdtw
