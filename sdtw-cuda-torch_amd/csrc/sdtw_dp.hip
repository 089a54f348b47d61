// sdtw_dp.hip -- wavefront-kernel dispatch, the scratch-reset kernel, and the R table
// pack / unpack kernels.  The wavefront kernels themselves live in sdtw_dp.hpp and are
// instantiated per (direction, arithmetic, cost source) in sdtw_dp_{fwd,bwd}_*.hip.
#include "sdtw_dp.hpp"

namespace sdtw {

// Zero the ticket and error flag; mark every entry of the cross-workgroup rows empty.
__global__ void prep_kernel(int* ticket, int* err, unsigned long long* rows, int64_t nwords,
                            unsigned long long lo, unsigned long long hi) {
    prep_rows((int64_t)blockIdx.x * blockDim.x + threadIdx.x, (int64_t)gridDim.x * blockDim.x,
              ticket, err, rows, nwords, lo, hi);
}

hipError_t launch_dp_prep(const DPParams& P, bool bwd, hipStream_t st) {
    const int64_t entries = (int64_t)P.B * P.G * P.RW;
    const int64_t nwords = bwd || P.lin ? 2 * entries : entries;  // 16-byte entries
    const unsigned long long lo = bwd ? (unsigned long long)kEmpty32 : kEmpty64;
    const unsigned long long hi = bwd ? 0ull : kEmpty64;
    if (P.x2_fill) {  // with the fused recursions' row norms (and the gradient mode's zeroing)
        const int64_t ngy = bwd && P.gy_out ? (int64_t)P.B * P.M * P.K : 0;
        const int64_t ncl = !bwd && P.D_out && P.clamped ? (int64_t)P.B : 0;
        return launch_prep_norms(P.ticket, P.err, reinterpret_cast<unsigned long long*>(P.gring),
                                 nwords, lo, hi, P.x, P.x2_fill, (int64_t)P.B * P.N, P.y,
                                 P.y2_fill, (int64_t)P.B * P.M, P.K,
                                 reinterpret_cast<unsigned*>(P.gy_out), ngy,
                                 reinterpret_cast<unsigned*>(P.clamped), ncl, st);
    }
    int64_t blocks = (nwords + 255) / 256;
    blocks = blocks < 1 ? 1 : (blocks > 2048 ? 2048 : blocks);
    hipLaunchKernelGGL(prep_kernel, dim3((unsigned)blocks), dim3(256), 0, st, P.ticket, P.err,
                       reinterpret_cast<unsigned long long*>(P.gring), nwords, lo, hi);
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
