// sdtw_bary.hip -- device kernels of the barycenter loop (sdtw_barycenter_f32).
//
// One iteration of the reference's loop (barycenters.py:116-139) is: the Soft-DTW losses
// of the barycenter against every sequence, the weighted loss, its gradient, gradient-norm
// clipping to 1, an Adam step and the cosine learning-rate schedule.  The recursions run on
// the engine's fused kernels, which read the barycenter from a (B, N, K) copy, one per pair
// (the reference's barycenter.unsqueeze(0).expand(B, -1, -1)); these kernels do the rest:
//   * bary_broadcast_kernel: that copy, written once before the first iteration;
//   * bary_grad_kernel: grad = sum_b gx[b] (the fused backward ran with gout = weights, so
//     gx[b] is already w_b * d sdtw_b / d x) and each workgroup's partial sum of grad^2;
//   * bary_adam_kernel: the norm from the partials (the same fixed-order reduction in every
//     workgroup, so all of them clip by the same coefficient), the clip, the Adam update
//     (torch's Adam with betas (0.9, 0.999), eps 1e-8, no weight decay, written from the
//     published algorithm: m <- m + (1 - b1)(g - m), v <- b2 v + (1 - b2) g^2,
//     p <- p - (lr / bc1) m / (sqrt(v) / sqrt(bc2) + eps)), the new barycenter written into
//     every pair's copy for the next iteration, and the weighted loss sum_b w_b out_b of the
//     iterate before the update.
#include "sdtw_internal.hpp"

namespace sdtw {

__global__ void bary_broadcast_kernel(const float* __restrict__ bary, float* __restrict__ xb,
                                      int64_t B, int64_t NK) {
    const int64_t total = B * NK;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x)
        xb[e] = bary[e % NK];
}

constexpr int kUpdThreads = 256;

static __device__ __forceinline__ float block_sum(float v, float* red) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float t = 0.0f;
    for (int k = 0; k < kUpdThreads / 64; ++k) t += red[k];
    return t;
}

__global__ void __launch_bounds__(kUpdThreads)
bary_grad_kernel(const float* __restrict__ gx, float* __restrict__ gbuf,
                 float* __restrict__ part, int B, int NK) {
    __shared__ float red[kUpdThreads / 64];
    const int e = (int)blockIdx.x * kUpdThreads + (int)threadIdx.x;
    float g = 0.0f;
    if (e < NK) {
#pragma unroll 8
        for (int b = 0; b < B; ++b) g += gx[(int64_t)b * NK + e];
        gbuf[e] = g;
    }
    const float ss = block_sum(g * g, red);
    if (threadIdx.x == 0) part[blockIdx.x] = ss;
}

__global__ void __launch_bounds__(kUpdThreads)
bary_adam_kernel(const float* __restrict__ gbuf, const float* __restrict__ part, int nparts,
                 const float* __restrict__ out, const float* __restrict__ w,
                 float* __restrict__ bary, float* __restrict__ xb, float* __restrict__ m,
                 float* __restrict__ v, float* __restrict__ loss, int B, int NK, BaryStep s) {
    __shared__ float red[kUpdThreads / 64];
    float ss = 0.0f;
    for (int k = (int)threadIdx.x; k < nparts; k += kUpdThreads) ss += part[k];
    const float tot = block_sum(ss, red);
    // clip_grad_norm_(max_norm): coefficient max_norm / (norm + 1e-6), at most 1
    const float clip = fminf(s.max_norm / (sqrtf(tot) + 1e-6f), 1.0f);
    const int e = (int)blockIdx.x * kUpdThreads + (int)threadIdx.x;
    if (e < NK) {
        const float g = gbuf[e] * clip;
        const float mo = m[e];
        const float mn = mo + s.one_m_b1 * (g - mo);
        const float vn = v[e] * s.b2 + s.one_m_b2 * g * g;
        m[e] = mn;
        v[e] = vn;
        const float den = sqrtf(vn) / s.bc2_sqrt + s.eps;
        const float p = bary[e] + s.neg_step * (mn / den);
        bary[e] = p;
        for (int b = 0; b < B; ++b) xb[(int64_t)b * NK + e] = p;
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        float l = 0.0f;
        for (int b = 0; b < B; ++b) l += w[b] * out[b];
        *loss = l;
    }
}

__global__ void fill_zero_kernel(float* __restrict__ p, int64_t n) {
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n;
         e += (int64_t)gridDim.x * blockDim.x)
        p[e] = 0.0f;
}

hipError_t launch_fill_zero(float* p, int64_t n, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    int64_t blocks = (n + 255) / 256;
    blocks = blocks > 1024 ? 1024 : blocks;
    hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)blocks), dim3(256), 0, st, p, n);
    return hipGetLastError();
}

hipError_t launch_bary_broadcast(const float* bary, float* xb, int64_t B, int64_t NK,
                                 hipStream_t st) {
    const int64_t total = B * NK;
    int64_t blocks = (total + 255) / 256;
    blocks = blocks < 1 ? 1 : (blocks > 4096 ? 4096 : blocks);
    hipLaunchKernelGGL(bary_broadcast_kernel, dim3((unsigned)blocks), dim3(256), 0, st, bary, xb,
                       B, NK);
    return hipGetLastError();
}

int bary_parts(int64_t NK) { return (int)((NK + kUpdThreads - 1) / kUpdThreads); }

hipError_t launch_bary_update(const float* gx, const float* out, const float* w, float* bary,
                              float* xb, float* m, float* v, float* gbuf, float* part,
                              float* loss, int B, int NK, const BaryStep& s, hipStream_t st) {
    const int nb = bary_parts(NK);
    hipLaunchKernelGGL(bary_grad_kernel, dim3((unsigned)nb), dim3(kUpdThreads), 0, st, gx, gbuf,
                       part, B, NK);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(bary_adam_kernel, dim3((unsigned)nb), dim3(kUpdThreads), 0, st, gbuf, part,
                       nb, out, w, bary, xb, m, v, loss, B, NK, s);
    return hipGetLastError();
}

}  // namespace sdtw
