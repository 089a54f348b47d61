// sdtw_bary.hip -- device kernels of the barycenter loop (sdtw_barycenter_f32).
//
// One iteration of the reference's loop (barycenters.py:116-139) is: the Soft-DTW losses
// of the barycenter against every sequence, the weighted loss, its gradient, gradient-norm
// clipping to 1, an Adam step and the cosine learning-rate schedule.  The recursions run on
// the engine's fused kernels; these two kernels do the rest on the device:
//   * bary_broadcast_kernel: the barycenter (N, K) copied to every pair, (B, N, K) -- the
//     reference's barycenter.unsqueeze(0).expand(B, -1, -1);
//   * bary_update_kernel: grad = sum_b gx[b] (the fused backward ran with gout = weights, so
//     gx[b] is already w_b * d sdtw_b / d x), the clip, the Adam update (torch's Adam with
//     betas (0.9, 0.999), eps 1e-8, no weight decay, written from the published algorithm:
//     m <- m + (1 - b1)(g - m), v <- b2 v + (1 - b2) g^2, p <- p - (lr / bc1) m / (sqrt(v) / sqrt(bc2)
//     + eps)), and the weighted loss sum_b w_b out_b of the iterate before the update.
#include "sdtw_internal.hpp"

namespace sdtw {

__global__ void bary_broadcast_kernel(const float* __restrict__ bary, float* __restrict__ xb,
                                      int64_t B, int64_t NK) {
    const int64_t total = B * NK;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x)
        xb[e] = bary[e % NK];
}

constexpr int kUpdThreads = 1024;

__global__ void __launch_bounds__(kUpdThreads)
bary_update_kernel(const float* __restrict__ gx, const float* __restrict__ out,
                   const float* __restrict__ w, float* __restrict__ bary, float* __restrict__ m,
                   float* __restrict__ v, float* __restrict__ gbuf, float* __restrict__ loss,
                   int B, int NK, BaryStep s) {
    __shared__ float red[kUpdThreads / 64];
    const int tid = threadIdx.x;
    // the gradient (sum over pairs in pair order) and its squared norm
    float ss = 0.0f;
    for (int e = tid; e < NK; e += kUpdThreads) {
        float g = 0.0f;
        for (int b = 0; b < B; ++b) g += gx[(int64_t)b * NK + e];
        gbuf[e] = g;
        ss = fmaf(g, g, ss);
    }
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    float tot = 0.0f;
    for (int k = 0; k < kUpdThreads / 64; ++k) tot += red[k];
    // clip_grad_norm_(max_norm): coefficient max_norm / (norm + 1e-6), at most 1
    const float clip = fminf(s.max_norm / (sqrtf(tot) + 1e-6f), 1.0f);
    for (int e = tid; e < NK; e += kUpdThreads) {
        const float g = gbuf[e] * clip;
        const float mo = m[e];
        const float mn = mo + s.one_m_b1 * (g - mo);
        const float vn = v[e] * s.b2 + s.one_m_b2 * g * g;
        m[e] = mn;
        v[e] = vn;
        const float den = sqrtf(vn) / s.bc2_sqrt + s.eps;
        bary[e] = bary[e] + s.neg_step * (mn / den);
    }
    if (tid == 0) {
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

hipError_t launch_bary_update(const float* gx, const float* out, const float* w, float* bary,
                              float* m, float* v, float* gbuf, float* loss, int B, int NK,
                              const BaryStep& s, hipStream_t st) {
    hipLaunchKernelGGL(bary_update_kernel, dim3(1), dim3(kUpdThreads), 0, st, gx, out, w, bary, m,
                       v, gbuf, loss, B, NK, s);
    return hipGetLastError();
}

}  // namespace sdtw
