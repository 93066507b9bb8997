// Adam step over several parameter tensors in one launch.
//
// The reference trains with torch.optim.Adam over per-group learning rates
// (gaussian_trace/model.py:172-189).  torch's multi-tensor implementations
// spend tens of microseconds per step on this path's ~10^5 parameters; here
// every tensor of the step is one row of the grid (blockIdx.y), and the
// per-tensor scalars travel in the kernel arguments.
//
// Per element, as torch's single-tensor Adam (torch/optim/adam.py,
// _single_tensor_adam, non-capturable, amsgrad off, maximize off):
//   g   = grad + weight_decay * param           (only when weight_decay != 0)
//   m   = lerp(m, g, 1 - beta1)                 (m + (1 - beta1) * (g - m))
//   v   = v * beta2 + (1 - beta2) * g * g
//   p  -= step_size * m / (sqrt(v) / sqrt(bias_correction2) + eps)
// with step_size = lr / bias_correction1 formed on the host in double.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/cubicsplat_hip.h"

namespace cs {

struct AdamTensorArgs {
    float* p;
    const float* g;
    float* m;
    float* v;
    int64_t n;
    float step_size;
    float bc2_sqrt;
    float weight_decay;
    float pad;
};

struct AdamLaunchArgs {
    AdamTensorArgs t[CS_ADAM_MAX_TENSORS];
    float beta2, one_minus_beta1, one_minus_beta2, eps;
};

constexpr int kAdamThreads = 256;
constexpr int kAdamItems = 4;

__global__ __launch_bounds__(kAdamThreads) void k_adam(AdamLaunchArgs a) {
    const AdamTensorArgs& t = a.t[blockIdx.y];
    const float omb1 = a.one_minus_beta1, omb2 = a.one_minus_beta2;
    const int64_t base = (int64_t)blockIdx.x * (kAdamThreads * kAdamItems) + threadIdx.x;
#pragma unroll
    for (int k = 0; k < kAdamItems; ++k) {
        const int64_t i = base + (int64_t)k * kAdamThreads;
        if (i >= t.n) break;
        float g = t.g[i];
        const float p = t.p[i];
        if (t.weight_decay != 0.0f) g = g + t.weight_decay * p;
        float m = t.m[i];
        m = m + omb1 * (g - m);
        const float v = t.v[i] * a.beta2 + omb2 * (g * g);
        const float denom = __builtin_sqrtf(v) / t.bc2_sqrt + a.eps;
        t.m[i] = m;
        t.v[i] = v;
        t.p[i] = p - t.step_size * (m / denom);
    }
}

// Adan step (manbo/optim.py:70-190 with adan_step_from_grad_kernel,
// ops/optim.py:8-113) over several tensors in one launch, per element with the
// reference kernel's fp32 expressions:
//   g     = grad * clip
//   ngod  = step == 1 ? 0 : neg_pre_grad + g         (g_t - g_{t-1})
//   m     = m * beta1 + g * (1 - beta1)
//   d     = d * beta2 + ngod * (1 - beta2)
//   ngod2 = ngod * beta2 + g
//   n     = n * beta3 + ngod2 * ngod2 * (1 - beta3)
//   denom = sqrt(n) / sqrt(bias_correction3) + eps
//   p    -= (lr / bc1) * m / denom, then (lr * beta2 / bc2) * d / denom, with
//           the weight decay as p (1 - lr wd) first (no_prox) or p / (1 + lr wd)
//           last; neg_pre_grad = -g.
// clip: the global-norm clip factor, a device scalar or (NULL) the tensor's
// host value.
struct AdanTensorArgs {
    float* p;
    const float* g;
    float* m;
    float* n;
    float* d;
    float* npg;
    int64_t numel;
    float beta1, beta2, beta3, bc1, bc2, bc3_sqrt, lr, wd, eps, clip;
    int32_t first, no_prox;
};

struct AdanLaunchArgs {
    AdanTensorArgs t[CS_ADAM_MAX_TENSORS];
    const float* clip;
};

__global__ __launch_bounds__(kAdamThreads) void k_adan(AdanLaunchArgs a) {
    const AdanTensorArgs& t = a.t[blockIdx.y];
    const float clip = a.clip ? *a.clip : t.clip;
    const float one = 1.0f;
    const float step_size = t.lr / t.bc1;
    const float step_size_diff = t.lr * t.beta2 / t.bc2;
    const int64_t base = (int64_t)blockIdx.x * (kAdamThreads * kAdamItems) + threadIdx.x;
#pragma unroll
    for (int k = 0; k < kAdamItems; ++k) {
        const int64_t i = base + (int64_t)k * kAdamThreads;
        if (i >= t.numel) break;
        const float p = t.p[i];
        const float g = t.g[i] * clip;
        const float ngod = t.first ? 0.0f : t.npg[i] + g;
        const float m = t.m[i] * t.beta1 + g * (one - t.beta1);
        const float d = t.d[i] * t.beta2 + ngod * (one - t.beta2);
        const float ngod2 = ngod * t.beta2 + g;
        const float n = t.n[i] * t.beta3 + ngod2 * ngod2 * (one - t.beta3);
        const float denom = __builtin_sqrtf(n) / t.bc3_sqrt + t.eps;
        float q = p;
        if (t.no_prox) {
            q = q * (one - t.lr * t.wd);
            q = q - step_size * m / denom;
            q = q - step_size_diff * d / denom;
        } else {
            q = q - step_size * m / denom;
            q = q - step_size_diff * d / denom;
            q = q / (one + t.lr * t.wd);
        }
        t.p[i] = q;
        t.m[i] = m;
        t.d[i] = d;
        t.n[i] = n;
        t.npg[i] = -g;
    }
}

}  // namespace cs

using namespace cs;

extern "C" int cs_adan_step(int32_t ntensors, float* const* params, const float* const* grads,
                            float* const* exp_avgs, float* const* exp_avg_sqs,
                            float* const* exp_avg_diffs, float* const* neg_pre_grads,
                            const int64_t* numels, const float* scalars, const int32_t* flags,
                            const float* clip, hipStream_t stream) {
    if (ntensors < 0 || ntensors > CS_ADAM_MAX_TENSORS) return CS_ERR_ARGS;
    if (ntensors == 0) return CS_OK;
    if (!params || !grads || !exp_avgs || !exp_avg_sqs || !exp_avg_diffs || !neg_pre_grads ||
        !numels || !scalars || !flags)
        return CS_ERR_ARGS;
    AdanLaunchArgs a{};
    int64_t nmax = 0;
    for (int k = 0; k < ntensors; ++k) {
        const float* sc = scalars + 10 * k;
        if (numels[k] < 0) return CS_ERR_ARGS;
        if (numels[k] > 0 && (!params[k] || !grads[k] || !exp_avgs[k] || !exp_avg_sqs[k] ||
                              !exp_avg_diffs[k] || !neg_pre_grads[k]))
            return CS_ERR_ARGS;
        a.t[k] = AdanTensorArgs{params[k], grads[k], exp_avgs[k], exp_avg_sqs[k],
                                exp_avg_diffs[k], neg_pre_grads[k], numels[k], sc[0], sc[1],
                                sc[2], sc[3], sc[4], sc[5], sc[6], sc[7], sc[8], sc[9],
                                flags[2 * k], flags[2 * k + 1]};
        nmax = numels[k] > nmax ? numels[k] : nmax;
    }
    a.clip = clip;
    if (nmax == 0) return CS_OK;
    const int64_t per_block = kAdamThreads * kAdamItems;
    const int64_t gx = (nmax + per_block - 1) / per_block;
    if (gx > INT32_MAX) return CS_ERR_ARGS;
    hipLaunchKernelGGL(k_adan, dim3((unsigned)gx, (unsigned)ntensors), dim3(kAdamThreads), 0,
                       stream, a);
    return hipGetLastError() == hipSuccess ? CS_OK : CS_ERR_HIP;
}

extern "C" int cs_adam_step(int32_t ntensors, float* const* params, const float* const* grads,
                            float* const* exp_avgs, float* const* exp_avg_sqs,
                            const int64_t* numels, const float* step_sizes,
                            const float* bias_correction2_sqrts, const float* weight_decays,
                            double beta1, double beta2, double eps, hipStream_t stream) {
    if (ntensors < 0 || ntensors > CS_ADAM_MAX_TENSORS) return CS_ERR_ARGS;
    if (ntensors == 0) return CS_OK;
    if (!params || !grads || !exp_avgs || !exp_avg_sqs || !numels || !step_sizes ||
        !bias_correction2_sqrts || !weight_decays)
        return CS_ERR_ARGS;
    AdamLaunchArgs a{};
    int64_t nmax = 0;
    for (int k = 0; k < ntensors; ++k) {
        if (numels[k] < 0 || !(bias_correction2_sqrts[k] > 0.0f)) return CS_ERR_ARGS;
        if (numels[k] > 0 && (!params[k] || !grads[k] || !exp_avgs[k] || !exp_avg_sqs[k]))
            return CS_ERR_ARGS;
        a.t[k] = AdamTensorArgs{params[k], grads[k], exp_avgs[k], exp_avg_sqs[k], numels[k],
                                step_sizes[k], bias_correction2_sqrts[k], weight_decays[k], 0.0f};
        nmax = numels[k] > nmax ? numels[k] : nmax;
    }
    // As torch does with its Python-float hyperparameters: 1 - beta in
    // double, each scalar rounded to fp32 once.
    a.beta2 = (float)beta2;
    a.one_minus_beta1 = (float)(1.0 - beta1);
    a.one_minus_beta2 = (float)(1.0 - beta2);
    a.eps = (float)eps;
    if (nmax == 0) return CS_OK;
    const int64_t per_block = kAdamThreads * kAdamItems;
    const int64_t gx = (nmax + per_block - 1) / per_block;
    if (gx > INT32_MAX) return CS_ERR_ARGS;
    hipLaunchKernelGGL(k_adam, dim3((unsigned)gx, (unsigned)ntensors), dim3(kAdamThreads), 0,
                       stream, a);
    return hipGetLastError() == hipSuccess ? CS_OK : CS_ERR_HIP;
}
