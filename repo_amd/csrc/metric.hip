// MSE and SSIM losses (forward and backward) for MI355X.
//
// MSE: one launch; each workgroup reduces a contiguous chunk with 16-byte
// loads, writes its partial, and the last workgroup to finish (ticket
// counter) sums the partials in index order, so the result is deterministic.
//
// SSIM: valid-window SSIM of ops/metric.py:205-341 with the 2D Gaussian
// window applied separably (the reference window is the outer product of one
// normalized 1D Gaussian, metric.py:47-61): a 32x32 output tile stages its
// (32+win-1)^2 inputs in LDS, a horizontal pass produces the five windowed
// moments per row, a vertical pass finishes them.  The backward (absent from
// the reference) uses the per-pixel partials A = dS/dmu_x, B = dS/dE[x^2],
// C = dS/dE[xy] and one transposed separable correlation.
#include "cs_common.h"
#include "../../include/cubicsplat_hip.h"

namespace cs {

constexpr int kMseThreads = 256;
constexpr int kMseItems = 16;  // float elements per thread
constexpr int kMseChunk = kMseThreads * kMseItems;

__device__ __forceinline__ float block_sum_256(float v, float* sh) {
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    if (lane == 0) sh[w] = v;
    __syncthreads();
    float r = 0.0f;
    if (threadIdx.x == 0) r = (sh[0] + sh[1]) + (sh[2] + sh[3]);
    __syncthreads();
    return r;
}

// Sums partials[0..n) in a fixed order with one workgroup; result in thread 0.
__device__ __forceinline__ float block_sum_partials(const float* __restrict__ partials, int n,
                                                   float* sh) {
    float acc = 0.0f;
    for (int i = threadIdx.x; i < n; i += kMseThreads) acc += partials[i];
    return block_sum_256(acc, sh);
}

__global__ __launch_bounds__(kMseThreads) void k_mse_fwd(const float* __restrict__ x,
                                                        const float* __restrict__ y, int64_t n,
                                                        float* __restrict__ partials,
                                                        uint32_t* __restrict__ ticket,
                                                        float* __restrict__ loss) {
    __shared__ float sh[4];
    __shared__ bool last;
    const int64_t base = (int64_t)blockIdx.x * kMseChunk;
    float acc = 0.0f;
    const bool aligned = ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) & 15) == 0;
    if (aligned && base + kMseChunk <= n) {
        const float4* x4 = reinterpret_cast<const float4*>(x + base);
        const float4* y4 = reinterpret_cast<const float4*>(y + base);
#pragma unroll
        for (int k = 0; k < kMseItems / 4; ++k) {
            const float4 a = x4[k * kMseThreads + threadIdx.x];
            const float4 b = y4[k * kMseThreads + threadIdx.x];
            const float d0 = a.x - b.x, d1 = a.y - b.y, d2 = a.z - b.z, d3 = a.w - b.w;
            acc = __builtin_fmaf(d0, d0, acc);
            acc = __builtin_fmaf(d1, d1, acc);
            acc = __builtin_fmaf(d2, d2, acc);
            acc = __builtin_fmaf(d3, d3, acc);
        }
    } else {
        for (int k = 0; k < kMseItems; ++k) {
            const int64_t i = base + (int64_t)k * kMseThreads + threadIdx.x;
            if (i < n) {
                const float d = x[i] - y[i];
                acc = __builtin_fmaf(d, d, acc);
            }
        }
    }
    const float bs = block_sum_256(acc, sh);
    if (threadIdx.x == 0) {
        partials[blockIdx.x] = bs;
        __threadfence();
        last = atomicAdd(ticket, 1u) == gridDim.x - 1;
    }
    __syncthreads();
    if (last) {
        __threadfence();
        const float tot = block_sum_partials(partials, gridDim.x, sh);
        if (threadIdx.x == 0) {
            *loss = tot / (float)n;
            *ticket = 0u;
        }
    }
}

__global__ __launch_bounds__(256) void k_mse_bwd(const float* __restrict__ x,
                                                const float* __restrict__ y, int64_t n,
                                                const float* __restrict__ grad_loss, float two_n,
                                                float* __restrict__ gx, float* __restrict__ gy) {
    const float s = (*grad_loss) * two_n;
    const int64_t i4 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
    if (i4 + 4 <= n && ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) & 15) == 0 &&
        ((reinterpret_cast<uintptr_t>(gx) | reinterpret_cast<uintptr_t>(gy)) & 15) == 0) {
        const float4 a = *reinterpret_cast<const float4*>(x + i4);
        const float4 b = *reinterpret_cast<const float4*>(y + i4);
        const float4 d = make_float4(s * (a.x - b.x), s * (a.y - b.y), s * (a.z - b.z),
                                     s * (a.w - b.w));
        if (gx) *reinterpret_cast<float4*>(gx + i4) = d;
        if (gy) *reinterpret_cast<float4*>(gy + i4) = make_float4(-d.x, -d.y, -d.z, -d.w);
    } else {
        for (int64_t i = i4; i < i4 + 4 && i < n; ++i) {
            const float d = s * (x[i] - y[i]);
            if (gx) gx[i] = d;
            if (gy) gy[i] = -d;
        }
    }
}

// ------------------------------------------------------------------ SSIM

constexpr int kSsimOT = 32;  // output tile edge

template <int WIN>
struct SsimTile {
    static constexpr int IT = kSsimOT + WIN - 1;  // staged input tile edge
    static constexpr int ITP = IT + 1;             // padded LDS row
};

template <int WIN>
__global__ __launch_bounds__(256) void k_ssim_fwd(const float* __restrict__ x,
                                                 const float* __restrict__ y, int h, int w,
                                                 int oh, int ow,
                                                 const float* __restrict__ win1d, float c1,
                                                 float c2, float* __restrict__ partials,
                                                 uint32_t* __restrict__ ticket,
                                                 float* __restrict__ out,
                                                 float* __restrict__ abc, int nc) {
    constexpr int IT = SsimTile<WIN>::IT, ITP = SsimTile<WIN>::ITP;
    __shared__ float xs[IT][ITP];
    __shared__ float ys[IT][ITP];
    __shared__ float hm[5][IT][kSsimOT + 1];
    __shared__ float gw[WIN];
    __shared__ float sh[4];
    __shared__ bool last;
    const int c = blockIdx.z;
    const int ox0 = blockIdx.x * kSsimOT, oy0 = blockIdx.y * kSsimOT;
    const float* xc = x + (size_t)c * h * w;
    const float* yc = y + (size_t)c * h * w;
    if (threadIdx.x < WIN) gw[threadIdx.x] = win1d[threadIdx.x];
    for (int idx = threadIdx.x; idx < IT * IT; idx += 256) {
        const int r = idx / IT, q = idx - r * IT;
        const int gy = oy0 + r, gx = ox0 + q;
        const bool in = gy < h && gx < w;
        xs[r][q] = in ? xc[(size_t)gy * w + gx] : 0.0f;
        ys[r][q] = in ? yc[(size_t)gy * w + gx] : 0.0f;
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < IT * kSsimOT; idx += 256) {
        const int r = idx / kSsimOT, q = idx - r * kSsimOT;
        float m0 = 0.f, m1 = 0.f, m2 = 0.f, m3 = 0.f, m4 = 0.f;
#pragma unroll
        for (int k = 0; k < WIN; ++k) {
            const float g = gw[k];
            const float a = xs[r][q + k], b = ys[r][q + k];
            m0 = __builtin_fmaf(g, a, m0);
            m1 = __builtin_fmaf(g, b, m1);
            m2 = __builtin_fmaf(g, a * a, m2);
            m3 = __builtin_fmaf(g, b * b, m3);
            m4 = __builtin_fmaf(g, a * b, m4);
        }
        hm[0][r][q] = m0; hm[1][r][q] = m1; hm[2][r][q] = m2; hm[3][r][q] = m3; hm[4][r][q] = m4;
    }
    __syncthreads();
    float acc = 0.0f;
    const size_t plane = (size_t)oh * ow;
    for (int idx = threadIdx.x; idx < kSsimOT * kSsimOT; idx += 256) {
        const int r = idx / kSsimOT, q = idx - r * kSsimOT;
        const int oy = oy0 + r, ox = ox0 + q;
        if (oy >= oh || ox >= ow) continue;
        float mu1 = 0.f, mu2 = 0.f, ex2 = 0.f, ey2 = 0.f, exy = 0.f;
#pragma unroll
        for (int k = 0; k < WIN; ++k) {
            const float g = gw[k];
            mu1 = __builtin_fmaf(g, hm[0][r + k][q], mu1);
            mu2 = __builtin_fmaf(g, hm[1][r + k][q], mu2);
            ex2 = __builtin_fmaf(g, hm[2][r + k][q], ex2);
            ey2 = __builtin_fmaf(g, hm[3][r + k][q], ey2);
            exy = __builtin_fmaf(g, hm[4][r + k][q], exy);
        }
        const float mu1_sq = mu1 * mu1, mu2_sq = mu2 * mu2, mu12 = mu1 * mu2;
        const float s1 = ex2 - mu1_sq, s2 = ey2 - mu2_sq, s12 = exy - mu12;
        const float n1 = 2.0f * mu12 + c1, d1 = mu1_sq + mu2_sq + c1;
        const float n2 = 2.0f * s12 + c2, d2 = s1 + s2 + c2;
        const float l = n1 / d1, cs_ = n2 / d2;
        acc += l * cs_;
        if (abc) {
            const float dl = 2.0f * (mu2 - l * mu1) / d1;
            const float dcs = 2.0f * (mu1 * cs_ - mu2) / d2;
            const size_t o = (size_t)c * plane + (size_t)oy * ow + ox;
            const size_t stride = (size_t)nc * plane;
            abc[o] = cs_ * dl + l * dcs;
            abc[stride + o] = -l * cs_ / d2;
            abc[2 * stride + o] = 2.0f * l / d2;
        }
    }
    const float bs = block_sum_256(acc, sh);
    const int nblk = gridDim.x * gridDim.y * gridDim.z;
    const int bid = (blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x;
    if (threadIdx.x == 0) {
        partials[bid] = bs;
        __threadfence();
        last = atomicAdd(ticket, 1u) == (uint32_t)nblk - 1;
    }
    __syncthreads();
    if (last) {
        __threadfence();
        const float tot = block_sum_partials(partials, nblk, sh);
        if (threadIdx.x == 0) {
            *out = tot / ((float)nc * (float)plane);
            *ticket = 0u;
        }
    }
}

template <int WIN>
__global__ __launch_bounds__(256) void k_ssim_bwd(const float* __restrict__ x,
                                                 const float* __restrict__ y, int h, int w,
                                                 int oh, int ow,
                                                 const float* __restrict__ win1d,
                                                 const float* __restrict__ abc,
                                                 const float* __restrict__ grad_out, float inv_cnt,
                                                 int nc, float* __restrict__ gx) {
    constexpr int IT = SsimTile<WIN>::IT, ITP = SsimTile<WIN>::ITP;
    __shared__ float as[3][IT][ITP];
    __shared__ float hs[3][IT][kSsimOT + 1];
    __shared__ float gw[WIN];
    const int c = blockIdx.z;
    const int px0 = blockIdx.x * kSsimOT, py0 = blockIdx.y * kSsimOT;
    const size_t plane = (size_t)oh * ow;
    const size_t stride = (size_t)nc * plane;
    const float* A = abc + (size_t)c * plane;
    if (threadIdx.x < WIN) gw[threadIdx.x] = win1d[threadIdx.x];
    // Tile of A, B, C for map pixels o in [p - (WIN-1), p].
    for (int idx = threadIdx.x; idx < IT * IT; idx += 256) {
        const int r = idx / IT, q = idx - r * IT;
        const int oy = py0 - (WIN - 1) + r, ox = px0 - (WIN - 1) + q;
        const bool in = oy >= 0 && oy < oh && ox >= 0 && ox < ow;
        const size_t o = in ? (size_t)oy * ow + ox : 0;
        as[0][r][q] = in ? A[o] : 0.0f;
        as[1][r][q] = in ? A[stride + o] : 0.0f;
        as[2][r][q] = in ? A[2 * stride + o] : 0.0f;
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < IT * kSsimOT; idx += 256) {
        const int r = idx / kSsimOT, q = idx - r * kSsimOT;
        float s0 = 0.f, s1 = 0.f, s2 = 0.f;
#pragma unroll
        for (int k = 0; k < WIN; ++k) {
            const float g = gw[k];
            s0 = __builtin_fmaf(g, as[0][r][q + WIN - 1 - k], s0);
            s1 = __builtin_fmaf(g, as[1][r][q + WIN - 1 - k], s1);
            s2 = __builtin_fmaf(g, as[2][r][q + WIN - 1 - k], s2);
        }
        hs[0][r][q] = s0; hs[1][r][q] = s1; hs[2][r][q] = s2;
    }
    __syncthreads();
    const float scale = (*grad_out) * inv_cnt;
    const float* xc = x + (size_t)c * h * w;
    const float* yc = y + (size_t)c * h * w;
    float* gc = gx + (size_t)c * h * w;
    for (int idx = threadIdx.x; idx < kSsimOT * kSsimOT; idx += 256) {
        const int r = idx / kSsimOT, q = idx - r * kSsimOT;
        const int py = py0 + r, px = px0 + q;
        if (py >= h || px >= w) continue;
        float ga = 0.f, gb = 0.f, gcc = 0.f;
#pragma unroll
        for (int k = 0; k < WIN; ++k) {
            const float g = gw[k];
            ga = __builtin_fmaf(g, hs[0][r + WIN - 1 - k][q], ga);
            gb = __builtin_fmaf(g, hs[1][r + WIN - 1 - k][q], gb);
            gcc = __builtin_fmaf(g, hs[2][r + WIN - 1 - k][q], gcc);
        }
        const size_t pi = (size_t)py * w + px;
        const float xv = xc[pi], yv = yc[pi];
        gc[pi] = scale * (ga + 2.0f * xv * gb + yv * gcc);
    }
}

}  // namespace cs

using namespace cs;

static int metric_status() { return hipGetLastError() == hipSuccess ? CS_OK : CS_ERR_HIP; }

extern "C" size_t cs_mse_partials_elems(int64_t n) {
    return (size_t)((n + kMseChunk - 1) / kMseChunk > 0 ? (n + kMseChunk - 1) / kMseChunk : 1);
}

extern "C" int cs_mse_forward(const float* x, const float* y, int64_t n, float* partials,
                              uint32_t* ticket, float* loss, hipStream_t stream) {
    if (n <= 0) return CS_ERR_ARGS;
    const int64_t nb = (n + kMseChunk - 1) / kMseChunk;
    if (nb > 0x7fffffff) return CS_ERR_ARGS;
    hipLaunchKernelGGL(k_mse_fwd, dim3((unsigned)nb), dim3(kMseThreads), 0, stream, x, y, n,
                       partials, ticket, loss);
    return metric_status();
}

extern "C" int cs_mse_backward(const float* x, const float* y, int64_t n, const float* grad_loss,
                               float* grad_x, float* grad_y, hipStream_t stream) {
    if (n <= 0) return CS_ERR_ARGS;
    const int64_t threads = (n + 3) / 4;
    const int64_t nb = (threads + 255) / 256;
    hipLaunchKernelGGL(k_mse_bwd, dim3((unsigned)nb), dim3(256), 0, stream, x, y, n, grad_loss,
                       (float)(2.0 / (double)n), grad_x, grad_y);
    return metric_status();
}

extern "C" size_t cs_ssim_partials_elems(int32_t nc, int32_t h, int32_t w) {
    const int64_t oh = h, ow = w;  // upper bound for any window
    return (size_t)(((ow + kSsimOT - 1) / kSsimOT) * ((oh + kSsimOT - 1) / kSsimOT) * nc);
}

#define CS_SSIM_DISPATCH(WIN_, CALL) \
    case WIN_: CALL(WIN_); break;

extern "C" int cs_ssim(const float* x, const float* y, int32_t nc, int32_t h, int32_t w,
                       const float* win1d, int32_t win, float c1, float c2, float* partials,
                       uint32_t* ticket, float* out, float* abc, hipStream_t stream) {
    if (nc <= 0 || win <= 0 || (win & 1) == 0 || win > 15 || h < win || w < win)
        return CS_ERR_ARGS;
    const int oh = h - win + 1, ow = w - win + 1;
    const dim3 grid((ow + kSsimOT - 1) / kSsimOT, (oh + kSsimOT - 1) / kSsimOT, nc);
#define CS_SSIM_FWD(W_)                                                                       \
    hipLaunchKernelGGL(k_ssim_fwd<W_>, grid, dim3(256), 0, stream, x, y, h, w, oh, ow, win1d, \
                       c1, c2, partials, ticket, out, abc, nc)
    switch (win) {
        CS_SSIM_DISPATCH(1, CS_SSIM_FWD)
        CS_SSIM_DISPATCH(3, CS_SSIM_FWD)
        CS_SSIM_DISPATCH(5, CS_SSIM_FWD)
        CS_SSIM_DISPATCH(7, CS_SSIM_FWD)
        CS_SSIM_DISPATCH(9, CS_SSIM_FWD)
        CS_SSIM_DISPATCH(11, CS_SSIM_FWD)
        CS_SSIM_DISPATCH(13, CS_SSIM_FWD)
        CS_SSIM_DISPATCH(15, CS_SSIM_FWD)
        default: return CS_ERR_ARGS;
    }
#undef CS_SSIM_FWD
    return metric_status();
}

extern "C" int cs_ssim_backward(const float* x, const float* y, int32_t nc, int32_t h, int32_t w,
                                const float* win1d, int32_t win, const float* abc,
                                const float* grad_out, float* grad_x, hipStream_t stream) {
    if (nc <= 0 || win <= 0 || (win & 1) == 0 || win > 15 || h < win || w < win)
        return CS_ERR_ARGS;
    const int oh = h - win + 1, ow = w - win + 1;
    const float inv_cnt = 1.0f / ((float)nc * (float)oh * (float)ow);
    const dim3 grid((w + kSsimOT - 1) / kSsimOT, (h + kSsimOT - 1) / kSsimOT, nc);
#define CS_SSIM_BWD(W_)                                                                     \
    hipLaunchKernelGGL(k_ssim_bwd<W_>, grid, dim3(256), 0, stream, x, y, h, w, oh, ow, win1d, \
                       abc, grad_out, inv_cnt, nc, grad_x)
    switch (win) {
        CS_SSIM_DISPATCH(1, CS_SSIM_BWD)
        CS_SSIM_DISPATCH(3, CS_SSIM_BWD)
        CS_SSIM_DISPATCH(5, CS_SSIM_BWD)
        CS_SSIM_DISPATCH(7, CS_SSIM_BWD)
        CS_SSIM_DISPATCH(9, CS_SSIM_BWD)
        CS_SSIM_DISPATCH(11, CS_SSIM_BWD)
        CS_SSIM_DISPATCH(13, CS_SSIM_BWD)
        CS_SSIM_DISPATCH(15, CS_SSIM_BWD)
        default: return CS_ERR_ARGS;
    }
#undef CS_SSIM_BWD
    return metric_status();
}
