// MSE and SSIM losses (forward and backward) for MI355X.
//
// Reductions are two launches: workgroups write partial sums, one workgroup
// adds them in index order (deterministic).  A last-workgroup ticket would
// save the launch but puts every workgroup's atomic on one device-scope
// address, which serializes outside the XCD L2s.
//
// SSIM: valid-window SSIM of ops/metric.py:205-341 with the 2D Gaussian window
// applied separably (the reference window is the outer product of one
// normalized 1D Gaussian, metric.py:47-61).  A 32x32 output tile stages its
// (32+win-1)^2 inputs in LDS; the horizontal pass gives each thread an 8-wide
// strip (the 8+win-1 inputs are read once), the vertical pass a 4-tall strip
// of the five moments (taken about a per-tile constant, see k_ssim_fwd).  The backward (absent from the reference) uses the
// per-pixel partials A = dS/dmu_x, B = dS/dE[x^2], C = dS/dE[xy] and one
// transposed separable correlation, blocked the same way.
#include "cs_common.h"
#include "../../include/cubicsplat_hip.h"

namespace cs {

constexpr int kMseThreads = 256;
constexpr int kMseItems = 16;  // float elements per thread
constexpr int kMseChunk = kMseThreads * kMseItems;
constexpr int kFinalThreads = 1024;

__device__ __forceinline__ float block_sum(float v, float* sh) {
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    if (lane == 0) sh[w] = v;
    __syncthreads();
    float r = 0.0f;
    if (threadIdx.x == 0) {
        const int nw = (blockDim.x + 63) >> 6;
        for (int k = 0; k < nw; ++k) r += sh[k];
    }
    __syncthreads();
    return r;
}

// out = scale * sum(partials[0..n)), one workgroup, fixed order.
__global__ __launch_bounds__(kFinalThreads) void k_sum_partials(const float* __restrict__ partials,
                                                               int n, float scale,
                                                               float* __restrict__ out) {
    __shared__ float sh[kFinalThreads / kWave];
    float acc = 0.0f;
    for (int i = threadIdx.x; i < n; i += kFinalThreads) acc += partials[i];
    const float tot = block_sum(acc, sh);
    if (threadIdx.x == 0) *out = tot * scale;
}

__global__ __launch_bounds__(kMseThreads) void k_mse_partial(const float* __restrict__ x,
                                                            const float* __restrict__ y, int64_t n,
                                                            float* __restrict__ partials) {
    __shared__ float sh[kMseThreads / kWave];
    const int64_t base = (int64_t)blockIdx.x * kMseChunk;
    float acc = 0.0f;
    const bool aligned = ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) & 15) == 0;
    if (aligned && base + kMseChunk <= n) {
        const float4* x4 = reinterpret_cast<const float4*>(x + base);
        const float4* y4 = reinterpret_cast<const float4*>(y + base);
        float4 a[kMseItems / 4], b[kMseItems / 4];
#pragma unroll
        for (int k = 0; k < kMseItems / 4; ++k) {
            a[k] = x4[k * kMseThreads + threadIdx.x];
            b[k] = y4[k * kMseThreads + threadIdx.x];
        }
#pragma unroll
        for (int k = 0; k < kMseItems / 4; ++k) {
            const float d0 = a[k].x - b[k].x, d1 = a[k].y - b[k].y;
            const float d2 = a[k].z - b[k].z, d3 = a[k].w - b[k].w;
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
    const float bs = block_sum(acc, sh);
    if (threadIdx.x == 0) partials[blockIdx.x] = bs;
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

constexpr int kSsimOT = 32;   // output tile edge
constexpr int kHStrip = 8;    // horizontal-pass outputs per thread
constexpr int kVStrip = 4;    // vertical-pass outputs per thread

template <int WIN>
struct SsimTile {
    static constexpr int IT = kSsimOT + WIN - 1;  // staged input tile edge
    static constexpr int ITP = IT + 1;             // padded LDS row
    static constexpr int HP = kSsimOT + 1;         // padded horizontal-result row
};

// Loads a (IT x IT) tile starting at (y0, x0) of `src` (h x w) into LDS,
// zero outside the image.  256 threads as 4 rows x 64 columns.
template <int IT, int ITP>
__device__ __forceinline__ void load_tile(const float* __restrict__ src, int h, int w, int y0,
                                          int x0, float (*dst)[ITP]) {
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    for (int r = ty; r < IT; r += 4) {
        const int gy = y0 + r;
        const bool rin = gy >= 0 && gy < h;
        for (int c = tx; c < IT; c += 64) {
            const int gx = x0 + c;
            dst[r][c] = (rin && gx >= 0 && gx < w) ? src[(size_t)gy * w + gx] : 0.0f;
        }
    }
}

template <int WIN>
__global__ __launch_bounds__(256) void k_ssim_fwd(const float* __restrict__ x,
                                                 const float* __restrict__ y, int h, int w,
                                                 int oh, int ow,
                                                 const float* __restrict__ win1d, float c1,
                                                 float c2, float* __restrict__ partials,
                                                 float* __restrict__ abc, int nc) {
    constexpr int IT = SsimTile<WIN>::IT, ITP = SsimTile<WIN>::ITP, HP = SsimTile<WIN>::HP;
    __shared__ float xs[IT][ITP];
    __shared__ float ys[IT][ITP];
    __shared__ float hm[5][IT][HP];
    __shared__ float gw[WIN];
    __shared__ float sh[4];
    const int c = blockIdx.z;
    const int ox0 = blockIdx.x * kSsimOT, oy0 = blockIdx.y * kSsimOT;
    if (threadIdx.x < WIN) gw[threadIdx.x] = win1d[threadIdx.x];
    load_tile<IT, ITP>(x + (size_t)c * h * w, h, w, oy0, ox0, xs);
    load_tile<IT, ITP>(y + (size_t)c * h * w, h, w, oy0, ox0, ys);
    __syncthreads();
    // Moments are taken of x - kx and y - ky, with kx, ky one staged value per
    // workgroup: sigma^2 = E[(x-k)^2] - (mu-k)^2 holds for any constant k and
    // avoids the cancellation of E[x^2] - mu^2 in flat regions (where it
    // would leave fp32 noise of order 1e-7 against c2 = 9e-4).
    const float kx = xs[IT / 2][IT / 2], ky = ys[IT / 2][IT / 2];
    // Horizontal: thread -> (row, 8-wide strip); IT rows x 4 strips.
    for (int item = threadIdx.x; item < IT * (kSsimOT / kHStrip); item += 256) {
        const int r = item >> 2, q0 = (item & 3) * kHStrip;
        float a[kHStrip + WIN - 1], b[kHStrip + WIN - 1];
#pragma unroll
        for (int k = 0; k < kHStrip + WIN - 1; ++k) {
            a[k] = xs[r][q0 + k] - kx;
            b[k] = ys[r][q0 + k] - ky;
        }
#pragma unroll
        for (int o = 0; o < kHStrip; ++o) {
            float m0 = 0.f, m1 = 0.f, m2 = 0.f, m3 = 0.f, m4 = 0.f;
#pragma unroll
            for (int k = 0; k < WIN; ++k) {
                const float g = gw[k];
                const float av = a[o + k], bv = b[o + k];
                m0 = __builtin_fmaf(g, av, m0);
                m1 = __builtin_fmaf(g, bv, m1);
                m2 = __builtin_fmaf(g, av * av, m2);
                m3 = __builtin_fmaf(g, bv * bv, m3);
                m4 = __builtin_fmaf(g, av * bv, m4);
            }
            hm[0][r][q0 + o] = m0;
            hm[1][r][q0 + o] = m1;
            hm[2][r][q0 + o] = m2;
            hm[3][r][q0 + o] = m3;
            hm[4][r][q0 + o] = m4;
        }
    }
    __syncthreads();
    // Vertical: thread -> (column, 4-tall strip); 32 columns x 8 strips.
    const int q = threadIdx.x & 31, r0 = (threadIdx.x >> 5) * kVStrip;
    float mom[5][kVStrip];
#pragma unroll
    for (int m = 0; m < 5; ++m)
#pragma unroll
        for (int o = 0; o < kVStrip; ++o) mom[m][o] = 0.0f;
#pragma unroll
    for (int k = 0; k < kVStrip + WIN - 1; ++k) {
        float v[5];
#pragma unroll
        for (int m = 0; m < 5; ++m) v[m] = hm[m][r0 + k][q];
#pragma unroll
        for (int o = 0; o < kVStrip; ++o) {
            const int t = k - o;
            if (t >= 0 && t < WIN) {
                const float g = gw[t];
#pragma unroll
                for (int m = 0; m < 5; ++m) mom[m][o] = __builtin_fmaf(g, v[m], mom[m][o]);
            }
        }
    }
    float acc = 0.0f;
    const size_t plane = (size_t)oh * ow;
    const size_t stride = (size_t)nc * plane;
    const int ox = ox0 + q;
#pragma unroll
    for (int o = 0; o < kVStrip; ++o) {
        const int oy = oy0 + r0 + o;
        if (oy >= oh || ox >= ow) continue;
        const float m1 = mom[0][o], m2 = mom[1][o];  // shifted means
        const float s1 = mom[2][o] - m1 * m1, s2 = mom[3][o] - m2 * m2;
        const float s12 = mom[4][o] - m1 * m2;
        const float mu1 = m1 + kx, mu2 = m2 + ky;
        const float mu1_sq = mu1 * mu1, mu2_sq = mu2 * mu2, mu12 = mu1 * mu2;
        const float n1 = 2.0f * mu12 + c1, d1 = mu1_sq + mu2_sq + c1;
        const float n2 = 2.0f * s12 + c2, d2 = s1 + s2 + c2;
        const float l = n1 / d1, cs_ = n2 / d2;
        acc += l * cs_;
        if (abc) {
            const float dl = 2.0f * (mu2 - l * mu1) / d1;
            const float dcs = 2.0f * (mu1 * cs_ - mu2) / d2;
            const size_t oi = (size_t)c * plane + (size_t)oy * ow + ox;
            abc[oi] = cs_ * dl + l * dcs;
            abc[stride + oi] = -l * cs_ / d2;
            abc[2 * stride + oi] = 2.0f * l / d2;
        }
    }
    const float bs = block_sum(acc, sh);
    if (threadIdx.x == 0)
        partials[(blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x] = bs;
}

template <int WIN>
__global__ __launch_bounds__(256) void k_ssim_bwd(const float* __restrict__ x,
                                                 const float* __restrict__ y, int h, int w,
                                                 int oh, int ow,
                                                 const float* __restrict__ win1d,
                                                 const float* __restrict__ abc,
                                                 const float* __restrict__ grad_out, float inv_cnt,
                                                 int nc, float* __restrict__ gx) {
    constexpr int IT = SsimTile<WIN>::IT, ITP = SsimTile<WIN>::ITP, HP = SsimTile<WIN>::HP;
    __shared__ float as[3][IT][ITP];
    __shared__ float hs[3][IT][HP];
    __shared__ float gw[WIN];
    const int c = blockIdx.z;
    const int px0 = blockIdx.x * kSsimOT, py0 = blockIdx.y * kSsimOT;
    const size_t plane = (size_t)oh * ow;
    const size_t stride = (size_t)nc * plane;
    if (threadIdx.x < WIN) gw[threadIdx.x] = win1d[threadIdx.x];
    // Map pixels o in [p - (WIN-1), p] of A, B, C.
    for (int m = 0; m < 3; ++m)
        load_tile<IT, ITP>(abc + m * stride + (size_t)c * plane, oh, ow, py0 - (WIN - 1),
                           px0 - (WIN - 1), as[m]);
    __syncthreads();
    // Horizontal full correlation: hs[r][q] = sum_k g[k] as[r][q + WIN-1-k].
    for (int item = threadIdx.x; item < IT * (kSsimOT / kHStrip); item += 256) {
        const int r = item >> 2, q0 = (item & 3) * kHStrip;
#pragma unroll
        for (int m = 0; m < 3; ++m) {
            float a[kHStrip + WIN - 1];
#pragma unroll
            for (int k = 0; k < kHStrip + WIN - 1; ++k) a[k] = as[m][r][q0 + k];
#pragma unroll
            for (int o = 0; o < kHStrip; ++o) {
                float s = 0.0f;
#pragma unroll
                for (int k = 0; k < WIN; ++k) s = __builtin_fmaf(gw[k], a[o + WIN - 1 - k], s);
                hs[m][r][q0 + o] = s;
            }
        }
    }
    __syncthreads();
    const int q = threadIdx.x & 31, r0 = (threadIdx.x >> 5) * kVStrip;
    float gsum[3][kVStrip];
#pragma unroll
    for (int m = 0; m < 3; ++m)
#pragma unroll
        for (int o = 0; o < kVStrip; ++o) gsum[m][o] = 0.0f;
#pragma unroll
    for (int k = 0; k < kVStrip + WIN - 1; ++k) {
        float v[3];
#pragma unroll
        for (int m = 0; m < 3; ++m) v[m] = hs[m][r0 + k][q];
#pragma unroll
        for (int o = 0; o < kVStrip; ++o) {
            const int t = o + WIN - 1 - k;
            if (t >= 0 && t < WIN) {
                const float g = gw[t];
#pragma unroll
                for (int m = 0; m < 3; ++m) gsum[m][o] = __builtin_fmaf(g, v[m], gsum[m][o]);
            }
        }
    }
    const float scale = (*grad_out) * inv_cnt;
    const float* xc = x + (size_t)c * h * w;
    const float* yc = y + (size_t)c * h * w;
    float* gc = gx + (size_t)c * h * w;
    const int px = px0 + q;
#pragma unroll
    for (int o = 0; o < kVStrip; ++o) {
        const int py = py0 + r0 + o;
        if (py >= h || px >= w) continue;
        const size_t pi = (size_t)py * w + px;
        gc[pi] = scale * (gsum[0][o] + 2.0f * xc[pi] * gsum[1][o] + yc[pi] * gsum[2][o]);
    }
}

}  // namespace cs

using namespace cs;

static int metric_status() { return hipGetLastError() == hipSuccess ? CS_OK : CS_ERR_HIP; }

extern "C" size_t cs_mse_partials_elems(int64_t n) {
    const int64_t nb = (n + kMseChunk - 1) / kMseChunk;
    return (size_t)(nb > 0 ? nb : 1);
}

extern "C" int cs_mse_forward(const float* x, const float* y, int64_t n, float* partials,
                              float* loss, hipStream_t stream) {
    if (n <= 0) return CS_ERR_ARGS;
    const int64_t nb = (n + kMseChunk - 1) / kMseChunk;
    if (nb > 0x7fffffff) return CS_ERR_ARGS;
    hipLaunchKernelGGL(k_mse_partial, dim3((unsigned)nb), dim3(kMseThreads), 0, stream, x, y, n,
                       partials);
    hipLaunchKernelGGL(k_sum_partials, dim3(1), dim3(kFinalThreads), 0, stream, partials, (int)nb,
                       1.0f / (float)n, loss);
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
                       float* out, float* abc, hipStream_t stream) {
    if (nc <= 0 || win <= 0 || (win & 1) == 0 || win > 15 || h < win || w < win)
        return CS_ERR_ARGS;
    const int oh = h - win + 1, ow = w - win + 1;
    const dim3 grid((ow + kSsimOT - 1) / kSsimOT, (oh + kSsimOT - 1) / kSsimOT, nc);
#define CS_SSIM_FWD(W_)                                                                       \
    hipLaunchKernelGGL(k_ssim_fwd<W_>, grid, dim3(256), 0, stream, x, y, h, w, oh, ow, win1d, \
                       c1, c2, partials, abc, nc)
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
    const int nblk = (int)(grid.x * grid.y * grid.z);
    hipLaunchKernelGGL(k_sum_partials, dim3(1), dim3(kFinalThreads), 0, stream, partials, nblk,
                       1.0f / ((float)nc * (float)oh * (float)ow), out);
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
