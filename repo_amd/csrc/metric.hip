// MSE and SSIM losses (forward and backward) for MI355X.
//
// Reductions are two launches: workgroups write partial sums, one workgroup
// adds them in index order (deterministic).  A last-workgroup ticket would
// save the launch but puts every workgroup's atomic on one device-scope
// address, which serializes outside the XCD L2s.
//
// SSIM: valid-window SSIM of ops/metric.py:205-341 with the 2D Gaussian window
// applied separably (the reference window is the outer product of one
// normalized 1D Gaussian, metric.py:47-61): a horizontal pass over input rows
// into LDS, then a vertical pass, blocked in register strips (see k_ssim_fwd).
// Moments are taken about a per-tile constant.  The backward (absent from the
// reference) uses the per-pixel partials A = dS/dmu_x, B = dS/dE[x^2],
// C = dS/dE[xy] and one transposed separable correlation, blocked the same
// way.
#include <mutex>

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

// grad = scale (lhs - rhs), the expression of mse_backward_diff_kernel
// (ops/metric.py:166-202), four elements per thread.
__global__ __launch_bounds__(256) void k_scaled_diff(const float* __restrict__ lhs,
                                                    const float* __restrict__ rhs, int64_t n,
                                                    float scale, float* __restrict__ grad) {
    const int64_t i4 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
    if (i4 + 4 <= n &&
        ((reinterpret_cast<uintptr_t>(lhs) | reinterpret_cast<uintptr_t>(rhs) |
          reinterpret_cast<uintptr_t>(grad)) & 15) == 0) {
        const float4 a = *reinterpret_cast<const float4*>(lhs + i4);
        const float4 b = *reinterpret_cast<const float4*>(rhs + i4);
        *reinterpret_cast<float4*>(grad + i4) = make_float4(
            scale * (a.x - b.x), scale * (a.y - b.y), scale * (a.z - b.z), scale * (a.w - b.w));
    } else {
        for (int64_t i = i4; i < i4 + 4 && i < n; ++i) grad[i] = scale * (lhs[i] - rhs[i]);
    }
}

// Partial sums of x over chunks of kMseChunk elements (one per workgroup).
__global__ __launch_bounds__(kMseThreads) void k_sum_partial(const float* __restrict__ x,
                                                            int64_t n,
                                                            float* __restrict__ partials) {
    __shared__ float sh[kMseThreads / kWave];
    const int64_t base = (int64_t)blockIdx.x * kMseChunk;
    float acc = 0.0f;
    if ((reinterpret_cast<uintptr_t>(x) & 15) == 0 && base + kMseChunk <= n) {
        const float4* x4 = reinterpret_cast<const float4*>(x + base);
        float4 a[kMseItems / 4];
#pragma unroll
        for (int k = 0; k < kMseItems / 4; ++k) a[k] = x4[k * kMseThreads + threadIdx.x];
#pragma unroll
        for (int k = 0; k < kMseItems / 4; ++k) acc += (a[k].x + a[k].y) + (a[k].z + a[k].w);
    } else {
        for (int k = 0; k < kMseItems; ++k) {
            const int64_t i = base + (int64_t)k * kMseThreads + threadIdx.x;
            if (i < n) acc += x[i];
        }
    }
    const float bs = block_sum(acc, sh);
    if (threadIdx.x == 0) partials[blockIdx.x] = bs;
}

// ------------------------------------------------------------------ SSIM

// Output tile: 32 columns x 48 rows per 256-thread workgroup.  The horizontal
// pass gives each thread a row and an 8-wide column strip (IT = 48 + win - 1
// rows x 4 strips, 232 items for win 11) and reads its inputs straight from
// global memory (through the vector cache, float4 where the strip is inside
// the image); only the horizontal results live in LDS.  The vertical pass
// gives each thread a column and a 6-tall row strip (32 x 8 items).
constexpr int kSsimTiledMaxWin = 15;  // widest window of the tiled kernels
constexpr int64_t kSsimMaxMapPlane = 1ll << 30;  // floats of one map plane (oh x padded ow)
constexpr int kSsimTW = 32;   // output tile width
constexpr int kSsimTH = 48;   // output tile height
constexpr int kHStrip = 8;    // horizontal-pass outputs per thread
constexpr int kVStrip = 6;    // vertical-pass outputs per thread
static_assert(kSsimTW * (kSsimTH / kVStrip) == 256, "vertical pass covers the tile");

template <int WIN>
struct SsimTile {
    static constexpr int IT = kSsimTH + WIN - 1;   // input rows per tile
    static constexpr int HP = kSsimTW + 1;         // padded horizontal-result row
    static constexpr int NIN = kHStrip + WIN - 1;  // inputs per horizontal strip
    // The backward's strips start WIN-1 map columns before a multiple of 8.
    static constexpr int BOFF = (4 - (WIN - 1) % 4) % 4;
};

// clamp(v, lo, hi) as torch.clamp computes it for ordered values (lo <= hi,
// v not NaN), when CLAMP: the median of the three, one instruction.
template <bool CLAMP>
__device__ __forceinline__ float clamp_if(float v, float lo, float hi) {
    return CLAMP ? __builtin_amdgcn_fmed3f(v, lo, hi) : v;
}

// Loads columns gx0 .. gx0 + N of M rows (rows[m], each of an image with w
// valid columns and inside it: zero outside the columns; with CLAMP0 the
// values of row 0 inside are clamped to [lo, hi], the zeros outside are not).
// The callers handle rows outside the image themselves (their results are
// zero rows), so that the values loaded here need no zero defaults.  When the
// rows are 16-byte aligned (vec_ok), gx0 - OFF is a multiple of 4 and the
// rounded-up strips lie inside the rows, it uses float4 loads starting OFF
// columns early, every row's loads issued before the first is used (one
// memory round trip for all of them).
template <int M, int N, int OFF, bool CLAMP0 = false>
__device__ __forceinline__ void load_strips(const float* const (&rows)[M], int w, int gx0,
                                            bool vec_ok, float (&dst)[M][N], float lo = 0.0f,
                                            float hi = 0.0f) {
    constexpr int NV4 = (N + OFF + 3) / 4;
    const int s0 = gx0 - OFF;
    if (vec_ok && s0 >= 0 && s0 + 4 * NV4 <= w) {
        float4 q[M][NV4];
#pragma unroll
        for (int m = 0; m < M; ++m)
#pragma unroll
            for (int v = 0; v < NV4; ++v)
                q[m][v] = *reinterpret_cast<const float4*>(rows[m] + s0 + 4 * v);
#pragma unroll
        for (int m = 0; m < M; ++m) {
            float t[4 * NV4];
#pragma unroll
            for (int v = 0; v < NV4; ++v) {
                t[4 * v] = q[m][v].x;
                t[4 * v + 1] = q[m][v].y;
                t[4 * v + 2] = q[m][v].z;
                t[4 * v + 3] = q[m][v].w;
            }
#pragma unroll
            for (int k = 0; k < N; ++k)
                dst[m][k] = m == 0 ? clamp_if<CLAMP0>(t[OFF + k], lo, hi) : t[OFF + k];
        }
    } else {
#pragma unroll
        for (int m = 0; m < M; ++m)
#pragma unroll
            for (int k = 0; k < N; ++k) {
                const int gx = gx0 + k;
                const float v = (gx >= 0 && gx < w) ? rows[m][gx] : 0.0f;
                dst[m][k] = (m == 0 && gx >= 0 && gx < w) ? clamp_if<CLAMP0>(v, lo, hi) : v;
            }
    }
}

// Tile (channel, row, column) of workgroup b over nt = ntx * nty * nc tiles,
// XCD-aware.  With an HWC image the channel is the fastest index, so the three
// channels of one spatial tile run back to back on one XCD and share the L2
// lines of the interleaved image and gradient.
template <bool HWC>
__device__ __forceinline__ void ssim_tile(int b, int ntx, int nty, int nc, int& c, int& ty,
                                          int& tx) {
    const int tile = xcd_tile(b, ntx * nty * nc);
    int sp;
    if (HWC) {
        c = tile % nc;
        sp = tile / nc;
    } else {
        c = tile / (ntx * nty);
        sp = tile - c * ntx * nty;
    }
    ty = sp / ntx;
    tx = sp - ty * ntx;
}

// Row stride of the per-pixel maps A, B, C (rows padded to 16 bytes).
__host__ __device__ __forceinline__ int abc_ld(int ow) { return (ow + 3) & ~3; }

// SSIM at one map pixel from its four filtered moments about (kx, ky) (means
// m1, m2 of x - kx and y - ky, E of the squared sum and of the product), and,
// when `grad`, the partials A = dS/dmu_x, B = dS/dE[x^2], C = dS/dE[xy].
struct SsimPixel {
    float s, a, b, c;
};

__device__ __forceinline__ SsimPixel ssim_pixel(float m1, float m2, float mss, float mxy, float kx,
                                                float ky, float c1, float c2, bool grad) {
    // sigma_x^2 + sigma_y^2 from the one filtered E[x^2 + y^2].
    const float s1s2 = mss - __builtin_fmaf(m2, m2, m1 * m1);
    const float s12 = __builtin_fmaf(-m1, m2, mxy);
    const float mu1 = m1 + kx, mu2 = m2 + ky;
    const float n1 = __builtin_fmaf(mu1 + mu1, mu2, c1);
    const float d1 = __builtin_fmaf(mu1, mu1, __builtin_fmaf(mu2, mu2, c1));
    const float n2 = __builtin_fmaf(2.0f, s12, c2), d2 = s1s2 + c2;
    // The hardware reciprocal (within 1 ulp): d1 >= c1 and d2 >= c2 up to
    // rounding, so both are positive normals; the loss and its gradient are
    // compared to float64 at 1e-5 / 1e-4, far above this rounding.
    const float r1 = __builtin_amdgcn_rcpf(d1), r2 = __builtin_amdgcn_rcpf(d2);
    const float l = n1 * r1, cs_ = n2 * r2;
    SsimPixel o;
    o.s = l * cs_;
    o.a = o.b = o.c = 0.0f;
    if (grad) {
        // dl/dmu1 = 2 (mu2 - l mu1) r1 and dcs/dmu1 = 2 (mu1 cs - mu2) r2, so
        // A = cs dl + l dcs = 2 (cs r1 (mu2 - l mu1) + l r2 (mu1 cs - mu2));
        // B = -l cs r2 and C = 2 l r2.
        const float t = __builtin_fmaf(-l, mu1, mu2), u = __builtin_fmaf(mu1, cs_, -mu2);
        const float p = cs_ * r1, q = l * r2;
        o.a = 2.0f * __builtin_fmaf(p, t, q * u);
        o.b = -(cs_ * q);
        o.c = q + q;
    }
    return o;
}

// mse_partials (optional): each workgroup also sums (x - y)^2 over its
// anchor inputs -- rows [oy0, oy0 + 48) and columns [ox0, ox0 + 32), extended
// to the image's last row / column in the last tile row / column -- so every
// input is counted once and no separate MSE pass is needed.
// CLAMP: x is read as clamp(x, lo, hi) (the caller's clamp glue, applied on
// load instead of in a pass of its own).
// GRAD: abc is given (the three maps are written).
template <int WIN, bool CLAMP, bool GRAD>
__global__ __launch_bounds__(256) void k_ssim_fwd(const float* __restrict__ x,
                                                 const float* __restrict__ y, int h, int w,
                                                 int oh, int ow,
                                                 const float* __restrict__ win1d, float c1,
                                                 float c2, float* __restrict__ partials,
                                                 float* __restrict__ abc, int nc,
                                                 float* __restrict__ mse_partials, float lo,
                                                 float hi) {
    using TT = SsimTile<WIN>;
    constexpr int IT = TT::IT, HP = TT::HP, NIN = TT::NIN;
    // Four filtered moments: x, y, x^2 + y^2 and xy (SSIM needs the two
    // variances only as their sum, so E[x^2] and E[y^2] are filtered as one).
    __shared__ float hm[4][IT][HP];
    __shared__ float sh[4];
    // 1D grid over (channel, tile row, tile column), XCD-aware.
    const int ntx = (ow + kSsimTW - 1) / kSsimTW, nty = (oh + kSsimTH - 1) / kSsimTH;
    int c, ty, tx;
    ssim_tile<false>(blockIdx.x, ntx, nty, nc, c, ty, tx);
    const int tile = (c * nty + ty) * ntx + tx;
    const int ox0 = tx * kSsimTW, oy0 = ty * kSsimTH;
    const float* xc = x + (size_t)c * h * w;
    const float* yc = y + (size_t)c * h * w;
    float g[WIN];
#pragma unroll
    for (int k = 0; k < WIN; ++k) g[k] = win1d[k];
    // Moments are taken of x - kx and y - ky, with kx, ky one input value per
    // workgroup: sigma^2 = E[(x-k)^2] - (mu-k)^2 holds for any constant k and
    // avoids the cancellation of E[x^2] - mu^2 in flat regions (where it
    // would leave fp32 noise of order 1e-7 against c2 = 9e-4).
    const size_t kpix = (size_t)min(oy0 + kSsimTH / 2, h - 1) * w + min(ox0 + kSsimTW / 2, w - 1);
    const float kx = clamp_if<CLAMP>(xc[kpix], lo, hi), ky = yc[kpix];
    const bool vec_ok = ((w & 3) == 0) &&
                        ((reinterpret_cast<uintptr_t>(xc) | reinterpret_cast<uintptr_t>(yc)) & 15) == 0;
    // MSE anchor: rows [0, mse_rows) of the tile's input rows; columns
    // [q0, q0 + 8) of each strip, the last strip of the last tile column up
    // to the end of its inputs (zeros past the image add nothing).
    const int mse_rows = ty == nty - 1 ? IT : kSsimTH;
    float mse = 0.0f;
    // Horizontal: thread -> (row, 8-wide strip).
    for (int item = threadIdx.x; item < IT * (kSsimTW / kHStrip); item += 256) {
        const int r = item >> 2, q0 = (item & 3) * kHStrip;
        if (oy0 + r >= h) {
            // Input rows past the image (the last tile row's windows): only
            // output rows past the valid map read them.
#pragma unroll
            for (int o = 0; o < kHStrip; ++o) {
                hm[0][r][q0 + o] = 0.0f;
                hm[1][r][q0 + o] = 0.0f;
                hm[2][r][q0 + o] = 0.0f;
                hm[3][r][q0 + o] = 0.0f;
            }
            continue;
        }
        float ab_in[2][NIN];
        {
            const size_t ro = (size_t)(oy0 + r) * w;
            const float* const rows[2] = {xc + ro, yc + ro};
            load_strips<2, NIN, 0, CLAMP>(rows, w, ox0 + q0, vec_ok, ab_in, lo, hi);
        }
        float (&a)[NIN] = ab_in[0];
        float (&b)[NIN] = ab_in[1];
        if (mse_partials && r < mse_rows) {
            // The strip's own 8 columns; the last strip of the last tile
            // column also takes the inputs past them (to the end of its
            // inputs), in the same order as one loop over all of them.
#pragma unroll
            for (int k = 0; k < kHStrip; ++k) {
                const float d = a[k] - b[k];
                mse = __builtin_fmaf(d, d, mse);
            }
            if (tx == ntx - 1 && q0 + kHStrip == kSsimTW) {
#pragma unroll
                for (int k = kHStrip; k < NIN; ++k) {
                    const float d = a[k] - b[k];
                    mse = __builtin_fmaf(d, d, mse);
                }
            }
        }
        float ss[NIN], ab[NIN];
#pragma unroll
        for (int k = 0; k < NIN; ++k) {
            a[k] -= kx;
            b[k] -= ky;
            ss[k] = __builtin_fmaf(b[k], b[k], a[k] * a[k]);
            ab[k] = a[k] * b[k];
        }
#pragma unroll
        for (int o = 0; o < kHStrip; ++o) {
            float m0 = 0.f, m1 = 0.f, m2 = 0.f, m3 = 0.f;
#pragma unroll
            for (int k = 0; k < WIN; ++k) {
                m0 = __builtin_fmaf(g[k], a[o + k], m0);
                m1 = __builtin_fmaf(g[k], b[o + k], m1);
                m2 = __builtin_fmaf(g[k], ss[o + k], m2);
                m3 = __builtin_fmaf(g[k], ab[o + k], m3);
            }
            hm[0][r][q0 + o] = m0;
            hm[1][r][q0 + o] = m1;
            hm[2][r][q0 + o] = m2;
            hm[3][r][q0 + o] = m3;
        }
    }
    __syncthreads();
    // Vertical: thread -> (column, 6-tall strip).
    const int q = threadIdx.x & (kSsimTW - 1), r0 = (threadIdx.x / kSsimTW) * kVStrip;
    float mom[4][kVStrip];
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int o = 0; o < kVStrip; ++o) mom[m][o] = 0.0f;
#pragma unroll
    for (int k = 0; k < kVStrip + WIN - 1; ++k) {
        float v[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) v[m] = hm[m][r0 + k][q];
#pragma unroll
        for (int o = 0; o < kVStrip; ++o) {
            const int t = k - o;
            if (t >= 0 && t < WIN) {
#pragma unroll
                for (int m = 0; m < 4; ++m) mom[m][o] = __builtin_fmaf(g[t], v[m], mom[m][o]);
            }
        }
    }
    float acc = 0.0f;
    const int ld = abc_ld(ow);
    const size_t plane = (size_t)oh * ld;
    const size_t stride = (size_t)nc * plane;
    // The maps of channel c from workgroup-uniform bases, at 32-bit byte
    // offsets within a plane (the launch checks that a plane's bytes fit).
    char* const map_a = reinterpret_cast<char*>(abc + (size_t)c * plane);
    char* const map_b = map_a + stride * sizeof(float);
    char* const map_c = map_b + stride * sizeof(float);
    const int ox = ox0 + q;
    const int oy_s = oy0 + r0;
    const uint32_t ob0 = ((uint32_t)oy_s * (uint32_t)ld + (uint32_t)ox) * 4u;
#pragma unroll
    for (int o = 0; o < kVStrip; ++o) {
        if (oy_s + o >= oh || ox >= ow) continue;
        const SsimPixel sp = ssim_pixel(mom[0][o], mom[1][o], mom[2][o], mom[3][o], kx, ky, c1,
                                        c2, GRAD);
        acc += sp.s;
        if (GRAD) {
            const uint32_t ob = ob0 + (uint32_t)(o * ld) * 4u;
            *reinterpret_cast<float*>(map_a + ob) = sp.a;
            *reinterpret_cast<float*>(map_b + ob) = sp.b;
            *reinterpret_cast<float*>(map_c + ob) = sp.c;
        }
    }
    const float bs = block_sum(acc, sh);
    if (threadIdx.x == 0) partials[tile] = bs;
    if (mse_partials) {
        const float ms = block_sum(mse, sh);
        if (threadIdx.x == 0) mse_partials[tile] = ms;
    }
}

// grad_x[p] = scale * sum over map pixels o of the window w(p - o) times
// (A[o] + 2 x[p] B[o] + y[p] C[o]): a full (transposed) correlation of the
// three maps, blocked like the forward (horizontal strips read the maps from
// global memory, vertical strips from LDS).
// XL, the layout of x: 0, nc planes read as they are; 1 (HWC), the [h, w, 3]
// image the forward read as clamp(x, lo, hi); 2, three [h, w] planes read as
// clamp(x, lo, hi).  With a clamp, gx is the gradient with respect to x
// itself, zero where x lies outside [lo, hi] (the clamp's gradient as torch
// defines it).  gx: planes, or, for XL 1 without gx_planar, [h, w, 3]
// (planes let each channel tile write whole lines).
template <int WIN, int XL>
__global__ __launch_bounds__(256) void k_ssim_bwd(const float* __restrict__ x,
                                                 const float* __restrict__ y, int h, int w,
                                                 int oh, int ow,
                                                 const float* __restrict__ win1d,
                                                 const float* __restrict__ abc,
                                                 const float* __restrict__ grad_out, int go_per_map,
                                                 float ssim_coef, float mse_coef, int nc, float lo,
                                                 float hi, int gx_planar, float* __restrict__ gx) {
    using TT = SsimTile<WIN>;
    constexpr int IT = TT::IT, HP = TT::HP, NIN = TT::NIN;
    __shared__ float hs[3][IT][HP];
    // 1D grid over (channel, tile row, tile column), XCD-aware.
    const int ntx = (w + kSsimTW - 1) / kSsimTW, nty = (h + kSsimTH - 1) / kSsimTH;
    int c, ty, tx;
    ssim_tile<XL == 1>(blockIdx.x, ntx, nty, nc, c, ty, tx);
    const int px0 = tx * kSsimTW, py0 = ty * kSsimTH;
    const size_t ld = abc_ld(ow);
    const size_t plane = (size_t)oh * ld;
    const size_t stride = (size_t)nc * plane;
    float g[WIN];
#pragma unroll
    for (int k = 0; k < WIN; ++k) g[k] = win1d[k];
    const bool vec_ok = (reinterpret_cast<uintptr_t>(abc) & 15) == 0;
    // Horizontal full correlation over map columns px0 - (WIN-1) + [0, 32 + WIN - 1):
    // hs[r][q] = sum_k g[k] M[r][q + WIN-1-k], map rows py0 - (WIN-1) + r.
    for (int item = threadIdx.x; item < IT * (kSsimTW / kHStrip); item += 256) {
        const int r = item >> 2, q0 = (item & 3) * kHStrip;
        const int my = py0 - (WIN - 1) + r, mx0 = px0 - (WIN - 1) + q0;
        if (my < 0 || my >= oh) {
            // Map rows outside the map: the correlation's zero padding.
#pragma unroll
            for (int m = 0; m < 3; ++m)
#pragma unroll
                for (int o = 0; o < kHStrip; ++o) hs[m][r][q0 + o] = 0.0f;
            continue;
        }
        // One map at a time: loading the three strips together would take
        // 60 more registers and cost this HBM-bound kernel a wave per SIMD
        // (measured slower).
        const float* const m0 = abc + (size_t)c * plane + (size_t)my * ld;
#pragma unroll
        for (int m = 0; m < 3; ++m) {
            float a1[1][NIN];
            const float* const rows[1] = {m0 + m * stride};
            load_strips<1, NIN, TT::BOFF>(rows, ow, mx0, vec_ok, a1);
#pragma unroll
            for (int o = 0; o < kHStrip; ++o) {
                float s = 0.0f;
#pragma unroll
                for (int k = 0; k < WIN; ++k) s = __builtin_fmaf(g[k], a1[0][o + WIN - 1 - k], s);
                hs[m][r][q0 + o] = s;
            }
        }
    }
    __syncthreads();
    const int q = threadIdx.x & (kSsimTW - 1), r0 = (threadIdx.x / kSsimTW) * kVStrip;
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
#pragma unroll
                for (int m = 0; m < 3; ++m) gsum[m][o] = __builtin_fmaf(g[t], v[m], gsum[m][o]);
            }
        }
    }
    // grad = g * ssim_coef * (SSIM-mean term) [+ g * mse_coef * (x - y) when
    // the MSE gradient is fused in]; g is the map's own incoming gradient
    // when go_per_map.
    const float go = grad_out[go_per_map ? c : 0];
    const float scale = go * ssim_coef, mscale = go * mse_coef;
    const float* yc = y + (size_t)c * h * w;
    const int px = px0 + q;
#pragma unroll
    for (int o = 0; o < kVStrip; ++o) {
        const int py = py0 + r0 + o;
        if (py >= h || px >= w) continue;
        const size_t pi = (size_t)py * w + px;
        const float xr = XL == 1 ? x[3 * pi + c] : x[(size_t)c * h * w + pi];
        const float xv = clamp_if<XL != 0>(xr, lo, hi), yv = yc[pi];
        float gv = scale * (gsum[0][o] + 2.0f * xv * gsum[1][o] + yv * gsum[2][o]);
        if (mse_coef != 0.0f) gv = __builtin_fmaf(mscale, xv - yv, gv);
        if (XL != 0) gv = ((xr >= lo) & (xr <= hi)) ? gv : 0.0f;
        gx[(XL == 1 && !gx_planar) ? 3 * pi + c : (size_t)c * h * w + pi] = gv;
    }
}

// Windows wider than the tiled kernels take (any odd size up to the image):
// two passes through a scratch buffer, one thread per output of each pass.
// Moments are taken about one constant per map (its centre pixel), as the
// tiled kernel takes them about one per tile.
constexpr int kSsimGenThreads = 256;

__device__ __forceinline__ void map_shift(const float* __restrict__ xc,
                                          const float* __restrict__ yc, int h, int w, float& kx,
                                          float& ky) {
    const size_t k = (size_t)(h / 2) * w + w / 2;
    kx = xc[k];
    ky = yc[k];
}

// hm[m][c][row][ox] = sum_k g[k] f_m(row, ox + k) for f = x - kx, y - ky,
// (x - kx)^2 + (y - ky)^2, (x - kx)(y - ky): [4, nc, h, ow].
__global__ __launch_bounds__(kSsimGenThreads) void k_ssim_gen_h(
    const float* __restrict__ x, const float* __restrict__ y, int nc, int h, int w, int ow,
    const float* __restrict__ win1d, int win, float* __restrict__ hm) {
    const int64_t total = (int64_t)nc * h * ow;
    const int64_t i = (int64_t)blockIdx.x * kSsimGenThreads + threadIdx.x;
    if (i >= total) return;
    const int ox = (int)(i % ow);
    const int64_t rc = i / ow;
    const int row = (int)(rc % h), c = (int)(rc / h);
    const float* xc = x + (size_t)c * h * w;
    const float* yc = y + (size_t)c * h * w;
    float kx, ky;
    map_shift(xc, yc, h, w, kx, ky);
    const float* xr = xc + (size_t)row * w + ox;
    const float* yr = yc + (size_t)row * w + ox;
    float m0 = 0.0f, m1 = 0.0f, m2 = 0.0f, m3 = 0.0f;
    for (int k = 0; k < win; ++k) {
        const float g = win1d[k];
        const float a = xr[k] - kx, b = yr[k] - ky;
        m0 = __builtin_fmaf(g, a, m0);
        m1 = __builtin_fmaf(g, b, m1);
        m2 = __builtin_fmaf(g, __builtin_fmaf(b, b, a * a), m2);
        m3 = __builtin_fmaf(g, a * b, m3);
    }
    hm[i] = m0;
    hm[total + i] = m1;
    hm[2 * total + i] = m2;
    hm[3 * total + i] = m3;
}

// The vertical pass of hm and the SSIM of each output; workgroup b of map c
// (blocks_per_map per map) writes partials[c * blocks_per_map + b].
__global__ __launch_bounds__(kSsimGenThreads) void k_ssim_gen_v(
    const float* __restrict__ x, const float* __restrict__ y, const float* __restrict__ hm,
    int nc, int h, int w, int oh, int ow, const float* __restrict__ win1d, int win, float c1,
    float c2, int blocks_per_map, float* __restrict__ partials, float* __restrict__ abc) {
    __shared__ float sh[4];
    const int c = blockIdx.x / blocks_per_map, b = blockIdx.x - c * blocks_per_map;
    const int64_t j = (int64_t)b * kSsimGenThreads + threadIdx.x;
    float acc = 0.0f;
    if (j < (int64_t)oh * ow) {
        const int oy = (int)(j / ow), ox = (int)(j - (int64_t)oy * ow);
        float kx, ky;
        map_shift(x + (size_t)c * h * w, y + (size_t)c * h * w, h, w, kx, ky);
        const size_t plane = (size_t)nc * h * ow;
        const float* col = hm + ((size_t)c * h + oy) * ow + ox;
        float m0 = 0.0f, m1 = 0.0f, m2 = 0.0f, m3 = 0.0f;
        for (int k = 0; k < win; ++k) {
            const float g = win1d[k];
            const float* q = col + (size_t)k * ow;
            m0 = __builtin_fmaf(g, q[0], m0);
            m1 = __builtin_fmaf(g, q[plane], m1);
            m2 = __builtin_fmaf(g, q[2 * plane], m2);
            m3 = __builtin_fmaf(g, q[3 * plane], m3);
        }
        const SsimPixel sp = ssim_pixel(m0, m1, m2, m3, kx, ky, c1, c2, abc != nullptr);
        acc = sp.s;
        if (abc) {
            const size_t ld = abc_ld(ow);
            const size_t mplane = (size_t)oh * ld, stride = (size_t)nc * mplane;
            const size_t oi = (size_t)c * mplane + (size_t)oy * ld + ox;
            abc[oi] = sp.a;
            abc[stride + oi] = sp.b;
            abc[2 * stride + oi] = sp.c;
        }
    }
    const float bs = block_sum(acc, sh);
    if (threadIdx.x == 0) partials[blockIdx.x] = bs;
}

// hs[m][c][oy][px] = sum over 0 <= px - k < ow of g[k] M_m[c][oy][px - k]
// (M = A, B, C): [3, nc, oh, w].
__global__ __launch_bounds__(kSsimGenThreads) void k_ssim_gen_bh(
    const float* __restrict__ abc, int nc, int oh, int ow, int w, const float* __restrict__ win1d,
    int win, float* __restrict__ hs) {
    const int64_t total = (int64_t)nc * oh * w;
    const int64_t i = (int64_t)blockIdx.x * kSsimGenThreads + threadIdx.x;
    if (i >= total) return;
    const int px = (int)(i % w);
    const int64_t rc = i / w;
    const int oy = (int)(rc % oh), c = (int)(rc / oh);
    const size_t ld = abc_ld(ow);
    const size_t plane = (size_t)oh * ld, stride = (size_t)nc * plane;
    const float* row = abc + (size_t)c * plane + (size_t)oy * ld;
    float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f;
    const int k0 = max(0, px - ow + 1), k1 = min(win - 1, px);
    for (int k = k0; k <= k1; ++k) {
        const float g = win1d[k];
        const float* q = row + (px - k);
        s0 = __builtin_fmaf(g, q[0], s0);
        s1 = __builtin_fmaf(g, q[stride], s1);
        s2 = __builtin_fmaf(g, q[2 * stride], s2);
    }
    hs[i] = s0;
    hs[total + i] = s1;
    hs[2 * total + i] = s2;
}

// grad_x[c][py][px] = go * ssim_coef * (SA + 2 x SB + y SC), S_m = sum over
// 0 <= py - k < oh of g[k] hs[m][c][py - k][px]; go = grad_out[c] when
// go_per_map, else *grad_out.
__global__ __launch_bounds__(kSsimGenThreads) void k_ssim_gen_bv(
    const float* __restrict__ x, const float* __restrict__ y, const float* __restrict__ hs,
    int nc, int h, int w, int oh, const float* __restrict__ win1d, int win,
    const float* __restrict__ grad_out, int go_per_map, float ssim_coef,
    float* __restrict__ gx) {
    const int64_t total = (int64_t)nc * h * w;
    const int64_t i = (int64_t)blockIdx.x * kSsimGenThreads + threadIdx.x;
    if (i >= total) return;
    const int px = (int)(i % w);
    const int64_t rc = i / w;
    const int py = (int)(rc % h), c = (int)(rc / h);
    const size_t plane = (size_t)nc * oh * w;
    const float* col = hs + (size_t)c * oh * w + px;
    float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f;
    const int k0 = max(0, py - oh + 1), k1 = min(win - 1, py);
    for (int k = k0; k <= k1; ++k) {
        const float g = win1d[k];
        const float* q = col + (size_t)(py - k) * w;
        s0 = __builtin_fmaf(g, q[0], s0);
        s1 = __builtin_fmaf(g, q[plane], s1);
        s2 = __builtin_fmaf(g, q[2 * plane], s2);
    }
    const float go = grad_out[go_per_map ? c : 0];
    gx[i] = go * ssim_coef * (s0 + 2.0f * x[i] * s1 + y[i] * s2);
}

// out[c] = inv * (sum of partials [c * per_map, (c + 1) * per_map)), one
// workgroup per map, fixed summation order.
__global__ __launch_bounds__(256) void k_ssim_map_sums(const float* __restrict__ partials,
                                                      int per_map, float inv,
                                                      float* __restrict__ out) {
    __shared__ float sh[4];
    const float* p = partials + (size_t)blockIdx.x * per_map;
    float s = 0.0f;
    for (int t = threadIdx.x; t < per_map; t += 256) s += p[t];
    const float bs = block_sum(s, sh);
    if (threadIdx.x == 0) out[blockIdx.x] = bs * inv;
}

// loss = mse_sum * inv_n + w * (1 - ssim_sum * inv_m); out[1] = MSE, out[2] =
// SSIM.  One workgroup, fixed summation order.
__global__ __launch_bounds__(kFinalThreads) void k_mse_ssim_combine(
    const float* __restrict__ mse_partials, int n_mse, const float* __restrict__ ssim_partials,
    int n_ssim, float inv_n, float inv_m, float weight, float* __restrict__ out) {
    __shared__ float sh[kFinalThreads / kWave];
    // Each thread adds its elements in index order, eight of each array
    // loaded before the first addition (one memory round trip per eight).
    constexpr int kU = 8;
    float a = 0.0f, b = 0.0f;
    const int n = max(n_mse, n_ssim);
    for (int i0 = threadIdx.x; i0 < n; i0 += kU * kFinalThreads) {
        float va[kU], vb[kU];
#pragma unroll
        for (int k = 0; k < kU; ++k) {
            const int i = i0 + k * kFinalThreads;
            va[k] = i < n_mse ? mse_partials[i] : 0.0f;
            vb[k] = i < n_ssim ? ssim_partials[i] : 0.0f;
        }
#pragma unroll
        for (int k = 0; k < kU; ++k) {
            a += va[k];
            b += vb[k];
        }
    }
    const float ta = block_sum(a, sh);
    const float tb = block_sum(b, sh);
    if (threadIdx.x == 0) {
        const float mse = ta * inv_n, ss = tb * inv_m;
        out[0] = mse + weight * (1.0f - ss);
        out[1] = mse;
        out[2] = ss;
    }
}

// out[c][i][j] = clamp(img[i][j][c], lo, hi) for an [h, w, 3] image (the
// caller's clamp(0, 1).permute(2, 0, 1) glue, gaussian_trace/render.py:1309-1310).
__global__ __launch_bounds__(256) void k_clamp_hwc_to_chw(const float* __restrict__ img, int64_t hw,
                                                         float lo, float hi,
                                                         float* __restrict__ out) {
    const int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= hw) return;
    const float r = img[3 * p], g = img[3 * p + 1], b = img[3 * p + 2];
    out[p] = fminf(fmaxf(r, lo), hi);
    out[hw + p] = fminf(fmaxf(g, lo), hi);
    out[2 * hw + p] = fminf(fmaxf(b, lo), hi);
}

// grad_img[i][j][c] = grad[c][i][j] where lo <= img <= hi, else 0 (the
// gradient of clamp as torch defines it).
__global__ __launch_bounds__(256) void k_clamp_hwc_to_chw_bwd(const float* __restrict__ img,
                                                             const float* __restrict__ grad,
                                                             int64_t hw, float lo, float hi,
                                                             float* __restrict__ grad_img) {
    const int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= hw) return;
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        const float v = img[3 * p + c];
        const bool pass = (v >= lo) & (v <= hi);
        grad_img[3 * p + c] = pass ? grad[c * hw + p] : 0.0f;
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

// ------------------------------------------- MSE forward without allocation

// Partial sums of cs_mse_forward_noalloc: a file-scope device array, one copy
// per GPU, held until the process ends.  Host code never passes the array's
// name to a kernel (on the host it is only a stand-in for the symbol); it
// passes the device address hipGetSymbolAddress returns for the current GPU.
constexpr int kNoAllocMsePartials = 65536;   // 256 KiB: n up to 2^28 elements
static __device__ __align__(256) float scratch[kNoAllocMsePartials];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
float* g_scratch_ptr[kMaxDevices];   // scratch's address on each device (null: not looked up)

// scratch's device address on the current GPU, looked up once per device.
int scratch_on_current_device(float** out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return CS_ERR_HIP;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return CS_ERR_HIP;
        g_scratch_ptr[dev] = static_cast<float*>(p);
    }
    *out = g_scratch_ptr[dev];
    return CS_OK;
}
}  // namespace

extern "C" int64_t cs_mse_forward_noalloc_max_elems(void) {
    return (int64_t)kNoAllocMsePartials * kMseChunk;
}

extern "C" int cs_mse_forward_noalloc(const float* x, const float* y, int64_t n, float* loss,
                                      hipStream_t stream) {
    if (n <= 0 || n > cs_mse_forward_noalloc_max_elems() || !x || !y || !loss)
        return CS_ERR_ARGS;
    float* partials = nullptr;
    const int rc = scratch_on_current_device(&partials);
    if (rc) return rc;
    // Every partial the second launch reads is written by the first, so the
    // array needs no clearing between calls.
    const int64_t nb = (n + kMseChunk - 1) / kMseChunk;
    hipLaunchKernelGGL(k_mse_partial, dim3((unsigned)nb), dim3(kMseThreads), 0, stream, x, y, n,
                       partials);
    hipLaunchKernelGGL(k_sum_partials, dim3(1), dim3(kFinalThreads), 0, stream, partials, (int)nb,
                       1.0f / (float)n, loss);
    return metric_status();
}

extern "C" int cs_mse_backward_diff(const float* lhs, const float* rhs, int64_t n, float scale,
                                    float* grad, hipStream_t stream) {
    if (n < 0 || (n > 0 && (!lhs || !rhs || !grad))) return CS_ERR_ARGS;
    if (n == 0) return CS_OK;
    const int64_t nb = ((n + 3) / 4 + 255) / 256;
    if (nb > 0x7fffffff) return CS_ERR_ARGS;
    hipLaunchKernelGGL(k_scaled_diff, dim3((unsigned)nb), dim3(256), 0, stream, lhs, rhs, n, scale,
                       grad);
    return metric_status();
}

extern "C" size_t cs_reduce_sum_partials_elems(int64_t n) { return cs_mse_partials_elems(n); }

extern "C" int cs_reduce_sum_f32(const float* x, int64_t n, float* partials, float* out,
                                 hipStream_t stream) {
    if (n <= 0 || !x || !partials || !out) return CS_ERR_ARGS;
    const int64_t nb = (n + kMseChunk - 1) / kMseChunk;
    if (nb > 0x7fffffff) return CS_ERR_ARGS;
    hipLaunchKernelGGL(k_sum_partial, dim3((unsigned)nb), dim3(kMseThreads), 0, stream, x, n,
                       partials);
    hipLaunchKernelGGL(k_sum_partials, dim3(1), dim3(kFinalThreads), 0, stream, partials, (int)nb,
                       1.0f, out);
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

// Partials per map: one per output tile (tiled windows) or per 256 outputs
// (wider windows); h x w outputs bound both for any window.
static int64_t ssim_partials_per_map(int64_t oh, int64_t ow, int win) {
    if (win <= kSsimTiledMaxWin)
        return ((ow + kSsimTW - 1) / kSsimTW) * ((oh + kSsimTH - 1) / kSsimTH);
    return (oh * ow + kSsimGenThreads - 1) / kSsimGenThreads;
}

extern "C" size_t cs_ssim_partials_elems(int32_t nc, int32_t h, int32_t w) {
    if (nc <= 0 || h <= 0 || w <= 0) return 0;
    return (size_t)nc * (size_t)ssim_partials_per_map(h, w, kSsimTiledMaxWin + 2);
}

extern "C" size_t cs_ssim_scratch_elems(int32_t nc, int32_t h, int32_t w, int32_t win) {
    if (nc <= 0 || win <= kSsimTiledMaxWin || h < win || w < win) return 0;
    const int64_t oh = h - win + 1, ow = w - win + 1;
    const int64_t fwd = 4 * (int64_t)nc * h * ow, bwd = 3 * (int64_t)nc * oh * w;
    return (size_t)(fwd > bwd ? fwd : bwd);
}

extern "C" size_t cs_ssim_abc_elems(int32_t nc, int32_t h, int32_t w, int32_t win) {
    if (nc <= 0 || win <= 0 || h < win || w < win) return 0;
    const int64_t oh = h - win + 1, ow = w - win + 1;
    return (size_t)(3 * (int64_t)nc * oh * abc_ld((int)ow));
}

#define CS_SSIM_DISPATCH(WIN_, CALL) \
    case WIN_: CALL(WIN_); break;

static bool ssim_args_ok(int32_t nc, int32_t h, int32_t w, int32_t win) {
    return nc > 0 && win > 0 && (win & 1) == 1 && h >= win && w >= win;
}

// The fused losses take the tiled kernels' windows only.
static bool ssim_tiled_ok(int32_t nc, int32_t h, int32_t w, int32_t win) {
    return ssim_args_ok(nc, h, w, win) && win <= kSsimTiledMaxWin;
}

// SSIM partial sums (one per output tile) and, when abc != null, the maps;
// with `clamp`, x is read as clamp(x, lo, hi).
template <bool CLAMP>
static int launch_ssim_fwd(const float* x, const float* y, int32_t nc, int32_t h, int32_t w,
                           const float* win1d, int32_t win, float c1, float c2,
                           float* partials, float* abc, hipStream_t stream, int* nblk,
                           float* mse_partials = nullptr, float lo = 0.0f, float hi = 0.0f) {
    const int oh = h - win + 1, ow = w - win + 1;
    // The map stores address a plane with 32-bit byte offsets.
    if (abc && (int64_t)oh * abc_ld(ow) > kSsimMaxMapPlane) return CS_ERR_ARGS;
    const dim3 grid(((ow + kSsimTW - 1) / kSsimTW) * ((oh + kSsimTH - 1) / kSsimTH) * nc);
#define CS_SSIM_FWD(W_)                                                                       \
    hipLaunchKernelGGL((abc ? k_ssim_fwd<W_, CLAMP, true> : k_ssim_fwd<W_, CLAMP, false>),     \
                       grid, dim3(256), 0, stream, x, y, h, w, oh, ow, win1d, c1, c2, partials, \
                       abc, nc, mse_partials, lo, hi)
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
    *nblk = (int)(grid.x * grid.y * grid.z);
    return CS_OK;
}

template <int XL>
static int launch_ssim_bwd(const float* x, const float* y, int32_t nc, int32_t h, int32_t w,
                           const float* win1d, int32_t win, const float* abc,
                           const float* grad_out, int go_per_map, float ssim_coef,
                           float mse_coef, float* grad_x, hipStream_t stream, float lo = 0.0f,
                           float hi = 1.0f, int gx_planar = 0) {
    const int oh = h - win + 1, ow = w - win + 1;
    const dim3 grid(((w + kSsimTW - 1) / kSsimTW) * ((h + kSsimTH - 1) / kSsimTH) * nc);
#define CS_SSIM_BWD(W_)                                                                        \
    hipLaunchKernelGGL((k_ssim_bwd<W_, XL>), grid, dim3(256), 0, stream, x, y, h, w, oh, ow,  \
                       win1d, abc, grad_out, go_per_map, ssim_coef, mse_coef, nc, lo, hi,     \
                       gx_planar, grad_x)
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
    return CS_OK;
}

extern "C" int cs_ssim(const float* x, const float* y, int32_t nc, int32_t h, int32_t w,
                       const float* win1d, int32_t win, float c1, float c2, int32_t per_map,
                       float* partials, float* out, float* abc, float* scratch,
                       hipStream_t stream) {
    if (!ssim_args_ok(nc, h, w, win)) return CS_ERR_ARGS;
    const int oh = h - win + 1, ow = w - win + 1;
    const int64_t per = ssim_partials_per_map(oh, ow, win);
    if (win <= kSsimTiledMaxWin) {
        int nblk = 0;
        const int rc = launch_ssim_fwd<false>(x, y, nc, h, w, win1d, win, c1, c2, partials,
                                              abc, stream, &nblk);
        if (rc) return rc;
    } else {
        if (!scratch) return CS_ERR_ARGS;
        const int64_t nh = (int64_t)nc * h * ow;
        hipLaunchKernelGGL(k_ssim_gen_h,
                           dim3((unsigned)((nh + kSsimGenThreads - 1) / kSsimGenThreads)),
                           dim3(kSsimGenThreads), 0, stream, x, y, nc, h, w, ow, win1d, win,
                           scratch);
        hipLaunchKernelGGL(k_ssim_gen_v, dim3((unsigned)(per * nc)), dim3(kSsimGenThreads), 0,
                           stream, x, y, scratch, nc, h, w, oh, ow, win1d, win, c1, c2, (int)per,
                           partials, abc);
    }
    if (per_map)
        hipLaunchKernelGGL(k_ssim_map_sums, dim3((unsigned)nc), dim3(256), 0, stream, partials,
                           (int)per, 1.0f / ((float)oh * (float)ow), out);
    else
        hipLaunchKernelGGL(k_sum_partials, dim3(1), dim3(kFinalThreads), 0, stream, partials,
                           (int)(per * nc), 1.0f / ((float)nc * (float)oh * (float)ow), out);
    return metric_status();
}

extern "C" int cs_ssim_backward(const float* x, const float* y, int32_t nc, int32_t h, int32_t w,
                                const float* win1d, int32_t win, const float* abc,
                                const float* grad_out, int32_t per_map, float* grad_x,
                                float* scratch, hipStream_t stream) {
    if (!ssim_args_ok(nc, h, w, win)) return CS_ERR_ARGS;
    const int oh = h - win + 1, ow = w - win + 1;
    const float inv_cnt =
        per_map ? 1.0f / ((float)oh * (float)ow) : 1.0f / ((float)nc * (float)oh * (float)ow);
    if (win <= kSsimTiledMaxWin) {
        const int rc = launch_ssim_bwd<0>(x, y, nc, h, w, win1d, win, abc, grad_out, per_map,
                                          inv_cnt, 0.0f, grad_x, stream);
        return rc ? rc : metric_status();
    }
    if (!scratch) return CS_ERR_ARGS;
    const int64_t nh = (int64_t)nc * oh * w, nx = (int64_t)nc * h * w;
    hipLaunchKernelGGL(k_ssim_gen_bh, dim3((unsigned)((nh + kSsimGenThreads - 1) / kSsimGenThreads)),
                       dim3(kSsimGenThreads), 0, stream, abc, nc, oh, ow, w, win1d, win, scratch);
    hipLaunchKernelGGL(k_ssim_gen_bv, dim3((unsigned)((nx + kSsimGenThreads - 1) / kSsimGenThreads)),
                       dim3(kSsimGenThreads), 0, stream, x, y, scratch, nc, h, w, oh, win1d, win,
                       grad_out, per_map, inv_cnt, grad_x);
    return metric_status();
}

extern "C" size_t cs_mse_ssim_partials_elems(int32_t nc, int32_t h, int32_t w) {
    return 2 * cs_ssim_partials_elems(nc, h, w);
}

// MSE + w (1 - SSIM): the SSIM forward also sums (x - y)^2 over each tile's
// anchor inputs (so the MSE needs no pass of its own); one workgroup then
// combines both sets of tile partials.  CLAMP: x read as clamp(x, lo, hi).
template <bool CLAMP>
static int mse_ssim_loss(const float* x, const float* y, int32_t nc, int32_t h, int32_t w,
                         const float* win1d, int32_t win, float c1, float c2, float ssim_weight,
                         float* partials, float* out, float* abc, hipStream_t stream,
                         float lo = 0.0f, float hi = 0.0f) {
    if (!ssim_tiled_ok(nc, h, w, win)) return CS_ERR_ARGS;
    const int64_t n = (int64_t)nc * h * w;
    const int oh = h - win + 1, ow = w - win + 1;
    const float inv_n = 1.0f / (float)n, inv_m = 1.0f / ((float)nc * (float)oh * (float)ow);
    float* ssim_partials = partials;
    float* mse_partials = partials + cs_ssim_partials_elems(nc, h, w);
    int nblk = 0;
    const int rc = launch_ssim_fwd<CLAMP>(x, y, nc, h, w, win1d, win, c1, c2, ssim_partials, abc,
                                          stream, &nblk, mse_partials, lo, hi);
    if (rc) return rc;
    hipLaunchKernelGGL(k_mse_ssim_combine, dim3(1), dim3(kFinalThreads), 0, stream, mse_partials,
                       nblk, ssim_partials, nblk, inv_n, inv_m, ssim_weight, out);
    return metric_status();
}

template <int XL>
static int mse_ssim_backward(const float* x, const float* y, int32_t nc, int32_t h, int32_t w,
                             float lo, float hi, const float* win1d, int32_t win,
                             const float* abc, float ssim_weight, const float* grad_loss,
                             float* grad_x, hipStream_t stream, int gx_planar = 0) {
    if (!ssim_tiled_ok(nc, h, w, win)) return CS_ERR_ARGS;
    const int oh = h - win + 1, ow = w - win + 1;
    const float inv_cnt = 1.0f / ((float)nc * (float)oh * (float)ow);
    const float mse_coef = (float)(2.0 / ((double)nc * h * w));
    const int rc = launch_ssim_bwd<XL>(x, y, nc, h, w, win1d, win, abc, grad_loss, 0,
                                        -ssim_weight * inv_cnt, mse_coef, grad_x, stream, lo, hi,
                                        gx_planar);
    return rc ? rc : metric_status();
}

extern "C" int cs_mse_ssim_loss(const float* x, const float* y, int32_t nc, int32_t h, int32_t w,
                                const float* win1d, int32_t win, float c1, float c2,
                                float ssim_weight, float* partials, float* out, float* abc,
                                hipStream_t stream) {
    return mse_ssim_loss<false>(x, y, nc, h, w, win1d, win, c1, c2, ssim_weight, partials, out,
                                abc, stream);
}

extern "C" int cs_mse_ssim_backward(const float* x, const float* y, int32_t nc, int32_t h,
                                    int32_t w, const float* win1d, int32_t win, const float* abc,
                                    float ssim_weight, const float* grad_loss, float* grad_x,
                                    hipStream_t stream) {
    return mse_ssim_backward<0>(x, y, nc, h, w, 0.0f, 0.0f, win1d, win, abc, ssim_weight,
                                grad_loss, grad_x, stream);
}

extern "C" int cs_clamp_mse_ssim_loss(const float* img, int32_t img_planar, const float* y,
                                      int32_t h, int32_t w, float lo, float hi,
                                      const float* win1d, int32_t win, float c1, float c2,
                                      float ssim_weight, float* x, float* partials, float* out,
                                      float* abc, hipStream_t stream) {
    if (!ssim_tiled_ok(3, h, w, win)) return CS_ERR_ARGS;
    // Planes: the SSIM forward reads them clamped; no copy.
    if (img_planar)
        return mse_ssim_loss<true>(img, y, 3, h, w, win1d, win, c1, c2, ssim_weight, partials,
                                   out, abc, stream, lo, hi);
    if (!x) return CS_ERR_ARGS;
    const int64_t hw = (int64_t)h * w;
    hipLaunchKernelGGL(k_clamp_hwc_to_chw, dim3((unsigned)((hw + 255) / 256)), dim3(256), 0,
                       stream, img, hw, lo, hi, x);
    return mse_ssim_loss<false>(x, y, 3, h, w, win1d, win, c1, c2, ssim_weight, partials, out,
                                abc, stream);
}

extern "C" int cs_clamp_mse_ssim_backward(const float* img, int32_t img_planar, const float* y,
                                          int32_t h, int32_t w, float lo, float hi,
                                          const float* win1d, int32_t win, const float* abc,
                                          float ssim_weight, const float* grad_loss,
                                          float* grad_img, int32_t grad_planar,
                                          hipStream_t stream) {
    if (img_planar) {
        // The gradient of a planar image is written as planes.
        if (!grad_planar) return CS_ERR_ARGS;
        return mse_ssim_backward<2>(img, y, 3, h, w, lo, hi, win1d, win, abc, ssim_weight,
                                    grad_loss, grad_img, stream, 1);
    }
    return mse_ssim_backward<1>(img, y, 3, h, w, lo, hi, win1d, win, abc, ssim_weight,
                                grad_loss, grad_img, stream, grad_planar ? 1 : 0);
}

extern "C" int cs_clamp_hwc_to_nchw(const float* img, int32_t h, int32_t w, float lo, float hi,
                                    float* out, hipStream_t stream) {
    if (h <= 0 || w <= 0) return CS_ERR_ARGS;
    const int64_t hw = (int64_t)h * w;
    hipLaunchKernelGGL(k_clamp_hwc_to_chw, dim3((unsigned)((hw + 255) / 256)), dim3(256), 0,
                       stream, img, hw, lo, hi, out);
    return metric_status();
}

extern "C" int cs_clamp_hwc_to_nchw_backward(const float* img, const float* grad, int32_t h,
                                             int32_t w, float lo, float hi, float* grad_img,
                                             hipStream_t stream) {
    if (h <= 0 || w <= 0) return CS_ERR_ARGS;
    const int64_t hw = (int64_t)h * w;
    hipLaunchKernelGGL(k_clamp_hwc_to_chw_bwd, dim3((unsigned)((hw + 255) / 256)), dim3(256), 0,
                       stream, img, grad, hw, lo, hi, grad_img);
    return metric_status();
}
