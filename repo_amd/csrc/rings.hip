// Closed control rings -> piecewise cubic Hermite segments (forward and
// backward), the step before binning in the reference's closed-fill model
// (gaussian_trace/render.py:755-777 -> ops/cubic_splatting.py:486-543).
//
// A ring has K control points (K >= 4, K even).  Branch b in {0, 1} is the
// Bezier curve of degree kb - 1 = K/2 on control points b (kb - 1) + i (mod K),
// i < kb, so the two branches share their end points and close the ring.  Each
// branch is cut at subdiv + 1 samples t_s into cubic Hermite pieces:
//   P0 = B(t_s), P3 = B(t_s+1), P1 = P0 + B'(t_s) dt/3, P2 = P3 - B'(t_s+1) dt/3,
// with B' = (kb - 1) sum_i d_i (c_{i+1} - c_i) from the derivative basis d.
//
// Forward: one thread per output segment (cubic_splatting.py:137-268, same
// operation order).  Backward: the reference scatters each segment's
// gradient into the control points with atomics (:271-383); here one thread
// per (ring, control point) gathers the terms of every segment that uses the
// point, so the result is deterministic and needs no zero-initialised output.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/cubicsplat_hip.h"

namespace cs {

constexpr int kRingThreads = 256;

__device__ __forceinline__ int wrap(int i, int K) { return i >= K ? i - K : i; }

__global__ __launch_bounds__(kRingThreads) void k_ring_fwd(
    const float2* __restrict__ cp, int ncurves, int K, int sub, const float* __restrict__ basis,
    const float* __restrict__ dbasis, const float* __restrict__ dt, float* __restrict__ out) {
    const int64_t sid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int per_curve = 2 * sub;
    if (sid >= (int64_t)ncurves * per_curve) return;
    const int curve = (int)(sid / per_curve);
    const int local = (int)(sid - (int64_t)curve * per_curve);
    const int branch = local / sub, s = local - branch * sub;
    const int kb = (K + 2) / 2;
    const int base = branch * (kb - 1);
    const float2* c = cp + (size_t)curve * K;
    const float* w0 = basis + (size_t)s * kb;
    const float* w1 = w0 + kb;
    float p0x = 0.0f, p0y = 0.0f, p3x = 0.0f, p3y = 0.0f;
    for (int i = 0; i < kb; ++i) {
        const float2 q = c[wrap(base + i, K)];
        p0x = p0x + w0[i] * q.x;
        p0y = p0y + w0[i] * q.y;
        p3x = p3x + w1[i] * q.x;
        p3y = p3y + w1[i] * q.y;
    }
    const float* d0 = dbasis + (size_t)s * (kb - 1);
    const float* d1 = d0 + (kb - 1);
    float d0x = 0.0f, d0y = 0.0f, d1x = 0.0f, d1y = 0.0f;
    for (int i = 0; i < kb - 1; ++i) {
        const float2 a = c[wrap(base + i, K)], b = c[wrap(base + i + 1, K)];
        const float dx = b.x - a.x, dy = b.y - a.y;
        d0x = d0x + d0[i] * dx;
        d0y = d0y + d0[i] * dy;
        d1x = d1x + d1[i] * dx;
        d1y = d1y + d1[i] * dy;
    }
    const float deg = (float)(kb - 1);
    d0x = d0x * deg;
    d0y = d0y * deg;
    d1x = d1x * deg;
    d1y = d1y * deg;
    const float third = dt[s] * (float)(1.0 / 3.0);
    float4* o = reinterpret_cast<float4*>(out + (size_t)sid * 8);
    o[0] = make_float4(p0x, p0y, p0x + d0x * third, p0y + d0y * third);
    o[1] = make_float4(p3x - d1x * third, p3y - d1y * third, p3x, p3y);
}

// Gradient of one control point: for each branch that contains it (local
// index i) and each of the branch's segments s, the reference's terms
//   (g0 w_s[i] + g3 w_s+1[i])                    g0 = gP0 + gP1, g3 = gP3 + gP2
//   - dcoef(i) (i < kb - 1) + dcoef(i - 1) (i > 0),
//   dcoef(j) = (kb - 1) (gP1 dt/3 d_s[j] - gP2 dt/3 d_s+1[j]).
__global__ __launch_bounds__(kRingThreads) void k_ring_bwd(
    const float* __restrict__ grad_seg, int ncurves, int K, int sub,
    const float* __restrict__ basis, const float* __restrict__ dbasis,
    const float* __restrict__ dt, float2* __restrict__ grad_cp) {
    const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (tid >= (int64_t)ncurves * K) return;
    const int curve = (int)(tid / K);
    const int j = (int)(tid - (int64_t)curve * K);
    const int kb = (K + 2) / 2;
    const float deg = (float)(kb - 1);
    float ax = 0.0f, ay = 0.0f;
    for (int branch = 0; branch < 2; ++branch) {
        int i = j - branch * (kb - 1);
        if (i < 0) i += K;
        if (i >= kb) continue;
        const float* g = grad_seg + ((size_t)curve * 2 * sub + (size_t)branch * sub) * 8;
        for (int s = 0; s < sub; ++s, g += 8) {
            const float4 a = reinterpret_cast<const float4*>(g)[0];  // P0, P1
            const float4 b = reinterpret_cast<const float4*>(g)[1];  // P2, P3
            const float third = dt[s] * (float)(1.0 / 3.0);
            const float w0 = basis[(size_t)s * kb + i], w1 = basis[(size_t)(s + 1) * kb + i];
            ax += (a.x + a.z) * w0 + (b.z + b.x) * w1;
            ay += (a.y + a.w) * w0 + (b.w + b.y) * w1;
            const float gd0x = a.z * third, gd0y = a.w * third;
            const float gd1x = -b.x * third, gd1y = -b.y * third;
            const float* d0 = dbasis + (size_t)s * (kb - 1);
            const float* d1 = d0 + (kb - 1);
            if (i < kb - 1) {
                ax -= deg * (gd0x * d0[i] + gd1x * d1[i]);
                ay -= deg * (gd0y * d0[i] + gd1y * d1[i]);
            }
            if (i > 0) {
                ax += deg * (gd0x * d0[i - 1] + gd1x * d1[i - 1]);
                ay += deg * (gd0y * d0[i - 1] + gd1y * d1[i - 1]);
            }
        }
    }
    grad_cp[tid] = make_float2(ax, ay);
}

}  // namespace cs

using namespace cs;

static bool ring_args_ok(int32_t ncurves, int32_t K, int32_t subdiv) {
    return ncurves >= 0 && K >= 4 && (K - 2) % 2 == 0 && subdiv > 0;
}

static bool aligned(const void* p, uintptr_t a) {
    return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0;
}

extern "C" int cs_closed_ring_segments(const float* control_points, int32_t num_curves,
                                       int32_t K, int32_t subdiv, const float* basis,
                                       const float* deriv_basis, const float* dt,
                                       float* out_segments, hipStream_t stream) {
    if (!ring_args_ok(num_curves, K, subdiv) || !aligned(control_points, 8) ||
        !aligned(out_segments, 16))
        return CS_ERR_ARGS;
    const int64_t n = (int64_t)num_curves * 2 * subdiv;
    if (n == 0) return CS_OK;
    hipLaunchKernelGGL(k_ring_fwd, dim3((unsigned)((n + kRingThreads - 1) / kRingThreads)),
                       dim3(kRingThreads), 0, stream,
                       reinterpret_cast<const float2*>(control_points), num_curves, K, subdiv,
                       basis, deriv_basis, dt, out_segments);
    return hipGetLastError() == hipSuccess ? CS_OK : CS_ERR_HIP;
}

extern "C" int cs_closed_ring_segments_backward(const float* grad_segments, int32_t num_curves,
                                                int32_t K, int32_t subdiv, const float* basis,
                                                const float* deriv_basis, const float* dt,
                                                float* grad_control_points, hipStream_t stream) {
    if (!ring_args_ok(num_curves, K, subdiv) || !aligned(grad_segments, 16) ||
        !aligned(grad_control_points, 8))
        return CS_ERR_ARGS;
    const int64_t n = (int64_t)num_curves * K;
    if (n == 0) return CS_OK;
    hipLaunchKernelGGL(k_ring_bwd, dim3((unsigned)((n + kRingThreads - 1) / kRingThreads)),
                       dim3(kRingThreads), 0, stream, grad_segments, num_curves, K, subdiv, basis,
                       deriv_basis, dt, reinterpret_cast<float2*>(grad_control_points));
    return hipGetLastError() == hipSuccess ? CS_OK : CS_ERR_HIP;
}
