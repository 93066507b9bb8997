// 2D Gaussian splats: the kernels behind GsRenderFunction
// (tilelang_renderer.py:149-490) and the op-level functions of
// ops/forward2d.py, ops/backward2d.py, ops/intersects.py and ops/rasterize.py.
//
//   k_gs_project      forward2d.py:14-164, one thread per Gaussian
//   k_gs_pack         per-Gaussian 48-byte raster records (GsRec)
//   k_gs_raster_fwd   rasterize.py:18-157: one workgroup per tile, one pixel
//                     per lane; each wave walks the tile's list on its own
//                     with scalar loads of ids and records, and leaves the
//                     walk when all of its pixels are done
//   k_gs_raster_bwd   rasterize.py:160-529: each wave walks back from the
//                     largest final index of its pixels; per entry the wave
//                     sums its pixels' terms with two 8-way DPP reductions and
//                     eight lanes add them with float atomics
//   k_gs_project_bwd  backward2d.py:8-151 (with the meta scaling of
//                     tilelang_renderer.py:111-116)
//   k_gs_map_ref      intersects.py:12-226 in the reference's int64 layout
//
// Arithmetic follows the spec shared with oracle/gs_oracle.c (cs_common.h):
// the forward's outputs are bit-identical to it.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/cubicsplat_hip.h"
#include "cs_common.h"

namespace cs {

constexpr int kGsThreads = 256;
constexpr float kGsAlphaCapFwd = (float)0.999;  // rasterize.py:49
constexpr float kGsAlphaCapBwd = (float)0.99;   // rasterize.py:246
constexpr float kGsAlphaMin = (float)(1.0 / 255.0);
constexpr float kGsTStop = (float)1e-4;

static_assert(sizeof(GsRec) == 48, "GsRec is read as 12 dwords");

__global__ __launch_bounds__(kGsThreads) void k_gs_project(
    const float2* __restrict__ means, const float2* __restrict__ scales,
    const float* __restrict__ rot, int n, int img_h, int img_w, int block_x, int block_y,
    int tbx, int tby, float2* __restrict__ xys, float* __restrict__ depths,
    int32_t* __restrict__ radii, float* __restrict__ conics, int32_t* __restrict__ tiles_hit) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float ox = 0.5f * (float)img_w, oy = 0.5f * (float)img_h;
    const float2 m = means[i], s = scales[i];
    const float cx = ox * m.x + ox, cy = oy * m.y + oy;
    float sr, cr;
    spec_sincosf(rot[i], &sr, &cr);
    const float m00 = cr * s.x, m01 = sr * s.y, m10 = -sr * s.x, m11 = cr * s.y;
    const float cxx = m00 * m00 + m01 * m01;
    const float cxy = m00 * m10 + m01 * m11;
    const float cyy = m10 * m10 + m11 * m11;
    const float det = cxx * cyy - cxy * cxy;
    float ox_ = 0.0f, oy_ = 0.0f, q0 = 0.0f, q1 = 0.0f, q2 = 0.0f;
    int32_t rad = 0, area = 0;
    if (det != 0.0f) {
        const float inv_det = 1.0f / det;
        const float qx = cyy * inv_det, qy = -cxy * inv_det, qz = cxx * inv_det;
        const float b = 0.5f * (cxx + cyy);
        const float delta = fmaxf(0.1f, b * b - det);
        const float sd = __builtin_sqrtf(delta);
        const float radius = __builtin_ceilf(3.0f * __builtin_sqrtf(fmaxf(b + sd, b - sd)));
        const int4 r = gs_tile_rect(cx, cy, qx, qy, qz, radius, block_x, block_y, tbx, tby);
        const int32_t a = (r.z - r.x) * (r.w - r.y);
        if (a > 0) {
            ox_ = cx;
            oy_ = cy;
            q0 = qx;
            q1 = qy;
            q2 = qz;
            rad = f2i_sat(radius);
            area = a;
        }
    }
    xys[i] = make_float2(ox_, oy_);
    depths[i] = 0.0f;
    radii[i] = rad;
    conics[3 * i] = q0;
    conics[3 * i + 1] = q1;
    conics[3 * i + 2] = q2;
    tiles_hit[i] = area;
}

__global__ __launch_bounds__(kGsThreads) void k_gs_pack(const float2* __restrict__ xys,
                                                        const float* __restrict__ conics,
                                                        const float* __restrict__ colors,
                                                        const float* __restrict__ opac, int n,
                                                        GsRec* __restrict__ recs) {
    const int g = blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= n) return;
    const float2 p = xys[g];
    const float qa = conics[3 * g], qb = conics[3 * g + 1], qc = conics[3 * g + 2];
    const float o = opac[g];
    float4* dst = reinterpret_cast<float4*>(recs + g);
    dst[0] = make_float4(p.x, p.y, 0.5f * qa, qb);
    dst[1] = make_float4(0.5f * qc, o, gs_alpha_cut(o), colors[3 * g]);
    dst[2] = make_float4(colors[3 * g + 1], colors[3 * g + 2], qa, qc);
}

// The lane's pixel: index k = threadIdx.x of the tile's block_x x block_y
// pixels in row-major order, at (px, py) = (j, i) (rasterize.py:84-88).
struct GsPixel {
    int i, j;
    bool inside;
};

__device__ __forceinline__ GsPixel gs_pixel(int tile, int tbx, int bx, int by, int img_h,
                                            int img_w) {
    const int ty = tile / tbx, tx = tile - ty * tbx;
    const int k = threadIdx.x;
    const int ly = k / bx, lx = k - ly * bx;
    GsPixel P;
    P.i = ty * by + ly;
    P.j = tx * bx + lx;
    P.inside = k < bx * by && P.i < img_h && P.j < img_w;
    return P;
}

// sigma = dx (a dx + b dy) + c dy^2, the spec form of rasterize.py:111-114.
__device__ __forceinline__ float gs_sigma(const GsRec& R, float px, float py, float& dx,
                                          float& dy) {
    dx = R.x - px;
    dy = R.y - py;
    return __builtin_fmaf(dx, __builtin_fmaf(R.a, dx, R.b * dy), (R.c * dy) * dy);
}

__global__ __launch_bounds__(1024) void k_gs_raster_fwd(
    const int32_t* __restrict__ ids_g, const int32_t* __restrict__ bins_g,
    const GsRec* __restrict__ recs_g, const float* __restrict__ bg, int img_h, int img_w, int bx,
    int by, int tbx, int ntiles, float* __restrict__ out, float* __restrict__ final_T,
    int32_t* __restrict__ final_idx) {
    const int tile = xcd_tile(blockIdx.x, ntiles);
    const GsPixel P = gs_pixel(tile, tbx, bx, by, img_h, img_w);
    const cptr<int32_t> ids = as_const(ids_g);
    const cptr<GsRec> recs = as_const(recs_g);
    const cptr<int32_t> bins = as_const(bins_g);
    const int g0 = bins[2 * tile], g1 = bins[2 * tile + 1];
    const float px = (float)P.j, py = (float)P.i;
    float T = 1.0f, c0 = 0.0f, c1 = 0.0f, c2 = 0.0f;
    int cur = 0;
    bool done = !P.inside;
    for (int e = g0; e < g1; ++e) {
        if (__ballot(!done) == 0) break;
        const GsRec R = recs[ids[e]];
        if (done) continue;
        float dx, dy;
        const float sigma = gs_sigma(R, px, py, dx, dy);
        if (sigma < 0.0f || sigma > R.cut) continue;
        const float alpha = fminf(kGsAlphaCapFwd, R.opac * spec_expf(-sigma));
        if (alpha < kGsAlphaMin) continue;
        const float nT = T * (1.0f - alpha);
        const float vis = alpha * T;
        c0 = __builtin_fmaf(R.r, vis, c0);
        c1 = __builtin_fmaf(R.g, vis, c1);
        c2 = __builtin_fmaf(R.bl, vis, c2);
        T = nT;
        cur = e;
        if (nT <= kGsTStop) done = true;
    }
    if (!P.inside) return;
    const size_t p = (size_t)P.i * img_w + P.j;
    final_T[p] = T;
    final_idx[p] = cur;
    out[3 * p] = __builtin_fmaf(T, bg[0], c0);
    out[3 * p + 1] = __builtin_fmaf(T, bg[1], c1);
    out[3 * p + 2] = __builtin_fmaf(T, bg[2], c2);
}

__global__ __launch_bounds__(1024) void k_gs_raster_bwd(
    const int32_t* __restrict__ ids_g, const int32_t* __restrict__ meta_g,
    const int32_t* __restrict__ bins_g, const GsRec* __restrict__ recs_g,
    const float* __restrict__ bg, int img_h, int img_w, int bx, int by, int tbx, int ntiles,
    const float* __restrict__ final_T, const int32_t* __restrict__ final_idx,
    const float* __restrict__ v_out, const float* __restrict__ v_out_alpha,
    float* __restrict__ v_xy, float* __restrict__ v_conic, float* __restrict__ v_rgb,
    float* __restrict__ v_opac, float* __restrict__ contrib_rgb,
    float* __restrict__ isect_contrib) {
    const int tile = xcd_tile(blockIdx.x, ntiles);
    const GsPixel P = gs_pixel(tile, tbx, bx, by, img_h, img_w);
    const cptr<int32_t> ids = as_const(ids_g);
    const cptr<int32_t> meta = as_const(meta_g);
    const cptr<GsRec> recs = as_const(recs_g);
    const cptr<int32_t> bins = as_const(bins_g);
    const int g0 = bins[2 * tile], g1 = bins[2 * tile + 1];
    const float px = (float)P.j, py = (float)P.i;
    const size_t p = P.inside ? (size_t)P.i * img_w + P.j : 0;
    float T = 0.0f, v0 = 0.0f, v1 = 0.0f, v2 = 0.0f, va = 0.0f;
    int fidx = -1;
    if (P.inside) {
        T = final_T[p];
        fidx = final_idx[p];
        v0 = v_out[3 * p];
        v1 = v_out[3 * p + 1];
        v2 = v_out[3 * p + 2];
        if (v_out_alpha) va = v_out_alpha[p];
    }
    const float T_final = T;
    const float bg_dot = bg[0] * v0 + bg[1] * v1 + bg[2] * v2;
    // T_final ra (va - bg.v) is the background's share of d alpha.
    const float bg_term = va - bg_dot;
    float b0 = 0.0f, b1 = 0.0f, b2 = 0.0f;
    const bool want_contrib = contrib_rgb != nullptr || isect_contrib != nullptr;
    const int lane = threadIdx.x & (kWave - 1);
    const int slot = reduce8_slot(lane & 7);
    const bool adder = (lane & ~7) == 8;
    const int gstart = min(g1 - 1, __builtin_amdgcn_readfirstlane(wave_max_i(fidx)));
    for (int e = gstart; e >= g0; --e) {
        const int g = ids[e];
        const GsRec R = recs[g];
        const bool geom = meta_g == nullptr || meta[e] != 0;
        float dx, dy;
        const float sigma = gs_sigma(R, px, py, dx, dy);
        bool valid = e <= fidx && !(sigma < 0.0f) && !(sigma > R.cut);
        float vis = 0.0f, alpha = 0.0f;
        if (valid) {
            vis = spec_expf(-sigma);
            alpha = fminf(kGsAlphaCapBwd, R.opac * vis);
            valid = alpha >= kGsAlphaMin;
        }
        if (__ballot(valid) == 0) continue;
        float pv[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
        float pw[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
        if (valid) {
            const float ra = __builtin_amdgcn_rcpf(1.0f - alpha);
            T = T * ra;
            const float fac = alpha * T;
            pv[0] = fac * v0;
            pv[1] = fac * v1;
            pv[2] = fac * v2;
            if (want_contrib) {
                pw[1] = fac * R.r;
                pw[2] = fac * R.g;
                pw[3] = fac * R.bl;
                pw[4] = pw[1] + pw[2] + pw[3];
            }
            float v_alpha = __builtin_fmaf(R.r, T, -(b0 * ra)) * v0;
            v_alpha = __builtin_fmaf(__builtin_fmaf(R.g, T, -(b1 * ra)), v1, v_alpha);
            v_alpha = __builtin_fmaf(__builtin_fmaf(R.bl, T, -(b2 * ra)), v2, v_alpha);
            v_alpha = __builtin_fmaf(T_final * ra, bg_term, v_alpha);
            b0 = __builtin_fmaf(R.r, fac, b0);
            b1 = __builtin_fmaf(R.g, fac, b1);
            b2 = __builtin_fmaf(R.bl, fac, b2);
            pv[3] = vis * v_alpha;
            if (geom) {
                const float v_sigma = -R.opac * vis * v_alpha;
                const float hs = 0.5f * v_sigma;
                pv[4] = hs * dx * dx;
                pv[5] = hs * dx * dy;
                pv[6] = hs * dy * dy;
                pv[7] = v_sigma * __builtin_fmaf(R.pad0, dx, R.b * dy);
                pw[0] = v_sigma * __builtin_fmaf(R.b, dx, R.pad1 * dy);
            }
        }
        {
            const float t = wave_reduce8(pv);
            if (adder) {
                float* dst = slot < 3 ? v_rgb + 3 * g + slot
                           : slot == 3 ? v_opac + g
                           : slot < 7 ? v_conic + 3 * g + (slot - 4)
                                      : v_xy + 2 * g;
                if (slot < 4 || geom) atomicAdd(dst, t);
            }
        }
        if (geom || want_contrib) {
            const float t = wave_reduce8(pw);
            if (adder) {
                if (slot == 0 && geom) atomicAdd(v_xy + 2 * g + 1, t);
                if (slot >= 1 && slot <= 3 && contrib_rgb)
                    atomicAdd(contrib_rgb + 3 * g + (slot - 1), t);
                if (slot == 4 && isect_contrib) atomicAdd(isect_contrib + e, t);
            }
        }
    }
}

__global__ __launch_bounds__(kGsThreads) void k_gs_project_bwd(
    const float2* __restrict__ scales, const float* __restrict__ rot,
    const int32_t* __restrict__ radii, const float* __restrict__ conics,
    const float2* __restrict__ v_xy, const float* __restrict__ v_conic,
    const int32_t* __restrict__ meta, int n, int img_h, int img_w, float* __restrict__ v_cov2d,
    float2* __restrict__ v_mean, float2* __restrict__ v_scale, float* __restrict__ v_rot) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float g11 = 0.0f, g12 = 0.0f, g22 = 0.0f, vs0 = 0.0f, vs1 = 0.0f, vr = 0.0f;
    float vm0 = 0.0f, vm1 = 0.0f;
    if (radii[i] > 0) {
        // tilelang_renderer.py:111-116: v_xy and v_conic times the meta flag.
        const float keep = meta ? (float)meta[i] : 1.0f;
        const float c0 = conics[3 * i], c1 = conics[3 * i + 1], c2 = conics[3 * i + 2];
        const float q0 = v_conic[3 * i] * keep, q1 = v_conic[3 * i + 1] * keep,
                    q2 = v_conic[3 * i + 2] * keep;
        const float h00 = c0 * q0 + c1 * q1, h01 = c0 * q1 + c1 * q2;
        const float h10 = c1 * q0 + c2 * q1, h11 = c1 * q1 + c2 * q2;
        g11 = -(h00 * c0 + h01 * c1);
        g12 = -(h10 * c0 + h11 * c1) - (h00 * c1 + h01 * c2);
        g22 = -(h10 * c1 + h11 * c2);
        const float2 s = scales[i];
        float sn, cs_;
        spec_sincosf(rot[i], &sn, &cs_);
        vs0 = g11 * (2.0f * s.x * cs_ * cs_) + 2.0f * g12 * (-2.0f * s.x * sn * cs_) +
              g22 * (2.0f * s.x * sn * sn);
        vs1 = g11 * (2.0f * s.y * sn * sn) + 2.0f * g12 * (2.0f * s.y * cs_ * sn) +
              g22 * (2.0f * s.y * cs_ * cs_);
        const float m00 = cs_ * s.x, m01 = sn * s.y, m10 = -sn * s.x, m11 = cs_ * s.y;
        const float a00 = -sn * s.x, a01 = cs_ * s.y, a10 = -cs_ * s.x, a11 = -sn * s.y;
        const float t1_00 = a00 * m00 + a01 * m01, t1_10 = a10 * m00 + a11 * m01,
                    t1_11 = a10 * m10 + a11 * m11;
        const float b00 = m00 * s.x, b01 = m01 * s.y, b10 = m10 * s.x, b11 = m11 * s.y;
        const float t2_00 = b00 * -sn + b01 * cs_, t2_10 = b10 * -sn + b11 * cs_,
                    t2_11 = b10 * -cs_ + b11 * -sn;
        vr = g11 * (t1_00 + t2_00) + 2.0f * g12 * (t1_10 + t2_10) + g22 * (t1_11 + t2_11);
        const float2 vx = v_xy[i];
        vm0 = vx.x * keep * (0.5f * (float)img_w);
        vm1 = vx.y * keep * (0.5f * (float)img_h);
    }
    if (v_cov2d) {
        v_cov2d[3 * i] = g11;
        v_cov2d[3 * i + 1] = g12;
        v_cov2d[3 * i + 2] = g22;
    }
    v_mean[i] = make_float2(vm0, vm1);
    v_scale[i] = make_float2(vs0, vs1);
    v_rot[i] = vr;
}

// intersects.py:12-226: Gaussian g writes its rectangle's tiles row-major at
// [cum[g-1], cum[g-1] + area), key (tile << 32) | depth bits.  Writes outside
// [0, num_intersects) are dropped (the reference assumes they cannot occur).
__global__ __launch_bounds__(kGsThreads) void k_gs_map_ref(
    const float* __restrict__ xys, const float* __restrict__ conics,
    const float* __restrict__ depths, const int32_t* __restrict__ radii,
    const int32_t* __restrict__ cum, int n, int64_t num_isects, int bx, int by, int tbx,
    int tby, int64_t* __restrict__ isect_ids, int32_t* __restrict__ gauss_ids) {
    const int g = blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= n || radii[g] <= 0) return;
    const float rf = (float)radii[g];
    const int4 r = conics ? gs_tile_rect(xys[2 * g], xys[2 * g + 1], conics[3 * g],
                                         conics[3 * g + 1], conics[3 * g + 2], rf, bx, by, tbx,
                                         tby)
                          : gs_tile_rect(xys[2 * g], xys[2 * g + 1], 0.0f, 0.0f, 0.0f, rf, bx,
                                         by, tbx, tby);
    const int w = r.z - r.x, h = r.w - r.y;
    if (w * h <= 0) return;
    const int64_t base = g == 0 ? 0 : (int64_t)cum[g - 1];
    const int64_t key_lo = (int64_t)__builtin_bit_cast(uint32_t, depths[g]);
    for (int row = 0; row < h; ++row) {
        for (int col = 0; col < w; ++col) {
            const int64_t o = base + (int64_t)row * w + col;
            if (o < 0 || o >= num_isects) continue;
            const int64_t t = (int64_t)(r.y + row) * tbx + r.x + col;
            isect_ids[o] = (t << 32) | key_lo;
            gauss_ids[o] = g;
        }
    }
}

}  // namespace cs

using namespace cs;

static inline int gs_blocks(int64_t n) { return (int)((n + kGsThreads - 1) / kGsThreads); }

static int gs_status() { return hipGetLastError() == hipSuccess ? CS_OK : CS_ERR_HIP; }

static bool gs_dims_ok(int32_t img_h, int32_t img_w, int32_t block_x, int32_t block_y) {
    return img_h > 0 && img_w > 0 && block_x > 0 && block_y > 0 && block_x * block_y <= 1024;
}

static bool al(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

extern "C" int cs_gs_project_forward(const float* means2d, const float* scales2d,
                                     const float* rotation, int32_t n, int32_t img_h,
                                     int32_t img_w, int32_t block_x, int32_t block_y, float* xys,
                                     float* depths, int32_t* radii, float* conics,
                                     int32_t* num_tiles_hit, hipStream_t stream) {
    if (n < 0 || !gs_dims_ok(img_h, img_w, block_x, block_y) || !al(means2d, 8) ||
        !al(scales2d, 8) || !al(xys, 8))
        return CS_ERR_ARGS;
    if (n == 0) return CS_OK;
    const int tbx = (img_w + block_x - 1) / block_x, tby = (img_h + block_y - 1) / block_y;
    hipLaunchKernelGGL(k_gs_project, dim3(gs_blocks(n)), dim3(kGsThreads), 0, stream,
                       reinterpret_cast<const float2*>(means2d),
                       reinterpret_cast<const float2*>(scales2d), rotation, n, img_h, img_w,
                       block_x, block_y, tbx, tby, reinterpret_cast<float2*>(xys), depths, radii,
                       conics, num_tiles_hit);
    return gs_status();
}

extern "C" int cs_gs_pack_records(const float* xys, const float* conics, const float* colors,
                                  const float* opacities, int32_t n, void* records,
                                  hipStream_t stream) {
    if (n < 0 || !al(xys, 8) || !al(records, 16)) return CS_ERR_ARGS;
    if (n == 0) return CS_OK;
    hipLaunchKernelGGL(k_gs_pack, dim3(gs_blocks(n)), dim3(kGsThreads), 0, stream,
                       reinterpret_cast<const float2*>(xys), conics, colors, opacities, n,
                       reinterpret_cast<GsRec*>(records));
    return gs_status();
}

static inline int gs_wg(int32_t block_x, int32_t block_y) {
    return (block_x * block_y + kWave - 1) / kWave * kWave;
}

extern "C" int cs_gs_rasterize_forward(const int32_t* gaussian_ids_sorted,
                                       const int32_t* tile_bins, const void* records,
                                       const float* background, int32_t img_h, int32_t img_w,
                                       int32_t block_x, int32_t block_y, float* out_img,
                                       float* final_Ts, int32_t* final_idx,
                                       hipStream_t stream) {
    if (!gs_dims_ok(img_h, img_w, block_x, block_y) || !al(records, 16)) return CS_ERR_ARGS;
    const int tbx = (img_w + block_x - 1) / block_x, tby = (img_h + block_y - 1) / block_y;
    const int ntiles = tbx * tby;
    hipLaunchKernelGGL(k_gs_raster_fwd, dim3(ntiles), dim3(gs_wg(block_x, block_y)), 0, stream,
                       gaussian_ids_sorted, tile_bins, reinterpret_cast<const GsRec*>(records),
                       background, img_h, img_w, block_x, block_y, tbx, ntiles, out_img,
                       final_Ts, final_idx);
    return gs_status();
}

extern "C" int cs_gs_rasterize_backward(
    const int32_t* gaussian_ids_sorted, const int32_t* intersect_meta_sorted,
    const int32_t* tile_bins, const void* records, const float* background, int32_t img_h,
    int32_t img_w, int32_t block_x, int32_t block_y, const float* final_Ts,
    const int32_t* final_idx, const float* v_output, const float* v_output_alpha, float* v_xy,
    float* v_conic, float* v_rgb, float* v_opacity, float* contrib_rgb, float* isect_contrib,
    hipStream_t stream) {
    if (!gs_dims_ok(img_h, img_w, block_x, block_y) || !al(records, 16)) return CS_ERR_ARGS;
    const int tbx = (img_w + block_x - 1) / block_x, tby = (img_h + block_y - 1) / block_y;
    const int ntiles = tbx * tby;
    hipLaunchKernelGGL(k_gs_raster_bwd, dim3(ntiles), dim3(gs_wg(block_x, block_y)), 0, stream,
                       gaussian_ids_sorted, intersect_meta_sorted, tile_bins,
                       reinterpret_cast<const GsRec*>(records), background, img_h, img_w,
                       block_x, block_y, tbx, ntiles, final_Ts, final_idx, v_output,
                       v_output_alpha, v_xy, v_conic, v_rgb, v_opacity, contrib_rgb,
                       isect_contrib);
    return gs_status();
}

extern "C" int cs_gs_project_backward(const float* scales2d, const float* rotation,
                                      const int32_t* radii, const float* conics,
                                      const float* v_xy, const float* v_conic,
                                      const int32_t* gaussian_meta, int32_t n, int32_t img_h,
                                      int32_t img_w, float* v_cov2d, float* v_mean2d,
                                      float* v_scale, float* v_rot, hipStream_t stream) {
    if (n < 0 || img_h <= 0 || img_w <= 0 || !al(scales2d, 8) || !al(v_xy, 8) ||
        !al(v_mean2d, 8) || !al(v_scale, 8))
        return CS_ERR_ARGS;
    if (n == 0) return CS_OK;
    hipLaunchKernelGGL(k_gs_project_bwd, dim3(gs_blocks(n)), dim3(kGsThreads), 0, stream,
                       reinterpret_cast<const float2*>(scales2d), rotation, radii, conics,
                       reinterpret_cast<const float2*>(v_xy), v_conic, gaussian_meta, n, img_h,
                       img_w, v_cov2d, reinterpret_cast<float2*>(v_mean2d),
                       reinterpret_cast<float2*>(v_scale), v_rot);
    return gs_status();
}

extern "C" int cs_gs_map_to_intersects(const float* xys, const float* conics,
                                       const float* depths, const int32_t* radii,
                                       const int32_t* cum_tiles_hit, int32_t n,
                                       int64_t num_intersects, int32_t tile_bound_x,
                                       int32_t tile_bound_y, int32_t block_x, int32_t block_y,
                                       int64_t* isect_ids, int32_t* gaussian_ids,
                                       hipStream_t stream) {
    if (n < 0 || num_intersects < 0 || tile_bound_x <= 0 || tile_bound_y <= 0 || block_x <= 0 ||
        block_y <= 0)
        return CS_ERR_ARGS;
    if (n == 0 || num_intersects == 0) return CS_OK;
    hipLaunchKernelGGL(k_gs_map_ref, dim3(gs_blocks(n)), dim3(kGsThreads), 0, stream, xys, conics,
                       depths, radii, cum_tiles_hit, n, num_intersects, block_x, block_y,
                       tile_bound_x, tile_bound_y, isect_ids, gaussian_ids);
    return gs_status();
}
