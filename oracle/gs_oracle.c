/*
 * CPU restatement of the reference's 2D Gaussian splat path (the renderer
 * behind manbo/tilelang_renderer.py GsRenderFunction).
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (repo_amd/, manbo/) may
 * link, load or call this file; only tests/ use it, always as the checker.
 *
 * Arithmetic spec (shared with the HIP kernels): fp32 IEEE + - * / sqrt in
 * the reference's expression order, no implicit contraction (fmaf only where
 * written), exp = cs_expf (cs_oracle.c), sin/cos = orc_sincosf below (the same
 * function as the GPU's spec_sincosf), float->int truncating and saturating.
 * The raster's quadratic form and colour sums follow the spec forms written
 * at gs_sigma and orc_gs_raster_forward.  Forward outputs are therefore
 * bit-identical; gradient sums accumulate in double here.
 *
 * Reference files followed (under /root/reference/manbo/ops/):
 *   forward2d.py:14-164   project_gaussians_2d_scale_rot_forward_kernel -> orc_gs_project
 *   intersects.py:12-121  map_gaussian_to_intersects_kernel (tile rectangle) -> orc_gs_rects
 *   rasterize.py:18-157   rasterize_forward_kernel  -> orc_gs_raster_forward
 *   rasterize.py:160-529  rasterize_backward_kernel -> orc_gs_raster_backward
 *   backward2d.py:8-151   project_gaussians_2d_scale_rot_backward_kernel -> orc_gs_project_backward
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

float cs_expf(float x);

/* The spec sin/cos (three-part Cody-Waite reduction by pi/2 with fmaf, Cephes
 * single-precision polynomials on |r| <= pi/4). */
void orc_sincosf(float x, float *sn, float *cs)
{
    if (!(x - x == 0.0f)) {
        *sn = x - x;
        *cs = x - x;
        return;
    }
    const float kf = rintf(x * 0.636619746685028076171875f);
    float r = fmaf(kf, -1.57079637050628662109375f, x);
    r = fmaf(kf, 4.37113882867379300296306610107421875e-08f, r);
    r = fmaf(kf, 1.77635683940025046467781066894531250e-15f, r);
    const float z = r * r;
    float ps = fmaf(-1.9515295891e-4f, z, 8.3321608736e-3f);
    ps = fmaf(ps, z, -1.6666654611e-1f);
    const float s = fmaf(ps * z, r, r);
    float pc = fmaf(2.443315711809948e-5f, z, -1.388731625493765e-3f);
    pc = fmaf(pc, z, 4.166664568298827e-2f);
    const float c = fmaf(pc * z, z, fmaf(-0.5f, z, 1.0f));
    const int q = (int)kf & 3;
    *sn = q == 0 ? s : q == 1 ? c : q == 2 ? -s : -c;
    *cs = q == 0 ? c : q == 1 ? -s : q == 2 ? -c : s;
}

void orc_sincosf_n(const float *x, int32_t n, float *sn, float *cs)
{
    for (int32_t i = 0; i < n; ++i) orc_sincosf(x[i], sn + i, cs + i);
}

static inline int32_t gs_f2i(float x)
{
    if (!(x == x)) return 0;
    if (x >= 2147483648.0f) return INT32_MAX;
    if (x < -2147483648.0f) return INT32_MIN;
    return (int32_t)x;
}

static inline int32_t gs_clampi(int32_t v, int32_t lo, int32_t hi)
{
    return v < lo ? lo : (v > hi ? hi : v);
}

#define GS_ANISO 3.0f
#define GS_CONIC_EPS ((float)1e-12)

/* Tile rectangle of a Gaussian from its centre, conic and radius
 * (forward2d.py:97-151 and intersects.py:42-95, identical expressions). */
static void gs_rect(float cx, float cy, float qxx, float qxy, float qyy, float radius,
                    int32_t block_x, int32_t block_y, int32_t tbx, int32_t tby, int32_t r[4])
{
    const float q_det = qxx * qyy - qxy * qxy;
    float rx = radius, ry = radius;
    if (qxx > 0.0f && qyy > 0.0f && q_det > GS_CONIC_EPS) {
        rx = GS_ANISO * sqrtf(qyy / q_det);
        ry = GS_ANISO * sqrtf(qxx / q_det);
    }
    const float tcx = cx / (float)block_x, tcy = cy / (float)block_y;
    const float trx = rx / (float)block_x, try_ = ry / (float)block_y;
    r[0] = gs_clampi(gs_f2i(tcx - trx), 0, tbx);
    r[2] = gs_clampi(gs_f2i(tcx + trx + 1.0f), 0, tbx);
    r[1] = gs_clampi(gs_f2i(tcy - try_), 0, tby);
    r[3] = gs_clampi(gs_f2i(tcy + try_ + 1.0f), 0, tby);
}

/* project_gaussians_2d_scale_rot_forward_kernel (forward2d.py:14-164). */
void orc_gs_project(const float *means, const float *scales, const float *rot, int32_t n,
                    int32_t img_h, int32_t img_w, int32_t block_x, int32_t block_y,
                    float *xys, float *depths, int32_t *radii, float *conics,
                    int32_t *num_tiles_hit)
{
    const int32_t tbx = (img_w + block_x - 1) / block_x, tby = (img_h + block_y - 1) / block_y;
    const float ox = 0.5f * (float)img_w, oy = 0.5f * (float)img_h;
    for (int32_t i = 0; i < n; ++i) {
        const float mx = means[2 * i], my = means[2 * i + 1];
        const float sx = scales[2 * i], sy = scales[2 * i + 1];
        const float cx = ox * mx + ox, cy = oy * my + oy;
        float sr, cr;
        orc_sincosf(rot[i], &sr, &cr);
        const float m00 = cr * sx, m01 = sr * sy, m10 = -sr * sx, m11 = cr * sy;
        const float cxx = m00 * m00 + m01 * m01;
        const float cxy = m00 * m10 + m01 * m11;
        const float cyy = m10 * m10 + m11 * m11;
        const float det = cxx * cyy - cxy * cxy;
        float o[3] = {0.0f, 0.0f, 0.0f}, px = 0.0f, py = 0.0f;
        int32_t rad = 0, tiles = 0;
        if (det != 0.0f) {
            const float inv_det = 1.0f / det;
            const float qx = cyy * inv_det, qy = -cxy * inv_det, qz = cxx * inv_det;
            const float b = 0.5f * (cxx + cyy);
            const float delta = fmaxf(0.1f, b * b - det);
            const float sd = sqrtf(delta);
            const float v1 = b + sd, v2 = b - sd;
            const float radius = ceilf(3.0f * sqrtf(fmaxf(v1, v2)));
            int32_t r[4];
            gs_rect(cx, cy, qx, qy, qz, radius, block_x, block_y, tbx, tby, r);
            const int32_t area = (r[2] - r[0]) * (r[3] - r[1]);
            if (area > 0) {
                px = cx;
                py = cy;
                o[0] = qx;
                o[1] = qy;
                o[2] = qz;
                rad = gs_f2i(radius);
                tiles = area;
            }
        }
        xys[2 * i] = px;
        xys[2 * i + 1] = py;
        depths[i] = 0.0f;
        radii[i] = rad;
        conics[3 * i] = o[0];
        conics[3 * i + 1] = o[1];
        conics[3 * i + 2] = o[2];
        num_tiles_hit[i] = tiles;
    }
}

/* The tile rectangle map_gaussian_to_intersects_kernel emits for each
 * Gaussian (intersects.py:34-121): empty (0,0,0,0) when radius <= 0 or the
 * area is not positive. */
void orc_gs_rects(const float *xys, const float *conics, const int32_t *radii, int32_t n,
                  int32_t block_x, int32_t block_y, int32_t tbx, int32_t tby, int32_t *rects)
{
    for (int32_t i = 0; i < n; ++i) {
        int32_t r[4] = {0, 0, 0, 0};
        if (radii[i] > 0) {
            gs_rect(xys[2 * i], xys[2 * i + 1], conics[3 * i], conics[3 * i + 1],
                    conics[3 * i + 2], (float)radii[i], block_x, block_y, tbx, tby, r);
            if ((r[2] - r[0]) * (r[3] - r[1]) <= 0) r[0] = r[1] = r[2] = r[3] = 0;
        }
        memcpy(rects + 4 * i, r, sizeof(r));
    }
}

/* The spec's per-pixel quadratic form.  The reference evaluates
 * 0.5 (qxx dx^2 + qyy dy^2) + qxy dx dy (rasterize.py:111-114); the spec
 * halves qxx and qyy once per Gaussian (a, c) and evaluates
 * dx (a dx + b dy) + c dy^2 with two fmaf, the same quadratic form. */
static inline float gs_sigma(const float *xy, const float *q, float px, float py, float *dx,
                             float *dy)
{
    const float a = 0.5f * q[0], b = q[1], c = 0.5f * q[2];
    *dx = xy[0] - px;
    *dy = xy[1] - py;
    return fmaf(*dx, fmaf(a, *dx, b * *dy), (c * *dy) * *dy);
}

#define GS_ALPHA_MIN ((float)(1.0 / 255.0))

/* rasterize_forward_kernel (rasterize.py:18-157), pixel rows [row0, row1):
 * pixel (i, j) at (px, py) = (j, i) walks its tile's list in order, skips
 * sigma < 0 and alpha = min(0.999, o exp(-sigma)) < 1/255, composites
 * front to back and stops after the entry that takes T to 1e-4 or below.
 * Colour sums and the background term use fmaf (spec). */
void orc_gs_raster_forward(const int32_t *ids, const int32_t *bins, const float *xys,
                           const float *conics, const float *colors, const float *opac,
                           const float *bg, int32_t img_h, int32_t img_w, int32_t block_x,
                           int32_t block_y, int32_t row0, int32_t row1, float *out,
                           float *final_T, int32_t *final_idx)
{
    const int32_t tbx = (img_w + block_x - 1) / block_x;
    (void)img_h;
    for (int32_t i = row0; i < row1; ++i) {
        for (int32_t j = 0; j < img_w; ++j) {
            const int32_t tile = (i / block_y) * tbx + j / block_x;
            const int32_t g0 = bins[2 * tile], g1 = bins[2 * tile + 1];
            const float px = (float)j, py = (float)i;
            float T = 1.0f, c0 = 0.0f, c1 = 0.0f, c2 = 0.0f;
            int32_t cur = 0;
            for (int32_t e = g0; e < g1; ++e) {
                const int32_t g = ids[e];
                float dx, dy;
                const float sigma = gs_sigma(xys + 2 * g, conics + 3 * g, px, py, &dx, &dy);
                if (sigma < 0.0f) continue;
                const float alpha = fminf((float)0.999, opac[g] * cs_expf(-sigma));
                if (alpha < GS_ALPHA_MIN) continue;
                const float nT = T * (1.0f - alpha);
                const float vis = alpha * T;
                c0 = fmaf(colors[3 * g], vis, c0);
                c1 = fmaf(colors[3 * g + 1], vis, c1);
                c2 = fmaf(colors[3 * g + 2], vis, c2);
                T = nT;
                cur = e;
                if (nT <= (float)1e-4) break;
            }
            const size_t p = (size_t)i * img_w + j;
            final_T[p] = T;
            final_idx[p] = cur;
            out[3 * p] = fmaf(T, bg[0], c0);
            out[3 * p + 1] = fmaf(T, bg[1], c1);
            out[3 * p + 2] = fmaf(T, bg[2], c2);
        }
    }
}

/* rasterize_backward_kernel (rasterize.py:160-529), pixel rows [row0, row1),
 * per-pixel terms in fp32 as the reference forms them, sums in double:
 * v_xy [N,2], v_conic [N,3], v_rgb [N,3], v_opacity [N] (zeroed by the
 * caller), optional contrib_rgb [N,3] and isect_contrib [I].  v_out_alpha
 * NULL reads as zeros; meta (per intersection) NULL enables every
 * intersection's geometry gradients.  The alpha cap is 0.99 here (the
 * forward's is 0.999), as in the reference. */
void orc_gs_raster_backward(const int32_t *ids, const int32_t *meta, const int32_t *bins,
                            const float *xys, const float *conics, const float *colors,
                            const float *opac, const float *bg, int32_t img_h, int32_t img_w,
                            int32_t block_x, int32_t block_y, int32_t row0, int32_t row1,
                            const float *final_T, const int32_t *final_idx, const float *v_out,
                            const float *v_out_alpha, double *v_xy, double *v_conic,
                            double *v_rgb, double *v_opacity, double *contrib_rgb,
                            double *isect_contrib)
{
    const int32_t tbx = (img_w + block_x - 1) / block_x;
    (void)img_h;
    for (int32_t i = row0; i < row1; ++i) {
        for (int32_t j = 0; j < img_w; ++j) {
            const int32_t tile = (i / block_y) * tbx + j / block_x;
            const int32_t g0 = bins[2 * tile], g1 = bins[2 * tile + 1];
            const size_t p = (size_t)i * img_w + j;
            const float px = (float)j, py = (float)i;
            float T = final_T[p];
            const float T_final = T;
            const int32_t fidx = final_idx[p];
            const float v0 = v_out[3 * p], v1 = v_out[3 * p + 1], v2 = v_out[3 * p + 2];
            const float va_out = v_out_alpha ? v_out_alpha[p] : 0.0f;
            const float bg_dot = bg[0] * v0 + bg[1] * v1 + bg[2] * v2;
            float b0 = 0.0f, b1 = 0.0f, b2 = 0.0f;
            for (int32_t e = (g1 - 1 < fidx ? g1 - 1 : fidx); e >= g0; --e) {
                const int32_t g = ids[e];
                const float *q = conics + 3 * g;
                float dx, dy;
                const float sigma = gs_sigma(xys + 2 * g, q, px, py, &dx, &dy);
                if (sigma < 0.0f) continue;
                const float vis = cs_expf(-sigma);
                const float o = opac[g];
                const float alpha = fminf((float)0.99, o * vis);
                if (alpha < GS_ALPHA_MIN) continue;
                const float ra = 1.0f / (1.0f - alpha);
                T = T * ra;
                const float fac = alpha * T;
                const float *rgb = colors + 3 * g;
                v_rgb[3 * g] += (double)(fac * v0);
                v_rgb[3 * g + 1] += (double)(fac * v1);
                v_rgb[3 * g + 2] += (double)(fac * v2);
                const double c0 = (double)(fac * rgb[0]), c1 = (double)(fac * rgb[1]),
                             c2 = (double)(fac * rgb[2]);
                if (contrib_rgb) {
                    contrib_rgb[3 * g] += c0;
                    contrib_rgb[3 * g + 1] += c1;
                    contrib_rgb[3 * g + 2] += c2;
                }
                if (isect_contrib) isect_contrib[e] += c0 + c1 + c2;
                float v_alpha = (rgb[0] * T - b0 * ra) * v0;
                v_alpha = v_alpha + (rgb[1] * T - b1 * ra) * v1;
                v_alpha = v_alpha + (rgb[2] * T - b2 * ra) * v2;
                v_alpha = v_alpha + T_final * ra * (va_out - bg_dot);
                b0 += rgb[0] * fac;
                b1 += rgb[1] * fac;
                b2 += rgb[2] * fac;
                v_opacity[g] += (double)(vis * v_alpha);
                if (!meta || meta[e] != 0) {
                    const float v_sigma = -o * vis * v_alpha;
                    v_conic[3 * g] += (double)(0.5f * v_sigma * dx * dx);
                    v_conic[3 * g + 1] += (double)(0.5f * v_sigma * dx * dy);
                    v_conic[3 * g + 2] += (double)(0.5f * v_sigma * dy * dy);
                    v_xy[2 * g] += (double)(v_sigma * (q[0] * dx + q[1] * dy));
                    v_xy[2 * g + 1] += (double)(v_sigma * (q[1] * dx + q[2] * dy));
                }
            }
        }
    }
}

/* project_gaussians_2d_scale_rot_backward_kernel (backward2d.py:8-151) in
 * double from fp32 inputs: v_cov2d [N,3], v_mean2d [N,2], v_scale [N,2],
 * v_rot [N]. */
void orc_gs_project_backward(const float *scales, const float *rot, const int32_t *radii,
                             const float *conics, const double *v_xy, const double *v_conic,
                             const int32_t *meta, int32_t n, int32_t img_h, int32_t img_w,
                             double *v_cov2d, double *v_mean2d, double *v_scale, double *v_rot)
{
    for (int32_t i = 0; i < n; ++i) {
        double *vc = v_cov2d + 3 * i;
        vc[0] = vc[1] = vc[2] = 0.0;
        v_mean2d[2 * i] = v_mean2d[2 * i + 1] = 0.0;
        v_scale[2 * i] = v_scale[2 * i + 1] = 0.0;
        v_rot[i] = 0.0;
        if (radii[i] <= 0) continue;
        const double c0 = conics[3 * i], c1 = conics[3 * i + 1], c2 = conics[3 * i + 2];
        /* tilelang_renderer.py:111-116: v_xy, v_conic scaled by the meta flag. */
        const double keep = meta ? (double)(float)meta[i] : 1.0;
        const double g0 = v_conic[3 * i] * keep, g1 = v_conic[3 * i + 1] * keep,
                     g2 = v_conic[3 * i + 2] * keep;
        const double h00 = c0 * g0 + c1 * g1, h01 = c0 * g1 + c1 * g2;
        const double h10 = c1 * g0 + c2 * g1, h11 = c1 * g1 + c2 * g2;
        const double g11 = -(h00 * c0 + h01 * c1);
        const double g12 = -(h10 * c0 + h11 * c1) - (h00 * c1 + h01 * c2);
        const double g22 = -(h10 * c1 + h11 * c2);
        vc[0] = g11;
        vc[1] = g12;
        vc[2] = g22;
        float sf, cf;
        orc_sincosf(rot[i], &sf, &cf);
        const double s = sf, c = cf, sx = scales[2 * i], sy = scales[2 * i + 1];
        v_scale[2 * i] = g11 * (2 * sx * c * c) + 2 * g12 * (-2 * sx * s * c) + g22 * (2 * sx * s * s);
        v_scale[2 * i + 1] = g11 * (2 * sy * s * s) + 2 * g12 * (2 * sy * c * s) + g22 * (2 * sy * c * c);
        const double m00 = c * sx, m01 = s * sy, m10 = -s * sx, m11 = c * sy;
        const double a00 = -s * sx, a01 = c * sy, a10 = -c * sx, a11 = -s * sy;
        const double t1_00 = a00 * m00 + a01 * m01, t1_10 = a10 * m00 + a11 * m01,
                     t1_11 = a10 * m10 + a11 * m11;
        const double b00 = m00 * sx, b01 = m01 * sy, b10 = m10 * sx, b11 = m11 * sy;
        const double t2_00 = b00 * -s + b01 * c, t2_10 = b10 * -s + b11 * c,
                     t2_11 = b10 * -c + b11 * -s;
        v_rot[i] = g11 * (t1_00 + t2_00) + 2 * g12 * (t1_10 + t2_10) + g22 * (t1_11 + t2_11);
        v_mean2d[2 * i] = v_xy[2 * i] * keep * (0.5 * (double)img_w);
        v_mean2d[2 * i + 1] = v_xy[2 * i + 1] * keep * (0.5 * (double)img_h);
    }
}
