// Shared device-side definitions for the CubicSplat MI355X kernels (gfx950,
// wave64).  Every floating-point expression below is part of the arithmetic
// spec that the CPU oracle also follows: IEEE-rounded + - * / sqrt, no
// implicit contraction (the library is built with -ffp-contract=off), fused
// multiply-adds only where fmaf() is written out.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cs {

constexpr int kWave = 64;
constexpr int kTile = 16;            // 16x16 pixel tiles, one workgroup each
// Raster launch shape: two pixels per lane (rows r and r + 4 of one column),
// so a wave owns 8 tile rows and a tile is two waves.
constexpr int kPix = 2;
constexpr int kWaveRows = 4 * kPix;
constexpr int kRasterThreads = kTile * kTile / kPix;
static_assert(kPix == 2, "the backward's segment-leader walk assumes two pixels per lane");

// Constants the reference writes as Python floats, rounded once from double.
constexpr float kEps = (float)1e-6;
constexpr float kAlphaCap = (float)0.999;
constexpr float kAlphaMin = (float)(1.0 / 255.0);
constexpr float kTStop = (float)1e-4;
constexpr float kWidthMin = (float)1e-4;

// Integer cull ranges.  A range holds every pixel index k (column or row)
// whose centre k + 0.5 can matter, widened by one pixel beyond its fp32 bound,
// so integer tests on it are conservative.  It is stored as (lo, span) with
// span = hi - lo + ext, where ext + 1 is the wave's extent along that axis
// (16 columns, kWaveRows rows): [lo, hi] then meets the wave's [last - ext, last]
// exactly when 0 <= last - lo <= span, which span_hits tests with one OR and a
// sign check (no unpacking).  An empty range has span < ext.
constexpr int kWaveColsExt = kTile - 1;      // a wave spans 16 columns
constexpr int kWaveRowsExt = kWaveRows - 1;  // and kWaveRows rows
constexpr int32_t kRangeLimit = 1 << 20;

__device__ __forceinline__ bool span_hits(int32_t lo, int32_t span, int32_t last) {
    const int32_t t = last - lo;
    return (t | (span - t)) >= 0;
}

// One flattened polyline edge, 32 bytes: endpoints, direction v = p1 - p0 and
// u = v / max(|v|^2, eps) (multiply by the correctly rounded reciprocal).
struct alignas(16) EdgeRec {
    float x0, y0, x1, y1;
    float vx, vy, ux, uy;
};

// The cull ranges of one edge, 16 bytes, each range packed as two int16
// (low half lo, high half span): near rows, crossing rows (exactly the rows k
// whose centre k + 0.5 lies in [min(y0, y1), max(y0, y1)), the rows where the
// +x ray crossing test can count the edge; a subset of the near rows), near
// columns, then flags.  Kept apart from the geometry so that the forward reads only
// geometry and the backward reads the ranges of a whole primitive with one
// vector load.  Packing limits pixel indices to int16, so images are at most
// kMaxImageDim on a side.
struct alignas(16) EdgeCull {
    int32_t ny, cy, nx, flags;
};

// EdgeCull.flags bit: the edge's x coordinates lie within +-kFarCrossMaxX, so
// for any wave whose near columns it misses, the sign of its crossing cross
// product is decided by geometry alone.  Such an edge lies at least D + 1 >=
// 1.25 px (D >= 0.25 px) horizontally from every pixel of the wave, on one
// side: |cr| = |vy| |x_c - px| >= 1.25 |vy|, while the fp32 evaluation of cr
// = fma(wy, vx, -(wx vy)) differs from the exact value by at most
// 2^-24 |vy| (2 |wx| + |vx|) (|wy| <= |vy| on a crossing row), which stays
// below 1.25 |vy| for |x| <= 2^20 and pixel centres below 16384.  Its term is
// then +1 / -1 on every row it spans when it lies right of the wave and 0
// when it lies left, exactly as the per-pixel test evaluates it.
constexpr int32_t kCullFarCrossExact = 1;
// EdgeCull.flags bit: y1 > y0, so the edge's crossings count +1 (else -1).
constexpr int32_t kCullUp = 2;
constexpr float kFarCrossMaxX = 1048576.0f;
constexpr int kMaxImageDim = 16384;

__device__ __forceinline__ int32_t pack_lo_span(int32_t lo, int32_t span) {
    return (int32_t)(((uint32_t)span << 16) | ((uint32_t)lo & 0xffffu));
}
__device__ __forceinline__ int32_t packed_lo(int32_t v) { return (int32_t)(v << 16) >> 16; }
__device__ __forceinline__ int32_t packed_span(int32_t v) { return v >> 16; }

// Per-edge record of the adaptive (de Casteljau) flattening, 16 bytes: the
// edge's cubic segment and the parameter interval [t0, t1] of the leaf cubic
// it is the chord of (cubic_splatting.py:1812-1828).  The backward folds an
// edge's endpoint gradients into its segment's control points with the
// Bernstein weights at t0 and t1 (cubic_splatting.py:2432-2485).
struct alignas(16) EdgeAux {
    int32_t seg;
    float t0, t1;
    int32_t pad;
};

// Raster log (forward -> backward).  For every (list entry g, wave of tile
// rows) the forward processes, log_index[2 g + wave] holds one of
//   >= 0          the record's position in the log pool, in 16-byte units;
//   kLogEmpty     no pixel of the wave is inside the primitive or within its
//                 exact-coverage distance: the entry contributes nothing;
//   kLogMissing   not recorded (the pool was full): the backward recomputes
//                 the entry's geometry with the forward's edge walk;
//   kLogInside    every pixel of the wave is inside the fill and farther than
//                 the cull distance from its edges (coverage 1, no record).
// A record is a header (the per-pixel inside bits of the winding test, zero
// for strokes, and the exact bits of the live pixels whose coverage needs the
// exact distance, each as one 64-bit lane mask per pixel row of the lanes)
// followed by one (best edge, coverage bits) pair per exact pixel, packed in
// lane order: the exact pixels of row 0, then those of row 1.  The pool's
// first 16 bytes hold the number of 16-byte units reserved so far (starting
// at 1); each wave reserves kLogBlockUnits at a time with one atomic and
// fills its block in order.
constexpr int32_t kLogEmpty = -1;
constexpr int32_t kLogMissing = -2;
constexpr int32_t kLogInside = -3;   // every pixel inside, none near an edge
constexpr uint32_t kLogHeaderUnits = 2;
constexpr uint32_t kLogBlockUnits = 128;     // 2 KiB; a record is at most 66 units
constexpr uint32_t kLogMaxUnits = 1u << 31;  // pool capacity limit (32 GiB)

struct alignas(16) LogHeader {
    uint32_t inside[2 * kPix];
    uint32_t exact[2 * kPix];
};

// Per cubic segment: the unions of its edges' ranges, plus the last pixel
// column that can lie left of one of its vertices (for open chains).
struct alignas(16) SegRec {
    int32_t ny_lo, ny_span, cy_lo, cy_span;
    int32_t nx_lo, nx_span, x_last, pad;
};

// Per-primitive raster record, built once per forward.
struct alignas(16) PrimRec {
    float r, g, b, opacity;
    float inv_sigma2;   // max(inv_sigma2, eps)
    float inv_sigma;    // sqrt(max(inv_sigma2, eps))
    float half_sw;      // stroke half width max(0, sw) / 2 (0 for fill)
    float cull_d;       // beyond this distance a pixel's result does not depend on it
    int32_t e0, e1;     // edge range (all edges of the primitive's segments)
    int32_t rule;       // 0 even-odd, else nonzero (fill)
    int32_t closed;     // 1 if the edge chain is closed
    int32_t ny_lo, ny_span, cy_lo, cy_span;  // unions over the segments
    int32_t nx_lo, nx_span, x_last;
    float cull_out;     // the same for pixels outside a fill (alpha < 1/255 beyond it)
};

// Read-only data for the raster kernels, reached through the constant address
// space so that wave-uniform loads compile to scalar (SMEM) loads even in
// kernels that also issue global atomics.
// (The host pass that parses the kernels has no address spaces.)
#if defined(__HIP_DEVICE_COMPILE__)
#define CS_CONST __attribute__((address_space(4)))
#else
#define CS_CONST
#endif
template <class T>
using cptr = const CS_CONST T*;
template <class T>
__device__ __forceinline__ cptr<T> as_const(const T* p) {
    return (cptr<T>)p;
}

// exp(x): n = rint(x log2 e), r = x - n ln2 (two-part Cody-Waite), e^r by a
// degree-7 Taylor polynomial in Horner form, scaled by 2^n in two exact steps.
__device__ __forceinline__ float spec_expf(float x) {
    if (!(x == x)) return x;
    if (x > 88.72283935546875f) return __builtin_huge_valf();
    if (x < -103.97208404541015625f) return 0.0f;
    const float kf = __builtin_rintf(x * 1.44269502162933349609375f);
    float r = __builtin_fmaf(kf, -0.693145751953125f, x);
    r = __builtin_fmaf(kf, -1.428606765330187045037746429443359375e-06f, r);
    float p = 1.98412698412698e-04f;
    p = __builtin_fmaf(p, r, 1.38888888888889e-03f);
    p = __builtin_fmaf(p, r, 8.33333333333333e-03f);
    p = __builtin_fmaf(p, r, 4.16666666666667e-02f);
    p = __builtin_fmaf(p, r, 1.66666666666667e-01f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    const int k = (int)kf;
    const int k1 = k >> 1;
    const int k2 = k - k1;
    const float s1 = __builtin_bit_cast(float, (uint32_t)(k1 + 127) << 23);
    const float s2 = __builtin_bit_cast(float, (uint32_t)(k2 + 127) << 23);
    return (p * s1) * s2;
}

// spec_expf for |x| <= 87: the same reduction and polynomial, without the
// NaN and range tests, and the final scaling by 2^k as one ldexp, which is
// exact (and equals the two-step scaling) while p 2^k is a normal float.
__device__ __forceinline__ float spec_expf_mid(float x) {
    const float kf = __builtin_rintf(x * 1.44269502162933349609375f);
    float r = __builtin_fmaf(kf, -0.693145751953125f, x);
    r = __builtin_fmaf(kf, -1.428606765330187045037746429443359375e-06f, r);
    float p = 1.98412698412698e-04f;
    p = __builtin_fmaf(p, r, 1.38888888888889e-03f);
    p = __builtin_fmaf(p, r, 8.33333333333333e-03f);
    p = __builtin_fmaf(p, r, 4.16666666666667e-02f);
    p = __builtin_fmaf(p, r, 1.66666666666667e-01f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    return __builtin_ldexpf(p, (int)kf);
}

// Correctly rounded sqrt(x) for finite x >= 2^-96 and x = +0: the hardware
// square root (within 1 ulp) corrected by the residual of its neighbours,
// the IEEE expansion without its denormal-range scaling and special-value
// selects.  Below 2^-96 it stays within a few ulp of sqrt(x) < 2^-48.
__device__ __forceinline__ float sqrt_rn(float x) {
    const float s = __builtin_amdgcn_sqrtf(x);
    const float s_dn = __builtin_bit_cast(float, __builtin_bit_cast(int, s) - 1);
    const float s_up = __builtin_bit_cast(float, __builtin_bit_cast(int, s) + 1);
    const float r_dn = __builtin_fmaf(-s_dn, s, x);
    const float r_up = __builtin_fmaf(-s_up, s, x);
    const float t = r_dn <= 0.0f ? s_dn : s;
    return r_up > 0.0f ? s_up : t;
}

// Correctly rounded 1 / y for normal y in [1, 2^90]: the hardware reciprocal
// refined by the fused Newton steps of the IEEE division, which needs its
// operand scaling and special-value fixup only outside that range.
__device__ __forceinline__ float rcp_rn(float y) {
    const float r0 = __builtin_amdgcn_rcpf(y);
    const float r1 = __builtin_fmaf(__builtin_fmaf(-y, r0, 1.0f), r0, r0);
    const float q1 = __builtin_fmaf(__builtin_fmaf(-y, r1, 1.0f), r1, r1);
    return __builtin_fmaf(__builtin_fmaf(-y, q1, 1.0f), r1, q1);
}

// sin and cos of x in fp32: k = rint(x 2/pi), r = x - k pi/2 by a three-part
// Cody-Waite reduction with fused multiply-adds, then the single-precision
// sin/cos polynomials of the Cephes library (S. L. Moshier, sinf.c/cosf.c)
// on |r| <= pi/4 and the quadrant k mod 4.  Within 2 ulp-scale absolute error
// of the true values for |x| up to ~1e5; deterministic everywhere (NaN and
// inf give NaN).
__device__ __forceinline__ void spec_sincosf(float x, float* sn, float* cs) {
    if (!(x - x == 0.0f)) {
        *sn = x - x;
        *cs = x - x;
        return;
    }
    const float kf = __builtin_rintf(x * 0.636619746685028076171875f);
    float r = __builtin_fmaf(kf, -1.57079637050628662109375f, x);
    r = __builtin_fmaf(kf, 4.37113882867379300296306610107421875e-08f, r);
    r = __builtin_fmaf(kf, 1.77635683940025046467781066894531250e-15f, r);
    const float z = r * r;
    float ps = __builtin_fmaf(-1.9515295891e-4f, z, 8.3321608736e-3f);
    ps = __builtin_fmaf(ps, z, -1.6666654611e-1f);
    const float s = __builtin_fmaf(ps * z, r, r);
    float pc = __builtin_fmaf(2.443315711809948e-5f, z, -1.388731625493765e-3f);
    pc = __builtin_fmaf(pc, z, 4.166664568298827e-2f);
    const float c = __builtin_fmaf(pc * z, z, __builtin_fmaf(-0.5f, z, 1.0f));
    const int q = (int)kf & 3;
    *sn = q == 0 ? s : q == 1 ? c : q == 2 ? -s : -c;
    *cs = q == 0 ? c : q == 1 ? -s : q == 2 ? -c : s;
}

// Truncating float -> int32 with saturation, NaN -> 0.
__device__ __forceinline__ int32_t f2i_sat(float x) {
    if (!(x == x)) return 0;
    if (x >= 2147483648.0f) return INT32_MAX;
    if (x < -2147483648.0f) return INT32_MIN;
    return (int32_t)x;
}

// Workgroups are dispatched round-robin over the 8 XCDs (block b on XCD b % 8);
// this maps block b to tile index x * ceil-share + k so that each XCD gets a
// contiguous run of tiles and neighbouring tiles (which share input rows,
// halos or primitives) hit the same L2.  Bijective on [0, n) for any n.
__device__ __forceinline__ int xcd_tile(int b, int n) {
    const int q = n >> 3, r = n & 7;
    const int x = b & 7, k = b >> 3;
    return x * q + min(x, r) + k;
}

__device__ __forceinline__ int32_t clampi(int32_t v, int32_t lo, int32_t hi) {
    return v < lo ? lo : (v > hi ? hi : v);
}

// ------------------------------------------------------- 2D Gaussian splats

// Tile rectangle [x0, x1) x [y0, y1) of a Gaussian from its centre, conic
// (inverse covariance) and radius: the axis extents 3 sqrt(qyy / det Q),
// 3 sqrt(qxx / det Q) of a positive definite conic, else the radius
// (forward2d.py:97-151 and intersects.py:42-95 use the same expressions).
__device__ __forceinline__ int4 gs_tile_rect(float cx, float cy, float qxx, float qxy, float qyy,
                                             float radius, int block_x, int block_y, int tbx,
                                             int tby) {
    const float q_det = qxx * qyy - qxy * qxy;
    float rx = radius, ry = radius;
    if (qxx > 0.0f && qyy > 0.0f && q_det > (float)1e-12) {
        rx = 3.0f * __builtin_sqrtf(qyy / q_det);
        ry = 3.0f * __builtin_sqrtf(qxx / q_det);
    }
    const float bxf = (float)block_x, byf = (float)block_y;
    const float tcx = cx / bxf, tcy = cy / byf;
    const float trx = rx / bxf, try_ = ry / byf;
    return make_int4(clampi(f2i_sat(tcx - trx), 0, tbx), clampi(f2i_sat(tcy - try_), 0, tby),
                     clampi(f2i_sat(tcx + trx + 1.0f), 0, tbx),
                     clampi(f2i_sat(tcy + try_ + 1.0f), 0, tby));
}

// Raster record of one Gaussian, 48 bytes, read with scalar loads:
// centre, the conic's halves a = qxx / 2, c = qyy / 2 and b = qxy (so that
// sigma = a dx^2 + b dx dy + c dy^2 = dx (a dx + b dy) + c dy^2), opacity,
// the alpha cut (below), colour.
struct alignas(16) GsRec {
    float x, y, a, b, c, opac, cut, r, g, bl, pad0, pad1;
};

// Pixels with sigma > cut have opac * exp(-sigma) < 1/255 (alpha is then
// below the reference's 1/255 threshold, rasterize.py:116-117 and :371-373):
// cut = ln(255 opac) + 1/64 keeps a factor e^(-1/64) below the threshold,
// far more than the error of the logarithm, the exponential and the
// product.  Callers test !(sigma > cut), so a NaN sigma or opacity takes the
// exact path.
__device__ __forceinline__ float gs_alpha_cut(float opac) {
    return __logf(255.0f * opac) + 0.015625f;
}

__device__ __forceinline__ uint64_t ballot(bool p) { return __ballot(p); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

// DPP move with zero for out-of-row sources (row_shr) or row broadcast.
template <int CTRL, int ROW_MASK, bool ZERO_OOB>
__device__ __forceinline__ float dpp_f32(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xf,
                                           ZERO_OOB));
}

// Sum over the 64 lanes with six DPP adds; the total lands in lane 63.  Every
// lane must be active (call it outside divergent code, with non-contributing
// lanes holding 0).  row_shr 1,2,4,8 sums each 16-lane row into its lane 15;
// row_bcast:15 (rows 1,3) and row_bcast:31 (rows 2,3) combine the rows.
__device__ __forceinline__ float wave_sum_lane63(float x) {
    x += dpp_f32<0x111, 0xf, true>(x);
    x += dpp_f32<0x112, 0xf, true>(x);
    x += dpp_f32<0x114, 0xf, true>(x);
    x += dpp_f32<0x118, 0xf, true>(x);
    x += dpp_f32<0x142, 0xa, false>(x);
    x += dpp_f32<0x143, 0xc, false>(x);
    return x;
}

template <int CTRL, int ROW_MASK, bool ZERO_OOB>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROW_MASK, 0xf, ZERO_OOB);
}

// Inclusive sum over lanes 0..i in lane i, the same six DPP steps as
// wave_sum_lane63 (each lane's partial sums are its own prefix).  Every lane
// must be active.
__device__ __forceinline__ uint32_t wave_incl_scan_u32(uint32_t x) {
    x += dpp_u32<0x111, 0xf, true>(x);
    x += dpp_u32<0x112, 0xf, true>(x);
    x += dpp_u32<0x114, 0xf, true>(x);
    x += dpp_u32<0x118, 0xf, true>(x);
    x += dpp_u32<0x142, 0xa, false>(x);
    x += dpp_u32<0x143, 0xc, false>(x);
    return x;
}

// t + (t moved by `STRIDE` lanes) on the lower half of each 2*STRIDE group,
// with v_permlane16_swap / v_permlane32_swap: the swap exchanges the upper
// rows of its first register with the lower rows of its second, so swapping t
// against a zero register leaves t's lower part in the first and its upper
// part in the second, lane-aligned.  (Written as inline assembly with two
// separate in/out registers: the compiler builtin's second result is not
// reliable.  The s_nop covers the VALU-write to permlane-read hazard.)
template <int STRIDE>
__device__ __forceinline__ float row_pair_add(float t) {
    float a = t, b = 0.0f;
    if constexpr (STRIDE == 16)
        asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
    else
        asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
    return a + b;
}

// Eight sums over the 64 lanes at once (v[k] summed over lanes, k = 0..7).
// Three pairwise exchanges inside each 8-lane block (half-row mirror, xor 1,
// xor 2) each keep half of the values, so that afterwards lane b of a block
// holds the block's sum of v[reduce8_slot(b)]; a row shift by 8 and the
// permlane16/permlane32 swaps then add the eight blocks.  The result is valid
// on lanes 8..15, lane l holding the total of v[reduce8_slot(l & 7)].  26 VALU operations instead of eight
// separate wave sums; every lane must be active.
__device__ __forceinline__ int reduce8_slot(int b) {
    return 4 * ((b >> 2) & 1) + 2 * (b & 1) + ((b >> 1) & 1);
}

template <int CTRL>
__device__ __forceinline__ float dpp_all(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}

__device__ __forceinline__ float wave_reduce8(const float (&v)[8]) {
    const int b = threadIdx.x & 7;
    const bool p = (b >> 2) & 1, q = b & 1, r = (b >> 1) & 1;
    float w[4], u[2];
#pragma unroll
    for (int j = 0; j < 4; ++j) {  // half-row mirror: b <-> 7 - b
        const float keep = p ? v[j + 4] : v[j];
        const float send = p ? v[j] : v[j + 4];
        w[j] = keep + dpp_all<0x141>(send);
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {  // quad_perm [1,0,3,2]: b <-> b ^ 1
        const float keep = q ? w[j + 2] : w[j];
        const float send = q ? w[j] : w[j + 2];
        u[j] = keep + dpp_all<0xB1>(send);
    }
    const float keep = r ? u[1] : u[0];  // quad_perm [2,3,0,1]: b <-> b ^ 2
    const float send = r ? u[0] : u[1];
    float t = keep + dpp_all<0x4E>(send);
    t += dpp_f32<0x118, 0xf, true>(t);  // row_shr:8: lanes 8..15 add lanes 0..7
    t = row_pair_add<16>(t);  // rows 0+1 -> row 0, rows 2+3 -> row 2
    return row_pair_add<32>(t);  // lanes 0..31 + lanes 32..63 -> lanes 0..31
}

__device__ __forceinline__ int wave_max_i(int v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = max(v, __shfl_xor(v, off, kWave));
    return v;
}

// Squared distance from the axis-aligned rectangle [rx0,rx1]x[ry0,ry1] to the
// box [bx0,bx1]x[by0,by1] (0 when they overlap).
__device__ __forceinline__ float rect_box_d2(float rx0, float ry0, float rx1, float ry1, float bx0,
                                             float by0, float bx1, float by1) {
    const float dx = fmaxf(fmaxf(bx0 - rx1, rx0 - bx1), 0.0f);
    const float dy = fmaxf(fmaxf(by0 - ry1, ry0 - by1), 0.0f);
    return dx * dx + dy * dy;
}

}  // namespace cs
