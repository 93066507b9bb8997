// Tile binning for the cubic splat path on MI355X (gfx950).
//
// Pipeline (one forward):
//   k_project_flatten_wave  workgroup per 32 or 64 cubic segments: normalized ->
//                      pixel space, exact AABB -> padded 16x16 tile range
//                      (lane per segment), then uniform Bernstein flattening
//                      into 32-byte edge records and a per-segment vertex
//                      bounding box (lane per sample point).
//   k_prim_prep        thread per primitive: union of its segments' tile
//                      ranges, tile count, depth sort key, raster record;
//                      ranks each workgroup's 256 keys among themselves when
//                      the merge ranks the keys.
//   depth rank         stable rank of the 32-bit depth keys (ties by
//                      primitive id): all-pairs counting up to 8K
//                      primitives (in one launch with the primitive records,
//                      k_prim_prep_rank), merge of the ranked blocks by
//                      binary search up to 16K, LSD radix sort above.
//   k_tile_counts      per-tile counts of the primitives whose tile rectangle
//                      covers the tile, per row segment of 64 tiles; each
//                      segment's first slot and the total I in closed form.
//   k_tile_scatter     each tile's primitives, in rank order, into its slots;
//                      tile_bins [start, end) per tile.
//
// Listing each tile's primitives in depth-rank order yields exactly the order
// of the reference's single sort of (tile << 32 | depth_key) keys emitted
// primitive-major with a stable tie order (ties broken by primitive id).
#include "cs_common.h"
#include "../../include/cubicsplat_hip.h"

namespace cs {

static_assert(sizeof(SegRec) == CS_SEG_RECORD_BYTES, "segment record layout");

// ---------------------------------------------------------------- projection

struct SegProj {
    float px[4], py[4];
    int32_t tx0, ty0, tx1, ty1;
};

// One axis of the exact cubic AABB (cubic_splatting.py:606-688), reference op order.
__device__ __forceinline__ void axis_extent(float p0, float p1, float p2, float p3, float& mn,
                                            float& mx) {
    const float a = ((-p0 + 3.0f * p1) - 3.0f * p2) + p3;
    const float b = (3.0f * p0 - 6.0f * p1) + 3.0f * p2;
    const float c = -3.0f * p0 + 3.0f * p1;
    const float d = p0;
    float lo = fminf(p0, p3), hi = fmaxf(p0, p3);
    const float q2 = 3.0f * a, q1 = 2.0f * b, q0 = c;
    if (q2 > kEps || q2 < -kEps) {
        const float disc = q1 * q1 - 4.0f * q2 * q0;
        if (disc >= -kEps) {
            const float sd = __builtin_sqrtf(fmaxf(disc, 0.0f));
            const float inv2q2 = 1.0f / (2.0f * q2);
            const float t0 = (-q1 - sd) * inv2q2;
            const float t1 = (-q1 + sd) * inv2q2;
            if (t0 > 0.0f && t0 < 1.0f) {
                const float v = ((a * t0 + b) * t0 + c) * t0 + d;
                lo = fminf(lo, v);
                hi = fmaxf(hi, v);
            }
            if (t1 > 0.0f && t1 < 1.0f) {
                const float v = ((a * t1 + b) * t1 + c) * t1 + d;
                lo = fminf(lo, v);
                hi = fmaxf(hi, v);
            }
        }
    } else if (q1 > kEps || q1 < -kEps) {
        const float t = -q0 / q1;
        if (t > 0.0f && t < 1.0f) {
            const float v = ((a * t + b) * t + c) * t + d;
            lo = fminf(lo, v);
            hi = fmaxf(hi, v);
        }
    }
    mn = lo;
    mx = hi;
}

// cubic_splatting.py:588-745 for one segment.
__device__ __forceinline__ SegProj project_segment(const float* __restrict__ cn, float half_w,
                                                   float half_h, float half_sw, float support,
                                                   float aabb_pad, int aniso, int tbx, int tby,
                                                   float bxf, float byf) {
    SegProj r;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        r.px[k] = cn[2 * k] * half_w + half_w;
        r.py[k] = cn[2 * k + 1] * half_h + half_h;
    }
    float min_x, max_x, min_y, max_y;
    axis_extent(r.px[0], r.px[1], r.px[2], r.px[3], min_x, max_x);
    axis_extent(r.py[0], r.py[1], r.py[2], r.py[3], min_y, max_y);
    if (aniso) {
        const float cx = r.px[3] - r.px[0], cy = r.py[3] - r.py[0];
        const float chord2 = cx * cx + cy * cy;
        const float inv_chord = 1.0f / __builtin_sqrtf(fmaxf(chord2, kEps));
        const float nx = fmaxf((float)0.20, fabsf(cy) * inv_chord);
        const float ny = fmaxf((float)0.20, fabsf(cx) * inv_chord);
        const float radial = half_sw + support;
        const float pad_x = aabb_pad + radial * nx;
        const float pad_y = aabb_pad + radial * ny;
        min_x = min_x - pad_x;
        max_x = max_x + pad_x;
        min_y = min_y - pad_y;
        max_y = max_y + pad_y;
    } else {
        const float pad_i = fmaxf(aabb_pad, support);
        min_x = min_x - half_sw - pad_i;
        min_y = min_y - half_sw - pad_i;
        max_x = max_x + half_sw + pad_i;
        max_y = max_y + half_sw + pad_i;
    }
    r.tx0 = clampi(f2i_sat(min_x / bxf), 0, tbx);
    r.ty0 = clampi(f2i_sat(min_y / byf), 0, tby);
    r.tx1 = clampi(f2i_sat(max_x / bxf + 1.0f), 0, tbx);
    r.ty1 = clampi(f2i_sat(max_y / byf + 1.0f), 0, tby);
    return r;
}

// Largest p in [0, P-1] with offs[p] <= s (the primitive owning segment s).
__device__ __forceinline__ int owner_of(const int32_t* __restrict__ offs, int P, int s) {
    int lo = 0, hi = P - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (offs[mid] <= s) lo = mid; else hi = mid - 1;
    }
    return lo;
}

// owner_of for segment base + lane, where base is the first of a wave's 64
// consecutive segments; every lane of the wave must be active.  The first
// segment's owner by a 64-way search (one offset per lane per step, so
// ceil(log64 P) dependent loads instead of log2 P), then each lane counts
// the primitive boundaries at or below its segment among the next 64 offsets
// (staged in sh[64]); a lane that finds all 64 below it (runs of primitives
// without segments) searches on its own.  Offsets that are not
// non-decreasing (reported through status) give some index in [0, P).
__device__ int wave_owner(const int32_t* __restrict__ offs, int P, int base, int32_t* sh) {
    const int lane = threadIdx.x & (kWave - 1);
    int lo = 0, hi = P - 1;   // wave-uniform; the owner lies in [lo, hi]
    while (hi - lo >= kWave) {
        const int step = (hi - lo + kWave) / kWave;
        const int idx = lo + lane * step;
        const uint64_t m = __ballot(idx <= hi && offs[idx] <= base);
        lo += m ? (kWave - 1 - __builtin_clzll(m)) * step : 0;
        hi = min(hi, lo + step - 1);
    }
    {
        const int idx = lo + lane;
        const uint64_t m = __ballot(idx <= hi && offs[idx] <= base);
        lo += m ? kWave - 1 - __builtin_clzll(m) : 0;
    }
    const int bi = lo + 1 + lane;
    sh[lane] = bi < P ? offs[bi] : INT32_MAX;
    const int seg = base + lane;
    int c = 0;
#pragma unroll
    for (int step = kWave / 2; step >= 1; step >>= 1)
        if (sh[c + step - 1] <= seg) c += step;
    if (c == kWave - 1 && sh[kWave - 1] <= seg) return owner_of(offs, P, seg);
    return lo + c;
}

// Conservative distance beyond which a pixel's coverage of this primitive is
// decided without its exact distance: fill -> alpha < 1/255 outside, coverage
// exactly 1.0f inside (1 / (1 + exp(-2 d inv_sigma)) evaluated in fp32 with
// the spec exp is exactly 1 for every d inv_sigma > 8.3177, found by a scan
// in fp32 steps; 8.5 leaves a 2% margin for the rounding of d); stroke ->
// alpha < 1/255.  The 1/4 pixel absorbs fp32 rounding of the cull tests.
__device__ __forceinline__ float cull_distance(int mode, float opacity, float inv_sigma,
                                               float half_sw) {
    if (!(opacity <= 3.0e38f)) return __builtin_huge_valf();
    const float lo = __logf(fmaxf(255.0f * opacity, 1.0f));
    if (mode == 0) return fmaxf(8.5f, 0.5f * (lo + 1.0f)) / inv_sigma + 0.25f;
    return half_sw + __builtin_sqrtf(2.0f * lo + 1.0f) / inv_sigma + 0.25f;
}

// The outside part of that bound for a fill: beyond it alpha < 1/255 (o cov
// <= o exp(-2 d inv_sigma) and 2 d inv_sigma >= ln(255 o) + 1), whatever the
// inside bound needs.  For strokes every pixel is outside: the cull distance.
__device__ __forceinline__ float cull_distance_outside(int mode, float opacity, float inv_sigma,
                                                       float half_sw) {
    if (mode != 0) return cull_distance(mode, opacity, inv_sigma, half_sw);
    if (!(opacity <= 3.0e38f)) return __builtin_huge_valf();
    const float lo = __logf(fmaxf(255.0f * opacity, 1.0f));
    return 0.5f * (lo + 1.0f) / inv_sigma + 0.25f;
}

struct PrimParams {
    float inv_sigma2;  // 1 / max(w^2, eps) (cubic_splatting.py:2820-2821)
    float inv_sigma;   // sqrt(max(inv_sigma2, eps))
    float half_sw;
    float cull_d;
};

__device__ __forceinline__ PrimParams prim_params(int mode, float aa_width, float opacity,
                                                  const float* __restrict__ stroke_widths,
                                                  int p) {
    PrimParams q;
    const float w = fmaxf(aa_width, kWidthMin);
    q.inv_sigma2 = 1.0f / fmaxf(w * w, kEps);
    q.inv_sigma = __builtin_sqrtf(fmaxf(q.inv_sigma2, kEps));
    q.half_sw = (mode == 1 && stroke_widths) ? fmaxf(0.0f, stroke_widths[p]) * 0.5f : 0.0f;
    q.cull_d = cull_distance(mode, opacity, q.inv_sigma, q.half_sw);
    return q;
}

__device__ __forceinline__ int32_t px_index(float v) {
    return f2i_sat(fminf(fmaxf(v, -40000.0f), 40000.0f));
}

// Inclusive range of pixel indices k whose centre k + 0.5 can lie in
// [lo - d, hi + d], widened by one pixel on each side.
struct IRange {
    int32_t lo, hi;
};

__device__ __forceinline__ IRange pixel_range(float lo, float hi, float d) {
    return IRange{px_index(floorf(lo - d - 0.5f)) - 1, px_index(ceilf(hi + d - 0.5f)) + 1};
}

// Rows k with lo <= k + 0.5 < hi, where the crossing test y0 <= py != y1 <= py
// (py = k + 0.5) can count an edge whose y-range is [lo, hi]: k from
// ceil(lo - 0.5) to ceil(hi - 0.5) - 1.  lo - 0.5 and hi - 0.5 are exact for
// magnitudes below 2^23; larger ones clamp past every pixel row.  Empty
// (hi < lo) when lo == hi or both are NaN.
__device__ __forceinline__ IRange crossing_rows(float lo, float hi) {
    return IRange{px_index(ceilf(lo - 0.5f)), px_index(ceilf(hi - 0.5f)) - 1};
}

__device__ __forceinline__ int32_t span_x(IRange r) { return r.hi - r.lo + kWaveColsExt; }
__device__ __forceinline__ int32_t span_y(IRange r) { return r.hi - r.lo + kWaveRowsExt; }

// (lo, span) as two int16.  Indices below -2 or above kMaxImageDim + 16 meet
// no wave of an image of at most kMaxImageDim pixels, so clamping them there
// keeps every test's result.
__device__ __forceinline__ int32_t packed_range(IRange r, int ext) {
    const int lo = clampi(r.lo, -2, kMaxImageDim + 16);
    const int hi = clampi(r.hi, -2, kMaxImageDim + 16);
    return pack_lo_span(lo, hi - lo + ext);
}

// packed_range of a range that may be empty; an empty one meets no wave
// (its first row lies past every image row).
__device__ __forceinline__ int32_t packed_range_or_empty(IRange r, int ext) {
    return r.hi < r.lo ? pack_lo_span(kMaxImageDim + 16, 0) : packed_range(r, ext);
}

// torch.linspace(0, 1, S)[i] as ATen's device kernel computes it.
__device__ __forceinline__ float linspace01(int S, int i) {
    const float step = 1.0f / (float)(S - 1);
    return i < (S >> 1) ? 0.0f + step * (float)i : 1.0f - step * (float)(S - i - 1);
}

// One edge's geometry and cull records (shared by both flattenings).
__device__ __forceinline__ void write_edge(float ax, float ay, float bx, float by, float D,
                                           EdgeRec* __restrict__ er, EdgeCull* __restrict__ ec) {
    const float vx = bx - ax, vy = by - ay;
    const float vv = vx * vx + vy * vy;
    const float ivv = 1.0f / fmaxf(vv, kEps);
    const float ex0 = fminf(ax, bx), ex1 = fmaxf(ax, bx);
    const float ey0 = fminf(ay, by), ey1 = fmaxf(ay, by);
    int4* o = reinterpret_cast<int4*>(er);
    o[0] = make_int4(__builtin_bit_cast(int, ax), __builtin_bit_cast(int, ay),
                     __builtin_bit_cast(int, bx), __builtin_bit_cast(int, by));
    o[1] = make_int4(__builtin_bit_cast(int, vx), __builtin_bit_cast(int, vy),
                     __builtin_bit_cast(int, vx * ivv), __builtin_bit_cast(int, vy * ivv));
    const IRange nx = pixel_range(ex0, ex1, D), ny = pixel_range(ey0, ey1, D);
    const IRange cy = crossing_rows(ey0, ey1);
    const int32_t flags =
        ((fabsf(ax) <= kFarCrossMaxX && fabsf(bx) <= kFarCrossMaxX) ? kCullFarCrossExact : 0) |
        (ay < by ? kCullUp : 0);
    *reinterpret_cast<int4*>(ec) =
        make_int4(packed_range(ny, kWaveRowsExt), packed_range_or_empty(cy, kWaveRowsExt),
                  packed_range(nx, kWaveColsExt), flags);
}

// Bounding box of a segment's polyline vertices -> its segment record.
struct VBox {
    float x0, y0, x1, y1;
};

__device__ __forceinline__ VBox vbox_empty() {
    const float inf = __builtin_huge_valf();
    return VBox{inf, inf, -inf, -inf};
}

__device__ __forceinline__ void vbox_add(VBox& b, float x, float y) {
    b.x0 = fminf(b.x0, x);
    b.x1 = fmaxf(b.x1, x);
    b.y0 = fminf(b.y0, y);
    b.y1 = fmaxf(b.y1, y);
}

__device__ __forceinline__ SegRec seg_record(const VBox& b, float D) {
    const IRange nx = pixel_range(b.x0, b.x1, D), ny = pixel_range(b.y0, b.y1, D);
    const IRange cy = pixel_range(b.y0, b.y1, 0.0f);
    SegRec sr;
    sr.ny_lo = ny.lo;
    sr.ny_span = span_y(ny);
    sr.cy_lo = cy.lo;
    sr.cy_span = span_y(cy);
    sr.nx_lo = nx.lo;
    sr.nx_span = span_x(nx);
    sr.x_last = px_index(ceilf(b.x1 - 0.5f)) + 1;
    sr.pad = 0;
    return sr;
}

// ------------------------------------------- adaptive (de Casteljau) flattening

// Control points of one cubic in pixel space.
struct Cub {
    float x[4], y[4];
};

__device__ __forceinline__ Cub load_cub(const float* __restrict__ c) {
    Cub r;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        r.x[k] = c[2 * k];
        r.y[k] = c[2 * k + 1];
    }
    return r;
}

// cubic_adaptive_flatness_flags_kernel (cubic_splatting.py:1863-1915): the
// larger distance of the inner control points from the chord line (or, for a
// chord shorter than sqrt(1e-6), from P0) is at most tol.
__device__ __forceinline__ bool cub_flat(const Cub& c, float tol) {
    const float lx = c.x[3] - c.x[0], ly = c.y[3] - c.y[0];
    const float chord2 = lx * lx + ly * ly;
    const float chord = __builtin_sqrtf(fmaxf(chord2, kEps));
    const float v1x = c.x[1] - c.x[0], v1y = c.y[1] - c.y[0];
    const float v2x = c.x[2] - c.x[0], v2y = c.y[2] - c.y[0];
    const float cross1 = fabsf(lx * v1y - ly * v1x);
    const float cross2 = fabsf(lx * v2y - ly * v2x);
    const float dline = fmaxf(cross1 / chord, cross2 / chord);
    float dmax = dline;
    if (chord2 <= kEps) {
        const float n1 = __builtin_sqrtf(fmaxf(v1x * v1x + v1y * v1y, 0.0f));
        const float n2 = __builtin_sqrtf(fmaxf(v2x * v2x + v2y * v2y, 0.0f));
        const float n3 = __builtin_sqrtf(fmaxf(chord2, 0.0f));
        dmax = fmaxf(n1, fmaxf(n2, n3));
    }
    return dmax <= tol;
}

// cubic_split_half_kernel (cubic_splatting.py:1968-2030): halves at t = 0.5.
__device__ __forceinline__ void cub_split(const Cub& c, Cub& l, Cub& r) {
#define CS_SPLIT_AXIS(A)                                   \
    {                                                      \
        const float p01 = 0.5f * (c.A[0] + c.A[1]);        \
        const float p12 = 0.5f * (c.A[1] + c.A[2]);        \
        const float p23 = 0.5f * (c.A[2] + c.A[3]);        \
        const float p012 = 0.5f * (p01 + p12);             \
        const float p123 = 0.5f * (p12 + p23);             \
        const float p0123 = 0.5f * (p012 + p123);          \
        l.A[0] = c.A[0];                                   \
        l.A[1] = p01;                                      \
        l.A[2] = p012;                                     \
        l.A[3] = p0123;                                    \
        r.A[0] = p0123;                                    \
        r.A[1] = p123;                                     \
        r.A[2] = p23;                                      \
        r.A[3] = c.A[3];                                   \
    }
    CS_SPLIT_AXIS(x)
    CS_SPLIT_AXIS(y)
#undef CS_SPLIT_AXIS
}

// Smallest d with 2^d >= n (n >= 1): the reference's
// ceil(log2(max(1, edges_per_segment))) (cubic_splatting.py:1733).
__host__ __device__ __forceinline__ int ceil_log2(int n) {
    int d = 0;
    while ((int64_t)1 << d < (int64_t)n) ++d;
    return d;
}

// The leaves of the reference's level-by-level subdivision
// (cubic_splatting.py:1747-1781) of one cubic, visited left to right (the
// order of its (segment, t0) sort, :1801-1809): node (d, k) covers
// [k / 2^d, (k + 1) / 2^d] and is a leaf when d == maxd or it is flat.  Each
// node's control points are recomputed from the root along the bits of k, so
// they are the same fp32 values the reference's repeated halving produces,
// with no stack.  leaf(c, d, k) is called once per leaf.
template <class F>
__device__ __forceinline__ void decas_leaves(const Cub& root, int maxd, float tol, F&& leaf) {
    int d = 0;
    uint32_t k = 0;
    for (;;) {
        Cub c = root;
        for (int i = d - 1; i >= 0; --i) {
            Cub l, r;
            cub_split(c, l, r);
            c = ((k >> i) & 1u) ? r : l;
        }
        if (d >= maxd || cub_flat(c, tol)) {
            leaf(c, d, k);
            while (d > 0 && (k & 1u)) {
                k >>= 1;
                --d;
            }
            if (d == 0) break;
            k += 1;
        } else {
            ++d;
            k <<= 1;
        }
    }
}

__device__ __forceinline__ uint32_t decas_count(const Cub& c, int maxd, float tol) {
    uint32_t n = 0;
    decas_leaves(c, maxd, tol, [&](const Cub&, int, uint32_t) { ++n; });
    return n;
}

// Leaf interval [k / 2^d, (k + 1) / 2^d] (exact: the reference's repeated
// midpoints 0.5 (t0 + t1) of dyadic values).
__device__ __forceinline__ float2 leaf_interval(int d, uint32_t k) {
    const float sc = __builtin_bit_cast(float, (uint32_t)(127 - d) << 23);
    return make_float2((float)k * sc, (float)(k + 1u) * sc);
}

// Flattening point at t: ((P0 b0 + P1 b1) + P2 b2) + P3 b3 with the cubic
// Bernstein weights, the reference's evaluation order.
__device__ __forceinline__ void bezier_point(const float (&X)[4], const float (&Y)[4], float t,
                                             float& x, float& y) {
    const float omt = 1.0f - t;
    const float b0 = omt * omt * omt;
    const float b1 = 3.0f * omt * omt * t;
    const float b2 = 3.0f * omt * t * t;
    const float b3 = t * t * t;
    x = X[0] * b0;
    x = x + X[1] * b1;
    x = x + X[2] * b2;
    x = x + X[3] * b3;
    y = Y[0] * b0;
    y = y + Y[1] * b1;
    y = y + Y[2] * b2;
    y = y + Y[3] * b3;
}

__global__ __launch_bounds__(256) void k_project_flatten(
    const float* __restrict__ cubics_norm, const int32_t* __restrict__ seg_offsets, int P,
    const float* __restrict__ aa_widths, const float* __restrict__ stroke_widths,
    const float* __restrict__ opacities, int mode, int nseg, int img_h, int img_w, int block_x,
    int block_y, float aabb_pad, int aniso, int S, float* __restrict__ cubics_px,
    int32_t* __restrict__ seg_tile_ranges, SegRec* __restrict__ seg_recs,
    EdgeRec* __restrict__ edges, EdgeCull* __restrict__ culls, int adaptive_maxd,
    float adaptive_tol, uint32_t* __restrict__ leaf_counts) {
    const int s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= nseg) return;
    const int p = owner_of(seg_offsets, P, s);
    const float w = fmaxf(aa_widths[p], kWidthMin);
    const float support = fmaxf(0.0f, w * 3.0f);
    const float half_sw = stroke_widths ? fmaxf(0.0f, stroke_widths[p]) * 0.5f : 0.0f;
    const float D = prim_params(mode, aa_widths[p], opacities[p], stroke_widths, p).cull_d;
    const int tbx = (img_w + block_x - 1) / block_x, tby = (img_h + block_y - 1) / block_y;
    const SegProj r = project_segment(cubics_norm + (size_t)s * 8, 0.5f * (float)img_w,
                                      0.5f * (float)img_h, half_sw, support, aabb_pad, aniso, tbx,
                                      tby, (float)block_x, (float)block_y);
    float4* cp = reinterpret_cast<float4*>(cubics_px + (size_t)s * 8);
    cp[0] = make_float4(r.px[0], r.py[0], r.px[1], r.py[1]);
    cp[1] = make_float4(r.px[2], r.py[2], r.px[3], r.py[3]);
    reinterpret_cast<int4*>(seg_tile_ranges)[s] = make_int4(r.tx0, r.ty0, r.tx1, r.ty1);

    if (leaf_counts) {
        // Adaptive flattening: count the leaves here; k_decas_emit writes
        // them once their offsets are known.
        Cub c;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            c.x[k] = r.px[k];
            c.y[k] = r.py[k];
        }
        leaf_counts[s] = decas_count(c, adaptive_maxd, adaptive_tol);
        return;
    }

    // Flatten: pts_i = ((P0 b0 + P1 b1) + P2 b2) + P3 b3 at t_i = linspace(0,1,S)[i].
    float prevx = 0.0f, prevy = 0.0f;
    VBox box = vbox_empty();
    EdgeRec* er = edges + (size_t)s * (S - 1);
    EdgeCull* ec = culls + (size_t)s * (S - 1);
    for (int i = 0; i < S; ++i) {
        float x, y;
        bezier_point(r.px, r.py, linspace01(S, i), x, y);
        vbox_add(box, x, y);
        if (i > 0) write_edge(prevx, prevy, x, y, D, er + (i - 1), ec + (i - 1));
        prevx = x;
        prevy = y;
    }
    seg_recs[s] = seg_record(box, D);
}

// Uniform flattening for S <= 64, one workgroup of four waves per 64
// consecutive segments.  Projection: lane j of wave 0 projects segment
// base + j (owning primitive, cull distance, exact AABB, tile range), writes
// its pixel-space control points and tile range, and stages the control
// points and cull distance in LDS.  Flattening: groups of L = 2^ceil(log2 S)
// lanes take the staged segments 64 / L at a time, the four waves taking
// turns; lane i of a group evaluates point min(i, S - 1) with the expression
// of k_project_flatten, takes point i + 1 from its neighbour and writes
// edge i (consecutive lanes write consecutive records); a butterfly min/max
// over the group gives the vertex box (min/max are order-independent) and
// lane 0 writes the segment record.  Each segment is projected once, not
// once per sample.  Thread 0 of the grid also sets the status words
// (k_status_init), which the later launches of the binning update.  Same
// outputs as k_project_flatten.
constexpr int kFlattenWaves = 4;
// Segments per workgroup for L sample lanes (at most a wave: wave 0 projects
// one per lane).  With few samples per segment, 32 puts more workgroups, and
// so more of the projection's dependent loads, in flight on each CU; with
// many, the flattening's vector work dominates and 64 does it in fewer steps.
__host__ __device__ constexpr int flatten_segs(int lanes) { return lanes >= 32 ? 64 : 32; }

template <int L>
__global__ __launch_bounds__(kWave * kFlattenWaves) void k_project_flatten_wave(
    const float* __restrict__ cubics_norm, const int32_t* __restrict__ seg_offsets, int P,
    const float* __restrict__ aa_widths, const float* __restrict__ stroke_widths,
    const float* __restrict__ opacities, int mode, int nseg, int img_h, int img_w, int block_x,
    int block_y, float aabb_pad, int aniso, int S, float* __restrict__ cubics_px,
    int32_t* __restrict__ seg_tile_ranges, SegRec* __restrict__ seg_recs,
    EdgeRec* __restrict__ edges, EdgeCull* __restrict__ culls, int32_t* __restrict__ status) {
    static_assert(L >= 2 && L <= kWave && (L & (L - 1)) == 0, "group of lanes");
    constexpr int G = kWave / L;  // segments per flattening step
    __shared__ float stage[9][kWave];
    __shared__ int32_t bounds[kWave];
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        status[0] = 0;
        status[1] = 0;
        status[2] = seg_offsets[0];
        status[3] = seg_offsets[P];
    }
    const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kWave));
    const int lane = threadIdx.x & (kWave - 1);
    constexpr int kSegs = flatten_segs(L);
    static_assert(kSegs <= kWave, "one projecting lane per segment");
    const int64_t base = (int64_t)blockIdx.x * kSegs;
    const int nw = (int)min((int64_t)kSegs, (int64_t)nseg - base);
    // The projecting lane's control points are loaded before the owner search,
    // whose dependent loads they do not wait for.
    float cub[8];
    if (w == 0 && lane < nw) {
        const float* c = cubics_norm + (size_t)(base + lane) * 8;
#pragma unroll
        for (int k = 0; k < 8; ++k) cub[k] = c[k];
    }
    const int p = w == 0 ? wave_owner(seg_offsets, P, (int)base, bounds) : 0;
    if (w == 0 && lane < nw) {
        const int s = (int)base + lane;
        const float wd = fmaxf(aa_widths[p], kWidthMin);
        const float support = fmaxf(0.0f, wd * 3.0f);
        const float half_sw = stroke_widths ? fmaxf(0.0f, stroke_widths[p]) * 0.5f : 0.0f;
        const float D = prim_params(mode, aa_widths[p], opacities[p], stroke_widths, p).cull_d;
        const int tbx = (img_w + block_x - 1) / block_x, tby = (img_h + block_y - 1) / block_y;
        const SegProj r = project_segment(cub, 0.5f * (float)img_w,
                                          0.5f * (float)img_h, half_sw, support, aabb_pad, aniso,
                                          tbx, tby, (float)block_x, (float)block_y);
        float4* cp = reinterpret_cast<float4*>(cubics_px + (size_t)s * 8);
        cp[0] = make_float4(r.px[0], r.py[0], r.px[1], r.py[1]);
        cp[1] = make_float4(r.px[2], r.py[2], r.px[3], r.py[3]);
        reinterpret_cast<int4*>(seg_tile_ranges)[s] = make_int4(r.tx0, r.ty0, r.tx1, r.ty1);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            stage[k][lane] = r.px[k];
            stage[4 + k][lane] = r.py[k];
        }
        stage[8][lane] = D;
    }
    __syncthreads();
    const int g = lane / L, i = lane & (L - 1);
    const float t = linspace01(S, min(i, S - 1));
    for (int q = w * G; q < nw; q += kFlattenWaves * G) {
        const int j = q + g;
        const bool seg_ok = j < nw;
        const int jc = seg_ok ? j : nw - 1;
        float X[4], Y[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            X[k] = stage[k][jc];
            Y[k] = stage[4 + k][jc];
        }
        const float D = stage[8][jc];
        float x, y;
        bezier_point(X, Y, t, x, y);
        const float nx = __shfl_down(x, 1, L), ny = __shfl_down(y, 1, L);
        const size_t s = (size_t)base + j;
        if (seg_ok && i < S - 1)
            write_edge(x, y, nx, ny, D, edges + s * (S - 1) + i, culls + s * (S - 1) + i);
        VBox box = vbox_empty();
        vbox_add(box, x, y);
#pragma unroll
        for (int off = L / 2; off >= 1; off >>= 1) {
            box.x0 = fminf(box.x0, __shfl_xor(box.x0, off, L));
            box.x1 = fmaxf(box.x1, __shfl_xor(box.x1, off, L));
            box.y0 = fminf(box.y0, __shfl_xor(box.y0, off, L));
            box.y1 = fmaxf(box.y1, __shfl_xor(box.y1, off, L));
        }
        if (seg_ok && i == 0) seg_recs[s] = seg_record(box, D);
    }
}

// Adaptive flattening, second pass (cubic_splatting.py:1729-1832): the leaves
// of segment s, left to right, as edges seg_edge_offsets[s] + i (chord P0 ->
// P3 of leaf i) with their records, the (segment, t0, t1) aux records and the
// segment record.
__global__ __launch_bounds__(256) void k_decas_emit(
    const float* __restrict__ cubics_px, const int32_t* __restrict__ seg_offsets, int P,
    const float* __restrict__ aa_widths, const float* __restrict__ stroke_widths,
    const float* __restrict__ opacities, int mode, int nseg, int maxd, float tol,
    const int32_t* __restrict__ seg_edge_offsets, EdgeRec* __restrict__ edges,
    EdgeCull* __restrict__ culls, EdgeAux* __restrict__ aux, SegRec* __restrict__ seg_recs) {
    const int s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= nseg) return;
    const int p = owner_of(seg_offsets, P, s);
    const float D = prim_params(mode, aa_widths[p], opacities[p], stroke_widths, p).cull_d;
    const Cub root = load_cub(cubics_px + (size_t)s * 8);
    const int base = seg_edge_offsets[s];
    int i = 0;
    VBox box = vbox_empty();
    vbox_add(box, root.x[0], root.y[0]);
    decas_leaves(root, maxd, tol, [&](const Cub& c, int d, uint32_t k) {
        const int e = base + i;
        write_edge(c.x[0], c.y[0], c.x[3], c.y[3], D, edges + e, culls + e);
        const float2 t = leaf_interval(d, k);
        *reinterpret_cast<int4*>(aux + e) =
            make_int4(s, __builtin_bit_cast(int, t.x), __builtin_bit_cast(int, t.y), 0);
        vbox_add(box, c.x[3], c.y[3]);
        ++i;
    });
    seg_recs[s] = seg_record(box, D);
}

// Reference-layout adaptive flattening (_flatten_cubics_to_edges,
// cubic_splatting.py:1729-1832): leaf counts, then edges_px [E,2,2] and
// edge_t_starts / edge_t_ends [E].
__global__ __launch_bounds__(256) void k_decas_count_ref(const float* __restrict__ cubics_px,
                                                         int nseg, int maxd, float tol,
                                                         uint32_t* __restrict__ leaf_counts) {
    const int s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= nseg) return;
    leaf_counts[s] = decas_count(load_cub(cubics_px + (size_t)s * 8), maxd, tol);
}

__global__ __launch_bounds__(256) void k_decas_emit_ref(
    const float* __restrict__ cubics_px, int nseg, int maxd, float tol,
    const int32_t* __restrict__ seg_edge_offsets, float* __restrict__ edges_px,
    float* __restrict__ t_starts, float* __restrict__ t_ends) {
    const int s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= nseg) return;
    const int base = seg_edge_offsets[s];
    int i = 0;
    decas_leaves(load_cub(cubics_px + (size_t)s * 8), maxd, tol,
                 [&](const Cub& c, int d, uint32_t k) {
                     const int e = base + i;
                     reinterpret_cast<float4*>(edges_px)[e] =
                         make_float4(c.x[0], c.y[0], c.x[3], c.y[3]);
                     const float2 t = leaf_interval(d, k);
                     t_starts[e] = t.x;
                     t_ends[e] = t.y;
                     ++i;
                 });
}

// Reference-layout uniform flattening (cubic_splatting.py:1709-1719): the
// same points as k_project_flatten, edges_px [nseg * (S - 1), 2, 2].
__global__ __launch_bounds__(256) void k_bernstein_ref(const float* __restrict__ cubics_px,
                                                       int nseg, int S,
                                                       float* __restrict__ edges_px) {
    const int s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= nseg) return;
    const Cub c = load_cub(cubics_px + (size_t)s * 8);
    float prevx = 0.0f, prevy = 0.0f;
    for (int i = 0; i < S; ++i) {
        float x, y;
        bezier_point(c.x, c.y, linspace01(S, i), x, y);
        if (i > 0)
            reinterpret_cast<float4*>(edges_px)[(size_t)s * (S - 1) + i - 1] =
                make_float4(prevx, prevy, x, y);
        prevx = x;
        prevy = y;
    }
}

// primitive_edge_offsets = segment_edge_offsets[primitive_seg_offsets]
// (cubic_splatting.py:1822-1826).
__global__ __launch_bounds__(256) void k_prim_edge_offsets(const int32_t* __restrict__ seo,
                                                           const int32_t* __restrict__ offs,
                                                           int n, int nseg,
                                                           int32_t* __restrict__ out) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = seo[clampi(offs[i], 0, nseg)];
}

__global__ __launch_bounds__(256) void k_flatness_flags(const float* __restrict__ cubics, int n,
                                                        float tol, int force,
                                                        uint8_t* __restrict__ out) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    out[i] = (force || cub_flat(load_cub(cubics + (size_t)i * 8), tol)) ? 1 : 0;
}

__global__ __launch_bounds__(256) void k_split_half(const float* __restrict__ cubics, int n,
                                                    float* __restrict__ left,
                                                    float* __restrict__ right) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    Cub l, r;
    cub_split(load_cub(cubics + (size_t)i * 8), l, r);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        left[(size_t)i * 8 + 2 * k] = l.x[k];
        left[(size_t)i * 8 + 2 * k + 1] = l.y[k];
        right[(size_t)i * 8 + 2 * k] = r.x[k];
        right[(size_t)i * 8 + 2 * k + 1] = r.y[k];
    }
}

// Depth ranks of at most kRankPairsMax keys: one launch of all-pairs
// counting.  Up to kRankSortMax: the first stage ranks each block of
// kRankBlock keys among themselves (k_prim_prep does it for the cubic path,
// k_rank_blocks for the others), the second merges the blocks.
constexpr int kRankPairsMax = 8192;
constexpr int kRankSortMax = 16384;
constexpr int kRankBlock = 256;

// Position of key ki (thread t) among the 256 keys of ks in (key, index)
// order.  Slots past a block's end hold the largest key: they sit after every
// real slot, so they never precede one.
// (key, index) as one 64-bit value: lexicographic order is integer order.
__device__ __forceinline__ uint64_t key_index(uint32_t key, int index) {
    return ((uint64_t)key << 32) | (uint32_t)index;
}

__device__ __forceinline__ int rank_in_block(const uint4* ks, uint32_t ki, int t) {
    const uint64_t kt = key_index(ki, t);
    int r = 0;
#pragma unroll 16
    for (int q = 0; q < kRankBlock / 4; ++q) {
        const uint4 k4 = ks[q];
        const int j = 4 * q;
        r += (int)(key_index(k4.x, j) < kt);
        r += (int)(key_index(k4.y, j + 1) < kt);
        r += (int)(key_index(k4.z, j + 2) < kt);
        r += (int)(key_index(k4.w, j + 3) < kt);
    }
    return r;
}

// One primitive's outputs of k_prim_prep.
struct PrimPrep {
    int4 tr;           // tile rectangle
    uint32_t area;     // tiles in it
    float inv_sigma2;  // clamped width's 1 / sigma^2
    uint32_t key;      // depth key
    bool bad;          // invalid CSR offsets
    PrimRec rec;
};

// Segments whose records prim_prep_compute_at reads in one round trip.
constexpr int kPrepSegGroup = 4;

// One primitive of k_prim_prep, computed (no stores), from its CSR offsets
// s0 = seg_offsets[p], s1 = seg_offsets[p + 1] (loaded by the caller, whose
// other loads can then overlap them).  Every load depends on p only, so with
// a wave-uniform p they are scalar loads.  The segments are read
// kPrepSegGroup at a time, every load of a group issued before the first is
// used; a group's positions past the last segment repeat the last one, which
// changes none of the minima, maxima and conjunctions taken over them.
__device__ __forceinline__ PrimPrep prim_prep_compute_at(
    const float* __restrict__ cubics_norm, const int32_t* __restrict__ seg_tile_ranges,
    const SegRec* __restrict__ seg_recs, const float* __restrict__ colors,
    const float* __restrict__ opacities, const float* __restrict__ depths,
    const int32_t* __restrict__ fill_rules, const float* __restrict__ aa_widths,
    const float* __restrict__ stroke_widths, int nseg, int eps,
    const int32_t* __restrict__ seg_edge_offsets, int tbx, int tby, int mode, int p, int s0,
    int s1) {
    PrimPrep o;
    // Invalid CSR offsets are reported through status[1] and clamped so that
    // no kernel reads outside the segment arrays.
    o.bad = s0 < 0 || s1 < s0 || s1 > nseg;
    if (o.bad) {
        s0 = clampi(s0, 0, nseg);
        s1 = clampi(s1, s0, nseg);
    }
    // cubic_splatting.py:2103-2135 (the tile rectangle), and the unions of
    // the segments' ranges and the chain's closure for the raster record.
    int mnx = tbx, mny = tby, mxx = 0, mxy = 0;
    int closed = 1;
    IRange nx{kRangeLimit, -kRangeLimit}, ny = nx, cy = nx;
    int32_t x_last = -kRangeLimit;
    for (int sc = s0; sc < s1; sc += kPrepSegGroup) {
        int4 tr[kPrepSegGroup];
        SegRec sr[kPrepSegGroup];
        float2 ae[kPrepSegGroup], bs[kPrepSegGroup];
#pragma unroll
        for (int u = 0; u < kPrepSegGroup; ++u) {
            const int s = min(sc + u, s1 - 1);
            const int nxt = (s + 1 < s1) ? s + 1 : s0;
            tr[u] = reinterpret_cast<const int4*>(seg_tile_ranges)[s];
            sr[u] = seg_recs[s];
            const float* ca = cubics_norm + (size_t)s * 8;
            const float* cb = cubics_norm + (size_t)nxt * 8;
            ae[u] = make_float2(ca[6], ca[7]);
            bs[u] = make_float2(cb[0], cb[1]);
        }
#pragma unroll
        for (int u = 0; u < kPrepSegGroup; ++u) {
            mnx = min(mnx, tr[u].x); mny = min(mny, tr[u].y);
            mxx = max(mxx, tr[u].z); mxy = max(mxy, tr[u].w);
            closed &= (ae[u].x == bs[u].x) & (ae[u].y == bs[u].y);
            nx.lo = min(nx.lo, sr[u].nx_lo);
            nx.hi = max(nx.hi, sr[u].nx_lo + sr[u].nx_span - kWaveColsExt);
            ny.lo = min(ny.lo, sr[u].ny_lo);
            ny.hi = max(ny.hi, sr[u].ny_lo + sr[u].ny_span - kWaveRowsExt);
            cy.lo = min(cy.lo, sr[u].cy_lo);
            cy.hi = max(cy.hi, sr[u].cy_lo + sr[u].cy_span - kWaveRowsExt);
            x_last = max(x_last, sr[u].x_last);
        }
    }
    o.tr = make_int4(0, 0, 0, 0);
    o.area = 0;
    if (s1 > s0) {
        o.tr = make_int4(mnx, mny, mxx, mxy);
        o.area = (uint32_t)(max(0, mxx - mnx) * max(0, mxy - mny));
    }

    // cubic_splatting.py:2820-2821 (widths clamp, inv_sigma2) and the cull distance.
    const PrimParams q = prim_params(mode, aa_widths[p], opacities[p], stroke_widths, p);
    o.inv_sigma2 = q.inv_sigma2;

    // cubic_splatting.py:801-805: float order as unsigned order.
    const int32_t bits = __builtin_bit_cast(int32_t, depths[p]);
    o.key = (uint32_t)(bits ^ ((bits >> 31) | (int32_t)0x80000000));

    PrimRec& rec = o.rec;
    rec.r = colors[3 * p];
    rec.g = colors[3 * p + 1];
    rec.b = colors[3 * p + 2];
    rec.opacity = opacities[p];
    rec.inv_sigma2 = fmaxf(q.inv_sigma2, kEps);
    rec.inv_sigma = q.inv_sigma;
    rec.half_sw = q.half_sw;
    rec.cull_d = q.cull_d;
    // Edge range: uniform flattening s * eps, adaptive the segment CSR.
    rec.e0 = seg_edge_offsets ? seg_edge_offsets[s0] : s0 * eps;
    rec.e1 = seg_edge_offsets ? seg_edge_offsets[s1] : s1 * eps;
    rec.rule = fill_rules ? fill_rules[p] : 1;
    rec.closed = closed;
    rec.ny_lo = ny.lo;
    rec.ny_span = span_y(ny);
    rec.cy_lo = cy.lo;
    rec.cy_span = span_y(cy);
    rec.nx_lo = nx.lo;
    rec.nx_span = span_x(nx);
    rec.x_last = x_last;
    rec.cull_out = cull_distance_outside(mode, opacities[p], q.inv_sigma, q.half_sw);
    return o;
}

__device__ __forceinline__ PrimPrep prim_prep_compute(
    const float* __restrict__ cubics_norm, const int32_t* __restrict__ seg_offsets,
    const int32_t* __restrict__ seg_tile_ranges, const SegRec* __restrict__ seg_recs,
    const float* __restrict__ colors, const float* __restrict__ opacities,
    const float* __restrict__ depths, const int32_t* __restrict__ fill_rules,
    const float* __restrict__ aa_widths, const float* __restrict__ stroke_widths, int nseg,
    int eps, const int32_t* __restrict__ seg_edge_offsets, int tbx, int tby, int mode, int p) {
    return prim_prep_compute_at(cubics_norm, seg_tile_ranges, seg_recs, colors, opacities,
                                depths, fill_rules, aa_widths, stroke_widths, nseg, eps,
                                seg_edge_offsets, tbx, tby, mode, p, seg_offsets[p],
                                seg_offsets[p + 1]);
}

// Stores primitive p's outputs of k_prim_prep.
__device__ __forceinline__ void prim_prep_store(const PrimPrep& o, int p,
                                                int32_t* __restrict__ status,
                                                int32_t* __restrict__ prim_tile_ranges,
                                                uint32_t* __restrict__ counts,
                                                float* __restrict__ inv_sigma2s,
                                                uint32_t* __restrict__ keys,
                                                int32_t* __restrict__ vals,
                                                PrimRec* __restrict__ recs) {
    if (o.bad) atomicOr(status + 1, 1);
    reinterpret_cast<int4*>(prim_tile_ranges)[p] = o.tr;
    counts[p] = o.area;
    inv_sigma2s[p] = o.inv_sigma2;
    keys[p] = o.key;
    vals[p] = p;
    recs[p] = o.rec;
}

__global__ __launch_bounds__(256) void k_prim_prep(
    const float* __restrict__ cubics_norm, const int32_t* __restrict__ seg_offsets, int P,
    const int32_t* __restrict__ seg_tile_ranges, const SegRec* __restrict__ seg_recs,
    const float* __restrict__ colors, const float* __restrict__ opacities,
    const float* __restrict__ depths, const int32_t* __restrict__ fill_rules,
    const float* __restrict__ aa_widths, const float* __restrict__ stroke_widths, int nseg,
    int eps, const int32_t* __restrict__ seg_edge_offsets, int tbx, int tby, int mode,
    int32_t* __restrict__ status,
    int32_t* __restrict__ prim_tile_ranges, uint32_t* __restrict__ counts,
    float* __restrict__ inv_sigma2s, uint32_t* __restrict__ keys, int32_t* __restrict__ vals,
    PrimRec* __restrict__ recs, uint32_t* __restrict__ block_sorted,
    int32_t* __restrict__ block_rank) {
    static_assert(kRankBlock == 256, "one rank block per workgroup");
    const int p = blockIdx.x * blockDim.x + threadIdx.x;
    uint32_t key = 0xffffffffu;
    if (p < P) {
        const PrimPrep o = prim_prep_compute(cubics_norm, seg_offsets, seg_tile_ranges, seg_recs,
                                             colors, opacities, depths, fill_rules, aa_widths,
                                             stroke_widths, nseg, eps, seg_edge_offsets, tbx,
                                             tby, mode, p);
        prim_prep_store(o, p, status, prim_tile_ranges, counts, inv_sigma2s, keys, vals, recs);
        key = o.key;
    }
    if (block_sorted) {
        // The first stage of the depth rank (as k_rank_blocks).
        __shared__ uint4 ks[kRankBlock / 4];
        reinterpret_cast<uint32_t*>(ks)[threadIdx.x] = key;
        __syncthreads();
        if (p < P) {
            const int r = rank_in_block(ks, key, (int)threadIdx.x);
            block_sorted[blockIdx.x * kRankBlock + r] = key;
            block_rank[p] = r;
        }
    }
}

// status = [intersection total, bad-offsets flag, offs[0], offs[P]].
__global__ void k_status_init(const int32_t* __restrict__ seg_offsets, int P,
                              int32_t* __restrict__ status) {
    status[0] = 0;
    status[1] = 0;
    status[2] = seg_offsets[0];
    status[3] = seg_offsets[P];
}

// ------------------------------------------------------------ exclusive scan

constexpr int kScanThreads = 1024;
constexpr int kScanItems = 4;
constexpr int kScanItemsLarge = 16;
constexpr int kScanChunk = kScanThreads * kScanItems;

// Exclusive scan of one value per thread over a 1024-thread block; returns the
// block total in *total.
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t v, uint32_t* sh, uint32_t* total) {
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const uint32_t incl = wave_incl_scan_u32(v);
    if (lane == kWave - 1) sh[w] = incl;
    __syncthreads();
    if (w == 0) {
        const uint32_t x = lane < (kScanThreads / kWave) ? sh[lane] : 0u;
        const uint32_t xi = wave_incl_scan_u32(x);
        if (lane < (kScanThreads / kWave)) sh[lane] = xi - x;
        if (lane == kWave - 1) sh[kScanThreads / kWave] = xi;
    }
    __syncthreads();
    const uint32_t r = sh[w] + incl - v;
    *total = sh[kScanThreads / kWave];
    __syncthreads();
    return r;
}

__global__ __launch_bounds__(kScanThreads) void k_scan_block_sums(const uint32_t* __restrict__ in,
                                                                 int n,
                                                                 uint32_t* __restrict__ sums) {
    __shared__ uint32_t sh[kScanThreads / kWave + 1];
    const size_t base = (size_t)blockIdx.x * kScanChunk + (size_t)threadIdx.x * kScanItems;
    uint32_t acc = 0;
#pragma unroll
    for (int k = 0; k < kScanItems; ++k)
        if (base + k < (size_t)n) acc += in[base + k];
    uint32_t total;
    block_excl_scan(acc, sh, &total);
    if (threadIdx.x == 0) sums[blockIdx.x] = total;
}

// Single block: exclusive scan of sums[0..nb) in place (chunks with a carry).
__global__ __launch_bounds__(kScanThreads) void k_scan_partials(uint32_t* __restrict__ sums,
                                                               int nb) {
    __shared__ uint32_t sh[kScanThreads / kWave + 1];
    uint32_t carry = 0;
    for (int c0 = 0; c0 < nb; c0 += kScanThreads) {
        const int i = c0 + threadIdx.x;
        const uint32_t v = i < nb ? sums[i] : 0u;
        uint32_t total;
        const uint32_t ex = block_excl_scan(v, sh, &total);
        if (i < nb) sums[i] = carry + ex;
        carry += total;
    }
}

// Exclusive scan of in[0..n) into out, ITEMS consecutive items per thread;
// block b adds the scanned block sum.  The last block writes the grand total
// to *total_out (if given).

template <int ITEMS>
__global__ __launch_bounds__(kScanThreads) void k_scan_apply(const uint32_t* __restrict__ in,
                                                            uint32_t* __restrict__ out, int n,
                                                            const uint32_t* __restrict__ sums,
                                                            int32_t* __restrict__ total_out) {
    __shared__ uint32_t sh[kScanThreads / kWave + 1];
    const size_t base =
        (size_t)blockIdx.x * kScanThreads * ITEMS + (size_t)threadIdx.x * ITEMS;
    uint32_t v[ITEMS];
    uint32_t acc = 0;
#pragma unroll
    for (int k = 0; k < ITEMS; ++k) {
        v[k] = (base + k < (size_t)n) ? in[base + k] : 0u;
        acc += v[k];
    }
    uint32_t total;
    uint32_t ex = block_excl_scan(acc, sh, &total);
    ex += sums ? sums[blockIdx.x] : 0u;
#pragma unroll
    for (int k = 0; k < ITEMS; ++k) {
        if (base + k < (size_t)n) out[base + k] = ex;
        ex += v[k];
    }
    if (total_out && blockIdx.x == gridDim.x - 1 && threadIdx.x == kScanThreads - 1)
        *total_out = (int32_t)ex;
}

// -------------------------------------------------------- stable radix sort

constexpr int kRsThreads = 256;
constexpr int kRsItems = 16;
constexpr int kRsTile = kRsThreads * kRsItems;

__global__ __launch_bounds__(kRsThreads) void k_rs_hist(const uint32_t* __restrict__ keys, int n,
                                                       int shift, int nblk,
                                                       uint32_t* __restrict__ counts) {
    __shared__ uint32_t h[256];
    h[threadIdx.x] = 0;
    __syncthreads();
    const int base = blockIdx.x * kRsTile;
#pragma unroll 4
    for (int k = 0; k < kRsItems; ++k) {
        const int idx = base + k * kRsThreads + threadIdx.x;
        if (idx < n) atomicAdd(&h[(keys[idx] >> shift) & 0xFFu], 1u);
    }
    __syncthreads();
    counts[(size_t)threadIdx.x * nblk + blockIdx.x] = h[threadIdx.x];
}

// Stable scatter of one 8-bit digit.  Items are ranked in rounds of 256 in
// input order: within a wave by matching digits with 8 ballots, across the
// block's waves through LDS counters, across rounds by running per-digit bases.
__global__ __launch_bounds__(kRsThreads) void k_rs_scatter(
    const uint32_t* __restrict__ kin, const int32_t* __restrict__ vin,
    uint32_t* __restrict__ kout, int32_t* __restrict__ vout, int n, int shift, int nblk,
    const uint32_t* __restrict__ offsets) {
    __shared__ uint32_t dbase[256];
    __shared__ uint32_t wc[kRsThreads / kWave][256];
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    dbase[t] = offsets[(size_t)t * nblk + blockIdx.x];
    const uint64_t below = __lanemask_lt();
    const int base = blockIdx.x * kRsTile;
    for (int k = 0; k < kRsItems; ++k) {
#pragma unroll
        for (int q = 0; q < kRsThreads / kWave; ++q) wc[q][t] = 0;
        __syncthreads();
        const int idx = base + k * kRsThreads + t;
        const bool valid = idx < n;
        const uint32_t key = valid ? kin[idx] : 0u;
        const int32_t val = valid ? vin[idx] : 0;
        const uint32_t d = (key >> shift) & 0xFFu;
        uint64_t peers = __ballot(valid);
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            const bool bit = (d >> b) & 1u;
            const uint64_t m = __ballot(bit);
            peers &= bit ? m : ~m;
        }
        const uint32_t rank = (uint32_t)__popcll(peers & below);
        if (valid && rank == 0) wc[w][d] = (uint32_t)__popcll(peers);
        __syncthreads();
        if (valid) {
            uint32_t off = dbase[d] + rank;
            for (int q = 0; q < w; ++q) off += wc[q][d];
            kout[off] = key;
            vout[off] = val;
        }
        __syncthreads();
        uint32_t add = 0;
#pragma unroll
        for (int q = 0; q < kRsThreads / kWave; ++q) add += wc[q][t];
        dbase[t] += add;
    }
}

// Stable sort of up to kRankSortMax keys (ascending, ties by index) in two
// launches.  k_rank_blocks: each 256-key block ranks its keys among
// themselves in LDS (the number of block keys that are smaller, or equal with
// a smaller index) and writes the block in sorted order.  k_rank_merge: a
// workgroup takes 64 keys and holds all sorted blocks in LDS (at most
// 64 KB); its 16 waves split the other blocks and, for each, count that
// block's keys that precede the key: keys <= it in earlier blocks (smaller
// indices), keys < it in later ones, each a binary search, four searches
// interleaved.
// In-block rank plus those counts is the key's position in the stable order:
// n log(256) n / 256 comparisons instead of n^2.
constexpr int kMergeKeys = kWave;  // keys per workgroup, 64 per key group
constexpr int kMergeWaves = 16;    // waves per key group, each a 16th of the blocks
constexpr int kMergeThreads = kMergeKeys * kMergeWaves;

__device__ __forceinline__ uint32_t wave_sum_u(uint32_t v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += (uint32_t)__shfl_xor((int)v, off, kWave);
    return v;
}

__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

__global__ __launch_bounds__(kRankBlock) void k_rank_blocks(const uint32_t* __restrict__ keys,
                                                           int n,
                                                           uint32_t* __restrict__ sorted_keys,
                                                           int32_t* __restrict__ block_rank) {
    __shared__ uint4 ks[kRankBlock / 4];
    const int t = threadIdx.x;
    const int base = blockIdx.x * kRankBlock;
    const int len = min(kRankBlock, n - base);
    const uint32_t ki = t < len ? keys[base + t] : 0xffffffffu;
    reinterpret_cast<uint32_t*>(ks)[t] = ki;
    __syncthreads();
    if (t >= len) return;
    const int r = rank_in_block(ks, ki, t);
    sorted_keys[base + r] = ki;
    block_rank[base + t] = r;
}

// Keys of the sorted block at sk[base, base + len) before ki: a prefix of
// the block (<= ki when `earlier`, < ki otherwise); steps 256, 128, ..., 1
// cover every count 0..256.
__device__ __forceinline__ int count_before(const uint32_t* sk, int base, int len, uint32_t ki,
                                            bool earlier) {
    int cnt = 0;
#pragma unroll
    for (int step = kRankBlock; step >= 1; step >>= 1) {
        const int probe = cnt + step;
        const uint32_t v = sk[base + min(probe, len) - 1];
        if (probe <= len && (earlier ? v <= ki : v < ki)) cnt = probe;
    }
    return cnt;
}

// PAIRS: kout[pos] = key i, vout[pos] = vals[i]; otherwise order[pos] = i and
// rank_rects[pos] = rects[i].
template <bool PAIRS>
__global__ __launch_bounds__(kMergeThreads) void k_rank_merge(
    const uint32_t* __restrict__ keys, const uint32_t* __restrict__ sorted_keys,
    const int32_t* __restrict__ block_rank, int n, const int32_t* __restrict__ vals,
    uint32_t* __restrict__ kout, int32_t* __restrict__ vout, const int4* __restrict__ rects,
    int32_t* __restrict__ order, int4* __restrict__ rank_rects) {
    __shared__ uint32_t sk[kRankSortMax];
    {
        // All loads in flight before the first LDS store.
        constexpr int kPer = kRankSortMax / kMergeThreads;
        uint32_t v[kPer];
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const int j = k * kMergeThreads + (int)threadIdx.x;
            if (k * kMergeThreads < n) v[k] = j < n ? sorted_keys[j] : 0u;
        }
#pragma unroll
        for (int k = 0; k < kPer; ++k)
            if (k * kMergeThreads < n) sk[k * kMergeThreads + threadIdx.x] = v[k];
    }
    __syncthreads();
    const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kWave));
    const int grp = wv / kMergeWaves, w = wv - grp * kMergeWaves;
    const int lane = threadIdx.x & (kWave - 1);
    const int i = blockIdx.x * kMergeKeys + grp * kWave + lane;
    const bool ok = i < n;
    const uint32_t ki = ok ? keys[i] : 0u;
    const int own = i / kRankBlock;
    const int nblocks = (n + kRankBlock - 1) / kRankBlock;
    int cnt = 0;
    // Wave w of the group takes blocks w, w + 16, ...; four searches per step.
    for (int b0 = w; b0 < nblocks; b0 += 4 * kMergeWaves) {
        int c[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int b = b0 + u * kMergeWaves;
            const int bb = min(b, nblocks - 1);
            const int base = bb * kRankBlock;
            const int len = min(kRankBlock, n - base);
            c[u] = count_before(sk, base, len, ki, bb < own);
            if (b >= nblocks || b == own) c[u] = 0;
        }
        cnt += (c[0] + c[1]) + (c[2] + c[3]);
    }
    // The partial counts reuse the key array once every search is done.
    __syncthreads();
    int* part = reinterpret_cast<int*>(sk);
    part[(grp * kMergeWaves + w) * kWave + lane] = cnt;
    __syncthreads();
    if (w != 0 || !ok) return;
    const int* pg = part + grp * kMergeWaves * kWave + lane;
    int sum = 0;
#pragma unroll
    for (int q = 0; q < kMergeWaves; ++q) sum += pg[q * kWave];
    const int pos = block_rank[i] + sum;
    if (PAIRS) {
        kout[pos] = ki;
        vout[pos] = vals[i];
    } else {
        order[pos] = i;
        rank_rects[pos] = rects[i];
    }
}

// Stable rank by counting, one wave per key, for at most kRankPairsMax keys:
// key i's position is the number of keys that are smaller, or equal with a
// smaller index.  Lanes count over interleaved (coalesced) 4-key slices of
// the key array, which every wave reads from cache, and one wave sum gives
// the position: n^2 comparisons in one launch, the cheapest form while n is
// small.  PAIRS and the outputs as for k_rank_merge.
template <bool PAIRS>
__global__ __launch_bounds__(256) void k_rank_allpairs(
    const uint32_t* __restrict__ keys, int n, const int32_t* __restrict__ vals,
    uint32_t* __restrict__ kout, int32_t* __restrict__ vout, const int4* __restrict__ rects,
    int32_t* __restrict__ order, int4* __restrict__ rank_rects) {
    const int i = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    if (i >= n) return;
    const int lane = threadIdx.x & (kWave - 1);
    const uint32_t ki = keys[i];
    const uint64_t kt = key_index(ki, i);
    int cnt = 0;
    const int n4 = n & ~3;
    const bool vec = (reinterpret_cast<uintptr_t>(keys) & 15) == 0;
    int j0 = 0;
    if (vec) {
#pragma unroll 4
        for (j0 = 4 * lane; j0 < n4; j0 += 4 * kWave) {
            const uint4 q = *reinterpret_cast<const uint4*>(keys + j0);
            cnt += (int)(key_index(q.x, j0) < kt);
            cnt += (int)(key_index(q.y, j0 + 1) < kt);
            cnt += (int)(key_index(q.z, j0 + 2) < kt);
            cnt += (int)(key_index(q.w, j0 + 3) < kt);
        }
        j0 = n4;
    }
    for (int j = j0 + lane; j < n; j += kWave) cnt += (int)(key_index(keys[j], j) < kt);
    const int pos = wave_sum_i(cnt);
    if (lane == 0) {
        if (PAIRS) {
            kout[pos] = ki;
            vout[pos] = vals[i];
        } else {
            order[pos] = i;
            rank_rects[pos] = rects[i];
        }
    }
}

// Depth key of a float: its order as unsigned order (cubic_splatting.py:801-805),
// as prim_prep_compute computes it.
__device__ __forceinline__ uint32_t depth_key(float d) {
    const int32_t bits = __builtin_bit_cast(int32_t, d);
    return (uint32_t)(bits ^ ((bits >> 31) | (int32_t)0x80000000));
}

// k_prim_prep and k_rank_allpairs<false> in one launch, for at most
// kRankPairsMax primitives: each wave takes kPrepRankPerWave consecutive
// primitives, lane k < kPrepRankPerWave computing primitive base + k's
// records, and counts for all of them the keys that precede each one's own
// (lane-parallel over the depths, each key computed once and compared with
// every primitive's; the keys come from the depths, since no other wave's
// keys are written yet); lane k then stores its primitive's records and
// writes order[pos] = p, rank_rects[pos] = its tile rectangle.  Several
// primitives per wave read the depths that many times less often and share
// the key computation among them.
constexpr int kPrepRankPerWave = 4;

__global__ __launch_bounds__(256) void k_prim_prep_rank(
    const float* __restrict__ cubics_norm, const int32_t* __restrict__ seg_offsets, int P,
    const int32_t* __restrict__ seg_tile_ranges, const SegRec* __restrict__ seg_recs,
    const float* __restrict__ colors, const float* __restrict__ opacities,
    const float* __restrict__ depths, const int32_t* __restrict__ fill_rules,
    const float* __restrict__ aa_widths, const float* __restrict__ stroke_widths, int nseg,
    int eps, const int32_t* __restrict__ seg_edge_offsets, int tbx, int tby, int mode,
    int32_t* __restrict__ status, int32_t* __restrict__ prim_tile_ranges,
    uint32_t* __restrict__ counts, float* __restrict__ inv_sigma2s, uint32_t* __restrict__ keys,
    int32_t* __restrict__ vals, PrimRec* __restrict__ recs, int32_t* __restrict__ order,
    int4* __restrict__ rank_rects) {
    constexpr int NP = kPrepRankPerWave;
    const int base =
        (blockIdx.x * 4 + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6))) * NP;
    if (base >= P) return;
    const int lane = threadIdx.x & (kWave - 1);
    const int p = base + lane;
    const bool mine = lane < NP && p < P;
    // Lane k's CSR offsets, loaded first so that they arrive with the depths.
    int s0 = 0, s1 = 0;
    if (mine) {
        s0 = seg_offsets[p];
        s1 = seg_offsets[p + 1];
    }
    // The primitives' (key, index) values, from their depths (the key
    // prim_prep_compute_at derives); past P the largest value (never stored).
    uint64_t kp[NP];
#pragma unroll
    for (int k = 0; k < NP; ++k)
        kp[k] = base + k < P ? key_index(depth_key(depths[base + k]), base + k) : ~0ull;
    // (key, index) pairs in lexicographic order: one 64-bit comparison each.
    int cnt[NP];
#pragma unroll
    for (int k = 0; k < NP; ++k) cnt[k] = 0;
    const int n4 = P & ~3;
    const bool vec = (reinterpret_cast<uintptr_t>(depths) & 15) == 0;
    int j0 = 0;
    if (vec) {
#pragma unroll 8
        for (j0 = 4 * lane; j0 < n4; j0 += 4 * kWave) {
            const float4 d = *reinterpret_cast<const float4*>(depths + j0);
            const uint64_t e0 = key_index(depth_key(d.x), j0);
            const uint64_t e1 = key_index(depth_key(d.y), j0 + 1);
            const uint64_t e2 = key_index(depth_key(d.z), j0 + 2);
            const uint64_t e3 = key_index(depth_key(d.w), j0 + 3);
#pragma unroll
            for (int k = 0; k < NP; ++k)
                cnt[k] += (int)(e0 < kp[k]) + (int)(e1 < kp[k]) + (int)(e2 < kp[k]) +
                          (int)(e3 < kp[k]);
        }
        j0 = n4;
    }
    for (int j = j0 + lane; j < P; j += kWave) {
        const uint64_t e = key_index(depth_key(depths[j]), j);
#pragma unroll
        for (int k = 0; k < NP; ++k) cnt[k] += (int)(e < kp[k]);
    }
    int pos = 0;
#pragma unroll
    for (int k = 0; k < NP; ++k) {
        const int t = wave_sum_i(cnt[k]);
        pos = lane == k ? t : pos;
    }
    if (mine) {
        const PrimPrep o = prim_prep_compute_at(cubics_norm, seg_tile_ranges, seg_recs, colors,
                                                opacities, depths, fill_rules, aa_widths,
                                                stroke_widths, nseg, eps, seg_edge_offsets, tbx,
                                                tby, mode, p, s0, s1);
        prim_prep_store(o, p, status, prim_tile_ranges, counts, inv_sigma2s, keys, vals, recs);
        order[pos] = p;
        rank_rects[pos] = o.tr;
    }
}

// rank_rects[r] = prim_rects[order[r]] (after the radix sort of many keys).
__global__ __launch_bounds__(256) void k_gather_rects(const int32_t* __restrict__ order, int n,
                                                     const int4* __restrict__ prim_rects,
                                                     int4* __restrict__ rank_rects) {
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r < n) rank_rects[r] = prim_rects[order[r]];
}

// ------------------------------------------------------------ emit and bins

__global__ __launch_bounds__(256) void k_fill_i32(int32_t* __restrict__ a, int n, int32_t v) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) a[i] = v;
}

// Per-tile lists without a global sort.  Primitives cover rectangles of
// tiles and arrive in depth-rank order (order[r], rank_rects[r]), so the list
// of tile t is the subsequence of ranks whose rectangle contains t.  The work
// is split two ways: a row segment of up to 64 tiles, and a slab of
// consecutive ranks (list_slabs: whole 1024-rank chunks, as many slabs as
// bring the launch to about a thousand workgroups), one workgroup per (slab,
// segment), so that small and large scenes fill the GPU and every rectangle
// is still read once per segment of its rows.
//   counting launch: each rectangle of the slab that meets the segment adds
//     +1 at its first column and -1 past its last in an LDS difference array,
//     whose prefix sum is the slab's count per tile: tile_count[slab][tile].
//     The segment's first slot (the entries of all tiles before it in
//     row-major order) is a sum over the rectangles in closed form -- each
//     one's tiles in the rows above plus those left of the segment in its
//     row -- taken per slab: seg_scratch[slab][segment]; the workgroups of
//     segment 0 add their slab's areas into the total I (integer atomics,
//     exact in any order; the total starts at 0).
//   scatter launch: a tile's list starts at the segment's first slot (the
//     sum over slabs) plus the totals of the tiles before it in the segment,
//     and the slab's entries follow those of the slabs before it (the slab-0
//     workgroup writes tile_bins); then the slab's ranks in chunks of
//     kListChunk:
//     1. each wave takes a contiguous slice of the chunk and tests its
//        rectangles against the segment; the hits (primitive id and column
//        range within the segment) go to one LDS list in rank order, each
//        wave's after the hits of the slices before it;
//     2. each wave owns kListTilesPerWave tile columns and reads that list 64
//        hits at a time: per owned tile a ballot of the hits whose range
//        contains it gives, in rank order, the tile's next entries, written
//        to consecutive slots (mbcnt) of its list.  (Staging them in LDS for
//        64-wide stores measured slower.)
constexpr int kSegTiles = kWave;
constexpr int kListWaves = 8;
constexpr int kListTilesPerWave = kSegTiles / kListWaves;
constexpr int kListChunk = 1024;
constexpr int kListSlice = kListChunk / kListWaves;
constexpr int kListSteps = kListSlice / kWave;
constexpr int kMaxSlabs = 64;

// Rank slabs of the list build: nslab slabs of `slab` ranks (a multiple of
// kListChunk; the last one shorter), as many as bring the launch to about
// kListTargetGroups workgroups over the nsegs row segments (at most
// kMaxSlabs, at most one per chunk): few segments take more, shorter slabs,
// many segments fewer, longer ones (each slab's workgroup reads its ranks
// once per segment either way).
struct ListSlabs {
    int slab, nslab;
};

constexpr int kListTargetGroups = 1024;

__host__ __device__ inline ListSlabs list_slabs(int P, int nsegs) {
    const int chunks = (P + kListChunk - 1) / kListChunk;
    int want = (kListTargetGroups + nsegs - 1) / (nsegs > 0 ? nsegs : 1);
    want = want < 1 ? 1 : (want > kMaxSlabs ? kMaxSlabs : want);
    want = want > chunks ? chunks : want;
    const int per = want > 0 ? (chunks + want - 1) / want : 1;
    ListSlabs s;
    s.slab = (per > 0 ? per : 1) * kListChunk;
    s.nslab = (P + s.slab - 1) / s.slab;
    if (s.nslab < 1) s.nslab = 1;
    return s;
}

__device__ __forceinline__ uint32_t lanes_below(uint64_t m) {
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                     __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

__device__ __forceinline__ bool rect_meets_row(const int4& q, int ty, int sx0, int sx1) {
    return q.y <= ty && ty < q.w && q.x < sx1 && q.z > sx0;
}

// Tiles of rectangle q (clipped to the tbx x tby grid) that precede tile
// (sx0, ty) in row-major order: its tiles in rows above ty and those left of
// column sx0 in row ty.  `total` receives all its tiles.
__device__ __forceinline__ uint32_t rect_tiles_before(const int4& q, int ty, int sx0, int tbx,
                                                      int tby, uint32_t& total) {
    const int x0 = max(q.x, 0), x1 = min(q.z, tbx), y0 = max(q.y, 0), y1 = min(q.w, tby);
    const uint32_t wd = (uint32_t)max(0, x1 - x0);
    total = (uint32_t)max(0, y1 - y0) * wd;
    const uint32_t above = (uint32_t)max(0, min(y1, ty) - y0) * wd;
    const bool in_row = y0 <= ty && ty < y1;
    return above + (in_row ? (uint32_t)max(0, min(x1, sx0) - x0) : 0u);
}

// Workgroup b's slab, segment, tile row and segment columns [sx0, sx1).
struct ListPart {
    int slab, seg, ty, sx0, sx1;
};

__device__ __forceinline__ ListPart list_part(int nsegs, int nsegcols, int tbx) {
    ListPart q;
    q.slab = (int)blockIdx.x / nsegs;
    q.seg = (int)blockIdx.x - q.slab * nsegs;
    q.ty = q.seg / nsegcols;
    q.sx0 = (q.seg - q.ty * nsegcols) * kSegTiles;
    q.sx1 = min(q.sx0 + kSegTiles, tbx);
    return q;
}

__global__ __launch_bounds__(kWave * kListWaves) void k_tile_counts(
    const int4* __restrict__ rank_rects, int P, int tbx, int tby, int nsegcols, int slab,
    uint32_t* __restrict__ tile_count, uint32_t* __restrict__ seg_scratch,
    int32_t* __restrict__ total_out) {
    __shared__ int diff[kSegTiles + 1];
    __shared__ uint32_t part[2][kListWaves];
    const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kWave));
    const int lane = threadIdx.x & (kWave - 1);
    const int nsegs = nsegcols * tby;
    const ListPart lp = list_part(nsegs, nsegcols, tbx);
    const int rb = lp.slab * slab, re = min(P, rb + slab);
    if (threadIdx.x <= kSegTiles) diff[threadIdx.x] = 0;
    __syncthreads();
    // Sums mod 2^32, as the list positions are formed (a total beyond int32 is
    // reported by the caller).
    uint32_t before = 0, total = 0;
    for (int r0 = rb + w * kWave * kListSteps; r0 < re; r0 += kListWaves * kWave * kListSteps) {
        int4 tr[kListSteps];
#pragma unroll
        for (int k = 0; k < kListSteps; ++k) {
            const int rr = r0 + k * kWave + lane;
            tr[k] = rr < re ? rank_rects[rr] : make_int4(0, 0, 0, 0);
        }
#pragma unroll
        for (int k = 0; k < kListSteps; ++k) {
            const int4 q = tr[k];
            uint32_t area;
            before += rect_tiles_before(q, lp.ty, lp.sx0, tbx, tby, area);
            total += area;
            if (rect_meets_row(q, lp.ty, lp.sx0, lp.sx1)) {
                atomicAdd(&diff[max(q.x, lp.sx0) - lp.sx0], 1);
                atomicAdd(&diff[min(q.z, lp.sx1) - lp.sx0], -1);
            }
        }
    }
    before = wave_sum_u(before);
    total = wave_sum_u(total);
    if (lane == 0) {
        part[0][w] = before;
        part[1][w] = total;
    }
    __syncthreads();
    if (w == 0) {
        const uint32_t n = wave_incl_scan_u32((uint32_t)diff[lane]);
        const bool tile_ok = lp.sx0 + lane < lp.sx1;
        const size_t tiles = (size_t)tbx * tby;
        if (tile_ok) tile_count[lp.slab * tiles + (size_t)lp.ty * tbx + lp.sx0 + lane] = n;
        if (lane == 0) {
            uint32_t b = 0, t = 0;
#pragma unroll
            for (int v = 0; v < kListWaves; ++v) {
                b += part[0][v];
                t += part[1][v];
            }
            seg_scratch[(size_t)lp.slab * nsegs + lp.seg] = b;
            if (lp.seg == 0) atomicAdd(reinterpret_cast<uint32_t*>(total_out), t);
        }
    }
}

__global__ __launch_bounds__(kWave * kListWaves) void k_tile_scatter(
    const int32_t* __restrict__ order, const int4* __restrict__ rank_rects, int P, int tbx,
    int tby, int nsegcols, int slab, int nslab, const uint32_t* __restrict__ tile_count,
    const uint32_t* __restrict__ seg_scratch, int32_t* __restrict__ prim_ids_sorted,
    int32_t* __restrict__ tile_bins, float* __restrict__ zero_buf, int64_t zero_n,
    const int32_t* __restrict__ total, int64_t capacity, int32_t* __restrict__ status_host) {
    __shared__ int32_t hit_pid[kListChunk];
    __shared__ uint32_t hit_cols[kListChunk];
    __shared__ int hit_n[kListWaves];
    __shared__ uint32_t tile_start[kSegTiles];
    // The four status words (final once the counting launch has ended) to the
    // caller's host buffer, which it reads after this launch.
    if (status_host && blockIdx.x == 0 && threadIdx.x < 4)
        status_host[threadIdx.x] = total[threadIdx.x];
    if (zero_buf) {
        const int64_t stride = (int64_t)gridDim.x * blockDim.x;
        for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < zero_n; i += stride)
            zero_buf[i] = 0.0f;
    }
    const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kWave));
    const int lane = threadIdx.x & (kWave - 1);
    const int nsegs = nsegcols * tby;
    const ListPart lp = list_part(nsegs, nsegcols, tbx);
    const int ty = lp.ty, sx0 = lp.sx0, sx1 = lp.sx1;
    const size_t tiles = (size_t)tbx * tby;
    const size_t row0 = (size_t)ty * tbx + sx0;
    if ((uint64_t)(uint32_t)*total > (uint64_t)capacity) {
        // The lists do not fit the caller's buffer: every tile reads as
        // empty, nothing is scattered, and the caller retries at full size.
        if (lp.slab == 0 && w == 0 && sx0 + lane < sx1) {
            tile_bins[2 * (row0 + lane)] = 0;
            tile_bins[2 * (row0 + lane) + 1] = 0;
        }
        return;
    }
    if (w == 0) {
        // The tile's count over all slabs, the slabs' counts before this one,
        // and the segment's first slot (summed over the slabs).
        const bool tile_ok = sx0 + lane < sx1;
        uint32_t n = 0, n_before = 0, seg_first = 0;
        // Eight slabs' loads in flight at a time (the loop would otherwise
        // wait for each load before issuing the next).
        for (int c0 = 0; c0 < nslab; c0 += 8) {
            uint32_t v[8], f[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const int c = c0 + k;
                v[k] = tile_ok && c < nslab ? tile_count[c * tiles + row0 + lane] : 0u;
                f[k] = c < nslab ? seg_scratch[(size_t)c * nsegs + lp.seg] : 0u;
            }
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                n += v[k];
                n_before += c0 + k < lp.slab ? v[k] : 0u;
                seg_first += f[k];
            }
        }
        const uint32_t start = seg_first + wave_incl_scan_u32(n) - n;
        tile_start[lane] = start + n_before;
        if (lp.slab == 0 && tile_ok) {
            // tile_bins.py:10-43: [start, end) per tile, (0, 0) when empty.
            tile_bins[2 * (row0 + lane)] = n ? (int32_t)start : 0;
            tile_bins[2 * (row0 + lane) + 1] = n ? (int32_t)(start + n) : 0;
        }
    }
    __syncthreads();
    uint32_t cur[kListTilesPerWave];
    int nst[kListTilesPerWave];
#pragma unroll
    for (int k = 0; k < kListTilesPerWave; ++k) {
        cur[k] = tile_start[w * kListTilesPerWave + k];
        nst[k] = 0;
    }

    const int rb = lp.slab * slab, re = min(P, rb + slab);
    for (int c0 = rb; c0 < re; c0 += kListChunk) {
        // 1. Compact the chunk's hits into one list (this wave's loads all
        //    in flight before the first test).
        const int r0 = c0 + w * kListSlice;
        const int r1 = min(r0 + kListSlice, re);
        int4 tr[kListSteps];
        int pid[kListSteps];
#pragma unroll
        for (int k = 0; k < kListSteps; ++k) {
            const int rr = r0 + k * kWave + lane;
            tr[k] = rr < r1 ? rank_rects[rr] : make_int4(0, 0, 0, 0);
            pid[k] = rr < r1 ? order[rr] : 0;
        }
        bool hit[kListSteps];
        int n_w = 0;
#pragma unroll
        for (int k = 0; k < kListSteps; ++k) {
            hit[k] = rect_meets_row(tr[k], ty, sx0, sx1);
            n_w += __builtin_popcountll(__ballot(hit[k]));
        }
        if (lane == 0) hit_n[w] = n_w;
        __syncthreads();
        int nh = 0, slot0 = 0;
#pragma unroll
        for (int v = 0; v < kListWaves; ++v) {
            const int c = hit_n[v];
            slot0 += v < w ? c : 0;
            nh += c;
        }
#pragma unroll
        for (int k = 0; k < kListSteps; ++k) {
            const uint64_t m = __ballot(hit[k]);
            if (hit[k]) {
                const int4 q = tr[k];
                const int slot = slot0 + (int)lanes_below(m);
                hit_pid[slot] = pid[k];
                hit_cols[slot] = (uint32_t)(max(q.x, sx0) - sx0) |
                                 ((uint32_t)(min(q.z, sx1) - sx0) << 16);
            }
            slot0 += __builtin_popcountll(m);
        }
        __syncthreads();
        // 2. The owned tiles' next entries, 64 hits at a time (the next
        //    group's LDS reads in flight).
        uint32_t cols_n = lane < nh ? hit_cols[lane] : 0u;
        int pid_n = lane < nh ? hit_pid[lane] : 0;
        for (int j = 0; j < nh; j += kWave) {
            const uint32_t cols = cols_n;
            const int pidv = pid_n;
            const int jn = j + kWave + lane;
            cols_n = jn < nh ? hit_cols[jn] : 0u;
            pid_n = jn < nh ? hit_pid[jn] : 0;
            const int x0 = (int)(cols & 0xffffu), x1 = (int)(cols >> 16);
#pragma unroll
            for (int k = 0; k < kListTilesPerWave; ++k) {
                const int col = w * kListTilesPerWave + k;
                const bool in = x0 <= col && col < x1;
                const uint64_t m = __ballot(in);
                if (in) prim_ids_sorted[cur[k] + lanes_below(m)] = pidv;
                cur[k] += (uint32_t)__builtin_popcountll(m);
            }
        }
        __syncthreads();
    }
}

// tile_bins.py:10-43 on the reference's int64 (tile << 32 | depth) keys.
__global__ __launch_bounds__(256) void k_tile_bins_i64(const int64_t* __restrict__ keys, int n,
                                                      int32_t* __restrict__ bins) {
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n) return;
    const int32_t cur = (int32_t)(keys[idx] >> 32);
    if (idx == 0) bins[2 * cur] = 0;
    if (idx == n - 1) bins[2 * cur + 1] = n;
    if (idx > 0) {
        const int32_t prev = (int32_t)(keys[idx - 1] >> 32);
        if (prev != cur) {
            bins[2 * prev + 1] = idx;
            bins[2 * cur] = idx;
        }
    }
}

// ------------------------------------------- reference-layout building blocks

// project_cubics_2d_forward_kernel (cubic_splatting.py:546-747), per segment.
__global__ __launch_bounds__(256) void k_project_ref(
    const float* __restrict__ cubics_norm, const float* __restrict__ stroke_widths,
    const float* __restrict__ support_radii, int nseg, int img_h, int img_w, int block_x,
    int block_y, float aabb_pad, int aniso, float* __restrict__ cubics_px,
    int32_t* __restrict__ tile_ranges, int32_t* __restrict__ num_tiles_hit) {
    const int s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= nseg) return;
    const int tbx = (img_w + block_x - 1) / block_x, tby = (img_h + block_y - 1) / block_y;
    const SegProj r = project_segment(
        cubics_norm + (size_t)s * 8, 0.5f * (float)img_w, 0.5f * (float)img_h,
        fmaxf(0.0f, stroke_widths[s]) * 0.5f, fmaxf(0.0f, support_radii[s]), aabb_pad, aniso,
        tbx, tby, (float)block_x, (float)block_y);
    float4* cp = reinterpret_cast<float4*>(cubics_px + (size_t)s * 8);
    cp[0] = make_float4(r.px[0], r.py[0], r.px[1], r.py[1]);
    cp[1] = make_float4(r.px[2], r.py[2], r.px[3], r.py[3]);
    reinterpret_cast<int4*>(tile_ranges)[s] = make_int4(r.tx0, r.ty0, r.tx1, r.ty1);
    num_tiles_hit[s] = max(0, (r.tx1 - r.tx0) * (r.ty1 - r.ty0));
}

// primitive_tile_ranges_from_segment_ranges_kernel (cubic_splatting.py:2071-2137).
__global__ __launch_bounds__(256) void k_prim_ranges_ref(const int32_t* __restrict__ seg_ranges,
                                                        const int32_t* __restrict__ offs, int P,
                                                        int tbx, int tby,
                                                        int32_t* __restrict__ prim_ranges,
                                                        int32_t* __restrict__ num_tiles_hit) {
    const int p = blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= P) return;
    const int s0 = offs[p], s1 = offs[p + 1];
    int4 tr = make_int4(0, 0, 0, 0);
    int area = 0;
    if (s1 > s0) {
        int mnx = tbx, mny = tby, mxx = 0, mxy = 0;
        for (int s = s0; s < s1; ++s) {
            const int4 r = reinterpret_cast<const int4*>(seg_ranges)[s];
            mnx = min(mnx, r.x); mny = min(mny, r.y);
            mxx = max(mxx, r.z); mxy = max(mxy, r.w);
        }
        tr = make_int4(mnx, mny, mxx, mxy);
        area = max(0, mxx - mnx) * max(0, mxy - mny);
    }
    reinterpret_cast<int4*>(prim_ranges)[p] = tr;
    num_tiles_hit[p] = area;
}

// map_cubic_to_intersects_kernel (cubic_splatting.py:750-819): wave per
// primitive, row-major over its tile rectangle, at offset cum[p-1].
__global__ __launch_bounds__(256) void k_map_ref(const int32_t* __restrict__ tile_ranges,
                                                const float* __restrict__ depths,
                                                const int32_t* __restrict__ cum, int P, int tbx,
                                                int64_t* __restrict__ isect_ids,
                                                int32_t* __restrict__ curve_ids) {
    const int lane = threadIdx.x & 63;
    const int waves = (gridDim.x * blockDim.x) >> 6;
    for (int p = (blockIdx.x * blockDim.x + threadIdx.x) >> 6; p < P; p += waves) {
        const int4 tr = reinterpret_cast<const int4*>(tile_ranges)[p];
        const int w = tr.z - tr.x, h = tr.w - tr.y;
        if (w * h <= 0) continue;
        const int base = p == 0 ? 0 : cum[p - 1];
        const int32_t bits = __builtin_bit_cast(int32_t, depths[p]);
        const int64_t dk =
            (int64_t)(uint32_t)(bits ^ ((bits >> 31) | (int32_t)0x80000000));
        for (int k = lane; k < w * h; k += kWave) {
            const int row = k / w, col = k - row * w;
            const int64_t tile = (int64_t)((tr.y + row) * tbx + tr.x + col);
            isect_ids[base + k] = (tile << 32) | dk;
            curve_ids[base + k] = p;
        }
    }
}

// _build_fill_isect_edge_ranges (cubic_splatting.py:1849-1860).
__global__ __launch_bounds__(256) void k_isect_edge_ranges(const int32_t* __restrict__ ids,
                                                          const int32_t* __restrict__ offs, int n,
                                                          int eps, int32_t* __restrict__ out) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int p = ids[i];
    out[2 * i] = offs[p] * eps;
    out[2 * i + 1] = offs[p + 1] * eps;
}

// ------------------------------------- raster records from reference layouts
//
// The reference's raster wrappers take flattened edges [E, 2, 2] and one edge
// range per intersection (rasterize_cubic_fill_forward_tilelang,
// ops/cubic_splatting.py:2181-2305; the backward :2572-2747).  The raster
// kernels here read per-primitive records, so each primitive's range is taken
// from its intersections (all of which must agree), and the edge and
// primitive records are built from the edges.

// range[ids[g]] = isect_edge_ranges[g]; status |= 1 for an id outside [0, P).
__global__ __launch_bounds__(256) void k_scatter_isect_ranges(const int32_t* __restrict__ ids,
                                                              const int2* __restrict__ ranges,
                                                              int64_t n, int P,
                                                              int2* __restrict__ prim_range,
                                                              int32_t* __restrict__ status) {
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= n) return;
    const int p = ids[g];
    if (p < 0 || p >= P) {
        atomicOr(status, 1);
        return;
    }
    prim_range[p] = ranges[g];
}

// status |= 2 where an intersection's range differs from its primitive's
// (or is not a range within [0, E]).
__global__ __launch_bounds__(256) void k_check_isect_ranges(const int32_t* __restrict__ ids,
                                                            const int2* __restrict__ ranges,
                                                            int64_t n, int P, int E,
                                                            const int2* __restrict__ prim_range,
                                                            int32_t* __restrict__ status) {
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= n) return;
    const int p = ids[g];
    if (p < 0 || p >= P) return;
    const int2 r = ranges[g], q = prim_range[p];
    if (r.x != q.x || r.y != q.y || r.x < 0 || r.y < r.x || r.y > E) atomicOr(status, 2);
}

// status |= 4 for a tile whose list range is not within [0, num_intersects].
__global__ __launch_bounds__(256) void k_check_tile_bins(const int2* __restrict__ bins, int T,
                                                         int64_t n, int32_t* __restrict__ status) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= T) return;
    const int2 b = bins[t];
    if (b.x < 0 || b.y < b.x || (int64_t)b.y > n) atomicOr(status, 4);
}

__device__ __forceinline__ float prim_cull_d_from_is2(int mode, float opacity, float inv_s2,
                                                     float half_sw) {
    return cull_distance(mode, opacity, __builtin_sqrtf(fmaxf(inv_s2, kEps)), half_sw);
}

__device__ __forceinline__ int2 clamp_range(int2 r, int E) {
    const int a = clampi(r.x, 0, E);
    return make_int2(a, clampi(r.y, a, E));
}

// Every edge's cull distance: the largest over the primitives whose range
// holds it (positive floats order as their bits).
__global__ __launch_bounds__(256) void k_edge_cull_d(const int2* __restrict__ prim_range, int P,
                                                     int E, int mode,
                                                     const float* __restrict__ opacities,
                                                     const float* __restrict__ inv_s2,
                                                     const float* __restrict__ stroke_widths,
                                                     int32_t* __restrict__ edge_d_bits) {
    const int p = blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= P) return;
    const float half_sw =
        (mode == 1 && stroke_widths) ? fmaxf(0.0f, stroke_widths[p]) * 0.5f : 0.0f;
    const float D = prim_cull_d_from_is2(mode, opacities[p], inv_s2[p], half_sw);
    const int2 r = clamp_range(prim_range[p], E);
    for (int e = r.x; e < r.y; ++e) atomicMax(edge_d_bits + e, __builtin_bit_cast(int32_t, D));
}

__global__ __launch_bounds__(256) void k_edges_from_px(const float4* __restrict__ edges_px, int E,
                                                       const int32_t* __restrict__ edge_d_bits,
                                                       EdgeRec* __restrict__ edges,
                                                       EdgeCull* __restrict__ culls) {
    const int e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= E) return;
    const float4 a = edges_px[e];
    write_edge(a.x, a.y, a.z, a.w, __builtin_bit_cast(float, edge_d_bits[e]), edges + e,
               culls + e);
}

// Primitive records as k_prim_prep makes them, with the ranges and the
// closed flag taken from the primitive's edges: the vertex box of its edges,
// and closed when each edge starts where the previous one ends and the last
// one ends where the first starts.
__global__ __launch_bounds__(256) void k_prim_recs_from_edges(
    const int2* __restrict__ prim_range, int P, int E, int mode,
    const float4* __restrict__ edges_px, const float* __restrict__ colors,
    const float* __restrict__ opacities, const float* __restrict__ inv_s2,
    const int32_t* __restrict__ fill_rules, const float* __restrict__ stroke_widths,
    PrimRec* __restrict__ recs) {
    const int p = blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= P) return;
    const int2 r = clamp_range(prim_range[p], E);
    PrimRec rec;
    rec.r = colors[3 * p];
    rec.g = colors[3 * p + 1];
    rec.b = colors[3 * p + 2];
    rec.opacity = opacities[p];
    rec.inv_sigma2 = fmaxf(inv_s2[p], kEps);
    rec.inv_sigma = __builtin_sqrtf(fmaxf(inv_s2[p], kEps));
    rec.half_sw = (mode == 1 && stroke_widths) ? fmaxf(0.0f, stroke_widths[p]) * 0.5f : 0.0f;
    rec.cull_d = cull_distance(mode, rec.opacity, rec.inv_sigma, rec.half_sw);
    rec.e0 = r.x;
    rec.e1 = r.y;
    rec.rule = fill_rules ? fill_rules[p] : 1;
    VBox box = vbox_empty();
    int closed = 1;
    for (int e = r.x; e < r.y; ++e) {
        const float4 a = edges_px[e];
        vbox_add(box, a.x, a.y);
        vbox_add(box, a.z, a.w);
        const float4 b = edges_px[e + 1 < r.y ? e + 1 : r.x];
        closed &= (a.z == b.x) & (a.w == b.y);
    }
    const SegRec sr = seg_record(box, rec.cull_d);
    rec.closed = closed;
    rec.ny_lo = sr.ny_lo;
    rec.ny_span = sr.ny_span;
    rec.cy_lo = sr.cy_lo;
    rec.cy_span = sr.cy_span;
    rec.nx_lo = sr.nx_lo;
    rec.nx_span = sr.nx_span;
    rec.x_last = r.y > r.x ? sr.x_last : -kRangeLimit;
    rec.cull_out = cull_distance_outside(mode, rec.opacity, rec.inv_sigma, rec.half_sw);
    recs[p] = rec;
}

// Per-edge (segment, t0, t1) records from the adaptive flattening's CSR
// (segment_edge_offsets, edge_t_starts, edge_t_ends; cubic_splatting.py:1812-1828).
__global__ __launch_bounds__(256) void k_edge_aux_from_csr(const int32_t* __restrict__ seo,
                                                          int nseg,
                                                          const float* __restrict__ t0,
                                                          const float* __restrict__ t1, int E,
                                                          EdgeAux* __restrict__ aux) {
    const int s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= nseg) return;
    const int a = clampi(seo[s], 0, E), b = clampi(seo[s + 1], a, E);
    for (int e = a; e < b; ++e) aux[e] = EdgeAux{s, t0[e], t1[e], 0};
}

}  // namespace cs

// ===================================================================== C ABI

using namespace cs;

static inline int blocks_for(int64_t n, int t) { return (int)((n + t - 1) / t); }

static int launch_status() {
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? CS_OK : CS_ERR_HIP;
}

extern "C" size_t cs_scan_temp_elems(int32_t n) {
    const int nb = blocks_for(n, kScanChunk);
    return (size_t)(nb > 1 ? nb : 1);
}

extern "C" int cs_scan_exclusive_u32(const uint32_t* in, uint32_t* out, int32_t n,
                                     uint32_t* temp, int32_t* total, hipStream_t stream) {
    if (n < 0) return CS_ERR_ARGS;
    if (n == 0) {
        if (total) {
            hipLaunchKernelGGL(k_fill_i32, dim3(1), dim3(256), 0, stream, total, 1, 0);
        }
        return launch_status();
    }
    const int nb = blocks_for(n, kScanChunk);
    if (nb == 1) {
        hipLaunchKernelGGL(k_scan_apply<kScanItems>, dim3(1), dim3(kScanThreads), 0, stream, in,
                           out, n, nullptr, total);
    } else if (n <= kScanThreads * kScanItemsLarge) {
        // One workgroup with more items per thread beats three launches.
        hipLaunchKernelGGL(k_scan_apply<kScanItemsLarge>, dim3(1), dim3(kScanThreads), 0, stream,
                           in, out, n, nullptr, total);
    } else {
        hipLaunchKernelGGL(k_scan_block_sums, dim3(nb), dim3(kScanThreads), 0, stream, in, n, temp);
        hipLaunchKernelGGL(k_scan_partials, dim3(1), dim3(kScanThreads), 0, stream, temp, nb);
        hipLaunchKernelGGL(k_scan_apply<kScanItems>, dim3(nb), dim3(kScanThreads), 0, stream, in,
                           out, n, temp, total);
    }
    return launch_status();
}

extern "C" size_t cs_radix_counts_elems(int32_t n) {
    const int nb = blocks_for(n > 0 ? n : 1, kRsTile);
    const size_t radix = (size_t)256 * nb;
    // The sort of at most kRankSortMax keys stages 2n words here.
    const size_t rank = n > kRankPairsMax && n <= kRankSortMax ? (size_t)2 * n : 0;
    return radix > rank ? radix : rank;
}

extern "C" int cs_radix_sort_pairs_u32(uint32_t* keys, int32_t* vals, uint32_t* keys_alt,
                                       int32_t* vals_alt, int32_t n, int32_t key_bits,
                                       uint32_t* counts, uint32_t* scan_temp,
                                       hipStream_t stream) {
    if (n < 0 || key_bits < 0 || key_bits > 32) return CS_ERR_ARGS;
    if (n <= 1 || key_bits == 0) return CS_OK;
    const int nb = blocks_for(n, kRsTile);
    const int passes = (key_bits + 7) / 8;
    if (n <= kRankSortMax) {
        // Ranked into the *_alt buffers and copied back; the block sort of
        // the merge path stages its sorted blocks in counts[0, n) and the
        // in-block ranks in counts[n, 2n).
        if (n <= kRankPairsMax) {
            hipLaunchKernelGGL(k_rank_allpairs<true>, dim3((n + 3) / 4), dim3(256), 0, stream,
                               keys, n, vals, keys_alt, vals_alt, (const int4*)nullptr,
                               (int32_t*)nullptr, (int4*)nullptr);
        } else {
            uint32_t* sorted = counts;
            int32_t* brank = reinterpret_cast<int32_t*>(counts + n);
            const int nblk = blocks_for(n, kRankBlock);
            hipLaunchKernelGGL(k_rank_blocks, dim3(nblk), dim3(kRankBlock), 0, stream, keys, n,
                               sorted, brank);
            hipLaunchKernelGGL(k_rank_merge<true>, dim3(blocks_for(n, kMergeKeys)),
                               dim3(kMergeThreads), 0, stream, keys, sorted, brank, n, vals,
                               keys_alt, vals_alt, (const int4*)nullptr, (int32_t*)nullptr,
                               (int4*)nullptr);
        }
        if (hipMemcpyAsync(keys, keys_alt, sizeof(uint32_t) * n, hipMemcpyDeviceToDevice,
                           stream) != hipSuccess ||
            hipMemcpyAsync(vals, vals_alt, sizeof(int32_t) * n, hipMemcpyDeviceToDevice,
                           stream) != hipSuccess)
            return CS_ERR_HIP;
        return launch_status();
    }
    uint32_t *ki = keys, *ko = keys_alt;
    int32_t *vi = vals, *vo = vals_alt;
    for (int ps = 0; ps < passes; ++ps) {
        const int shift = 8 * ps;
        hipLaunchKernelGGL(k_rs_hist, dim3(nb), dim3(kRsThreads), 0, stream, ki, n, shift, nb,
                           counts);
        int rc = cs_scan_exclusive_u32(counts, counts, 256 * nb, scan_temp, nullptr, stream);
        if (rc) return rc;
        hipLaunchKernelGGL(k_rs_scatter, dim3(nb), dim3(kRsThreads), 0, stream, ki, vi, ko, vo, n,
                           shift, nb, counts);
        uint32_t* tk = ki; ki = ko; ko = tk;
        int32_t* tv = vi; vi = vo; vo = tv;
    }
    if (ki != keys) {
        if (hipMemcpyAsync(keys, ki, sizeof(uint32_t) * n, hipMemcpyDeviceToDevice, stream) !=
                hipSuccess ||
            hipMemcpyAsync(vals, vi, sizeof(int32_t) * n, hipMemcpyDeviceToDevice, stream) !=
                hipSuccess)
            return CS_ERR_HIP;
    }
    return launch_status();
}


// Depth ranks, then the tile-list counts: order[r] = primitive with the r-th
// smallest key (ties by primitive id) and rank_rects[r] its tile rectangle
// (already written when `ranked`); per-tile counts, per-segment totals, then
// the segments' first slots; status[0] receives the intersection total.
static int rank_and_count(bool blocks_ranked, uint32_t* keys, int32_t* order,
                          const int4* prim_rects,
                          int4* rank_rects, int nprim, int tbx, int tby, uint32_t* keys_alt,
                          int32_t* vals_alt, uint32_t* radix_counts, uint32_t* scan_temp,
                          uint32_t* tile_count,
                          uint32_t* tile_scratch, int32_t* status, hipStream_t stream,
                          bool ranked = false) {
    if (ranked) {
    } else if (nprim <= kRankPairsMax) {
        hipLaunchKernelGGL(k_rank_allpairs<false>, dim3((nprim + 3) / 4), dim3(256), 0, stream,
                           keys, nprim, (const int32_t*)nullptr, (uint32_t*)nullptr,
                           (int32_t*)nullptr, prim_rects, order, rank_rects);
    } else if (nprim <= kRankSortMax) {
        // Block ranks into keys_alt / vals_alt (already there when
        // blocks_ranked: k_prim_prep wrote them).
        if (!blocks_ranked)
            hipLaunchKernelGGL(k_rank_blocks, dim3(blocks_for(nprim, kRankBlock)),
                               dim3(kRankBlock), 0, stream, keys, nprim, keys_alt, vals_alt);
        hipLaunchKernelGGL(k_rank_merge<false>, dim3(blocks_for(nprim, kMergeKeys)),
                           dim3(kMergeThreads), 0, stream, keys,
                           keys_alt, vals_alt, nprim, (const int32_t*)nullptr,
                           (uint32_t*)nullptr, (int32_t*)nullptr, prim_rects, order, rank_rects);
    } else {
        const int rc = cs_radix_sort_pairs_u32(keys, order, keys_alt, vals_alt, nprim, 32,
                                               radix_counts, scan_temp, stream);
        if (rc) return rc;
        hipLaunchKernelGGL(k_gather_rects, dim3(blocks_for(nprim, 256)), dim3(256), 0, stream,
                           order, nprim, prim_rects, rank_rects);
    }
    const int nsegcols = (tbx + kSegTiles - 1) / kSegTiles;
    const ListSlabs ls = list_slabs(nprim, nsegcols * tby);
    hipLaunchKernelGGL(k_tile_counts, dim3(nsegcols * tby * ls.nslab),
                       dim3(kWave * kListWaves), 0, stream, rank_rects, nprim, tbx, tby,
                       nsegcols, ls.slab, tile_count, tile_scratch, status);
    return launch_status();
}

// Flatness tolerance of the adaptive flattening, px
// (DEFAULT_DE_CASTELJAU_FLATNESS_TOL_PX, cubic_splatting.py:18, clamped at
// 1e-4 as :1731 does).
constexpr float kDecasTolPx = 0.5f;
// Deepest subdivision the adaptive entry points accept (2^24 edges per segment).
constexpr int kDecasMaxDepth = 24;

static int bin_prepare(const float* cubics_norm, const int32_t* seg_offsets, const float* colors,
                       const float* opacities, const float* depths, const int32_t* fill_rules,
                       const float* aa_widths, const float* stroke_widths, int32_t nseg,
                       int32_t nprim, int32_t img_h, int32_t img_w, int32_t block_x,
                       int32_t block_y, int32_t samples, float aabb_pad, int32_t aniso,
                       int32_t mode, float* cubics_px, int32_t* seg_tile_ranges, void* seg_recs,
                       void* edges, void* edge_culls, int32_t* prim_tile_ranges,
                       uint32_t* num_tiles_hit, float* inv_sigma2s, void* prim_recs,
                       uint32_t* keys, int32_t* order, uint32_t* keys_alt, int32_t* vals_alt,
                       uint32_t* radix_counts, uint32_t* scan_temp, int32_t* rank_tile_ranges,
                       uint32_t* tile_count, uint32_t* tile_scratch,
                       int32_t* status, int32_t* seg_edge_offsets, void* edge_aux,
                       uint32_t* leaf_counts, hipStream_t stream) {
    if (nseg < 0 || nprim <= 0 || img_h <= 0 || img_w <= 0 || block_x <= 0 || block_y <= 0 ||
        samples < 2 || (mode != 0 && mode != 1) || img_h > kMaxImageDim ||
        img_w > kMaxImageDim)
        return CS_ERR_ARGS;
    const bool adaptive = seg_edge_offsets != nullptr;
    const int eps = samples - 1;
    const int maxd = ceil_log2(eps);
    if (adaptive) {
        if (!edge_aux || !leaf_counts || maxd > kDecasMaxDepth ||
            (int64_t)nseg << maxd > (int64_t)INT32_MAX)
            return CS_ERR_ARGS;
    } else if ((int64_t)nseg * eps > (int64_t)INT32_MAX) {
        return CS_ERR_ARGS;
    }
    const int tbx = (img_w + block_x - 1) / block_x, tby = (img_h + block_y - 1) / block_y;
    if (!adaptive && nseg > 0 && samples <= kWave) {
        // One lane per sample point; the kernel also sets the status words.
        const int lanes = samples <= 2 ? 2 : 1 << ceil_log2(samples);
        const dim3 grid((unsigned)blocks_for(nseg, flatten_segs(lanes))),
            block(kWave * kFlattenWaves);
#define CS_FLATTEN_LANES(Lv)                                                                   \
    hipLaunchKernelGGL(k_project_flatten_wave<Lv>, grid, block, 0, stream, cubics_norm,       \
                       seg_offsets, nprim, aa_widths, stroke_widths, opacities, mode, nseg,    \
                       img_h, img_w, block_x, block_y, aabb_pad, aniso, samples, cubics_px,    \
                       seg_tile_ranges, reinterpret_cast<SegRec*>(seg_recs),                   \
                       reinterpret_cast<EdgeRec*>(edges), reinterpret_cast<EdgeCull*>(edge_culls), \
                       status)
        switch (lanes) {
            case 2: CS_FLATTEN_LANES(2); break;
            case 4: CS_FLATTEN_LANES(4); break;
            case 8: CS_FLATTEN_LANES(8); break;
            case 16: CS_FLATTEN_LANES(16); break;
            case 32: CS_FLATTEN_LANES(32); break;
            default: CS_FLATTEN_LANES(64); break;
        }
#undef CS_FLATTEN_LANES
    } else {
        hipLaunchKernelGGL(k_status_init, dim3(1), dim3(1), 0, stream, seg_offsets, nprim,
                           status);
    }
    if (nseg > 0 && (adaptive || samples > kWave))
        hipLaunchKernelGGL(k_project_flatten, dim3(blocks_for(nseg, 256)), dim3(256), 0, stream,
                           cubics_norm, seg_offsets, nprim, aa_widths, stroke_widths, opacities,
                           mode, nseg, img_h, img_w, block_x, block_y, aabb_pad, aniso, samples,
                           cubics_px, seg_tile_ranges, reinterpret_cast<SegRec*>(seg_recs),
                           reinterpret_cast<EdgeRec*>(edges),
                           reinterpret_cast<EdgeCull*>(edge_culls), maxd, kDecasTolPx,
                           adaptive ? leaf_counts : nullptr);
    if (adaptive) {
        int rc = cs_scan_exclusive_u32(leaf_counts, reinterpret_cast<uint32_t*>(seg_edge_offsets),
                                       nseg, scan_temp, seg_edge_offsets + nseg, stream);
        if (rc) return rc;
        if (nseg > 0)
            hipLaunchKernelGGL(k_decas_emit, dim3(blocks_for(nseg, 256)), dim3(256), 0, stream,
                               cubics_px, seg_offsets, nprim, aa_widths, stroke_widths,
                               opacities, mode, nseg, maxd, kDecasTolPx, seg_edge_offsets,
                               reinterpret_cast<EdgeRec*>(edges),
                               reinterpret_cast<EdgeCull*>(edge_culls),
                               reinterpret_cast<EdgeAux*>(edge_aux),
                               reinterpret_cast<SegRec*>(seg_recs));
    }
    if (nprim <= kRankPairsMax) {
        // Records and depth ranks in one launch.
        constexpr int per_block = 4 * kPrepRankPerWave;
        hipLaunchKernelGGL(k_prim_prep_rank, dim3((nprim + per_block - 1) / per_block),
                           dim3(256), 0, stream,
                           cubics_norm, seg_offsets, nprim, seg_tile_ranges,
                           reinterpret_cast<const SegRec*>(seg_recs), colors, opacities, depths,
                           fill_rules, aa_widths, stroke_widths, nseg, eps,
                           adaptive ? seg_edge_offsets : nullptr, tbx, tby, mode, status,
                           prim_tile_ranges, num_tiles_hit, inv_sigma2s, keys,
                           reinterpret_cast<int32_t*>(keys_alt),
                           reinterpret_cast<PrimRec*>(prim_recs), order,
                           reinterpret_cast<int4*>(rank_tile_ranges));
        return rank_and_count(true, keys, order, reinterpret_cast<const int4*>(prim_tile_ranges),
                              reinterpret_cast<int4*>(rank_tile_ranges), nprim, tbx, tby,
                              keys_alt, vals_alt, radix_counts, scan_temp, tile_count,
                              tile_scratch, status, stream, true);
    }
    hipLaunchKernelGGL(k_prim_prep, dim3(blocks_for(nprim, 256)), dim3(256), 0, stream,
                       cubics_norm, seg_offsets, nprim, seg_tile_ranges,
                       reinterpret_cast<const SegRec*>(seg_recs), colors, opacities, depths,
                       fill_rules, aa_widths, stroke_widths, nseg, eps,
                       adaptive ? seg_edge_offsets : nullptr, tbx, tby, mode, status,
                       prim_tile_ranges, num_tiles_hit, inv_sigma2s, keys, order,
                       reinterpret_cast<PrimRec*>(prim_recs),
                       nprim <= kRankSortMax ? keys_alt : nullptr,
                       nprim <= kRankSortMax ? vals_alt : nullptr);
    return rank_and_count(true, keys, order, reinterpret_cast<const int4*>(prim_tile_ranges),
                          reinterpret_cast<int4*>(rank_tile_ranges), nprim, tbx, tby, keys_alt,
                          vals_alt, radix_counts, scan_temp, tile_count,
                          tile_scratch, status, stream);
}

extern "C" int cs_bin_prepare(const float* cubics_norm, const int32_t* seg_offsets,
                              const float* colors, const float* opacities, const float* depths,
                              const int32_t* fill_rules, const float* aa_widths,
                              const float* stroke_widths, int32_t nseg, int32_t nprim,
                              int32_t img_h, int32_t img_w, int32_t block_x, int32_t block_y,
                              int32_t samples, float aabb_pad, int32_t aniso, int32_t mode,
                              float* cubics_px, int32_t* seg_tile_ranges, void* seg_recs,
                              void* edges, void* edge_culls, int32_t* prim_tile_ranges,
                              uint32_t* num_tiles_hit,
                              float* inv_sigma2s, void* prim_recs, uint32_t* keys,
                              int32_t* order, uint32_t* keys_alt, int32_t* vals_alt,
                              uint32_t* radix_counts, uint32_t* scan_temp,
                              int32_t* rank_tile_ranges, uint32_t* tile_count, uint32_t* tile_scratch, int32_t* status,
                              hipStream_t stream) {
    return bin_prepare(cubics_norm, seg_offsets, colors, opacities, depths, fill_rules,
                       aa_widths, stroke_widths, nseg, nprim, img_h, img_w, block_x, block_y,
                       samples, aabb_pad, aniso, mode, cubics_px, seg_tile_ranges, seg_recs,
                       edges, edge_culls, prim_tile_ranges, num_tiles_hit, inv_sigma2s,
                       prim_recs, keys, order, keys_alt, vals_alt, radix_counts, scan_temp,
                       rank_tile_ranges, tile_count, tile_scratch, status,
                       nullptr, nullptr, nullptr, stream);
}

extern "C" int32_t cs_de_casteljau_max_edges_per_segment(int32_t samples) {
    if (samples < 2) return 0;
    const int d = ceil_log2(samples - 1);
    return d > kDecasMaxDepth ? 0 : (1 << d);
}

extern "C" int cs_bin_prepare_de_casteljau(
    const float* cubics_norm, const int32_t* seg_offsets, const float* colors,
    const float* opacities, const float* depths, const int32_t* fill_rules,
    const float* aa_widths, const float* stroke_widths, int32_t nseg, int32_t nprim,
    int32_t img_h, int32_t img_w, int32_t block_x, int32_t block_y, int32_t samples,
    float aabb_pad, int32_t aniso, int32_t mode, float* cubics_px, int32_t* seg_tile_ranges,
    void* seg_recs, void* edges, void* edge_culls, int32_t* prim_tile_ranges,
    uint32_t* num_tiles_hit, float* inv_sigma2s, void* prim_recs, uint32_t* keys,
    int32_t* order, uint32_t* keys_alt, int32_t* vals_alt, uint32_t* radix_counts,
    uint32_t* scan_temp, int32_t* rank_tile_ranges, uint32_t* tile_count, uint32_t* tile_scratch, int32_t* status, int32_t* seg_edge_offsets,
    void* edge_aux, uint32_t* leaf_counts, hipStream_t stream) {
    if (!seg_edge_offsets) return CS_ERR_ARGS;
    return bin_prepare(cubics_norm, seg_offsets, colors, opacities, depths, fill_rules,
                       aa_widths, stroke_widths, nseg, nprim, img_h, img_w, block_x, block_y,
                       samples, aabb_pad, aniso, mode, cubics_px, seg_tile_ranges, seg_recs,
                       edges, edge_culls, prim_tile_ranges, num_tiles_hit, inv_sigma2s,
                       prim_recs, keys, order, keys_alt, vals_alt, radix_counts, scan_temp,
                       rank_tile_ranges, tile_count, tile_scratch, status,
                       seg_edge_offsets, edge_aux, leaf_counts, stream);
}

extern "C" int cs_flatten_cubics_de_casteljau(const float* cubics_px, const int32_t* seg_offsets,
                                              int32_t nprim, int32_t nseg, int32_t samples,
                                              uint32_t* leaf_counts, uint32_t* scan_temp,
                                              int32_t* segment_edge_offsets,
                                              int32_t* primitive_edge_offsets, float* edges_px,
                                              float* edge_t_starts, float* edge_t_ends,
                                              hipStream_t stream) {
    if (nseg < 0 || nprim < 0 || samples < 2 || !segment_edge_offsets) return CS_ERR_ARGS;
    const int maxd = ceil_log2(samples - 1);
    if (maxd > kDecasMaxDepth || (int64_t)nseg << maxd > (int64_t)INT32_MAX) return CS_ERR_ARGS;
    if (nseg > 0)
        hipLaunchKernelGGL(k_decas_count_ref, dim3(blocks_for(nseg, 256)), dim3(256), 0, stream,
                           cubics_px, nseg, maxd, kDecasTolPx, leaf_counts);
    int rc = cs_scan_exclusive_u32(leaf_counts, reinterpret_cast<uint32_t*>(segment_edge_offsets),
                                   nseg, scan_temp, segment_edge_offsets + nseg, stream);
    if (rc) return rc;
    if (nseg > 0)
        hipLaunchKernelGGL(k_decas_emit_ref, dim3(blocks_for(nseg, 256)), dim3(256), 0, stream,
                           cubics_px, nseg, maxd, kDecasTolPx, segment_edge_offsets, edges_px,
                           edge_t_starts, edge_t_ends);
    if (primitive_edge_offsets && nprim >= 0 && seg_offsets)
        hipLaunchKernelGGL(k_prim_edge_offsets, dim3(blocks_for(nprim + 1, 256)), dim3(256), 0,
                           stream, segment_edge_offsets, seg_offsets, nprim + 1, nseg,
                           primitive_edge_offsets);
    return launch_status();
}

extern "C" int cs_flatten_cubics_bernstein(const float* cubics_px, int32_t nseg,
                                           int32_t samples, float* edges_px,
                                           hipStream_t stream) {
    if (nseg < 0 || samples < 2 || (int64_t)nseg * (samples - 1) > (int64_t)INT32_MAX)
        return CS_ERR_ARGS;
    if (nseg == 0) return CS_OK;
    hipLaunchKernelGGL(k_bernstein_ref, dim3(blocks_for(nseg, 256)), dim3(256), 0, stream,
                       cubics_px, nseg, samples, edges_px);
    return launch_status();
}

extern "C" int cs_cubic_flatness_flags(const float* cubics, int32_t n, float tol_px,
                                       int32_t force_flat, uint8_t* out_flat,
                                       hipStream_t stream) {
    if (n < 0) return CS_ERR_ARGS;
    if (n == 0) return CS_OK;
    hipLaunchKernelGGL(k_flatness_flags, dim3(blocks_for(n, 256)), dim3(256), 0, stream, cubics,
                       n, fmaxf(1e-4f, tol_px), force_flat ? 1 : 0, out_flat);
    return launch_status();
}

extern "C" int cs_cubic_split_half(const float* cubics, int32_t n, float* left, float* right,
                                   hipStream_t stream) {
    if (n < 0) return CS_ERR_ARGS;
    if (n == 0) return CS_OK;
    hipLaunchKernelGGL(k_split_half, dim3(blocks_for(n, 256)), dim3(256), 0, stream, cubics, n,
                       left, right);
    return launch_status();
}

// 2D Gaussians: the tile rectangle map_gaussian_to_intersects_kernel emits
// (intersects.py:34-121; empty when radius <= 0 or the area is not positive)
// and the key of the sort, the raw depth bits (intersects.py:107-109), for
// tilelang_renderer.py:224-269.  Thread 0 also clears the status words.
__global__ __launch_bounds__(256) void k_gs_keys_rects(
    const float* __restrict__ xys, const float* __restrict__ conics,
    const int32_t* __restrict__ radii, const float* __restrict__ depths, int n, int bx, int by,
    int tbx, int tby, int4* __restrict__ rects, uint32_t* __restrict__ keys,
    int32_t* __restrict__ order, int32_t* __restrict__ status) {
    const int g = blockIdx.x * blockDim.x + threadIdx.x;
    if (g == 0) {
        status[0] = 0;
        status[1] = 0;
        status[2] = 0;
        status[3] = 0;
    }
    if (g >= n) return;
    int4 r = make_int4(0, 0, 0, 0);
    if (radii[g] > 0) {
        r = gs_tile_rect(xys[2 * g], xys[2 * g + 1], conics[3 * g], conics[3 * g + 1],
                         conics[3 * g + 2], (float)radii[g], bx, by, tbx, tby);
        if ((r.z - r.x) * (r.w - r.y) <= 0) r = make_int4(0, 0, 0, 0);
    }
    rects[g] = r;
    keys[g] = __builtin_bit_cast(uint32_t, depths[g]);
    order[g] = g;
}

extern "C" int cs_gs_bin_prepare(const float* xys, const float* conics, const int32_t* radii,
                                 const float* depths, int32_t n, int32_t img_h, int32_t img_w,
                                 int32_t block_x, int32_t block_y, int32_t* tile_rects,
                                 uint32_t* keys, int32_t* order, uint32_t* keys_alt,
                                 int32_t* vals_alt, uint32_t* radix_counts, uint32_t* scan_temp,
                                 int32_t* rank_tile_ranges, uint32_t* tile_count, uint32_t* tile_scratch, int32_t* status,
                                 hipStream_t stream) {
    if (n <= 0 || img_h <= 0 || img_w <= 0 || block_x <= 0 || block_y <= 0 ||
        (reinterpret_cast<uintptr_t>(tile_rects) & 15) != 0 ||
        (reinterpret_cast<uintptr_t>(rank_tile_ranges) & 15) != 0)
        return CS_ERR_ARGS;
    const int tbx = (img_w + block_x - 1) / block_x, tby = (img_h + block_y - 1) / block_y;
    hipLaunchKernelGGL(k_gs_keys_rects, dim3(blocks_for(n, 256)), dim3(256), 0, stream, xys,
                       conics, radii, depths, n, block_x, block_y, tbx, tby,
                       reinterpret_cast<int4*>(tile_rects), keys, order, status);
    return rank_and_count(false, keys, order, reinterpret_cast<const int4*>(tile_rects),
                          reinterpret_cast<int4*>(rank_tile_ranges), n, tbx, tby, keys_alt,
                          vals_alt, radix_counts, scan_temp, tile_count,
                          tile_scratch, status, stream);
}

extern "C" size_t cs_bin_list_elems(int32_t nprim, int32_t img_h, int32_t img_w, int32_t block_x,
                                     int32_t block_y) {
    if (nprim < 0 || img_h <= 0 || img_w <= 0 || block_x <= 0 || block_y <= 0) return 0;
    const size_t tiles = (size_t)((img_w + block_x - 1) / block_x) *
                         (size_t)((img_h + block_y - 1) / block_y);
    const int tbx = (img_w + block_x - 1) / block_x, tby = (img_h + block_y - 1) / block_y;
    const int nsegcols = (tbx + kSegTiles - 1) / kSegTiles;
    return (size_t)list_slabs(nprim, nsegcols * tby).nslab * tiles;
}

extern "C" int cs_bin_finish(const int32_t* order, const int32_t* rank_tile_ranges,
                             int32_t nprim, const int32_t* status, int64_t capacity,
                             int32_t img_h, int32_t img_w, int32_t block_x, int32_t block_y,
                             uint32_t* tile_count,
                             uint32_t* tile_scratch, int32_t* prim_ids_sorted,
                             int32_t* tile_bins, float* zero_buf, int64_t zero_n,
                             int32_t* status_host, hipStream_t stream) {
    if (nprim <= 0 || !status || capacity < 0 || img_h <= 0 || img_w <= 0 || block_x <= 0 ||
        block_y <= 0 || zero_n < 0 || (zero_n > 0 && !zero_buf))
        return CS_ERR_ARGS;
    const int tbx = (img_w + block_x - 1) / block_x, tby = (img_h + block_y - 1) / block_y;
    const int nsegcols = (tbx + kSegTiles - 1) / kSegTiles;
    const ListSlabs ls = list_slabs(nprim, nsegcols * tby);
    hipLaunchKernelGGL(k_tile_scatter, dim3(nsegcols * tby * ls.nslab),
                       dim3(kWave * kListWaves), 0, stream, order,
                       reinterpret_cast<const int4*>(rank_tile_ranges), nprim, tbx, tby, nsegcols,
                       ls.slab, ls.nslab, tile_count, tile_scratch, prim_ids_sorted, tile_bins,
                       zero_n > 0 ? zero_buf : nullptr, zero_n, status, capacity, status_host);
    return launch_status();
}

extern "C" int cs_project_cubics_2d_forward(const float* cubics_norm, const float* stroke_widths,
                                            const float* support_radii, int32_t nseg,
                                            int32_t img_h, int32_t img_w, int32_t block_x,
                                            int32_t block_y, float aabb_pad, int32_t aniso,
                                            float* cubics_px, int32_t* tile_ranges,
                                            int32_t* num_tiles_hit, hipStream_t stream) {
    if (nseg < 0 || img_h <= 0 || img_w <= 0 || block_x <= 0 || block_y <= 0) return CS_ERR_ARGS;
    if (nseg == 0) return CS_OK;
    hipLaunchKernelGGL(k_project_ref, dim3(blocks_for(nseg, 256)), dim3(256), 0, stream,
                       cubics_norm, stroke_widths, support_radii, nseg, img_h, img_w, block_x,
                       block_y, aabb_pad, aniso, cubics_px, tile_ranges, num_tiles_hit);
    return launch_status();
}

extern "C" int cs_primitive_tile_ranges(const int32_t* seg_tile_ranges, const int32_t* offs,
                                        int32_t nprim, int32_t tbx, int32_t tby,
                                        int32_t* prim_tile_ranges, int32_t* num_tiles_hit,
                                        hipStream_t stream) {
    if (nprim < 0) return CS_ERR_ARGS;
    if (nprim == 0) return CS_OK;
    hipLaunchKernelGGL(k_prim_ranges_ref, dim3(blocks_for(nprim, 256)), dim3(256), 0, stream,
                       seg_tile_ranges, offs, nprim, tbx, tby, prim_tile_ranges, num_tiles_hit);
    return launch_status();
}

extern "C" int cs_map_cubic_to_intersects(const int32_t* tile_ranges, const float* depths,
                                          const int32_t* cum_tiles_hit, int32_t nprim,
                                          int32_t tbx, int64_t* isect_ids, int32_t* curve_ids,
                                          hipStream_t stream) {
    if (nprim < 0 || tbx <= 0) return CS_ERR_ARGS;
    if (nprim == 0) return CS_OK;
    const int nb = blocks_for((int64_t)nprim * kWave, 256);
    hipLaunchKernelGGL(k_map_ref, dim3(nb < 65535 ? nb : 65535), dim3(256), 0, stream,
                       tile_ranges, depths, cum_tiles_hit, nprim, tbx, isect_ids, curve_ids);
    return launch_status();
}

extern "C" int cs_get_tile_bin_edges(const int64_t* isect_ids_sorted, int32_t num_intersects,
                                     int32_t num_rows, int32_t* tile_bins, hipStream_t stream) {
    if (num_intersects < 0 || num_rows < 0) return CS_ERR_ARGS;
    if (num_rows > 0)
        hipLaunchKernelGGL(k_fill_i32, dim3(blocks_for(2 * (int64_t)num_rows, 256)), dim3(256), 0,
                           stream, tile_bins, 2 * num_rows, 0);
    if (num_intersects > 0)
        hipLaunchKernelGGL(k_tile_bins_i64, dim3(blocks_for(num_intersects, 256)), dim3(256), 0,
                           stream, isect_ids_sorted, num_intersects, tile_bins);
    return launch_status();
}

extern "C" int cs_isect_edge_ranges(const int32_t* prim_ids_sorted, const int32_t* seg_offsets,
                                    int32_t num_intersects, int32_t edges_per_segment,
                                    int32_t* out, hipStream_t stream) {
    if (num_intersects < 0 || edges_per_segment < 1) return CS_ERR_ARGS;
    if (num_intersects == 0) return CS_OK;
    hipLaunchKernelGGL(k_isect_edge_ranges, dim3(blocks_for(num_intersects, 256)), dim3(256), 0,
                       stream, prim_ids_sorted, seg_offsets, num_intersects, edges_per_segment,
                       out);
    return launch_status();
}

extern "C" int cs_raster_records_from_edges(
    int32_t mode, const float* edges_px, int32_t num_edges, const int32_t* prim_ids_sorted,
    const int32_t* isect_edge_ranges, int64_t num_intersects, const float* colors,
    const float* opacities, const float* inv_sigma2s, const int32_t* fill_rules,
    const float* stroke_widths, int32_t nprim, const int32_t* tile_bins, int32_t num_tiles,
    int32_t* prim_edge_ranges, int32_t* edge_cull_d, int32_t* status, void* edges,
    void* edge_culls, void* prim_recs, hipStream_t stream) {
    if ((mode != 0 && mode != 1) || num_edges < 1 || nprim < 1 || num_intersects < 0 ||
        !status || (mode == 1 && !stroke_widths) || num_tiles < 0 || (num_tiles > 0 && !tile_bins))
        return CS_ERR_ARGS;
    int2* pr = reinterpret_cast<int2*>(prim_edge_ranges);
    hipLaunchKernelGGL(k_fill_i32, dim3(blocks_for(2 * (int64_t)nprim, 256)), dim3(256), 0, stream,
                       prim_edge_ranges, 2 * nprim, 0);
    hipLaunchKernelGGL(k_fill_i32, dim3(blocks_for(num_edges, 256)), dim3(256), 0, stream,
                       edge_cull_d, num_edges, 0);
    hipLaunchKernelGGL(k_fill_i32, dim3(1), dim3(256), 0, stream, status, 1, 0);
    if (num_intersects > 0) {
        const int nb = blocks_for(num_intersects, 256);
        const int2* rg = reinterpret_cast<const int2*>(isect_edge_ranges);
        hipLaunchKernelGGL(k_scatter_isect_ranges, dim3(nb), dim3(256), 0, stream, prim_ids_sorted,
                           rg, num_intersects, nprim, pr, status);
        hipLaunchKernelGGL(k_check_isect_ranges, dim3(nb), dim3(256), 0, stream, prim_ids_sorted,
                           rg, num_intersects, nprim, num_edges, pr, status);
    }
    if (num_tiles > 0)
        hipLaunchKernelGGL(k_check_tile_bins, dim3(blocks_for(num_tiles, 256)), dim3(256), 0,
                           stream, reinterpret_cast<const int2*>(tile_bins), num_tiles,
                           num_intersects, status);
    const int pb = blocks_for(nprim, 256);
    hipLaunchKernelGGL(k_edge_cull_d, dim3(pb), dim3(256), 0, stream, pr, nprim, num_edges, mode,
                       opacities, inv_sigma2s, stroke_widths, edge_cull_d);
    hipLaunchKernelGGL(k_edges_from_px, dim3(blocks_for(num_edges, 256)), dim3(256), 0, stream,
                       reinterpret_cast<const float4*>(edges_px), num_edges, edge_cull_d,
                       reinterpret_cast<EdgeRec*>(edges), reinterpret_cast<EdgeCull*>(edge_culls));
    hipLaunchKernelGGL(k_prim_recs_from_edges, dim3(pb), dim3(256), 0, stream, pr, nprim,
                       num_edges, mode, reinterpret_cast<const float4*>(edges_px), colors,
                       opacities, inv_sigma2s, fill_rules, stroke_widths,
                       reinterpret_cast<PrimRec*>(prim_recs));
    return launch_status();
}

extern "C" int cs_edge_aux_from_csr(const int32_t* segment_edge_offsets, int32_t nseg,
                                    const float* edge_t_starts, const float* edge_t_ends,
                                    int32_t num_edges, void* edge_aux, hipStream_t stream) {
    if (nseg < 0 || num_edges < 0 || !segment_edge_offsets) return CS_ERR_ARGS;
    if (nseg == 0) return CS_OK;
    hipLaunchKernelGGL(k_edge_aux_from_csr, dim3(blocks_for(nseg, 256)), dim3(256), 0, stream,
                       segment_edge_offsets, nseg, edge_t_starts, edge_t_ends, num_edges,
                       reinterpret_cast<EdgeAux*>(edge_aux));
    return launch_status();
}
