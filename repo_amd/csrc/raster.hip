// Forward and backward rasterization of flattened cubic primitives on MI355X.
//
// Launch: one 128-thread workgroup per 16x16 tile.  Unlike a block-synchronous
// design, each of the two waves owns eight tile rows (128 pixels, two per lane:
// rows r and r + 4 of one column) and walks the tile's sorted list on its own,
// so every per-entry scalar step, edge-record load and wave reduction serves
// 128 pixels.  The list entry, the primitive
// record and the edge geometry are wave-uniform, so they are read through the
// scalar cache and used as SGPR operands, and no LDS or workgroup barrier is
// needed.  A wave leaves the list when all of its pixels have reached the
// transmittance stop.
//
// Exactness-preserving culling per wave, on integer pixel ranges: geometry
// whose near ranges miss the wave's pixel rectangle is farther than the
// primitive's cull distance from every lane and cannot change any lane's
// result (outside: alpha < 1/255; inside: coverage is exactly 1.0f), so its
// distance terms are skipped; its crossing terms are skipped when its y-range
// misses the wave's eight pixel rows.  A primitive is tested as a whole with
// scalar instructions; its edges are tested lane-parallel (one edge per lane,
// one ballot per test), and the wave then evaluates only the edges that can
// matter.  Results stay bit-identical to evaluating every edge.
#include "cs_common.h"
#include "../../include/cubicsplat_hip.h"

namespace cs {

static_assert(sizeof(EdgeRec) == CS_EDGE_RECORD_BYTES, "edge record layout");
static_assert(sizeof(PrimRec) == CS_PRIM_RECORD_BYTES, "primitive record layout");
static_assert(sizeof(EdgeCull) == CS_EDGE_CULL_BYTES, "edge cull record layout");
static_assert(sizeof(EdgeAux) == CS_EDGE_AUX_BYTES, "edge aux record layout");
static_assert(sizeof(LogHeader) == 16 * kLogHeaderUnits, "raster log header layout");
static_assert(kLogBlockUnits * 16 == CS_RASTER_LOG_BLOCK_BYTES, "raster log block");

// Crossing parity equals winding & 1 (each crossing changes the winding by
// +-1), so only the winding number is tracked.
struct Geom {
    float min_d2;
    int winding;
    int best;
    float bproj, bdx, bdy;
};

// Wave-uniform integer pixel rectangle: columns [c0, c1], rows [r0, r1].
struct WaveRect {
    int c0, c1, r0, r1;
};

// Cull tests of a record's ranges against the wave (all wave-uniform).
template <class R>
__device__ __forceinline__ bool near_rows(const R& r, const WaveRect& W) {
    return span_hits(r.ny_lo, r.ny_span, W.r1);
}
template <class R>
__device__ __forceinline__ bool near_cols(const R& r, const WaveRect& W) {
    return span_hits(r.nx_lo, r.nx_span, W.c1);
}
template <class R>
__device__ __forceinline__ bool cross_rows(const R& r, const WaveRect& W) {
    return span_hits(r.cy_lo, r.cy_span, W.r1);
}
template <class R>
__device__ __forceinline__ bool near_wave(const R& r, const WaveRect& W) {
    return near_rows(r, W) && near_cols(r, W);
}

// Distance of one edge, with w = pixel - p0, cubic_splatting.py:1095-1118 /
// 1451-1484.  BEST 0 keeps the minimum, 1 also the best edge (the first strict
// minimum in visiting order), 2 also its projection and offset (for the
// gradients).  A NaN d2 leaves each variant unchanged, so all three keep the
// same minimum.
template <int BEST>
__device__ __forceinline__ void dist_term(const EdgeRec& E, int eid, float wx, float wy,
                                          Geom& G) {
    float proj = __builtin_fmaf(wx, E.ux, wy * E.uy);
    proj = fminf(fmaxf(proj, 0.0f), 1.0f);
    const float dx = __builtin_fmaf(proj, E.vx, -wx);
    const float dy = __builtin_fmaf(proj, E.vy, -wy);
    const float d2 = __builtin_fmaf(dx, dx, dy * dy);
    // Selects on one comparison, not a branch (a per-pixel branch costs an
    // exec-mask save and restore on every edge); a NaN d2 or a tie keeps the
    // current minimum.
    const bool lt = d2 < G.min_d2;
    if constexpr (BEST >= 1) G.best = lt ? eid : G.best;
    if constexpr (BEST == 2) {
        G.bproj = lt ? proj : G.bproj;
        G.bdx = lt ? dx : G.bdx;
        G.bdy = lt ? dy : G.bdy;
    }
    if constexpr (BEST >= 1) G.min_d2 = lt ? d2 : G.min_d2;
    else G.min_d2 = fminf(G.min_d2, d2);
}

// +x ray crossing of one edge, cubic_splatting.py:1119-1134 / 1485-1501.
// Upward crossing (y0 <= py < y1) counts +1 when the edge passes right of the
// pixel (cross product > 0), downward -1 when < 0.
__device__ __forceinline__ void cross_term(const EdgeRec& E, float wx, float wy, float py,
                                           Geom& G) {
    const bool b0 = E.y0 <= py, b1 = E.y1 <= py;
    const float cr = __builtin_fmaf(wy, E.vx, -(wx * E.vy));
    const bool hit = (b0 != b1) & ((b0 ? cr : -cr) > 0.0f);
    G.winding += (int)(hit & b0);
    G.winding -= (int)(hit & !b0);
}

// Primitive-level cull: true when no lane of the wave can be affected.
template <int MODE>
__device__ __forceinline__ bool prim_culled(const PrimRec& pr, const WaveRect& W) {
    if (near_wave(pr, W)) return false;
    if (MODE == 1 || pr.closed) return true;
    // Open chain in fill mode: the winding number can be non-zero left of the
    // vertices, but not when the rows miss their y-range or the wave lies
    // right of every vertex.
    return !cross_rows(pr, W) || W.c0 > pr.x_last;
}

// Lane's cull words of edge min(c + lane, e1 - 1) of a primitive whose edges
// end at e1.  Always issued (so that the compiler can count outstanding vector
// loads statically); lanes past e1 are masked at use.  Every list entry's
// primitive has at least one segment (a primitive without segments covers no
// tile), so the index is a valid edge.
__device__ __forceinline__ int4 load_culls(const EdgeCull* __restrict__ culls, int c, int e1) {
    const int lane = threadIdx.x & (kWave - 1);
    return *reinterpret_cast<const int4*>(culls + max(min(c + lane, e1 - 1), 0));
}

// Wave-uniform evaluation counters of the counting instantiation: distance
// terms and exact crossing terms evaluated (edge visits times the wave's
// active pixels), row-span crossing terms of far edges, list entries a wave
// processed past the primitive cull, and exact coverage evaluations (pixels
// within the cull distance).
struct EvalCounts {
    uint64_t dist, cross, row, entries, cover;
};

// Number of lanes below this one with their bit set in mask m.
__device__ __forceinline__ int lane_rank(uint64_t m) {
    return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                          __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// Number of the wave's pixels with `a` set (both pixels of every lane).
__device__ __forceinline__ int wave_count(const bool (&a)[kPix]) {
    int n = 0;
#pragma unroll
    for (int p = 0; p < kPix; ++p) n += __builtin_popcountll(__ballot(a[p]));
    return n;
}

// One edge record through the scalar cache as a single 32-byte load.
typedef float v8f __attribute__((ext_vector_type(8)));
__device__ __forceinline__ EdgeRec load_edge(cptr<EdgeRec> ec, int k) {
    const v8f v = *reinterpret_cast<cptr<v8f>>(ec + k);
    EdgeRec e;
    e.x0 = v[0];
    e.y0 = v[1];
    e.x1 = v[2];
    e.y1 = v[3];
    e.vx = v[4];
    e.vy = v[5];
    e.ux = v[6];
    e.uy = v[7];
    return e;
}

// Crossing term of an edge that lies entirely right of the wave (flag
// kCullFarCrossExact): +1 on the rows an upward edge spans, -1 for a
// downward one; cross_term evaluates to the same value there.
__device__ __forceinline__ void row_cross_term(const EdgeRec& E, float py, Geom& G) {
    const bool b0 = E.y0 <= py, b1 = E.y1 <= py;
    G.winding += (b0 != b1) ? (b0 ? 1 : -1) : 0;
}

// Edge classes of one 64-edge chunk starting at edge c (lane k: edge c + k,
// cull words q), as ballots.  All exact:
//   dist   near (distance can matter): distance term, and the crossing term
//          when the edge spans a row;
//   cross  exact crossing terms: spans a row and is near or not flagged;
//   right  far, spans a row, flagged, right of the wave: row-span crossing
//          term only (far, flagged, left: nothing -- its crossing term is 0).
struct ChunkMasks {
    uint64_t dist, cross, right;
};

template <bool CROSS>
__device__ __forceinline__ ChunkMasks chunk_masks(int4 q, int c, int e1, const WaveRect& W) {
    const bool in = c + (int)(threadIdx.x & (kWave - 1)) < e1;
    const bool dn = in && span_hits(packed_lo(q.x), packed_span(q.x), W.r1) &&
                    span_hits(packed_lo(q.z), packed_span(q.z), W.c1);
    ChunkMasks m;
    m.dist = __ballot(dn);
    m.cross = 0ull;
    m.right = 0ull;
    if constexpr (CROSS) {
        const bool cb = in && span_hits(packed_lo(q.y), packed_span(q.y), W.r1);
        const bool flagged = (q.w & kCullFarCrossExact) != 0;
        m.cross = __ballot(cb && (dn || !flagged));
        m.right = __ballot(cb && !dn && flagged && packed_lo(q.z) > W.c1);
    }
    return m;
}

// The edge walks of one chunk for the lane's pixels (one column px, rows
// py[p]).  Each edge record is loaded once through the scalar cache and
// evaluated for every pixel.
template <int MODE, int BEST, bool COUNT, bool CROSS>
__device__ __forceinline__ void chunk_geometry(const ChunkMasks& cm, int c,
                                               cptr<EdgeRec> edges, float px,
                                               const float (&py)[kPix], Geom (&G)[kPix],
                                               EvalCounts& n, int npix) {
    const uint64_t mdn = cm.dist, mcross = cm.cross, mright = cm.right;
    if constexpr (COUNT) {
        n.dist += (uint64_t)__builtin_popcountll(mdn) * npix;
        n.cross += (uint64_t)__builtin_popcountll(mcross) * npix;
        n.row += (uint64_t)__builtin_popcountll(mright) * npix;
    }
    const cptr<EdgeRec> ec = edges + c;
    if constexpr (BEST > 0) {
        // Distance terms in ascending edge order (the first strict minimum
        // wins ties); the crossing terms' order does not matter.
        for (uint64_t todo = mdn; todo; todo &= todo - 1) {
            const int k = (int)__builtin_ctzll(todo);
            const EdgeRec E = load_edge(ec, k);
            const float wx = px - E.x0;
            const bool cross = CROSS && ((mcross >> k) & 1);
#pragma unroll
            for (int p = 0; p < kPix; ++p) {
                const float wy = py[p] - E.y0;
                dist_term<BEST>(E, c + k, wx, wy, G[p]);
                if (cross) cross_term(E, wx, wy, py[p], G[p]);
            }
        }
    } else {
        // The minimum and the winding number do not depend on the order:
        // loops without per-edge tests.
        for (uint64_t todo = mdn & mcross; todo; todo &= todo - 1) {
            const EdgeRec E = load_edge(ec, (int)__builtin_ctzll(todo));
            const float wx = px - E.x0;
#pragma unroll
            for (int p = 0; p < kPix; ++p) {
                const float wy = py[p] - E.y0;
                dist_term<0>(E, 0, wx, wy, G[p]);
                cross_term(E, wx, wy, py[p], G[p]);
            }
        }
        for (uint64_t todo = mdn & ~mcross; todo; todo &= todo - 1) {
            const EdgeRec E = load_edge(ec, (int)__builtin_ctzll(todo));
            const float wx = px - E.x0;
#pragma unroll
            for (int p = 0; p < kPix; ++p) dist_term<0>(E, 0, wx, py[p] - E.y0, G[p]);
        }
    }
    if constexpr (CROSS) {
        for (uint64_t todo = mcross & ~mdn; todo; todo &= todo - 1) {
            const EdgeRec E = load_edge(ec, (int)__builtin_ctzll(todo));
            const float wx = px - E.x0;
#pragma unroll
            for (int p = 0; p < kPix; ++p) cross_term(E, wx, py[p] - E.y0, py[p], G[p]);
        }
        for (uint64_t todo = mright; todo; todo &= todo - 1) {
            const EdgeRec E = load_edge(ec, (int)__builtin_ctzll(todo));
#pragma unroll
            for (int p = 0; p < kPix; ++p) row_cross_term(E, py[p], G[p]);
        }
    }
}

// All edges of a primitive with per-edge culling decided lane-parallel: lane
// k holds the packed ranges of edge k of a 64-edge chunk (one vector load),
// tests them against the wave, and ballots give the edges whose distance
// and crossing terms can matter.  The wave then visits only those edges, in
// ascending index order (so the best edge is the first strict minimum, as in
// the reference), loading each one's geometry through the scalar cache.
// `first` holds the first chunk's masks (computed by the caller).
template <int MODE, int BEST, bool COUNT, bool CROSS>
__device__ __forceinline__ void prim_geometry(const PrimRec& pr, const WaveRect& W,
                                              const EdgeCull* __restrict__ culls,
                                              cptr<EdgeRec> edges, float px,
                                              const float (&py)[kPix], const ChunkMasks& first,
                                              Geom (&G)[kPix], EvalCounts& n, int npix) {
#pragma unroll
    for (int p = 0; p < kPix; ++p) {
        G[p].min_d2 = 1e30f;
        G[p].winding = 0;
        G[p].best = -1;
        G[p].bproj = 0.0f;
        G[p].bdx = 0.0f;
        G[p].bdy = 0.0f;
    }
    const int c0 = pr.e0, e1 = pr.e1;
    chunk_geometry<MODE, BEST, COUNT, CROSS>(first, c0, edges, px, py, G, n, npix);
    for (int c = c0 + kWave; c < e1; c += kWave)
        chunk_geometry<MODE, BEST, COUNT, CROSS>(
            chunk_masks<CROSS>(load_culls(culls, c, e1), c, e1, W), c, edges, px, py, G, n, npix);
}

struct Cov {
    float cov, dist, sgn, ed;
};

// Fill: cubic_splatting.py:1138-1170; stroke: cubic_polyline_splatting.py:219-226.
// A lane whose minimum over the evaluated edges exceeds its bound is decided
// without exp/div/sqrt: inside a fill beyond the cull distance its coverage is
// exactly 1.0f (1 + exp(-2 d inv_sigma) rounds to 1); outside (or for a
// stroke) beyond the smaller outside bound its alpha is below 1/255, which
// cov = 0 reproduces.  The exact branch only runs when some lane of the wave
// needs it.
// Winding-number mask of the fill rule: inside when (winding & mask) != 0
// (1: even-odd, all bits: nonzero).
__device__ __forceinline__ int rule_mask(const PrimRec& pr) { return pr.rule == 0 ? 1 : -1; }

template <int MODE>
__device__ __forceinline__ bool inside_of(const PrimRec& pr, const Geom& G) {
    return MODE == 0 && (G.winding & rule_mask(pr)) != 0;
}

// Squared distance beyond which the lane's coverage is decided in closed form:
// the cull distance inside a fill, the (smaller) outside bound elsewhere.
template <int MODE>
__device__ __forceinline__ bool needs_exact(const PrimRec& pr, const Geom& G, float D2_in,
                                            float D2_out) {
    return !(G.min_d2 > (inside_of<MODE>(pr, G) ? D2_in : D2_out));
}

template <int MODE>
__device__ __forceinline__ Cov coverage(const PrimRec& pr, const Geom& G, float D2_in,
                                        float D2_out) {
    Cov c;
    const bool inside = inside_of<MODE>(pr, G);
    c.sgn = inside ? -1.0f : 1.0f;
    c.cov = inside ? 1.0f : 0.0f;
    c.dist = 0.0f;
    c.ed = 0.0f;
    if (!(G.min_d2 > (inside ? D2_in : D2_out))) {
        c.dist = __builtin_sqrtf(fmaxf(G.min_d2, 0.0f));
        if (MODE == 0) {
            float logit = c.dist * pr.inv_sigma * 2.0f;
            if (inside) logit = -logit;
            logit = fmaxf(-60.0f, fminf(60.0f, logit));
            c.cov = 1.0f / (1.0f + spec_expf(logit));
        } else {
            c.ed = fmaxf(0.0f, c.dist - pr.half_sw);
            const float sigma = 0.5f * c.ed * c.ed * pr.inv_sigma2;
            c.cov = spec_expf(-sigma);
        }
    }
    return c;
}

__device__ __forceinline__ void flush_counts(const EvalCounts& n,
                                             unsigned long long* __restrict__ counts) {
    if ((threadIdx.x & (kWave - 1)) == 0) {
        atomicAdd(counts + 0, (unsigned long long)n.dist);
        atomicAdd(counts + 1, (unsigned long long)n.cross);
        atomicAdd(counts + 2, (unsigned long long)n.row);
        atomicAdd(counts + 3, (unsigned long long)n.entries);
        atomicAdd(counts + 4, (unsigned long long)n.cover);
    }
}

// The lane's pixels: column j, rows i[p] = first row of the wave + (lane >> 4)
// + 4 p, so that each wave covers an 8 x 16 block of its tile.
struct LanePixels {
    int j;
    int i[kPix];
    bool in_img[kPix];
    float px;
    float py[kPix];
};

__device__ __forceinline__ LanePixels lane_pixels(int r0, int c0, int img_h, int img_w) {
    LanePixels L;
    const int lane = threadIdx.x & (kWave - 1);
    L.j = c0 + (lane & 15);
    L.px = (float)L.j + 0.5f;
#pragma unroll
    for (int p = 0; p < kPix; ++p) {
        L.i[p] = r0 + (lane >> 4) + 4 * p;
        L.in_img[p] = (L.i[p] < img_h) & (L.j < img_w);
        L.py[p] = (float)L.i[p] + 0.5f;
    }
    return L;
}

// The raster's workgroups: one per 16x16 sub-block of the image (two waves
// of 16 x 8 pixels).  A tile of block_x x block_y pixels (multiples of 16)
// holds sbx x sby sub-blocks, whose 2 sbx sby waves all walk the tile's list.
// Largest tile: 16 sub-blocks (for example 64 x 64 pixels), 32 waves.
constexpr int kRasterMaxWavesPerTile = 32;

struct TileGrid {
    int tbx;    // tiles per row
    int sbtx;   // sub-blocks per row (ceil(img_w / 16))
    int nsb;    // sub-blocks in the image
    int sbx, sby;
    int waves;  // waves per tile, 2 sbx sby
    int ocap;   // positions per XCD of a tile order (order_cap(nsb))
};

// Positions per XCD of a heavy-first tile order for n sub-blocks: an eighth
// of them and an eighth of that again, so that each XCD's run of sub-blocks
// can be sized to an equal share of the cost (k_tile_order).
__host__ __device__ __forceinline__ int order_cap(int n) {
    const int q = (n + 7) >> 3;
    return q + (q >> 3) + 1;
}

struct SubBlock {
    int index;  // sub-block (the unit of the tile order and the wave costs), -1: none
    int tile;   // its tile
    int slot;   // this wave's slot among the tile's waves
    int r0, c0; // its first pixel row and column
};

// Sub-block of workgroup b: with a heavy-first order (cs_raster_tile_order,
// 8 ocap positions; the launch has 8 ocap workgroups, workgroup b on XCD
// b mod 8) the entry at position (b mod 8) ocap + b / 8, which is -1 for the
// positions past XCD b mod 8's run; else the XCD-contiguous order
// xcd_tile(b).  Any permutation gives the same results: sub-blocks are
// independent.
__device__ __forceinline__ SubBlock sub_block(const TileGrid& tg,
                                              const int32_t* __restrict__ tile_order, int wv) {
    SubBlock b;
    b.index = tile_order
                  ? __builtin_amdgcn_readfirstlane(
                        tile_order[(blockIdx.x & 7) * tg.ocap + (blockIdx.x >> 3)])
                  : xcd_tile(blockIdx.x, tg.nsb);
    const int sy = b.index / tg.sbtx, sx = b.index - sy * tg.sbtx;
    const int ty = sy / tg.sby, tx = sx / tg.sbx;
    b.tile = ty * tg.tbx + tx;
    b.slot = 2 * ((sy - ty * tg.sby) * tg.sbx + (sx - tx * tg.sbx)) + wv;
    b.r0 = sy * kTile;
    b.c0 = sx * kTile;
    return b;
}

// A wave's duration in ticks of the constant 100 MHz clock, stored in its
// slot of wave_cost [2 * sub-blocks] (two waves per sub-block) for the next
// ordering.
__device__ __forceinline__ void record_wave_cost(uint32_t* __restrict__ wave_cost, int sb,
                                                 uint64_t t_start) {
    if (wave_cost && (threadIdx.x & (kWave - 1)) == 0) {
        const uint64_t dt = __builtin_amdgcn_s_memrealtime() - t_start;
        wave_cost[2 * sb + (threadIdx.x >> 6)] = dt > 0xffffffffull ? 0xffffffffu : (uint32_t)dt;
    }
}

// Primitive-level cull of one lane's list entry (lane-parallel form of
// prim_culled): the record's near rows and columns (and, for an open chain in
// fill mode, its crossing rows and last vertex column) read with vector loads.
// All three loads are issued before any test, so that they take one memory
// round trip (a test between them would make each wait for the one before).
template <int MODE>
__device__ __forceinline__ bool prim_culled_lane(const PrimRec* __restrict__ p,
                                                 const WaveRect& W) {
    const int4 a = *reinterpret_cast<const int4*>(&p->ny_lo);  // ny_lo ny_span cy_lo cy_span
    const int4 b = *reinterpret_cast<const int4*>(&p->nx_lo);  // nx_lo nx_span x_last -
    const int closed = MODE == 1 ? 1 : p->closed;
    const bool near = span_hits(a.x, a.y, W.r1) & span_hits(b.x, b.y, W.c1);
    if (MODE == 1) return !near;
    return !near & ((closed != 0) | !span_hits(a.z, a.w, W.r1) | (W.c0 > b.z));
}

// Winding number at the pixel row r of a wave over the edges c + lane < e1 of
// one chunk, when none of them has a distance or exact crossing term for the
// wave (a far chunk): an edge whose crossing rows (exact) contain r is then
// flagged kCullFarCrossExact and misses the wave's near columns, so its
// crossing term there is +1 (upward) or -1 when it lies right of the wave and
// 0 when it lies left -- the values cross_term computes at every pixel of
// that row.  One lane per edge, two ballots; no edge geometry is read.
__device__ __forceinline__ int far_winding(int4 q, int c, int e1, const WaveRect& W) {
    const bool in = c + (int)(threadIdx.x & (kWave - 1)) < e1;
    const bool hit = in && span_hits(packed_lo(q.y), packed_span(q.y) - kWaveRowsExt, W.r0) &&
                     packed_lo(q.z) > W.c1;
    const bool up = (q.w & kCullUp) != 0;
    return __builtin_popcountll(__ballot(hit && up)) - __builtin_popcountll(__ballot(hit && !up));
}

// Far entry: no edge of the primitive lies within the cull distance of any of
// the wave's pixels (its near ranges miss the wave), and (fill) every edge
// whose y-range spans one of the wave's rows carries kCullFarCrossExact.
// Then no pixel needs the exact coverage, and every pixel has the same
// winding number: the winding number changes only across an edge, none
// crosses the wave's rectangle, and for such edges the fp32 crossing test at
// each pixel gives the geometric side (see kCullFarCrossExact).  `first`
// holds the masks of the first 64 edges and `w0` their far_winding (computed
// by the caller when first has no distance or exact crossing term): the
// entry is far when no edge has a distance or exact crossing term.  For a
// fill, `winding` receives the winding number of the wave's pixels.  Only a
// closed chain's crossing count is the same on every row of the wave: an
// open chain filled (no closing edge; a ring whose segments' shared end
// points an optimizer moved apart is one) changes it between rows where one
// of its edges ends right of the wave, so such entries take the edge walk,
// whose far edges count per row (row_cross_term).  (Comparing the counts of
// all eight rows instead was measured: slower than the edge walk.)
template <int MODE>
__device__ __forceinline__ bool entry_far(const PrimRec& pr, const WaveRect& W,
                                          const EdgeCull* __restrict__ culls,
                                          const ChunkMasks& first, int w0, int& winding) {
    if (first.dist | first.cross) return false;
    if (MODE == 0 && !pr.closed) return false;
    int w = MODE == 0 ? w0 : 0;
    for (int c = pr.e0 + kWave; c < pr.e1; c += kWave) {
        const int4 q = load_culls(culls, c, pr.e1);
        const ChunkMasks m = chunk_masks<MODE == 0>(q, c, pr.e1, W);
        if (m.dist | m.cross) return false;
        if (MODE == 0) w += far_winding(q, c, pr.e1, W);
    }
    winding = w;
    return true;
}

// Exact coverage from the squared distance: coverage()'s expressions and
// results, evaluated with sqrt_rn / spec_expf_mid / rcp_rn where they equal
// the IEEE square root, spec_expf and the IEEE division.  d2 >= +0 (or NaN,
// which fmaxf maps to 0); below 2^-96 sqrt_rn may differ from the IEEE root
// by a few ulp, but then dist inv_sigma 2 < 2^-48 1e4 2 < 2^-25 (widths are at
// least 1e-4), exp rounds to exactly 1 and the coverage is 0.5 either way.
// The logit is clamped to [-60, 60] (spec_expf_mid's range) and 1 + exp lies
// in [1, 2^87] (rcp_rn's).
template <int MODE>
__device__ __forceinline__ float exact_coverage(const PrimRec& pr, float d2, bool inside) {
    const float dist = sqrt_rn(fmaxf(d2, 0.0f));
    if (MODE == 0) {
        float logit = dist * pr.inv_sigma * 2.0f;
        if (inside) logit = -logit;
        logit = fmaxf(-60.0f, fminf(60.0f, logit));
        return rcp_rn(1.0f + spec_expf_mid(logit));
    } else {
        const float ed = fmaxf(0.0f, dist - pr.half_sw);
        const float sigma = 0.5f * ed * ed * pr.inv_sigma2;
        return spec_expf(-sigma);
    }
}

// A wave's position in the log pool: its current region [p, e) in 16-byte
// units, and whether the pool ran out (then nothing more is recorded).
struct LogCursor {
    uint32_t p, e;
    bool full;
};

// Position of a record of `units` (<= kLogBlockUnits) units.  A wave first
// fills its own region of the pool (`per_entry` units for each list entry of
// its tile, at a position fixed by the tile's list range, so no atomics);
// when a record does not fit there it reserves blocks of kLogBlockUnits from
// the shared counter (the next block is at `first` + *ctr).  kLogMissing when
// the pool is full.  Wave-uniform; every lane of the wave must be active.
__device__ __forceinline__ int32_t log_reserve(uint32_t* __restrict__ ctr, uint32_t first,
                                               uint32_t cap_units, LogCursor& c,
                                               uint32_t units) {
    if (c.full) return kLogMissing;
    if (c.p + units > c.e) {
        uint32_t base = 0;
        // An opaque copy of the lane index, so that the comparison is made
        // here rather than kept as a 64-bit lane mask in scalar registers for
        // the whole list walk (the forward has none to spare).
        int lane_o = (int)(threadIdx.x & (kWave - 1));
        asm volatile("" : "+v"(lane_o));
        if (lane_o == 0) base = first + atomicAdd(ctr, kLogBlockUnits);
        base = __builtin_amdgcn_readfirstlane(base);
        if ((uint64_t)base + kLogBlockUnits > cap_units) {
            c.full = true;
            return kLogMissing;
        }
        c.p = base;
        c.e = base + kLogBlockUnits;
    }
    const uint32_t r = c.p;
    c.p += units;
    return (int32_t)r;
}

// A wave's staged log records: LDS units [0, n) hold pool units
// [base, base + n).  Records are composed in LDS and copied to the pool in
// bulk (when the stage fills, when the next record goes to another region
// of the pool, and when the wave ends): global stores and loads share one
// completion counter, so log stores issued between the edge walks would make
// every following load wait for them.
constexpr uint32_t kLogStageUnits = 256;   // 4 KiB of LDS per wave

struct LogStage {
    uint32_t base, n;
};

__device__ __forceinline__ void log_flush(uint4* __restrict__ pool, const uint4* stage,
                                          LogStage& st) {
    // A wave-uniform loop (the lane test inside), so that the stage's
    // position and size stay scalar values.
    const uint32_t lane = threadIdx.x & (kWave - 1);
    for (uint32_t u0 = 0; u0 < st.n; u0 += kWave)
        if (u0 + lane < st.n) {
            // Streaming stores: the backward reads the log long after the
            // loss kernels, which want the caches for the image and target.
            const uint4 v = stage[u0 + lane];
            uint4* d = pool + st.base + u0 + lane;
            __builtin_nontemporal_store(v.x, &d->x);
            __builtin_nontemporal_store(v.y, &d->y);
            __builtin_nontemporal_store(v.z, &d->z);
            __builtin_nontemporal_store(v.w, &d->w);
        }
    st.n = 0;
}

__device__ __forceinline__ uint32_t pack_d2_inside(float d2, bool inside) {
    // d2 >= +0 or NaN: its sign bit is free to carry the inside flag.
    return (__builtin_bit_cast(uint32_t, d2) & 0x7fffffffu) | ((uint32_t)inside << 31);
}

// Front-to-back compositing of one entry at one pixel
// (cubic_splatting.py:1171-1183): unless the pixel has stopped, an alpha of at
// least 1/255 blends the colour at weight alpha T and multiplies T by
// 1 - alpha; the pixel stops once T reaches the transmittance stop.  Written
// with selects, so the lanes that skip the entry need no branch.
__device__ __forceinline__ void composite(const PrimRec& pr, float alpha, int g, float& T,
                                          float& C0, float& C1, float& C2, int& cur,
                                          bool& done) {
    const bool take = !done && alpha >= kAlphaMin;
    const float vis = alpha * T;
    const float nT = T * (1.0f - alpha);
    C0 = take ? __builtin_fmaf(pr.r, vis, C0) : C0;
    C1 = take ? __builtin_fmaf(pr.g, vis, C1) : C1;
    C2 = take ? __builtin_fmaf(pr.b, vis, C2) : C2;
    T = take ? nT : T;
    cur = take ? g : cur;
    done = done || (take && nT <= kTStop);
}

// The fields of a primitive record the forward uses after the primitive cull
// (three 16-byte scalar loads and one dword: colour, opacity, widths, cull
// distances, edge range, rule, closed flag); the cull ranges stay in memory (the cull
// reads them lane-parallel), so they take no scalar registers here.
__device__ __forceinline__ PrimRec load_prim_fwd(cptr<PrimRec> prims, int pid) {
    const cptr<float4> f = reinterpret_cast<cptr<float4>>(prims + pid);
    const float4 a = f[0], b = f[1];
    const int4 c = reinterpret_cast<cptr<int4>>(f)[2];
    PrimRec pr{};
    pr.r = a.x; pr.g = a.y; pr.b = a.z; pr.opacity = a.w;
    pr.inv_sigma2 = b.x; pr.inv_sigma = b.y; pr.half_sw = b.z; pr.cull_d = b.w;
    pr.e0 = c.x; pr.e1 = c.y; pr.rule = c.z; pr.closed = c.w;
    pr.cull_out = prims[pid].cull_out;
    return pr;
}

// Forward raster.  Each wave walks its tile's list in chunks of 64 entries:
// lane k tests entry k of the chunk against the wave's pixel rectangle
// (prim_culled_lane), and the wave then processes only the entries that can
// affect one of its pixels, in list order, until every pixel has reached the
// transmittance stop.  Per processed entry: the edge walk (prim_geometry),
// exact coverage for the pixels within the cull distance, the raster log
// record, compositing.  When both pixel rows of the lanes have exact pixels
// and they fit in one wave, they are gathered into lanes 0 .. n-1 with
// ds_permute, so the exact coverage (sqrt, exp, divide) runs once instead of
// once per row.  Eight waves per SIMD (the register budget that allows; a
// few scalar values then live in vector-register lanes): the edge walks wait
// on scalar loads, and more waves hide more of that wait.
// The forward's arguments that only its last instructions use (the image,
// T, index, wave cost and counter outputs).  The kernel takes them as its
// first argument, which the kernel-argument segment holds at offset 0, and
// reads them at the end through the segment pointer, so they hold no scalar
// registers during the list walk: at eight waves per SIMD a wave has 78 of
// them, and values that do not fit are kept in vector-register lanes, each
// reload a vector instruction.  LOG (the kernel's other specialization):
// the raster log is written, without a null test per entry.
struct FwdTail {
    const float* bg;
    float* out;
    float* out_planes;
    float* final_T;
    int32_t* final_idx;
    uint32_t* wave_cost;
    unsigned long long* counts;
    int out_planar;
    int img_h, img_w;
};
typedef const __attribute__((address_space(4))) FwdTail* KernargTail;

template <int MODE, bool COUNT, bool LOG>
__global__ __launch_bounds__(kRasterThreads) __attribute__((amdgpu_waves_per_eu(8))) void k_raster_fwd(
    FwdTail tail_arg, const int32_t* __restrict__ prim_ids_g, const int32_t* __restrict__ bins,
    const EdgeRec* __restrict__ edges_g, const EdgeCull* __restrict__ culls,
    const PrimRec* __restrict__ prims_g, int img_h, int img_w,
    TileGrid tg, const int32_t* __restrict__ tile_order,
    int32_t* __restrict__ log_index, uint4* __restrict__ log_pool, uint32_t* __restrict__ log_ctr,
    uint32_t log_first, uint32_t log_units, uint32_t log_per_entry) {
    (void)tail_arg;
    const uint64_t t_start = __builtin_amdgcn_s_memrealtime();
    const int lane = threadIdx.x & (kWave - 1);
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const SubBlock sb = sub_block(tg, tile_order, wv);
    if (sb.index < 0) return;  // a position past this XCD's run (whole workgroup)
    const int tile = sb.tile;
    const int r0 = sb.r0 + wv * kWaveRows;
    const LanePixels L = lane_pixels(r0, sb.c0, img_h, img_w);
    const WaveRect W{sb.c0, sb.c0 + kTile - 1, r0, r0 + kWaveRows - 1};
    const cptr<PrimRec> prims = as_const(prims_g);
    const cptr<EdgeRec> edges = as_const(edges_g);
    const int g0 = bins[2 * tile], g1 = bins[2 * tile + 1];
    float T[kPix], C0[kPix], C1[kPix], C2[kPix];
    int cur[kPix];
    bool done[kPix];
#pragma unroll
    for (int p = 0; p < kPix; ++p) {
        T[p] = 1.0f;
        C0[p] = C1[p] = C2[p] = 0.0f;
        cur[p] = 0;
        done[p] = !L.in_img[p];
    }
    EvalCounts n{};
    // This wave's own log region: per_entry units for each entry of the
    // tile's list, the tile's waves side by side.
    const uint32_t len = (uint32_t)(g1 - g0);
    const uint32_t own =
        1u + ((uint32_t)tg.waves * (uint32_t)g0 + (uint32_t)sb.slot * len) * log_per_entry;
    LogCursor lc{own, own + len * log_per_entry, false};
    __shared__ uint4 log_stage_all[kRasterThreads / kWave][kLogStageUnits];
    uint4* const stage = log_stage_all[wv];
    LogStage st{own, 0u};
    bool finished = false;
    for (int gc = g0; gc < g1 && !finished; gc += kWave) {
        const int gl = gc + lane;
        const bool in_list = gl < g1;
        const int pid_l = in_list ? prim_ids_g[gl] : 0;
        const bool keep = in_list && !prim_culled_lane<MODE>(prims_g + pid_l, W);
        uint64_t todo = __ballot(keep);
        // Entry gc + k's log index, held by lane k; stored once per chunk.
        int idx_l = kLogEmpty;
        uint64_t logged = 0;
        // The next entry's first 64 cull words are loaded one processed entry
        // ahead, so that vector load is in flight while this entry runs.
        int4 q_next = make_int4(0, -1, 0, -1);
        if (todo) {
            const int pid0 = __builtin_amdgcn_readlane(pid_l, (int)__builtin_ctzll(todo));
            q_next = load_culls(culls, prims[pid0].e0, prims[pid0].e1);
        }
        while (todo) {
            bool any_live = false;
#pragma unroll
            for (int p = 0; p < kPix; ++p) any_live |= !done[p];
            if (__ballot(any_live) == 0) {
                finished = true;
                break;
            }
            const int k = (int)__builtin_ctzll(todo);
            todo &= todo - 1;
            const int g = gc + k;
            const int pid = __builtin_amdgcn_readlane(pid_l, k);
            const PrimRec pr = load_prim_fwd(prims, pid);
            // Everything this entry needs from its first cull words is taken
            // before the next entry's load reuses their registers.
            const ChunkMasks cm0 = chunk_masks<MODE == 0>(q_next, pr.e0, pr.e1, W);
            const int w0 = (MODE == 0 && pr.closed && (cm0.dist | cm0.cross) == 0)
                               ? far_winding(q_next, pr.e0, pr.e1, W) : 0;
            if (todo) {
                const int pid2 = __builtin_amdgcn_readlane(pid_l, (int)__builtin_ctzll(todo));
                q_next = load_culls(culls, prims[pid2].e0, prims[pid2].e1);
            }
            const float D2 = pr.cull_d * pr.cull_d, D2o = pr.cull_out * pr.cull_out;
            int npix = 0;
            if constexpr (COUNT) {
                bool live[kPix];
#pragma unroll
                for (int p = 0; p < kPix; ++p) live[p] = !done[p];
                npix = wave_count(live);
                n.entries += 1;
            }
            int wnd = 0;
            // Coverage of each pixel; one compositing site below for every
            // path (so the pixels' state stays in the same registers).
            float cov[kPix];
            if (entry_far<MODE>(pr, W, culls, cm0, w0, wnd)) {
                // Uniform entry: outside (nothing to do) or, for a fill whose
                // winding number says inside, coverage 1 at every pixel.
                bool inside_all = false;
                if constexpr (MODE == 0) {
                    inside_all = (wnd & rule_mask(pr)) != 0;
                    if constexpr (COUNT) n.row += (uint64_t)(pr.e1 - pr.e0);
                }
                if (LOG) {
                    idx_l = lane == k ? (inside_all ? kLogInside : kLogEmpty) : idx_l;
                    logged |= 1ull << k;
                }
                if (!inside_all) continue;
#pragma unroll
                for (int p = 0; p < kPix; ++p) cov[p] = 1.0f;
            } else {
                Geom G[kPix];
                prim_geometry<MODE, 1, COUNT, MODE == 0>(pr, W, culls, edges, L.px, L.py, cm0, G,
                                                         n, npix);
                bool ex[kPix], ins[kPix];
#pragma unroll
                for (int p = 0; p < kPix; ++p) {
                    ins[p] = inside_of<MODE>(pr, G[p]);
                    ex[p] = !done[p] && !(G[p].min_d2 > (ins[p] ? D2 : D2o));
                    cov[p] = ins[p] ? 1.0f : 0.0f;   // closed form; exact pixels below
                }
                const uint64_t x0 = __ballot(ex[0]), x1 = __ballot(ex[kPix - 1]);
                const uint64_t in0 = MODE == 0 ? (uint64_t)__ballot(ins[0]) : 0ull;
                const uint64_t in1 = MODE == 0 ? (uint64_t)__ballot(ins[kPix - 1]) : 0ull;
                if ((in0 | in1 | x0 | x1) == 0) {
                    // No pixel inside or within the exact distance: every
                    // coverage is 0 and the entry changes nothing.
                    if (LOG) {
                        idx_l = lane == k ? kLogEmpty : idx_l;
                        logged |= 1ull << k;
                    }
                    continue;
                }
                const int n0 = __builtin_popcountll(x0), nx = n0 + __builtin_popcountll(x1);
                const int rk0 = lane_rank(x0), rk1 = lane_rank(x1);
                if constexpr (COUNT) n.cover += (uint64_t)nx;
                // Exact coverage.  gathered: lane j < nx holds exact pixel j (row 0's
                // in lane order, then row 1's) and its best edge.
                const bool gathered = n0 > 0 && nx > n0 && nx <= kWave;
                float cov_g = 0.0f;
                int best_g = 0;
                if (gathered) {
                    const int d0 = ex[0] ? rk0 : n0 + (lane - rk0);
                    const int nr1 = lane - rk1;
                    const int d1 = ex[1] ? n0 + rk1 : (nr1 < n0 ? nr1 : nr1 + (nx - n0));
                    const uint32_t a = (uint32_t)__builtin_amdgcn_ds_permute(
                        4 * d0, (int)pack_d2_inside(G[0].min_d2, ins[0]));
                    const uint32_t b = (uint32_t)__builtin_amdgcn_ds_permute(
                        4 * d1, (int)pack_d2_inside(G[1].min_d2, ins[1]));
                    const int ba = __builtin_amdgcn_ds_permute(4 * d0, G[0].best);
                    const int bb = __builtin_amdgcn_ds_permute(4 * d1, G[1].best);
                    const uint32_t v = lane < n0 ? a : b;
                    best_g = lane < n0 ? ba : bb;
                    if (lane < nx)
                        cov_g = exact_coverage<MODE>(
                            pr, __builtin_bit_cast(float, v & 0x7fffffffu), (v >> 31) != 0);
                    const float c0 = __builtin_bit_cast(
                        float,
                        __builtin_amdgcn_ds_bpermute(4 * rk0, __builtin_bit_cast(int, cov_g)));
                    const float c1 = __builtin_bit_cast(
                        float,
                        __builtin_amdgcn_ds_bpermute(4 * (n0 + rk1),
                                                     __builtin_bit_cast(int, cov_g)));
                    if (ex[0]) cov[0] = c0;
                    if (ex[1]) cov[1] = c1;
                } else {
#pragma unroll
                    for (int p = 0; p < kPix; ++p)
                        if (ex[p]) cov[p] = exact_coverage<MODE>(pr, G[p].min_d2, ins[p]);
                }
                // The log record of this entry and wave: inside and exact bits, and
                // each exact pixel's best edge and coverage, for the backward.
                if (LOG) {
                    const uint32_t units = kLogHeaderUnits + (uint32_t)((nx + 1) >> 1);
                    if (st.n + units > kLogStageUnits) log_flush(log_pool, stage, st);
                    const int32_t at = log_reserve(log_ctr, log_first, log_units, lc, units);
                    if (at >= 0) {
                        if ((uint32_t)at != st.base + st.n) {   // another region: flush first
                            log_flush(log_pool, stage, st);
                            st.base = (uint32_t)at;
                        }
                        uint4* rec = stage + st.n;
                        st.n += units;
                        int lane_o = lane;   // compared here, as in log_reserve
                        asm volatile("" : "+v"(lane_o));
                        if (lane_o == 0) {
                            rec[0] = make_uint4((uint32_t)in0, (uint32_t)(in0 >> 32),
                                                (uint32_t)in1, (uint32_t)(in1 >> 32));
                            rec[1] = make_uint4((uint32_t)x0, (uint32_t)(x0 >> 32), (uint32_t)x1,
                                                (uint32_t)(x1 >> 32));
                        }
                        int2* pairs = reinterpret_cast<int2*>(rec + kLogHeaderUnits);
                        if (gathered) {
                            if (lane < nx)
                                pairs[lane] = make_int2(best_g, __builtin_bit_cast(int, cov_g));
                        } else {
                            if (ex[0])
                                pairs[rk0] = make_int2(G[0].best, __builtin_bit_cast(int, cov[0]));
                            if (ex[1])
                                pairs[n0 + rk1] =
                                    make_int2(G[1].best, __builtin_bit_cast(int, cov[1]));
                        }
                    }
                    idx_l = lane == k ? at : idx_l;
                    logged |= 1ull << k;
                }
            }
#pragma unroll
            for (int p = 0; p < kPix; ++p)
                composite(pr, fminf(kAlphaCap, pr.opacity * cov[p]), g, T[p], C0[p], C1[p],
                          C2[p], cur[p], done[p]);
        }
        if ((logged >> lane) & 1u)
            __builtin_nontemporal_store(idx_l, log_index + (size_t)tg.waves * gl + sb.slot);
    }
    if (LOG) log_flush(log_pool, stage, st);
    const KernargTail kt = (KernargTail)__builtin_amdgcn_kernarg_segment_ptr();
    const float* const bg = kt->bg;
    float* const out = kt->out;
    float* const out_planes = kt->out_planes;
    float* const final_T = kt->final_T;
    int32_t* const final_idx = kt->final_idx;
    const int out_planar = kt->out_planar;
    img_h = kt->img_h;
    img_w = kt->img_w;
    // The image as [H, W, 3], or as three [H, W] planes (out_planar), and
    // optionally also as three planes at out_planes.
    const size_t np = (size_t)img_h * img_w;
    const size_t ch = out_planar ? np : 1;
#pragma unroll
    for (int p = 0; p < kPix; ++p) {
        if (!((L.i[p] < img_h) & (L.j < img_w))) continue;
        const size_t pix = (size_t)L.i[p] * img_w + L.j;
        __builtin_nontemporal_store(T[p], final_T + pix);
        __builtin_nontemporal_store(cur[p], final_idx + pix);
        const float o0 = __builtin_fmaf(T[p], bg[0], C0[p]);
        const float o1 = __builtin_fmaf(T[p], bg[1], C1[p]);
        const float o2 = __builtin_fmaf(T[p], bg[2], C2[p]);
        float* const o = out + (out_planar ? pix : 3 * pix);
        o[0] = o0;
        o[ch] = o1;
        o[2 * ch] = o2;
        if (out_planes) {
            out_planes[pix] = o0;
            out_planes[np + pix] = o1;
            out_planes[2 * np + pix] = o2;
        }
    }
    if constexpr (COUNT) flush_counts(n, kt->counts);
    record_wave_cost(kt->wave_cost, sb.index, t_start);
}

// First unit of the log pool: the counter of the shared blocks, which start
// after the waves' own regions.
__global__ void k_log_init(uint4* __restrict__ pool, uint32_t first_shared) {
    pool[0] = make_uint4(first_shared, 0u, 0u, 0u);
}

// n / eps for 0 <= n < 2^31 with magic = ceil(2^32 / eps) (eps >= 2): the
// high product is n/eps or one more, which one comparison corrects.
__device__ __forceinline__ int div_eps(int n, int eps, uint32_t magic) {
    if (eps == 1) return n;
    int q = (int)__umulhi((uint32_t)n, magic);
    if (q * eps > n) --q;
    return q;
}

// Quotients that only feed gradients (never the image, T or a decision) use
// the hardware reciprocal (within 1 ulp) instead of an IEEE division.
__device__ __forceinline__ float grad_rcp(float x) { return __builtin_amdgcn_rcpf(x); }

// Reference cubic-accumulation basis at t (cubic_splatting.py:2353-2371,
// :2446-2463).
__device__ __forceinline__ void basis_at(float t, float b[4]) {
    const float o = 1.0f - t;
    const float o2 = o * o, t2 = t * t;
    b[0] = o2 * o;
    b[1] = 3.0f * o2 * t;
    b[2] = 3.0f * o * t2;
    b[3] = t2 * t;
}

// The same at t = e / eps for edge e of a uniformly flattened segment.
__device__ __forceinline__ void seg_basis(int e, float inv_e, float b[4]) {
    basis_at((float)e * inv_e, b);
}

// Masks of a raster log record's header: per pixel row of the lanes, the
// inside bits and the exact bits.
struct LogHead {
    uint64_t in[kPix], xm[kPix];
};

// The header that lane k read (ha, hb: its first two units).
__device__ __forceinline__ LogHead log_head_lane(uint4 ha, uint4 hb, int k) {
    LogHead h;
    h.in[0] = ((uint64_t)__builtin_amdgcn_readlane(ha.y, k) << 32) |
              (uint32_t)__builtin_amdgcn_readlane(ha.x, k);
    h.in[1] = ((uint64_t)__builtin_amdgcn_readlane(ha.w, k) << 32) |
              (uint32_t)__builtin_amdgcn_readlane(ha.z, k);
    h.xm[0] = ((uint64_t)__builtin_amdgcn_readlane(hb.y, k) << 32) |
              (uint32_t)__builtin_amdgcn_readlane(hb.x, k);
    h.xm[1] = ((uint64_t)__builtin_amdgcn_readlane(hb.w, k) << 32) |
              (uint32_t)__builtin_amdgcn_readlane(hb.z, k);
    return h;
}

// The lane's (best edge, coverage) pairs of the record at unit `at` for its
// exact pixels (others keep their value).
__device__ __forceinline__ void log_pixels(const uint4* __restrict__ pool, int32_t at,
                                           const LogHead& h, int lane, int2 (&px)[kPix]) {
    const int2* pairs = reinterpret_cast<const int2*>(pool + at + kLogHeaderUnits);
#pragma unroll
    for (int p = 0; p < kPix; ++p)
        if ((h.xm[p] >> lane) & 1u)
            px[p] = pairs[(p == 0 ? 0 : __builtin_popcountll(h.xm[0])) + lane_rank(h.xm[p])];
}

// A wave's gradient contributions, collected in LDS and added to global
// memory in bulk (one 64-lane atomic instruction per 64 of them) when the
// buffer would overflow and when the wave ends.  One counter tracks a wave's
// outstanding vector loads and stores alike, so an atomic issued before a
// load makes the wait for that load wait for the atomic too: added right
// away, every entry's atomics would put an L2 round trip before the next
// entry's first load.  Entries with a null destination are skipped.
struct GradRec {
    float* dst;
    float v;
};
constexpr uint32_t kGradBufRecs = 256;   // 4 KiB of LDS per wave

// Per-primitive gradients (colour, opacity, inverse variance, stroke width)
// go, when the caller gives a scratch buffer, to one of kGradReplicas copies
// chosen by the workgroup's XCD (workgroup b runs on XCD b mod 8): a large
// primitive covers thousands of tiles, and their atomic additions to the same
// few addresses serialize; spread over the XCDs they do not.  A second launch
// adds the copies into the caller's arrays and clears them.
constexpr int kGradReplicas = 8;

// Largest edges-per-segment count whose accumulation weights the backward
// keeps in an LDS table.
constexpr int kBasisTable = 64;

template <int NV>
__global__ __launch_bounds__(256) void k_prim_rep_reduce(float* __restrict__ rep, int nprim,
                                                        float* __restrict__ v_col,
                                                        float* __restrict__ v_op,
                                                        float* __restrict__ v_is2,
                                                        float* __restrict__ v_sw) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)nprim * NV) return;
    const int p = (int)(i / NV), v = (int)(i - (int64_t)p * NV);
    float sum = 0.0f;
#pragma unroll
    for (int r = 0; r < kGradReplicas; ++r) {
        float* q = rep + (int64_t)r * nprim * NV + i;
        sum += *q;
        *q = 0.0f;
    }
    float* dst = v < 3 ? v_col + 3 * p + v : v == 3 ? v_op + p : v == 4 ? v_is2 + p : v_sw + p;
    *dst += sum;
}

// k_prim_rep_reduce and k_finalize in one launch, for a backward whose
// per-primitive gradients go straight to the epilogue (no hook between them):
// thread t < NV nprim adds value t % NV of primitive t / NV from its copies
// into the caller's array (the same sums as k_prim_rep_reduce) and clears
// them, and the thread of v_is2 takes v_aa from the final value (the
// expression of k_finalize); thread t < 8 nseg scales v_px[t] into v_norm[t].
// One value per thread keeps eight loads in flight per thread on about NV
// times the threads of one primitive per thread.
template <int NV>
__global__ __launch_bounds__(256) void k_prim_rep_finalize(
    float* __restrict__ rep, int nprim, float* __restrict__ v_col, float* __restrict__ v_op,
    float* __restrict__ v_is2, float* __restrict__ v_sw, const float* __restrict__ v_px,
    int nseg, float half_w, float half_h, const float* __restrict__ widths,
    float* __restrict__ v_norm, float* __restrict__ v_aa) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t < (int64_t)nseg * 8) v_norm[t] = v_px[t] * ((t & 1) ? half_h : half_w);
    if (t >= (int64_t)nprim * NV) return;
    const int p = (int)(t / NV), v = (int)(t - (int64_t)p * NV);
    float sum = 0.0f;
#pragma unroll
    for (int r = 0; r < kGradReplicas; ++r) {
        float* q = rep + (int64_t)r * nprim * NV + t;
        sum += *q;
        *q = 0.0f;
    }
    float* dst = v < 3 ? v_col + 3 * p + v : v == 3 ? v_op + p : v == 4 ? v_is2 + p : v_sw + p;
    const float tot = *dst + sum;
    *dst = tot;
    if (v == 4) {
        const float w = fmaxf(widths[p], kWidthMin);
        v_aa[p] = (-2.0f * tot) / fmaxf(w * w * w, (float)1e-12);
    }
}

struct GradBuf {
    GradRec* rec;
    uint32_t n;   // wave-uniform
};

__device__ __forceinline__ void grad_flush(GradBuf& gb) {
    const uint32_t lane = threadIdx.x & (kWave - 1);
    for (uint32_t i0 = 0; i0 < gb.n; i0 += kWave) {
        if (i0 + lane < gb.n) {
            const GradRec r = gb.rec[i0 + lane];
            if (r.dst) atomicAdd(r.dst, r.v);
        }
    }
    gb.n = 0;
}

// Records (dst, v) from the lanes with `add` (lanes 8..15 after
// wave_reduce8, each its slot); eight records per call.
__device__ __forceinline__ void grad_push8(GradBuf& gb, bool add, float* dst, float v) {
    if (gb.n + 8 > kGradBufRecs) grad_flush(gb);
    const int lane = threadIdx.x & (kWave - 1);
    if (lane >= 8 && lane < 16) gb.rec[gb.n + (lane - 8)] = GradRec{add ? dst : nullptr, v};
    gb.n += 8;
}

// Backward: the reverse traversal of cubic_splatting.py:1339-1649 (fill) and
// cubic_polyline_splatting.py:393-658 (stroke).  Per-pixel terms are those of
// the reference; the sums differ in how they are formed:
//   * per-primitive gradients: the lane's two pixels are added, then one DPP
//     wave reduction and one atomic addition per value, wave and entry
//     (issued in bulk from the wave's GradBuf);
//   * geometry: each pixel folds its best edge's endpoint gradients straight
//     into the 8 control-point gradients of the edge's cubic segment with the
//     reference's accumulation weights (cubic_splatting.py:2308-2396), then
//     the pixels that share a segment are summed (one leader pass per distinct
//     segment) and the 8 values are added to v_cubics_px (through GradBuf).
// ADAPTIVE: edges come from the de Casteljau flattening; an edge's segment and
// its leaf interval [t0, t1] are read from its aux record (the CSR weights of
// cubic_splatting.py:2432-2485) instead of being derived from its index.
// LEAN: the per-primitive sums go to the per-XCD copies (prim_rep given) and
// no contribution outputs are asked for, the case of a training step.  Without
// the other destinations' pointers and tests the kernel's wave-uniform values
// fit its scalar registers; the general instance keeps about 40 of them in
// vector-register lanes, and each reload is a vector instruction (config 3
// backward 92.5 -> 82.7 us).
template <int MODE, bool COUNT, bool ADAPTIVE, bool LEAN>
__global__ __launch_bounds__(kRasterThreads) __attribute__((amdgpu_waves_per_eu(7))) void k_raster_bwd(
    const int32_t* __restrict__ prim_ids_g, const int32_t* __restrict__ bins,
    const EdgeRec* __restrict__ edges_g, const EdgeCull* __restrict__ culls,
    const PrimRec* __restrict__ prims_g, const float* __restrict__ bg, int img_h, int img_w,
    TileGrid tg, const int32_t* __restrict__ tile_order, int eps, uint32_t eps_magic,
    const EdgeAux* __restrict__ edge_aux, const int32_t* __restrict__ log_index_g,
    const uint4* __restrict__ log_pool, const float* __restrict__ final_T,
    const int32_t* __restrict__ final_idx, const float* __restrict__ v_out, int v_planar,
    float* __restrict__ v_cubics, float* __restrict__ v_colors, float* __restrict__ v_opac,
    float* __restrict__ v_is2, float* __restrict__ v_sw, float* __restrict__ contrib_rgb,
    float* __restrict__ isect_contrib, float* __restrict__ prim_rep, int nprim,
    unsigned long long* __restrict__ counts) {
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const SubBlock sb = sub_block(tg, tile_order, wv);
    if (sb.index < 0) return;  // a position past this XCD's run (whole workgroup)
    const int tile = sb.tile;
    const int r0 = sb.r0 + wv * kWaveRows;
    const LanePixels L = lane_pixels(r0, sb.c0, img_h, img_w);
    const WaveRect W{sb.c0, sb.c0 + kTile - 1, r0, r0 + kWaveRows - 1};
    const cptr<int32_t> prim_ids = as_const(prim_ids_g);
    const cptr<PrimRec> prims = as_const(prims_g);
    const int g0 = bins[2 * tile], g1 = bins[2 * tile + 1];
    const float bg0 = bg[0], bg1 = bg[1], bg2 = bg[2];
    float T[kPix], T_final[kPix], v0[kPix], v1[kPix], v2[kPix], bg_dot[kPix];
    float b0[kPix], b1[kPix], b2[kPix];
    int fidx[kPix];
    int fmax = -1;
#pragma unroll
    for (int p = 0; p < kPix; ++p) {
        const bool in = L.in_img[p];
        const size_t pix = in ? (size_t)L.i[p] * img_w + L.j : 0;
        T[p] = in ? final_T[pix] : 1.0f;
        T_final[p] = T[p];
        fidx[p] = in ? final_idx[pix] : -1;
        // v_out: [H, W, 3] interleaved, or (v_planar) three [H, W] planes.
        const size_t hw = (size_t)img_h * img_w;
        const size_t o0 = v_planar ? pix : 3 * pix, step = v_planar ? hw : 1;
        v0[p] = in ? v_out[o0] : 0.0f;
        v1[p] = in ? v_out[o0 + step] : 0.0f;
        v2[p] = in ? v_out[o0 + 2 * step] : 0.0f;
        bg_dot[p] = __builtin_fmaf(bg2, v2[p], __builtin_fmaf(bg1, v1[p], bg0 * v0[p]));
        b0[p] = b1[p] = b2[p] = 0.0f;
        fmax = max(fmax, fidx[p]);
    }
    const bool want_contrib = !LEAN && ((contrib_rgb != nullptr) | (isect_contrib != nullptr));
    const float inv_e = 1.0f / (float)eps;
    EvalCounts n{};

    // The wave maximum is uniform; readfirstlane tells the compiler so, which
    // keeps every load that depends on the entry index scalar.
    const int gstart = min(g1 - 1, __builtin_amdgcn_readfirstlane(wave_max_i(fmax)));
    const int slot = reduce8_slot(lane & 7);
    const bool adder = (lane & ~7) == 8;
    __shared__ GradRec grad_rec_all[kRasterThreads / kWave][kGradBufRecs];
    // Uniform flattening with at most kBasisTable edges per segment: the
    // accumulation weights at t = e / eps for every e, computed once per
    // workgroup with seg_basis (so the same values) and read per pixel.
    __shared__ float4 basis_tab[kBasisTable + 1];
    const bool use_tab = !ADAPTIVE && eps <= kBasisTable;
    if (use_tab) {
        for (int e = (int)threadIdx.x; e <= eps; e += kRasterThreads) {
            float bb[4];
            seg_basis(e, inv_e, bb);
            basis_tab[e] = make_float4(bb[0], bb[1], bb[2], bb[3]);
        }
        __syncthreads();
    }
    GradBuf gbuf{grad_rec_all[wv], 0u};
    // Entries from gstart down to g0 in chunks of 64: lane k tests entry
    // gc - k with the forward's primitive cull, and the wave visits the
    // survivors in descending order -- exactly the entries the forward
    // processed at or below this wave's last contributing entry.
    for (int gc = gstart; gc >= g0; gc -= kWave) {
      const int gl = gc - lane;
      const bool in_list = gl >= g0;
      const int pid_l = in_list ? prim_ids_g[gl] : 0;
      // Lane k also reads entry gc - k's log index and, when it has a record,
      // the record's header, so that no entry waits for them.  Every entry at
      // or below gstart that passes the cull was processed by the forward,
      // so its index is written; the others are not read.
      // The entry's log index is loaded beside its cull fields (one round
      // trip for both) and kept only for entries that pass the cull.
      const int32_t at_ld = (in_list && log_index_g)
                                ? log_index_g[(size_t)tg.waves * gl + sb.slot] : kLogMissing;
      const bool kept = in_list && !prim_culled_lane<MODE>(prims_g + pid_l, W);
      const int32_t at_l = kept ? at_ld : kLogMissing;
      uint4 ha = make_uint4(0u, 0u, 0u, 0u), hb = ha;
      if (at_l >= 0) {
          ha = log_pool[at_l];
          hb = log_pool[at_l + 1];
      }
      uint64_t todo = __ballot(kept && at_l != kLogEmpty);
      while (todo) {
        const int k = (int)__builtin_ctzll(todo);
        todo &= todo - 1;
        const int g = gc - k;
        bool valid[kPix];
        bool any_valid = false;
#pragma unroll
        for (int p = 0; p < kPix; ++p) {
            valid[p] = L.in_img[p] & (g <= fidx[p]);
            any_valid |= valid[p];
        }
        if (__ballot(any_valid) == 0) continue;
        const int pid_cur = __builtin_amdgcn_readlane(pid_l, k);
        const PrimRec pr = prims[pid_cur];
        // The forward's log record of this entry and wave, if it has one
        // (entries without a contribution, kLogEmpty, are not visited).
        const int32_t at = __builtin_amdgcn_readlane(at_l, k);
        const bool uniform_inside = at == kLogInside;
        if constexpr (COUNT) n.entries += 1;
        // From the record: inside bits (the forward's winding test), exact
        // bits, and each exact pixel's best edge and coverage.  The best
        // edge's distance term is recomputed with the forward's expressions
        // (so min_d2 is the forward's minimum; the index is kept inside the
        // primitive's edge range); the coverage is the forward's own value.
        // Every other pixel is decided in closed form and needs no distance.
        // Without a record the forward's edge walk and coverage run again
        // (the same expressions, so the same values).
        Geom G[kPix];
        bool exact[kPix];
        float lcov[kPix];
        if (uniform_inside) {
#pragma unroll
            for (int p = 0; p < kPix; ++p) {
                G[p].winding = 1;
                G[p].best = pr.e0;
                G[p].min_d2 = G[p].bproj = G[p].bdx = G[p].bdy = 0.0f;
                exact[p] = false;
                lcov[p] = 1.0f;
            }
        } else if (at < 0) {
            const float D2 = pr.cull_d * pr.cull_d, D2o = pr.cull_out * pr.cull_out;
            int npix = 0;
            if constexpr (COUNT) npix = wave_count(valid);
            prim_geometry<MODE, 2, COUNT, MODE == 0>(
                pr, W, culls, as_const(edges_g), L.px, L.py,
                chunk_masks<MODE == 0>(load_culls(culls, pr.e0, pr.e1), pr.e0, pr.e1, W), G, n,
                npix);
#pragma unroll
            for (int p = 0; p < kPix; ++p) {
                const bool ins = inside_of<MODE>(pr, G[p]);
                exact[p] = !(G[p].min_d2 > (ins ? D2 : D2o));
                lcov[p] = exact[p] ? exact_coverage<MODE>(pr, G[p].min_d2, ins) : 0.0f;
                G[p].winding = (int)ins;
            }
        } else {
            const LogHead h = log_head_lane(ha, hb, k);
            int2 lpx[kPix] = {make_int2(0, 0), make_int2(0, 0)};
            log_pixels(log_pool, at, h, lane, lpx);
            if constexpr (COUNT)
                n.dist += (uint64_t)(__builtin_popcountll(h.xm[0]) +
                                     __builtin_popcountll(h.xm[1]));
            // Only exact pixels read G's distance fields (closed-form pixels
            // have dist 0 and no geometry gradient), so they are assigned
            // directly from the best edge: its d2 is the forward's minimum.
            const char* ebase = reinterpret_cast<const char*>(edges_g);
#pragma unroll
            for (int p = 0; p < kPix; ++p) {
                G[p].winding = (int)((h.in[p] >> lane) & 1u);
                exact[p] = (h.xm[p] >> lane) & 1u;
                lcov[p] = __builtin_bit_cast(float, lpx[p].y);
                const int e = min(max(lpx[p].x, pr.e0), pr.e1 - 1);
                G[p].best = e;
                G[p].min_d2 = G[p].bproj = G[p].bdx = G[p].bdy = 0.0f;
                if (exact[p]) {
                    const float4* er = reinterpret_cast<const float4*>(
                        ebase + (size_t)(uint32_t)e * sizeof(EdgeRec));
                    const float4 a = er[0], b = er[1];
                    const float wx = L.px - a.x, wy = L.py[p] - a.y;
                    float proj = __builtin_fmaf(wx, b.z, wy * b.w);
                    proj = fminf(fmaxf(proj, 0.0f), 1.0f);
                    const float dx = __builtin_fmaf(proj, b.x, -wx);
                    const float dy = __builtin_fmaf(proj, b.y, -wy);
                    G[p].min_d2 = __builtin_fmaf(dx, dx, dy * dy);
                    G[p].bproj = proj;
                    G[p].bdx = dx;
                    G[p].bdy = dy;
                }
            }
        }
        if constexpr (COUNT) {
            bool ex[kPix];
#pragma unroll
            for (int p = 0; p < kPix; ++p) ex[p] = valid[p] && exact[p];
            n.cover += (uint64_t)wave_count(ex);
        }
        // Per-primitive sums over the lane's pixels: v_r, v_g, v_b, v_opacity,
        // v_inv_sigma2, v_stroke; contribution sums r, g, b, r + g + b.
        float pv[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
        float cv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        float gx[kPix], gy[kPix];
        bool geom[kPix];
        bool contrib = false;
#pragma unroll
        for (int p = 0; p < kPix; ++p) {
            gx[p] = gy[p] = 0.0f;
            geom[p] = false;
            if (!valid[p]) continue;
            // coverage() of the forward: its value for exact pixels, the
            // closed form otherwise.  The distance only feeds gradients: a
            // fill's terms are proportional to it (hardware square root,
            // within 1 ulp), but a stroke's take dist - half_sw, which cancels
            // at the stroke's edge and is then scaled by inv_sigma2 (up to
            // 1e8 at the width floor), so strokes take the IEEE root.
            Cov c;
            const bool inside = inside_of<MODE>(pr, G[p]);
            c.sgn = inside ? -1.0f : 1.0f;
            c.cov = exact[p] ? lcov[p] : (inside ? 1.0f : 0.0f);
            const float d2c = fmaxf(G[p].min_d2, 0.0f);
            c.dist = !exact[p] ? 0.0f
                     : MODE == 1 ? sqrt_rn(d2c) : __builtin_amdgcn_sqrtf(d2c);
            c.ed = (MODE == 1 && exact[p]) ? fmaxf(0.0f, c.dist - pr.half_sw) : 0.0f;
            const float op = pr.opacity;
            const float alpha = fminf(kAlphaCap, op * c.cov);
            if (!(alpha >= kAlphaMin)) continue;
            contrib = true;
            const float ra = grad_rcp(1.0f - alpha);
            T[p] = T[p] * ra;
            const float fac = alpha * T[p];
            pv[0] = __builtin_fmaf(fac, v0[p], pv[0]);
            pv[1] = __builtin_fmaf(fac, v1[p], pv[1]);
            pv[2] = __builtin_fmaf(fac, v2[p], pv[2]);
            if (want_contrib) {
                const float cr = fac * pr.r, cg = fac * pr.g, cb = fac * pr.b;
                cv[0] += cr;
                cv[1] += cg;
                cv[2] += cb;
                cv[3] += cr + cg + cb;
            }
            float va = __builtin_fmaf(pr.r, T[p], -(b0[p] * ra)) * v0[p];
            va = __builtin_fmaf(__builtin_fmaf(pr.g, T[p], -(b1[p] * ra)), v1[p], va);
            va = __builtin_fmaf(__builtin_fmaf(pr.b, T[p], -(b2[p] * ra)), v2[p], va);
            va = __builtin_fmaf(T_final[p] * ra, -bg_dot[p], va);
            b0[p] = __builtin_fmaf(pr.r, fac, b0[p]);
            b1[p] = __builtin_fmaf(pr.g, fac, b1[p]);
            b2[p] = __builtin_fmaf(pr.b, fac, b2[p]);
            if (!(alpha < kAlphaCap)) continue;
            pv[3] = __builtin_fmaf(c.cov, va, pv[3]);
            if (MODE == 0) {
                const float v_cov = op * va;
                const float v_logit = -v_cov * c.cov * (1.0f - c.cov);
                const float v_is = v_logit * c.sgn * c.dist * 2.0f;
                pv[4] += v_is * 0.5f * grad_rcp(fmaxf(pr.inv_sigma, kEps));
                if (c.dist > kEps && G[p].best >= 0) {
                    const float v_dist = v_logit * c.sgn * pr.inv_sigma * 2.0f;
                    const float rd = grad_rcp(c.dist);
                    gx[p] = v_dist * G[p].bdx * rd;
                    gy[p] = v_dist * G[p].bdy * rd;
                    geom[p] = true;
                }
            } else {
                const float v_sigma = -op * c.cov * va;
                pv[4] += 0.5f * c.ed * c.ed * v_sigma;
                if (c.ed > 0.0f) {
                    const float v_e = v_sigma * c.ed * pr.inv_sigma2;
                    pv[5] += -0.5f * v_e;
                    if (c.dist > kEps && G[p].best >= 0) {
                        const float rd = grad_rcp(c.dist);
                        gx[p] = v_e * G[p].bdx * rd;
                        gy[p] = v_e * G[p].bdy * rd;
                        geom[p] = true;
                    }
                }
            }
        }
        if (__ballot(contrib) == 0) continue;
        // Per-primitive gradients: one 8-way transposed reduction; lanes 8..15
        // then hold the totals and each adds one of them.
        {
            constexpr int NV = MODE == 1 ? 6 : 5;
            const float t = wave_reduce8(pv);
            float* dst = (LEAN || prim_rep)
                             ? prim_rep + ((int64_t)(blockIdx.x % kGradReplicas) * nprim +
                                           pid_cur) * NV + slot
                       : slot < 3 ? v_colors + 3 * pid_cur + slot
                       : slot == 3 ? v_opac + pid_cur
                       : slot == 4 ? v_is2 + pid_cur
                                   : v_sw + pid_cur;
            grad_push8(gbuf, adder && slot < NV, dst, t);
        }
        if (want_contrib) {
            const float cw[8] = {cv[0], cv[1], cv[2], cv[3], 0.0f, 0.0f, 0.0f, 0.0f};
            const float t = wave_reduce8(cw);
            float* dst = slot < 3 ? (contrib_rgb ? contrib_rgb + 3 * pid_cur + slot : nullptr)
                                  : (isect_contrib ? isect_contrib + g : nullptr);
            grad_push8(gbuf, adder && slot < 4, dst, t);
        }
        // Geometry: endpoint gradients ((1-t) g, t g) of each pixel's best
        // edge, folded into its segment's control points.
        uint64_t pend[kPix];
        uint64_t any_pend = 0;
#pragma unroll
        for (int p = 0; p < kPix; ++p) {
            pend[p] = __ballot(geom[p]);
            any_pend |= pend[p];
        }
        if (any_pend == 0) continue;
        int gseg[kPix];
        float cp[kPix][8];
#pragma unroll
        for (int p = 0; p < kPix; ++p) {
            gseg[p] = -1;
#pragma unroll
            for (int k = 0; k < 8; ++k) cp[p][k] = 0.0f;
            if (!geom[p]) continue;
            float bs[4], be[4];
            if constexpr (ADAPTIVE) {
                const int4 ax = *reinterpret_cast<const int4*>(edge_aux + G[p].best);
                gseg[p] = ax.x;
                basis_at(__builtin_bit_cast(float, ax.y), bs);
                basis_at(__builtin_bit_cast(float, ax.z), be);
            } else {
                gseg[p] = div_eps(G[p].best, eps, eps_magic);
                const int el = G[p].best - gseg[p] * eps;
                if (use_tab) {
                    const float4 ta = basis_tab[el], tb = basis_tab[el + 1];
                    bs[0] = ta.x; bs[1] = ta.y; bs[2] = ta.z; bs[3] = ta.w;
                    be[0] = tb.x; be[1] = tb.y; be[2] = tb.z; be[3] = tb.w;
                } else {
                    seg_basis(el, inv_e, bs);
                    seg_basis(el + 1, inv_e, be);
                }
            }
            const float sx = (1.0f - G[p].bproj) * gx[p], sy = (1.0f - G[p].bproj) * gy[p];
            const float ex = G[p].bproj * gx[p], ey = G[p].bproj * gy[p];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                cp[p][2 * k] = __builtin_fmaf(ex, be[k], sx * bs[k]);
                cp[p][2 * k + 1] = __builtin_fmaf(ey, be[k], sy * bs[k]);
            }
        }
        while (any_pend) {
            // Leader: the lowest pending pixel (first pixel row before the
            // second); its segment is processed for every pixel that has it.
            const bool first_row = pend[0] != 0;
            const int leader = (int)__builtin_ctzll(first_row ? pend[0] : pend[kPix - 1]);
            const int s = __builtin_amdgcn_readlane(first_row ? gseg[0] : gseg[kPix - 1], leader);
            float sv[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
            any_pend = 0;
#pragma unroll
            for (int p = 0; p < kPix; ++p) {
                const bool mine = gseg[p] == s;
                pend[p] &= ~__ballot(mine);
                any_pend |= pend[p];
#pragma unroll
                for (int k = 0; k < 8; ++k) sv[k] += mine ? cp[p][k] : 0.0f;
            }
            const float t = wave_reduce8(sv);
            grad_push8(gbuf, adder, v_cubics + 8 * (size_t)s + slot, t);
        }
      }
    }
    grad_flush(gbuf);
    if constexpr (COUNT) flush_counts(n, counts);
}

// _accumulate_edge_grads_to_cubics_kernel (cubic_splatting.py:2308-2396) and
// the px -> normalized scaling (cubic_splatting.py:3096-3100).
__global__ __launch_bounds__(256) void k_accumulate(const float4* __restrict__ v_edges, int nseg,
                                                   int eps, float half_w, float half_h,
                                                   float* __restrict__ v_px,
                                                   float* __restrict__ v_norm) {
    const int s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= nseg) return;
    const float inv_e = 1.0f / (float)eps;

    float a[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int e = 0; e < eps; ++e) {
        float bs[4], be[4];
        seg_basis(e, inv_e, bs);
        seg_basis(e + 1, inv_e, be);
        const float4 gr = v_edges[(size_t)s * eps + e];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            a[2 * k] = __builtin_fmaf(gr.z, be[k], __builtin_fmaf(gr.x, bs[k], a[2 * k]));
            a[2 * k + 1] = __builtin_fmaf(gr.w, be[k], __builtin_fmaf(gr.y, bs[k], a[2 * k + 1]));
        }
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        v_px[(size_t)s * 8 + 2 * k] = a[2 * k];
        v_px[(size_t)s * 8 + 2 * k + 1] = a[2 * k + 1];
        if (v_norm) {
            v_norm[(size_t)s * 8 + 2 * k] = a[2 * k] * half_w;
            v_norm[(size_t)s * 8 + 2 * k + 1] = a[2 * k + 1] * half_h;
        }
    }
}

// _accumulate_edge_grads_to_cubics_csr_kernel (cubic_splatting.py:2399-2487):
// v_P_k = sum over the segment's edges of gs b_k(t0) + ge b_k(t1), fused with
// the px -> normalized scaling.
__global__ __launch_bounds__(256) void k_accumulate_csr(const float4* __restrict__ v_edges,
                                                       const float* __restrict__ t_starts,
                                                       const float* __restrict__ t_ends,
                                                       const int32_t* __restrict__ seo,
                                                       int nseg, float half_w, float half_h,
                                                       float* __restrict__ v_px,
                                                       float* __restrict__ v_norm) {
    const int s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= nseg) return;
    float a[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int e = seo[s]; e < seo[s + 1]; ++e) {
        float bs[4], be[4];
        basis_at(t_starts[e], bs);
        basis_at(t_ends[e], be);
        const float4 gr = v_edges[e];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            a[2 * k] = __builtin_fmaf(gr.z, be[k], __builtin_fmaf(gr.x, bs[k], a[2 * k]));
            a[2 * k + 1] = __builtin_fmaf(gr.w, be[k], __builtin_fmaf(gr.y, bs[k], a[2 * k + 1]));
        }
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        v_px[(size_t)s * 8 + k] = a[k];
        if (v_norm) v_norm[(size_t)s * 8 + k] = a[k] * ((k & 1) ? half_h : half_w);
    }
}

// v_cubics_norm = v_cubics_px * (W/2, H/2) (cubic_splatting.py:3096-3100) and
// v_aa_widths = -2 v_inv_sigma2 / max(w^3, 1e-12) (cubic_splatting.py:3103-3104),
// w = max(aa_width, 1e-4) (the clamp of cubic_splatting.py:2820).
__global__ __launch_bounds__(256) void k_finalize(const float* __restrict__ v_px, int nseg,
                                                 float half_w, float half_h,
                                                 const float* __restrict__ widths,
                                                 const float* __restrict__ v_is2, int P,
                                                 float* __restrict__ v_norm,
                                                 float* __restrict__ v_aa) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t < nseg * 8) v_norm[t] = v_px[t] * ((t & 1) ? half_h : half_w);
    if (t < P) {
        const float w = fmaxf(widths[t], kWidthMin);
        v_aa[t] = (-2.0f * v_is2[t]) / fmaxf(w * w * w, (float)1e-12);
    }
}

// Heavy-first tile order from the per-wave costs of a previous launch: a
// counting sort of tiles by a log-linear bucket of their cost (two waves
// summed; 128 buckets per octave), descending.  The order has order_cap(n)
// positions per XCD (XCD x's at x * cap .. x * cap + cap - 1, the rest -1),
// and workgroup b takes position (b mod 8) cap + b / 8, so the layout decides
// the schedule:
//   chunked (grid of 8, one workgroup per XCD): the tiles cut into eight
//     contiguous runs of about equal total cost (each at most cap tiles),
//     run x sorted onto XCD x's positions, so XCD x still works on its own
//     part of the image (L2 locality), starts with its longest tiles, and
//     the XCDs finish together;
//   global (grid of 1): rank r at position (r mod 8) cap + r / 8, so
//     workgroups take the longest tiles of the whole image first.
// The costs are read once, coalesced, and each tile's bucket is kept in LDS
// (16 bits per tile, up to kOrderLdsTiles tiles; larger ranges re-read the
// costs).  Neighbouring tiles cost about the same, so the counting and
// scatter passes visit tiles in the scrambled order i * kOrderStride mod m
// (a bijection: the stride is a prime above any tile count) and a wave's LDS
// atomics rarely share a bucket.  Order within a bucket is whatever the
// atomics give; every layout holds each tile once.
constexpr int kOrderThreads = 1024;
constexpr int kOrderBuckets = 4096;
constexpr int kOrderPerThread = kOrderBuckets / kOrderThreads;
constexpr int kOrderLdsTiles = 16384;
// A prime above the largest tile count (kMaxImageDim^2 / 256 = 2^20 tiles of
// 16x16), so i -> i * kOrderStride mod m is a bijection for every m.
constexpr uint64_t kOrderStride = 1048583;
static_assert(kOrderStride > (uint64_t)(kMaxImageDim / kTile) * (kMaxImageDim / kTile),
              "the tile-order stride must exceed every tile count");

__device__ __forceinline__ uint32_t cost_bucket(uint32_t c) {
    if (c == 0) return 0;
    const int e = 31 - __builtin_clz(c);                      // 0..31
    const uint32_t m = e >= 7 ? (c >> (e - 7)) & 127u : (c << (7 - e)) & 127u;
    return (uint32_t)e * 128u + m;                            // < 4096
}

// A tile's cost: its two waves' durations summed (saturating), averaged with
// the tile's previous cost when one is given.  One launch's durations vary by
// about a fifth from launch to launch (a wave's time depends on what runs
// beside it), so the running average predicts the next launch better.
struct TileCosts {
    const uint32_t* wave_cost;  // [2n] this launch's wave durations
    const uint32_t* prev;       // [n] previous costs, or null
};

__device__ __forceinline__ uint32_t tile_cost(const TileCosts& tc, int t) {
    const uint2 w = reinterpret_cast<const uint2*>(tc.wave_cost)[t];
    const uint32_t c = w.x + w.y < w.x ? 0xffffffffu : w.x + w.y;
    return tc.prev ? (uint32_t)(((uint64_t)tc.prev[t] + c + 1) >> 1) : c;
}

// Run boundaries bnd[0..8] of the chunked layout, from the tiles' costs in
// units of 16 ticks capped at 4095 (scale_cost; 12 bits, so the sums of up to
// 2^20 tiles fit 32 bits): bnd[k] the first tile whose preceding tiles cost at
// least floor(k total / 8), clamped so that every run holds at most cap tiles
// (a feasible choice: 8 cap >= n).  Every workgroup of the launch computes the
// same boundaries from the same costs.  Thread i sums the contiguous tiles
// [i per, i per + per); with per <= kOrderScanRegs the scaled costs are
// loaded coalesced and staged through LDS (the sort's bucket array, free until
// the sort) so that each thread reads its range from there; the block's
// prefix is a DPP scan per wave and the waves' totals.  The thread whose
// range takes the running cost across a mark finds its tile.
constexpr int kOrderScanRegs = 16;
constexpr int kOrderWaves = kOrderThreads / kWave;
static_assert(kOrderScanRegs * kOrderThreads <= kOrderLdsTiles, "staging fits the bucket array");

__device__ __forceinline__ uint32_t scale_cost(uint32_t c) { return min(c >> 4, 4095u); }

__device__ void order_bounds(const TileCosts& tc, int n, int cap, int* __restrict__ bnd,
                             uint16_t* __restrict__ stage, uint32_t* __restrict__ part) {
    const int tid = threadIdx.x, lane = tid & (kWave - 1), w = tid >> 6;
    const int per = (n + kOrderThreads - 1) / kOrderThreads;
    const int i0 = min(n, tid * per), i1 = min(n, i0 + per);
    const bool staged = per <= kOrderScanRegs;
    uint32_t c[kOrderScanRegs];
    uint32_t own = 0;
    if (staged) {
#pragma unroll
        for (int k = 0; k < kOrderScanRegs; ++k) {
            const int t = k * kOrderThreads + tid;
            if (t < n) stage[t] = (uint16_t)scale_cost(tile_cost(tc, t));
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < kOrderScanRegs; ++k) {
            c[k] = k < i1 - i0 ? (uint32_t)stage[i0 + k] : 0u;
            own += c[k];
        }
    } else {
        for (int i = i0; i < i1; ++i) own += scale_cost(tile_cost(tc, i));
    }
    const uint32_t incl = wave_incl_scan_u32(own);
    if (lane == kWave - 1) part[w] = incl;
    __syncthreads();
    uint32_t before = incl - own, total = 0;
    for (int x = 0; x < kOrderWaves; ++x) {
        const uint32_t px = part[x];
        before += x < w ? px : 0u;
        total += px;
    }
    for (int q = 1; q < 8; ++q) {
        const uint32_t mark = (uint32_t)((uint64_t)total * (uint64_t)q / 8ull);
        if (mark == 0) {
            if (tid == 0) bnd[q] = 0;
        } else if (before < mark && mark <= before + own) {
            uint32_t acc = before;
            int j = i0;
            if (staged) {
#pragma unroll
                for (int k = 0; k < kOrderScanRegs; ++k)
                    if (acc < mark) {
                        acc += c[k];
                        ++j;
                    }
            } else {
                while (acc < mark) acc += scale_cost(tile_cost(tc, j++));
            }
            bnd[q] = j;
        }
    }
    __syncthreads();
    if (tid == 0) {
        bnd[0] = 0;
        for (int k = 1; k < 8; ++k) {
            const int lo = max(bnd[k - 1], n - (8 - k) * cap);
            bnd[k] = min(max(bnd[k], lo), bnd[k - 1] + cap);
        }
        bnd[8] = n;
    }
    __syncthreads();
}

// cost_out (or null): the costs the order was made from, for the next order's
// average (never the same buffer as cost_in).
__global__ __launch_bounds__(kOrderThreads) void k_tile_order(const uint32_t* __restrict__ wave_cost,
                                                            const uint32_t* __restrict__ cost_in,
                                                            uint32_t* __restrict__ cost_out,
                                                            int n, int chunked,
                                                            int32_t* __restrict__ order) {
    const TileCosts tc{wave_cost, cost_in};
    __shared__ uint32_t start[kOrderBuckets];
    __shared__ uint16_t bucket[kOrderLdsTiles];
    __shared__ uint32_t part[kOrderThreads / kWave];
    __shared__ int bnd[9];
    const int tid = threadIdx.x;
    const int cap = order_cap(n);
    // This workgroup's tile range [lo, lo + m); its unused positions are -1.
    int lo = 0, m = n;
    if (chunked) {
        order_bounds(tc, n, cap, bnd, bucket, part);
        const int x = blockIdx.x;
        lo = bnd[x];
        m = bnd[x + 1] - lo;
        for (int k = m + tid; k < cap; k += kOrderThreads) order[x * cap + k] = -1;
    } else {
        for (int x = 0; x < 8; ++x)
            for (int k = ((n - x + 7) >> 3) + tid; k < cap; k += kOrderThreads)
                order[x * cap + k] = -1;
    }
    if (m <= 0) return;
    const bool cached = m <= kOrderLdsTiles;
    if (cost_out && !cached)
        for (int i = tid; i < m; i += kOrderThreads) cost_out[lo + i] = tile_cost(tc, lo + i);
    for (int i = tid; i < kOrderBuckets; i += kOrderThreads) start[i] = 0;
    if (cached) {
        // All of the thread's cost loads in flight at once.
        constexpr int kPer = kOrderLdsTiles / kOrderThreads;
        uint32_t wc[kPer];
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const int t = tid + k * kOrderThreads;
            wc[k] = t < m ? tile_cost(tc, lo + t) : 0u;
        }
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const int t = tid + k * kOrderThreads;
            if (t < m) {
                bucket[t] = (uint16_t)cost_bucket(wc[k]);
                if (cost_out) cost_out[lo + t] = wc[k];
            }
        }
    }
    __syncthreads();
    // Visit i of this thread: local tile i * stride mod m, advanced incrementally.
    const uint32_t t0 = (uint32_t)(((uint64_t)tid * kOrderStride) % (uint64_t)m);
    const uint32_t jump = (uint32_t)(((uint64_t)kOrderThreads * kOrderStride) % (uint64_t)m);
    for (int i = tid, t = (int)t0; i < m; i += kOrderThreads) {
        const uint32_t b = cached ? bucket[t] : cost_bucket(tile_cost(tc, lo + t));
        atomicAdd(&start[b], 1u);
        t += (int)jump;
        if (t >= m) t -= m;
    }
    __syncthreads();
    // Exclusive scan in descending bucket order: thread i owns descending
    // positions kOrderPerThread * i + k, i.e. buckets 4095 - 4i - k.
    uint32_t h[kOrderPerThread];
    uint32_t v = 0;
#pragma unroll
    for (int k = 0; k < kOrderPerThread; ++k) {
        h[k] = start[kOrderBuckets - 1 - kOrderPerThread * tid - k];
        v += h[k];
    }
    const uint32_t own = v;
    const int lane = tid & (kWave - 1), w = tid >> 6;
    for (int d = 1; d < kWave; d <<= 1) {
        const uint32_t o = __shfl_up(v, d);
        if (lane >= d) v += o;
    }
    if (lane == kWave - 1) part[w] = v;
    __syncthreads();
    uint32_t acc = 0;
    for (int k = 0; k < w; ++k) acc += part[k];
    acc += v - own;
#pragma unroll
    for (int k = 0; k < kOrderPerThread; ++k) {
        start[kOrderBuckets - 1 - kOrderPerThread * tid - k] = acc;
        acc += h[k];
    }
    __syncthreads();
    for (int i = tid, t = (int)t0; i < m; i += kOrderThreads) {
        const uint32_t b = cached ? bucket[t] : cost_bucket(tile_cost(tc, lo + t));
        const int rank = (int)atomicAdd(&start[b], 1u);
        order[chunked ? blockIdx.x * cap + rank : (rank & 7) * cap + (rank >> 3)] = lo + t;
        t += (int)jump;
        if (t >= m) t -= m;
    }
}

// ---------------------------------------------------------------------------
// Tiles of any size.  The 16 x 16 kernels above need tiles whose sides are
// multiples of 16; the reference takes any block_x x block_y and launches one
// thread per pixel of a tile (threads=(block_x, block_y),
// cubic_splatting.py:918-1194 and :1197-1651, cubic_polyline_splatting.py:
// 33-249 and :252-660).  These kernels keep that shape: one workgroup per
// tile, one lane per pixel (the workgroup rounded up to whole waves), each
// wave walking the tile's list and evaluating every edge of every entry at
// its pixels, with the expressions of the 16 x 16 kernels and the exact
// coverage everywhere (no culling, so no culling argument is needed for
// exactness).  Edge records and primitive records are wave-uniform scalar
// loads.
constexpr int kAnyMaxThreads = 1024;

struct AnyPixel {
    int i, j;
    bool valid;   // inside the tile and the image
    float px, py;
};

__device__ __forceinline__ AnyPixel any_pixel(int tile, int bx, int by, int tbx, int img_h,
                                              int img_w) {
    AnyPixel q;
    const int ty = tile / tbx, tx = tile - ty * tbx;
    const int t = (int)threadIdx.x;
    const bool in_tile = t < bx * by;
    const int li = in_tile ? t / bx : 0;
    const int lj = in_tile ? t - li * bx : 0;
    q.i = ty * by + li;
    q.j = tx * bx + lj;
    q.valid = in_tile && q.i < img_h && q.j < img_w;
    q.px = (float)q.j + 0.5f;
    q.py = (float)q.i + 0.5f;
    return q;
}

// Minimum distance (with the best edge, its projection and offset), and for
// fills the winding number, over edges [e0, e1) (cubic_splatting.py:1095-1134).
template <int MODE>
__device__ __forceinline__ Geom any_geometry(cptr<EdgeRec> edges, int e0, int e1, float px,
                                             float py) {
    Geom G;
    G.min_d2 = 1e30f;
    G.winding = 0;
    G.best = -1;
    G.bproj = G.bdx = G.bdy = 0.0f;
    for (int e = e0; e < e1; ++e) {
        const EdgeRec E = edges[e];
        const float wx = px - E.x0, wy = py - E.y0;
        dist_term<2>(E, e, wx, wy, G);
        if (MODE == 0) cross_term(E, wx, wy, py, G);
    }
    return G;
}

template <int MODE>
__global__ __launch_bounds__(kAnyMaxThreads) void k_raster_fwd_any(
    const int32_t* __restrict__ ids, const int32_t* __restrict__ bins,
    const EdgeRec* __restrict__ edges_g, const PrimRec* __restrict__ prims_g,
    const float* __restrict__ bg, int img_h, int img_w, int bx, int by, int tbx,
    float* __restrict__ out, int out_planar, float* __restrict__ out_planes,
    float* __restrict__ final_T, int32_t* __restrict__ final_idx) {
    const int tile = blockIdx.x;
    const AnyPixel q = any_pixel(tile, bx, by, tbx, img_h, img_w);
    const cptr<PrimRec> prims = as_const(prims_g);
    const cptr<EdgeRec> edges = as_const(edges_g);
    const int g0 = bins[2 * tile], g1 = bins[2 * tile + 1];
    float T = 1.0f, C0 = 0.0f, C1 = 0.0f, C2 = 0.0f;
    int cur = 0;
    bool done = !q.valid;
    for (int g = g0; g < g1; ++g) {
        if (__ballot(!done) == 0) break;
        const int pid = __builtin_amdgcn_readfirstlane(ids[g]);
        const PrimRec pr = load_prim_fwd(prims, pid);
        const Geom G = any_geometry<MODE>(edges, pr.e0, pr.e1, q.px, q.py);
        const Cov c = coverage<MODE>(pr, G, __builtin_huge_valf(), __builtin_huge_valf());
        composite(pr, fminf(kAlphaCap, pr.opacity * c.cov), g, T, C0, C1, C2, cur, done);
    }
    if (!q.valid) return;
    const size_t pix = (size_t)q.i * img_w + q.j;
    final_T[pix] = T;
    final_idx[pix] = cur;
    const size_t np = (size_t)img_h * img_w;
    const size_t ch = out_planar ? np : 1;
    const float o0 = __builtin_fmaf(T, bg[0], C0);
    const float o1 = __builtin_fmaf(T, bg[1], C1);
    const float o2 = __builtin_fmaf(T, bg[2], C2);
    float* const o = out + (out_planar ? pix : 3 * pix);
    o[0] = o0;
    o[ch] = o1;
    o[2 * ch] = o2;
    if (out_planes) {
        out_planes[pix] = o0;
        out_planes[np + pix] = o1;
        out_planes[2 * np + pix] = o2;
    }
}

__device__ __forceinline__ float any_wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

// Reverse walk over the entries at or below each pixel's final index,
// recomputing the geometry, the coverage and the transmittance
// (cubic_splatting.py:1339-1649).  Per-primitive gradients (and the
// contribution statistics) are summed over the wave and added by one lane;
// each pixel adds its best edge's endpoint gradients to v_edges [E] x
// (x0, y0, x1, y1), which the caller folds into the control points.
template <int MODE>
__global__ __launch_bounds__(kAnyMaxThreads) void k_raster_bwd_any(
    const int32_t* __restrict__ ids, const int32_t* __restrict__ bins,
    const EdgeRec* __restrict__ edges_g, const PrimRec* __restrict__ prims_g,
    const float* __restrict__ bg, int img_h, int img_w, int bx, int by, int tbx,
    const float* __restrict__ fT, const int32_t* __restrict__ fidx,
    const float* __restrict__ v_out, int v_planar, float* __restrict__ v_edges,
    float* __restrict__ v_col, float* __restrict__ v_op, float* __restrict__ v_is2,
    float* __restrict__ v_sw, float* __restrict__ c_rgb, float* __restrict__ c_isect) {
    const int tile = blockIdx.x;
    const AnyPixel q = any_pixel(tile, bx, by, tbx, img_h, img_w);
    const cptr<PrimRec> prims = as_const(prims_g);
    const cptr<EdgeRec> edges = as_const(edges_g);
    const int g0 = bins[2 * tile], g1 = bins[2 * tile + 1];
    const int lane = threadIdx.x & (kWave - 1);
    const size_t pix = q.valid ? (size_t)q.i * img_w + q.j : 0;
    float T = q.valid ? fT[pix] : 1.0f;
    const float T_final = T;
    const int last = q.valid ? fidx[pix] : g0 - 1;
    const size_t ch = v_planar ? (size_t)img_h * img_w : 1;
    const float* const vo = v_out + (v_planar ? pix : 3 * pix);
    const float v0 = q.valid ? vo[0] : 0.0f;
    const float v1 = q.valid ? vo[ch] : 0.0f;
    const float v2 = q.valid ? vo[2 * ch] : 0.0f;
    const float bg_dot = __builtin_fmaf(bg[2], v2, __builtin_fmaf(bg[1], v1, bg[0] * v0));
    float b0 = 0.0f, b1 = 0.0f, b2 = 0.0f;
    // The wave's last entry to visit: the largest final index among its pixels.
    int gmax = last;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) gmax = max(gmax, __shfl_xor(gmax, off, kWave));
    gmax = __builtin_amdgcn_readfirstlane(gmax < g1 - 1 ? gmax : g1 - 1);
    const bool want_contrib = (c_rgb != nullptr) | (c_isect != nullptr);
    for (int g = gmax; g >= g0; --g) {
        const int pid = __builtin_amdgcn_readfirstlane(ids[g]);
        const PrimRec pr = load_prim_fwd(prims, pid);
        const bool live = q.valid && g <= last;
        const Geom G = any_geometry<MODE>(edges, pr.e0, pr.e1, q.px, q.py);
        const Cov c = coverage<MODE>(pr, G, __builtin_huge_valf(), __builtin_huge_valf());
        const float op = pr.opacity;
        const float alpha = fminf(kAlphaCap, op * c.cov);
        const bool contrib = live && alpha >= kAlphaMin;
        if (__ballot(contrib) == 0) continue;
        float pv[6] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
        float cv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        float gx = 0.0f, gy = 0.0f;
        bool geom = false;
        if (contrib) {
            const float ra = 1.0f / (1.0f - alpha);
            T = T * ra;
            const float fac = alpha * T;
            pv[0] = fac * v0;
            pv[1] = fac * v1;
            pv[2] = fac * v2;
            if (want_contrib) {
                cv[0] = fac * pr.r;
                cv[1] = fac * pr.g;
                cv[2] = fac * pr.b;
                cv[3] = cv[0] + cv[1] + cv[2];
            }
            float va = __builtin_fmaf(pr.r, T, -(b0 * ra)) * v0;
            va = __builtin_fmaf(__builtin_fmaf(pr.g, T, -(b1 * ra)), v1, va);
            va = __builtin_fmaf(__builtin_fmaf(pr.b, T, -(b2 * ra)), v2, va);
            va = __builtin_fmaf(T_final * ra, -bg_dot, va);
            b0 = __builtin_fmaf(pr.r, fac, b0);
            b1 = __builtin_fmaf(pr.g, fac, b1);
            b2 = __builtin_fmaf(pr.b, fac, b2);
            if (alpha < kAlphaCap) {
                pv[3] = c.cov * va;
                if (MODE == 0) {
                    const float v_logit = -(op * va) * c.cov * (1.0f - c.cov);
                    pv[4] = v_logit * c.sgn * c.dist * 2.0f * 0.5f / fmaxf(pr.inv_sigma, kEps);
                    if (c.dist > kEps && G.best >= 0) {
                        const float v_dist = v_logit * c.sgn * pr.inv_sigma * 2.0f;
                        gx = v_dist * G.bdx / c.dist;
                        gy = v_dist * G.bdy / c.dist;
                        geom = true;
                    }
                } else {
                    const float v_sigma = -op * c.cov * va;
                    pv[4] = 0.5f * c.ed * c.ed * v_sigma;
                    if (c.ed > 0.0f) {
                        const float v_e = v_sigma * c.ed * pr.inv_sigma2;
                        pv[5] = -0.5f * v_e;
                        if (c.dist > kEps && G.best >= 0) {
                            gx = v_e * G.bdx / c.dist;
                            gy = v_e * G.bdy / c.dist;
                            geom = true;
                        }
                    }
                }
            }
        }
        constexpr int NV = MODE == 1 ? 6 : 5;
        float tot[6];
#pragma unroll
        for (int k = 0; k < NV; ++k) tot[k] = any_wave_sum(pv[k]);
        if (lane == 0) {
            atomicAdd(v_col + 3 * pid + 0, tot[0]);
            atomicAdd(v_col + 3 * pid + 1, tot[1]);
            atomicAdd(v_col + 3 * pid + 2, tot[2]);
            atomicAdd(v_op + pid, tot[3]);
            atomicAdd(v_is2 + pid, tot[4]);
            if (MODE == 1) atomicAdd(v_sw + pid, tot[5]);
        }
        if (want_contrib) {
            float ct[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) ct[k] = any_wave_sum(cv[k]);
            if (lane == 0) {
                if (c_rgb) {
                    atomicAdd(c_rgb + 3 * pid + 0, ct[0]);
                    atomicAdd(c_rgb + 3 * pid + 1, ct[1]);
                    atomicAdd(c_rgb + 3 * pid + 2, ct[2]);
                }
                if (c_isect) atomicAdd(c_isect + g, ct[3]);
            }
        }
        if (geom) {
            float* ve = v_edges + 4 * (size_t)G.best;
            atomicAdd(ve + 0, (1.0f - G.bproj) * gx);
            atomicAdd(ve + 1, (1.0f - G.bproj) * gy);
            atomicAdd(ve + 2, G.bproj * gx);
            atomicAdd(ve + 3, G.bproj * gy);
        }
    }
}

}  // namespace cs

using namespace cs;

static int raster_status() {
    return hipGetLastError() == hipSuccess ? CS_OK : CS_ERR_HIP;
}

struct RasterArgs {
    int mode, img_h, img_w, eps;
    TileGrid tg;
    const int32_t* ids;
    const int32_t* bins;
    const EdgeRec* E;
    const EdgeCull* C;
    const PrimRec* P;
    const float* bg;
    // forward outputs
    float* out;
    int out_planar;      // out as three [H, W] planes instead of [H, W, 3]
    float* out_planes;   // also the image as three [H, W] planes (or null)
    float* final_T;
    int32_t* final_idx;
    int32_t* log_index;     // raster log: written by the forward, read by the backward
    uint4* log_pool;
    uint32_t* log_ctr;      // shared-block counter (the next block at log_first + *log_ctr)
    uint32_t log_first;
    uint32_t log_units;     // pool capacity in 16-byte units
    uint32_t log_per_entry; // units of a wave's own region per list entry
    // backward inputs / outputs
    const float* fT;
    const int32_t* fidx;
    const float* v_out;
    int v_planar;        // v_out as three [H, W] planes instead of [H, W, 3]
    const EdgeAux* aux;  // adaptive flattening (eps == 0)
    float *v_cub, *v_col, *v_op, *v_is2, *v_sw, *c_rgb, *c_isect;
    float* prim_rep;  // per-primitive gradient copies (NULL: direct atomics)
    int nprim;
    // backward epilogue fused with the copies' reduction (NULL: none)
    const float* fin_widths;
    float *fin_norm, *fin_aa;
    int nseg;
    // evaluation counters of the counting entry points
    unsigned long long* counts;
    // heavy-first tile order (NULL: XCD order) and per-wave costs out (NULL: none)
    const int32_t* order;
    uint32_t* wave_cost;
    hipStream_t stream;
};

// Workgroups of a raster launch: one per sub-block, or with a tile order
// one per position of it (8 ocap, the positions past each XCD's run exit).
static unsigned raster_groups(const RasterArgs& a) {
    return (unsigned)(a.order ? 8 * a.tg.ocap : a.tg.nsb);
}

template <int MODE, bool COUNT>
static void launch_fwd(const RasterArgs& a) {
    const FwdTail tail{a.bg,        a.out,    a.out_planes, a.final_T, a.final_idx,
                       a.wave_cost, a.counts, a.out_planar, a.img_h,   a.img_w};
    auto kern = a.log_index ? k_raster_fwd<MODE, COUNT, true> : k_raster_fwd<MODE, COUNT, false>;
    hipLaunchKernelGGL(kern, dim3(raster_groups(a)), dim3(kRasterThreads), 0,
                       a.stream, tail, a.ids, a.bins, a.E, a.C, a.P, a.img_h, a.img_w, a.tg,
                       a.order, a.log_index, a.log_pool, a.log_ctr, a.log_first, a.log_units,
                       a.log_per_entry);
}

template <int MODE, bool COUNT, bool ADAPTIVE, bool LEAN>
static void launch_bwd4(const RasterArgs& a) {
    // ceil(2^32 / eps) for div_eps (unused when eps <= 1).
    const uint32_t magic =
        a.eps > 1 ? (uint32_t)((0x100000000ull + (uint64_t)(a.eps - 1)) / (uint64_t)a.eps) : 0u;
    hipLaunchKernelGGL((k_raster_bwd<MODE, COUNT, ADAPTIVE, LEAN>), dim3(raster_groups(a)),
                       dim3(kRasterThreads), 0, a.stream, a.ids, a.bins, a.E, a.C, a.P, a.bg,
                       a.img_h, a.img_w, a.tg, a.order, a.eps, magic, a.aux, a.log_index,
                       a.log_pool, a.fT, a.fidx,
                       a.v_out, a.v_planar,
                       a.v_cub, a.v_col,
                       a.v_op, a.v_is2, a.v_sw, a.c_rgb, a.c_isect, a.prim_rep, a.nprim,
                       a.counts);
    if (a.prim_rep && a.fin_norm) {
        constexpr int NV = MODE == 1 ? 6 : 5;
        const int64_t n = (int64_t)a.nseg * 8 > (int64_t)a.nprim * NV ? (int64_t)a.nseg * 8
                                                                       : (int64_t)a.nprim * NV;
        const float half_w = (float)(0.5 * (double)a.img_w), half_h = (float)(0.5 * (double)a.img_h);
        hipLaunchKernelGGL(k_prim_rep_finalize<NV>, dim3((unsigned)((n + 255) / 256)), dim3(256),
                           0, a.stream, a.prim_rep, a.nprim, a.v_col, a.v_op, a.v_is2, a.v_sw,
                           a.v_cub, a.nseg, half_w, half_h, a.fin_widths, a.fin_norm, a.fin_aa);
    } else if (a.prim_rep) {
        constexpr int NV = MODE == 1 ? 6 : 5;
        const int64_t n = (int64_t)a.nprim * NV;
        hipLaunchKernelGGL(k_prim_rep_reduce<NV>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                           a.stream, a.prim_rep, a.nprim, a.v_col, a.v_op, a.v_is2, a.v_sw);
    }
}

template <int MODE, bool COUNT, bool ADAPTIVE>
static void launch_bwd3(const RasterArgs& a) {
    if (!COUNT && a.prim_rep && !a.c_rgb && !a.c_isect)
        launch_bwd4<MODE, COUNT, ADAPTIVE, true>(a);
    else
        launch_bwd4<MODE, COUNT, ADAPTIVE, false>(a);
}

template <int MODE, bool COUNT>
static void launch_bwd(const RasterArgs& a) {
    if (a.aux) launch_bwd3<MODE, COUNT, true>(a);
    else launch_bwd3<MODE, COUNT, false>(a);
}

template <bool COUNT>
static void launch_fwd_mode(const RasterArgs& a) {
    if (a.mode == 0) launch_fwd<0, COUNT>(a);
    else launch_fwd<1, COUNT>(a);
}

template <bool COUNT>
static void launch_bwd_mode(const RasterArgs& a) {
    if (a.mode == 0) launch_bwd<0, COUNT>(a);
    else launch_bwd<1, COUNT>(a);
}

// Tiles of block_x x block_y pixels, both positive multiples of 16 (the
// 16x16 sub-blocks of the raster's workgroups), at most 16 waves per tile.
static bool tile_grid(int32_t img_h, int32_t img_w, int32_t block_x, int32_t block_y,
                      TileGrid& tg) {
    if (img_h <= 0 || img_w <= 0 || img_h > kMaxImageDim || img_w > kMaxImageDim ||
        block_x <= 0 || block_y <= 0 || block_x % kTile != 0 || block_y % kTile != 0)
        return false;
    tg.sbx = block_x / kTile;
    tg.sby = block_y / kTile;
    tg.waves = 2 * tg.sbx * tg.sby;
    if (tg.waves > kRasterMaxWavesPerTile) return false;
    tg.tbx = (img_w + block_x - 1) / block_x;
    tg.sbtx = (img_w + kTile - 1) / kTile;
    tg.nsb = tg.sbtx * ((img_h + kTile - 1) / kTile);
    tg.ocap = order_cap(tg.nsb);
    return true;
}

static RasterArgs raster_args(int32_t mode, const int32_t* ids, const int32_t* bins,
                              const void* edges, const void* edge_culls, const void* prims,
                              const float* bg, int32_t img_h, int32_t img_w, const TileGrid& tg,
                              int32_t eps, hipStream_t stream) {
    RasterArgs a{};
    a.mode = mode;
    a.tg = tg;
    a.img_h = img_h;
    a.img_w = img_w;
    a.eps = eps;
    a.ids = ids;
    a.bins = bins;
    a.E = reinterpret_cast<const EdgeRec*>(edges);
    a.C = reinterpret_cast<const EdgeCull*>(edge_culls);
    a.P = reinterpret_cast<const PrimRec*>(prims);
    a.bg = bg;
    a.stream = stream;
    return a;
}

static int rasterize_forward(int32_t mode, const int32_t* prim_ids_sorted,
                             const int32_t* tile_bins, const void* edges, const void* edge_culls,
                             const void* prim_recs, const float* background, int32_t img_h,
                             int32_t img_w, int32_t block_x, int32_t block_y,
                             int32_t edges_per_segment, float* out_img, int32_t out_planar,
                             float* out_planes, float* final_Ts, int32_t* final_idx,
                             int64_t num_entries,
                             int32_t* log_index, void* log_pool, int64_t log_pool_bytes,
                             int32_t log_entry_units, uint32_t* log_counter,
                             unsigned long long* eval_counts, const int32_t* tile_order,
                             uint32_t* wave_cost, hipStream_t stream) {
    // The primitive records hold each primitive's edge range, so the forward
    // does not use edges_per_segment (0 for adaptively flattened records).
    TileGrid tg;
    if ((mode != 0 && mode != 1) || edges_per_segment < 0 ||
        !tile_grid(img_h, img_w, block_x, block_y, tg))
        return CS_ERR_ARGS;
    // The waves' own regions take waves-per-tile * num_entries *
    // log_entry_units units after the counter; shared blocks follow.
    const int64_t units = log_index ? log_pool_bytes / 16 : 0;
    const int64_t cap = units < (int64_t)kLogMaxUnits ? units : (int64_t)kLogMaxUnits;
    const int64_t first_shared = 1 + (int64_t)tg.waves * num_entries * (int64_t)log_entry_units;
    if (log_index && (!log_pool || (reinterpret_cast<uintptr_t>(log_pool) & 15) != 0 ||
                      num_entries < 0 || log_entry_units < 0 || first_shared > cap))
        return CS_ERR_ARGS;
    RasterArgs a = raster_args(mode, prim_ids_sorted, tile_bins, edges, edge_culls, prim_recs,
                               background, img_h, img_w, tg, edges_per_segment, stream);
    a.out = out_img;
    a.out_planar = out_planar ? 1 : 0;
    a.out_planes = out_planes;
    a.final_T = final_Ts;
    a.final_idx = final_idx;
    a.log_index = log_index;
    a.log_pool = log_index ? reinterpret_cast<uint4*>(log_pool) : nullptr;
    a.log_units = (uint32_t)cap;
    a.log_per_entry = log_index ? (uint32_t)log_entry_units : 0u;
    a.counts = eval_counts;
    a.order = tile_order;
    a.wave_cost = wave_cost;
    // The shared blocks' counter: the caller's zeroed word, or the pool's first
    // unit, set to the first shared unit here.
    if (log_index && log_counter) {
        a.log_ctr = log_counter;
        a.log_first = (uint32_t)first_shared;
    } else if (log_index) {
        a.log_ctr = reinterpret_cast<uint32_t*>(a.log_pool);
        a.log_first = 0;
        hipLaunchKernelGGL(k_log_init, dim3(1), dim3(1), 0, stream, a.log_pool,
                           (uint32_t)first_shared);
    }
    if (eval_counts) launch_fwd_mode<true>(a);
    else launch_fwd_mode<false>(a);
    return raster_status();
}

extern "C" int cs_rasterize_forward(int32_t mode, const int32_t* prim_ids_sorted,
                                    const int32_t* tile_bins, const void* edges,
                                    const void* edge_culls, const void* prim_recs,
                                    const float* background, int32_t img_h, int32_t img_w,
                                    int32_t block_x, int32_t block_y, int32_t edges_per_segment,
                                    float* out_img, int32_t out_planar, float* out_planes,
                                    float* final_Ts, int32_t* final_idx, int64_t num_entries,
                                    int32_t* log_index,
                                    void* log_pool, int64_t log_pool_bytes,
                                    int32_t log_entry_units, uint32_t* log_counter,
                                    const int32_t* tile_order, uint32_t* wave_cost,
                                    hipStream_t stream) {
    return rasterize_forward(mode, prim_ids_sorted, tile_bins, edges, edge_culls, prim_recs,
                             background, img_h, img_w, block_x, block_y, edges_per_segment,
                             out_img, out_planar, out_planes, final_Ts,
                             final_idx, num_entries, log_index, log_pool, log_pool_bytes,
                             log_entry_units, log_counter, nullptr, tile_order, wave_cost,
                             stream);
}

extern "C" int cs_rasterize_forward_counted(int32_t mode, const int32_t* prim_ids_sorted,
                                            const int32_t* tile_bins, const void* edges,
                                            const void* edge_culls, const void* prim_recs,
                                            const float* background, int32_t img_h,
                                            int32_t img_w, int32_t block_x, int32_t block_y,
                                            int32_t edges_per_segment, float* out_img,
                                            int32_t out_planar, float* out_planes,
                                            float* final_Ts, int32_t* final_idx,
                                            int64_t num_entries,
                                            int32_t* log_index, void* log_pool,
                                            int64_t log_pool_bytes, int32_t log_entry_units,
                                            uint32_t* log_counter,
                                            unsigned long long* eval_counts,
                                            const int32_t* tile_order, uint32_t* wave_cost,
                                            hipStream_t stream) {
    if (!eval_counts) return CS_ERR_ARGS;
    return rasterize_forward(mode, prim_ids_sorted, tile_bins, edges, edge_culls, prim_recs,
                             background, img_h, img_w, block_x, block_y, edges_per_segment,
                             out_img, out_planar, out_planes, final_Ts,
                             final_idx, num_entries, log_index, log_pool, log_pool_bytes,
                             log_entry_units, log_counter, eval_counts, tile_order, wave_cost,
                             stream);
}

static int rasterize_backward(int32_t mode, const int32_t* prim_ids_sorted,
                              const int32_t* tile_bins, const void* edges,
                              const void* edge_culls, const void* prim_recs,
                              const float* background, int32_t img_h, int32_t img_w,
                              int32_t block_x, int32_t block_y,
                              int32_t edges_per_segment, const float* final_Ts,
                              const int32_t* final_idx, const float* v_output,
                              int32_t v_output_planar,
                              float* v_cubics_px, float* v_colors, float* v_opacities,
                              float* v_inv_sigma2s, float* v_stroke_widths,
                              float* curve_contrib_rgb, float* curve_isect_contrib,
                              const void* edge_aux, const int32_t* log_index,
                              const void* log_pool, unsigned long long* eval_counts,
                              int32_t nprim, float* prim_scratch,
                              const int32_t* tile_order, hipStream_t stream,
                              int32_t nseg = 0, const float* fin_widths = nullptr,
                              float* fin_norm = nullptr, float* fin_aa = nullptr) {
    TileGrid tg;
    if ((mode != 0 && mode != 1) || (edge_aux == nullptr && edges_per_segment < 1) ||
        !tile_grid(img_h, img_w, block_x, block_y, tg))
        return CS_ERR_ARGS;
    if (prim_scratch && (nprim <= 0 || !v_colors || !v_opacities || !v_inv_sigma2s))
        return CS_ERR_ARGS;
    if (mode == 1 && v_stroke_widths == nullptr) return CS_ERR_ARGS;
    if (log_index && !log_pool) return CS_ERR_ARGS;
    RasterArgs a = raster_args(mode, prim_ids_sorted, tile_bins, edges, edge_culls, prim_recs,
                               background, img_h, img_w, tg, edges_per_segment, stream);
    a.fT = final_Ts;
    a.fidx = final_idx;
    a.v_out = v_output;
    a.v_planar = v_output_planar ? 1 : 0;
    a.v_cub = v_cubics_px;
    a.v_col = v_colors;
    a.v_op = v_opacities;
    a.v_is2 = v_inv_sigma2s;
    a.v_sw = v_stroke_widths;
    a.c_rgb = curve_contrib_rgb;
    a.c_isect = curve_isect_contrib;
    a.aux = reinterpret_cast<const EdgeAux*>(edge_aux);
    if (edge_aux) a.eps = 0;
    a.log_index = const_cast<int32_t*>(log_index);
    a.log_pool = log_index ? reinterpret_cast<uint4*>(const_cast<void*>(log_pool)) : nullptr;
    a.counts = eval_counts;
    a.order = tile_order;
    a.prim_rep = prim_scratch;
    a.nprim = prim_scratch ? nprim : 0;
    a.nseg = nseg;
    a.fin_widths = fin_widths;
    a.fin_norm = fin_norm;
    a.fin_aa = fin_aa;
    if (eval_counts) launch_bwd_mode<true>(a);
    else launch_bwd_mode<false>(a);
    return raster_status();
}

extern "C" size_t cs_raster_prim_scratch_elems(int32_t nprim, int32_t mode) {
    if (nprim <= 0 || (mode != 0 && mode != 1)) return 0;
    return (size_t)kGradReplicas * (size_t)nprim * (mode == 1 ? 6u : 5u);
}

extern "C" int cs_rasterize_backward(int32_t mode, const int32_t* prim_ids_sorted,
                                     const int32_t* tile_bins, const void* edges,
                                     const void* edge_culls, const void* prim_recs,
                                     const float* background, int32_t img_h, int32_t img_w,
                                     int32_t block_x, int32_t block_y,
                                     int32_t edges_per_segment, const float* final_Ts,
                                     const int32_t* final_idx, const int32_t* log_index,
                                     const void* log_pool, const float* v_output,
                                     int32_t v_output_planar,
                                     float* v_cubics_px, float* v_colors, float* v_opacities,
                                     float* v_inv_sigma2s, float* v_stroke_widths,
                                     float* curve_contrib_rgb, float* curve_isect_contrib,
                                     int32_t nprim, float* prim_scratch,
                                     const int32_t* tile_order, hipStream_t stream) {
    return rasterize_backward(mode, prim_ids_sorted, tile_bins, edges, edge_culls, prim_recs,
                              background, img_h, img_w, block_x, block_y, edges_per_segment,
                              final_Ts, final_idx, v_output, v_output_planar, v_cubics_px,
                              v_colors, v_opacities,
                              v_inv_sigma2s, v_stroke_widths, curve_contrib_rgb,
                              curve_isect_contrib, nullptr, log_index, log_pool, nullptr, nprim,
                              prim_scratch, tile_order, stream);
}

extern "C" int cs_rasterize_backward_finalized(
    int32_t mode, const int32_t* prim_ids_sorted, const int32_t* tile_bins, const void* edges,
    const void* edge_culls, const void* prim_recs, const float* background, int32_t img_h,
    int32_t img_w, int32_t block_x, int32_t block_y, int32_t edges_per_segment,
    const float* final_Ts, const int32_t* final_idx, const int32_t* log_index,
    const void* log_pool, const float* v_output, int32_t v_output_planar, float* v_cubics_px,
    float* v_colors, float* v_opacities, float* v_inv_sigma2s, float* v_stroke_widths,
    int32_t nprim, float* prim_scratch, const int32_t* tile_order, int32_t nseg,
    const float* widths, float* v_cubics_norm, float* v_aa_widths, hipStream_t stream) {
    if (!prim_scratch || nseg < 0 || !widths || !v_cubics_norm || !v_aa_widths)
        return CS_ERR_ARGS;
    return rasterize_backward(mode, prim_ids_sorted, tile_bins, edges, edge_culls, prim_recs,
                              background, img_h, img_w, block_x, block_y, edges_per_segment,
                              final_Ts, final_idx, v_output, v_output_planar, v_cubics_px,
                              v_colors, v_opacities, v_inv_sigma2s, v_stroke_widths, nullptr,
                              nullptr, nullptr, log_index, log_pool, nullptr, nprim, prim_scratch,
                              tile_order, stream, nseg, widths, v_cubics_norm, v_aa_widths);
}

extern "C" int cs_rasterize_backward_de_casteljau(
    int32_t mode, const int32_t* prim_ids_sorted, const int32_t* tile_bins, const void* edges,
    const void* edge_culls, const void* prim_recs, const float* background, int32_t img_h,
    int32_t img_w, int32_t block_x, int32_t block_y, const void* edge_aux,
    const float* final_Ts, const int32_t* final_idx,
    const int32_t* log_index, const void* log_pool, const float* v_output,
    int32_t v_output_planar, float* v_cubics_px,
    float* v_colors, float* v_opacities, float* v_inv_sigma2s, float* v_stroke_widths,
    float* curve_contrib_rgb, float* curve_isect_contrib, int32_t nprim, float* prim_scratch,
    const int32_t* tile_order, hipStream_t stream) {
    if (!edge_aux) return CS_ERR_ARGS;
    return rasterize_backward(mode, prim_ids_sorted, tile_bins, edges, edge_culls, prim_recs,
                              background, img_h, img_w, block_x, block_y, 0, final_Ts,
                              final_idx, v_output, v_output_planar,
                              v_cubics_px, v_colors, v_opacities, v_inv_sigma2s, v_stroke_widths,
                              curve_contrib_rgb, curve_isect_contrib, edge_aux, log_index,
                              log_pool, nullptr, nprim, prim_scratch, tile_order, stream);
}

extern "C" int cs_rasterize_backward_counted(
    int32_t mode, const int32_t* prim_ids_sorted, const int32_t* tile_bins, const void* edges,
    const void* edge_culls, const void* prim_recs, const float* background, int32_t img_h,
    int32_t img_w, int32_t block_x, int32_t block_y, int32_t edges_per_segment,
    const float* final_Ts, const int32_t* final_idx,
    const int32_t* log_index, const void* log_pool, const float* v_output,
    int32_t v_output_planar, float* v_cubics_px,
    float* v_colors, float* v_opacities, float* v_inv_sigma2s, float* v_stroke_widths,
    float* curve_contrib_rgb, float* curve_isect_contrib, unsigned long long* eval_counts,
    int32_t nprim, float* prim_scratch, const int32_t* tile_order, hipStream_t stream) {
    if (!eval_counts) return CS_ERR_ARGS;
    return rasterize_backward(mode, prim_ids_sorted, tile_bins, edges, edge_culls, prim_recs,
                              background, img_h, img_w, block_x, block_y, edges_per_segment,
                              final_Ts, final_idx, v_output, v_output_planar, v_cubics_px,
                              v_colors, v_opacities, v_inv_sigma2s,
                              v_stroke_widths, curve_contrib_rgb, curve_isect_contrib, nullptr,
                              log_index, log_pool, eval_counts, nprim, prim_scratch, tile_order,
                              stream);
}

extern "C" size_t cs_raster_tile_order_elems(int32_t ntiles) {
    if (ntiles <= 0 || (uint64_t)ntiles >= kOrderStride) return 0;
    return (size_t)8 * (size_t)order_cap(ntiles);
}

static int tile_order_launch(const uint32_t* wave_cost, const uint32_t* cost_in,
                             uint32_t* cost_out, int32_t ntiles, int32_t chunked,
                             int32_t* tile_order, hipStream_t stream) {
    if (ntiles <= 0 || (uint64_t)ntiles >= kOrderStride || !wave_cost || !tile_order)
        return CS_ERR_ARGS;
    if (cost_in && cost_in == cost_out) return CS_ERR_ARGS;
    hipLaunchKernelGGL(k_tile_order, dim3(chunked ? 8 : 1), dim3(kOrderThreads), 0, stream,
                       wave_cost, cost_in, cost_out, ntiles, chunked ? 1 : 0, tile_order);
    return raster_status();
}

extern "C" int cs_raster_tile_order(const uint32_t* wave_cost, int32_t ntiles, int32_t chunked,
                                    int32_t* tile_order, hipStream_t stream) {
    return tile_order_launch(wave_cost, nullptr, nullptr, ntiles, chunked, tile_order, stream);
}

extern "C" int cs_raster_tile_order_averaged(const uint32_t* wave_cost, const uint32_t* cost_in,
                                             uint32_t* cost_out, int32_t ntiles,
                                             int32_t chunked, int32_t* tile_order,
                                             hipStream_t stream) {
    return tile_order_launch(wave_cost, cost_in, cost_out, ntiles, chunked, tile_order, stream);
}

extern "C" int cs_accumulate_edge_grads(const float* v_edges, int32_t nseg,
                                        int32_t edges_per_segment, int32_t img_h, int32_t img_w,
                                        float* v_cubics_px, float* v_cubics_norm,
                                        hipStream_t stream) {
    if (nseg < 0 || edges_per_segment < 1) return CS_ERR_ARGS;
    if (nseg == 0) return CS_OK;
    const float half_w = (float)(0.5 * (double)img_w), half_h = (float)(0.5 * (double)img_h);
    hipLaunchKernelGGL(k_accumulate, dim3((nseg + 255) / 256), dim3(256), 0, stream,
                       reinterpret_cast<const float4*>(v_edges), nseg, edges_per_segment, half_w,
                       half_h, v_cubics_px, v_cubics_norm);
    return raster_status();
}

extern "C" int cs_accumulate_edge_grads_csr(const float* v_edges, const float* edge_t_starts,
                                            const float* edge_t_ends,
                                            const int32_t* segment_edge_offsets, int32_t nseg,
                                            int32_t img_h, int32_t img_w, float* v_cubics_px,
                                            float* v_cubics_norm, hipStream_t stream) {
    if (nseg < 0 || !segment_edge_offsets) return CS_ERR_ARGS;
    if (nseg == 0) return CS_OK;
    const float half_w = (float)(0.5 * (double)img_w), half_h = (float)(0.5 * (double)img_h);
    hipLaunchKernelGGL(k_accumulate_csr, dim3((nseg + 255) / 256), dim3(256), 0, stream,
                       reinterpret_cast<const float4*>(v_edges), edge_t_starts, edge_t_ends,
                       segment_edge_offsets, nseg, half_w, half_h, v_cubics_px, v_cubics_norm);
    return raster_status();
}

extern "C" int cs_backward_finalize(const float* v_cubics_px, int32_t nseg, int32_t img_h,
                                    int32_t img_w, const float* widths,
                                    const float* v_inv_sigma2s, int32_t nprim,
                                    float* v_cubics_norm, float* v_aa_widths,
                                    hipStream_t stream) {
    if (nseg < 0 || nprim < 0) return CS_ERR_ARGS;
    const int64_t n = (int64_t)nseg * 8 > nprim ? (int64_t)nseg * 8 : nprim;
    if (n == 0) return CS_OK;
    const float half_w = (float)(0.5 * (double)img_w), half_h = (float)(0.5 * (double)img_h);
    hipLaunchKernelGGL(k_finalize, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream,
                       v_cubics_px, nseg, half_w, half_h, widths, v_inv_sigma2s, nprim,
                       v_cubics_norm, v_aa_widths);
    return raster_status();
}

// Tiles of any size (at most kAnyMaxThreads pixels): the grid is one
// workgroup per tile.
static bool any_tile_grid(int32_t img_h, int32_t img_w, int32_t block_x, int32_t block_y,
                          int& ntiles, int& tbx, int& threads) {
    if (img_h <= 0 || img_w <= 0 || img_h > kMaxImageDim || img_w > kMaxImageDim ||
        block_x <= 0 || block_y <= 0 || (int64_t)block_x * block_y > kAnyMaxThreads)
        return false;
    tbx = (img_w + block_x - 1) / block_x;
    ntiles = tbx * ((img_h + block_y - 1) / block_y);
    threads = ((block_x * block_y + kWave - 1) / kWave) * kWave;
    return true;
}

extern "C" int cs_rasterize_forward_any_tile(int32_t mode, const int32_t* prim_ids_sorted,
                                             const int32_t* tile_bins, const void* edges,
                                             const void* prim_recs, const float* background,
                                             int32_t img_h, int32_t img_w, int32_t block_x,
                                             int32_t block_y, float* out_img,
                                             int32_t out_planar, float* out_planes,
                                             float* final_Ts, int32_t* final_idx,
                                             hipStream_t stream) {
    int ntiles, tbx, threads;
    if ((mode != 0 && mode != 1) || !any_tile_grid(img_h, img_w, block_x, block_y, ntiles, tbx,
                                                    threads))
        return CS_ERR_ARGS;
    if (!tile_bins || !prim_recs || !edges || !background || !out_img || !final_Ts ||
        !final_idx)
        return CS_ERR_ARGS;
    const auto* E = reinterpret_cast<const EdgeRec*>(edges);
    const auto* P = reinterpret_cast<const PrimRec*>(prim_recs);
    if (mode == 0)
        hipLaunchKernelGGL(k_raster_fwd_any<0>, dim3(ntiles), dim3(threads), 0, stream,
                           prim_ids_sorted, tile_bins, E, P, background, img_h, img_w, block_x,
                           block_y, tbx, out_img, out_planar ? 1 : 0, out_planes, final_Ts,
                           final_idx);
    else
        hipLaunchKernelGGL(k_raster_fwd_any<1>, dim3(ntiles), dim3(threads), 0, stream,
                           prim_ids_sorted, tile_bins, E, P, background, img_h, img_w, block_x,
                           block_y, tbx, out_img, out_planar ? 1 : 0, out_planes, final_Ts,
                           final_idx);
    return raster_status();
}

extern "C" int cs_rasterize_backward_any_tile(
    int32_t mode, const int32_t* prim_ids_sorted, const int32_t* tile_bins, const void* edges,
    const void* prim_recs, const float* background, int32_t img_h, int32_t img_w,
    int32_t block_x, int32_t block_y, const float* final_Ts, const int32_t* final_idx,
    const float* v_output, int32_t v_output_planar, float* v_edges, float* v_colors,
    float* v_opacities, float* v_inv_sigma2s, float* v_stroke_widths,
    float* curve_contrib_rgb, float* curve_isect_contrib, hipStream_t stream) {
    int ntiles, tbx, threads;
    if ((mode != 0 && mode != 1) || !any_tile_grid(img_h, img_w, block_x, block_y, ntiles, tbx,
                                                    threads))
        return CS_ERR_ARGS;
    if (!tile_bins || !prim_recs || !edges || !background || !final_Ts || !final_idx ||
        !v_output || !v_edges || !v_colors || !v_opacities || !v_inv_sigma2s ||
        (mode == 1 && !v_stroke_widths))
        return CS_ERR_ARGS;
    const auto* E = reinterpret_cast<const EdgeRec*>(edges);
    const auto* P = reinterpret_cast<const PrimRec*>(prim_recs);
    const int planar = v_output_planar ? 1 : 0;
    if (mode == 0)
        hipLaunchKernelGGL(k_raster_bwd_any<0>, dim3(ntiles), dim3(threads), 0, stream,
                           prim_ids_sorted, tile_bins, E, P, background, img_h, img_w, block_x,
                           block_y, tbx, final_Ts, final_idx, v_output, planar, v_edges,
                           v_colors, v_opacities, v_inv_sigma2s, v_stroke_widths,
                           curve_contrib_rgb, curve_isect_contrib);
    else
        hipLaunchKernelGGL(k_raster_bwd_any<1>, dim3(ntiles), dim3(threads), 0, stream,
                           prim_ids_sorted, tile_bins, E, P, background, img_h, img_w, block_x,
                           block_y, tbx, final_Ts, final_idx, v_output, planar, v_edges,
                           v_colors, v_opacities, v_inv_sigma2s, v_stroke_widths,
                           curve_contrib_rgb, curve_isect_contrib);
    return raster_status();
}
