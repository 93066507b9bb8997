/*
 * C ABI of libcubicsplat_hip.so: the MI355X (gfx950) kernels of CubicSplat's
 * differentiable cubic rasterizer hot path.
 *
 * Conventions
 *   - Every pointer is a device pointer to caller-owned memory; the library
 *     allocates nothing and keeps no state between calls.
 *   - Every call only enqueues work on `stream` (no device-wide sync) and is
 *     safe to call from several host threads on different streams.
 *   - Layouts are the reference's (row-major, fp32/int32 unless stated).
 *   - Return value: CS_OK, or CS_ERR_ARGS for invalid sizes/arguments (nothing
 *     was enqueued), or CS_ERR_HIP when a launch failed.
 *
 * Reference citations are paths under /root/reference/manbo.
 */
#ifndef CUBICSPLAT_HIP_H
#define CUBICSPLAT_HIP_H

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CS_OK 0
#define CS_ERR_ARGS 1
#define CS_ERR_HIP 2

/* ---------------- building blocks ---------------- */

/* Temp element counts (uint32) for the scan and the radix sort of n items. */
size_t cs_scan_temp_elems(int32_t n);
size_t cs_radix_counts_elems(int32_t n);

/* Exclusive prefix sum of uint32 counts; *total (device int32, optional)
 * receives the sum.  Replaces torch.cumsum (ops/cubic_splatting.py:2877). */
int cs_scan_exclusive_u32(const uint32_t* in, uint32_t* out, int32_t n, uint32_t* temp,
                          int32_t* total, hipStream_t stream);

/* Stable LSD radix sort (8-bit digits) of (key, value) pairs on the low
 * key_bits bits; *_alt are same-size scratch.  Replaces torch.sort + gather
 * (ops/cubic_splatting.py:2895-2896). */
int cs_radix_sort_pairs_u32(uint32_t* keys, int32_t* vals, uint32_t* keys_alt,
                            int32_t* vals_alt, int32_t n, int32_t key_bits, uint32_t* counts,
                            uint32_t* scan_temp, hipStream_t stream);

/* ---------------- reference-layout kernels ---------------- */

/* project_cubics_2d_forward_kernel (ops/cubic_splatting.py:546-747). */
int cs_project_cubics_2d_forward(const float* cubics_norm, const float* stroke_widths,
                                 const float* support_radii, int32_t nseg, int32_t img_h,
                                 int32_t img_w, int32_t block_x, int32_t block_y, float aabb_pad,
                                 int32_t aniso, float* cubics_px, int32_t* tile_ranges,
                                 int32_t* num_tiles_hit, hipStream_t stream);

/* primitive_tile_ranges_from_segment_ranges_kernel (ops/cubic_splatting.py:2071-2137). */
int cs_primitive_tile_ranges(const int32_t* seg_tile_ranges, const int32_t* offs, int32_t nprim,
                             int32_t tbx, int32_t tby, int32_t* prim_tile_ranges,
                             int32_t* num_tiles_hit, hipStream_t stream);

/* map_cubic_to_intersects_kernel (ops/cubic_splatting.py:750-819): int64 keys
 * (tile << 32 | depth_key), primitive-major. */
int cs_map_cubic_to_intersects(const int32_t* tile_ranges, const float* depths,
                               const int32_t* cum_tiles_hit, int32_t nprim, int32_t tbx,
                               int64_t* isect_ids, int32_t* curve_ids, hipStream_t stream);

/* get_tile_bin_edges_kernel (ops/tile_bins.py:10-60); zero-fills num_rows rows first. */
int cs_get_tile_bin_edges(const int64_t* isect_ids_sorted, int32_t num_intersects,
                          int32_t num_rows, int32_t* tile_bins, hipStream_t stream);

/* _build_fill_isect_edge_ranges (ops/cubic_splatting.py:1849-1860) for
 * uniform flattening: [seg_offsets[p]*eps, seg_offsets[p+1]*eps]. */
int cs_isect_edge_ranges(const int32_t* prim_ids_sorted, const int32_t* seg_offsets,
                         int32_t num_intersects, int32_t edges_per_segment, int32_t* out,
                         hipStream_t stream);

/* ---------------- fused forward binning ---------------- */

/* Size in bytes of one flattened edge record (geometry), one edge cull
 * record, one segment record and one primitive record (opaque to callers;
 * the raster entry points read them).  The cull records pack pixel indices as
 * int16, so every entry point that takes them requires img_h, img_w <=
 * CS_MAX_IMAGE_DIM. */
#define CS_EDGE_RECORD_BYTES 32
#define CS_EDGE_CULL_BYTES 16
#define CS_SEG_RECORD_BYTES 32
#define CS_PRIM_RECORD_BYTES 80
#define CS_MAX_IMAGE_DIM 16384
/* Per-edge record of the adaptive flattening: int32 segment, float t0, t1, pad. */
#define CS_EDGE_AUX_BYTES 16

/* Stage 1 of _CubicFillSplatFunction.forward / _CubicPolylineSplatFunction.forward
 * (ops/cubic_splatting.py:2815-2880, ops/cubic_polyline_splatting.py:1027-1098):
 * project + exact AABB + tile ranges, uniform Bernstein flattening
 * (ops/cubic_splatting.py:1709-1719), per-primitive tile counts, depth ranks
 * (order[r] = primitive of depth rank r, ties by primitive id, and
 * rank_tile_ranges [nprim,4] its tile rectangle), per-tile list lengths per
 * rank slab (tile_count) and per-row-segment first slots per slab
 * (tile_scratch), each of cs_bin_list_elems(nprim, img_h, img_w, block_x,
 * block_y) elements,
 * and status[4] (device int32) = {intersection total, 1 if seg_offsets is not
 * a valid CSR of nseg segments (the kernels then clamp every range),
 * seg_offsets[0], seg_offsets[nprim]}.  T = ceil(W/block_x) * ceil(H/block_y).
 * keys, keys_alt, vals_alt hold nprim elements; radix_counts
 * cs_radix_counts_elems(nprim); scan_temp cs_scan_temp_elems(max(nprim, T)).
 * mode 0 = closed fill, 1 = open stroke (stroke_widths required). */
int cs_bin_prepare(const float* cubics_norm, const int32_t* seg_offsets, const float* colors,
                   const float* opacities, const float* depths, const int32_t* fill_rules,
                   const float* aa_widths, const float* stroke_widths, int32_t nseg,
                   int32_t nprim, int32_t img_h, int32_t img_w, int32_t block_x, int32_t block_y,
                   int32_t samples, float aabb_pad, int32_t aniso, int32_t mode,
                   float* cubics_px, int32_t* seg_tile_ranges, void* seg_recs, void* edges,
                   void* edge_culls, int32_t* prim_tile_ranges, uint32_t* num_tiles_hit,
                   float* inv_sigma2s, void* prim_recs, uint32_t* keys, int32_t* order,
                   uint32_t* keys_alt, int32_t* vals_alt, uint32_t* radix_counts,
                   uint32_t* scan_temp, int32_t* rank_tile_ranges, uint32_t* tile_count,
                   uint32_t* tile_scratch, int32_t* status,
                   hipStream_t stream);

/* ---------------- adaptive (de Casteljau) flattening ---------------- */

/* Edges per segment the adaptive flattening can emit at most: 2^d with
 * d = ceil(log2(samples - 1)) (the reference's max_depth,
 * ops/cubic_splatting.py:1733); 0 when samples < 2 or d > 24. */
int32_t cs_de_casteljau_max_edges_per_segment(int32_t samples);

/* cs_bin_prepare with flatten_method="de_casteljau"
 * (ops/cubic_splatting.py:1729-1832): each pixel-space cubic is halved at
 * t = 0.5 until it is flat within 0.5 px
 * (cubic_adaptive_flatness_flags_kernel, :1863-1915) or at depth d; its
 * leaves, left to right, become its edges (chord P0 -> P3).  edges,
 * edge_culls and edge_aux hold nseg * cs_de_casteljau_max_edges_per_segment
 * records; leaf_counts [nseg] is scratch; seg_edge_offsets [nseg + 1]
 * receives the segment CSR (seg_edge_offsets[nseg] = edge total); edge_aux
 * receives each edge's (segment, t0, t1).  scan_temp holds
 * cs_scan_temp_elems(max(nprim, T, nseg)).  The primitive records carry the
 * edge ranges, so cs_rasterize_forward reads them unchanged (pass
 * edges_per_segment 0); the backward is cs_rasterize_backward_de_casteljau. */
int cs_bin_prepare_de_casteljau(
    const float* cubics_norm, const int32_t* seg_offsets, const float* colors,
    const float* opacities, const float* depths, const int32_t* fill_rules,
    const float* aa_widths, const float* stroke_widths, int32_t nseg, int32_t nprim,
    int32_t img_h, int32_t img_w, int32_t block_x, int32_t block_y, int32_t samples,
    float aabb_pad, int32_t aniso, int32_t mode, float* cubics_px, int32_t* seg_tile_ranges,
    void* seg_recs, void* edges, void* edge_culls, int32_t* prim_tile_ranges,
    uint32_t* num_tiles_hit, float* inv_sigma2s, void* prim_recs, uint32_t* keys,
    int32_t* order, uint32_t* keys_alt, int32_t* vals_alt, uint32_t* radix_counts,
    uint32_t* scan_temp, int32_t* rank_tile_ranges, uint32_t* tile_count, uint32_t* tile_scratch,
    int32_t* status, int32_t* seg_edge_offsets,
    void* edge_aux, uint32_t* leaf_counts, hipStream_t stream);

/* _flatten_cubics_to_edges, de Casteljau branch (ops/cubic_splatting.py:1729-1832),
 * in the reference's layout: edges_px [E,2,2], edge_t_starts / edge_t_ends [E]
 * (capacity nseg * cs_de_casteljau_max_edges_per_segment(samples)),
 * segment_edge_offsets [nseg + 1] and, when not NULL, primitive_edge_offsets
 * [nprim + 1] = segment_edge_offsets[seg_offsets].  leaf_counts [nseg] and
 * scan_temp (cs_scan_temp_elems(nseg)) are scratch. */
int cs_flatten_cubics_de_casteljau(const float* cubics_px, const int32_t* seg_offsets,
                                   int32_t nprim, int32_t nseg, int32_t samples,
                                   uint32_t* leaf_counts, uint32_t* scan_temp,
                                   int32_t* segment_edge_offsets, int32_t* primitive_edge_offsets,
                                   float* edges_px, float* edge_t_starts, float* edge_t_ends,
                                   hipStream_t stream);

/* _flatten_cubics_to_edges, Bernstein branch (ops/cubic_splatting.py:1709-1719),
 * in the reference's layout: edges_px [nseg * (samples - 1), 2, 2], the
 * points of cs_bin_prepare's edge records. */
int cs_flatten_cubics_bernstein(const float* cubics_px, int32_t nseg, int32_t samples,
                                float* edges_px, hipStream_t stream);

/* cubic_adaptive_flatness_flags_kernel (ops/cubic_splatting.py:1863-1915):
 * out_flat[i] = 1 when cubic i [n,4,2] is flat within max(1e-4, tol_px) (or
 * force_flat), else 0. */
int cs_cubic_flatness_flags(const float* cubics, int32_t n, float tol_px, int32_t force_flat,
                            uint8_t* out_flat, hipStream_t stream);

/* cubic_split_half_kernel (ops/cubic_splatting.py:1968-2030): the halves of
 * each cubic [n,4,2] at t = 0.5. */
int cs_cubic_split_half(const float* cubics, int32_t n, float* left, float* right,
                        hipStream_t stream);

/* Stage 2 (ops/cubic_splatting.py:2888-2908, the sort of :2895-2896 and
 * get_tile_bin_edges of ops/tile_bins.py:10-60): each tile's primitives in
 * depth-rank order into primitive_ids_sorted and tile_bins [T,2] ((0, 0) for
 * empty tiles) -- the reference's values, bit-exact, without a global sort.
 * Inputs are stage 1's outputs, status included: the intersection total is
 * read on the device, so this call can be enqueued before the host has read
 * it.  primitive_ids_sorted holds `capacity` elements; when the total exceeds
 * it, nothing is written except empty tile_bins (the caller retries with a
 * larger buffer).  zero_buf (optional, zero_n floats) is cleared by the same
 * launch: the caller's gradient accumulators for cs_rasterize_backward, which
 * saves that step a separate fill.  status_host (optional): pinned host memory
 * (a device-accessible address of it, hipHostGetDevicePointer) that receives
 * the four status words; they are there once the launch has completed (an
 * event recorded after the call), with no separate device-to-host copy. */
/* Elements of the tile_count and tile_scratch buffers that cs_bin_prepare,
 * cs_bin_prepare_de_casteljau, cs_gs_bin_prepare and cs_bin_finish take:
 * the list build splits the depth ranks into at most 64 slabs of whole
 * 1024-rank chunks, about a thousand workgroups' worth (one workgroup per
 * slab and row segment of 64 tiles), and
 * keeps a count per slab and tile (no reference counterpart: the reference's
 * cumsum and sort need no such buffer, cubic_splatting.py:2877-2896). */
size_t cs_bin_list_elems(int32_t nprim, int32_t img_h, int32_t img_w, int32_t block_x,
                         int32_t block_y);

int cs_bin_finish(const int32_t* order, const int32_t* rank_tile_ranges, int32_t nprim,
                  const int32_t* status, int64_t capacity, int32_t img_h, int32_t img_w,
                  int32_t block_x, int32_t block_y, uint32_t* tile_count, uint32_t* tile_scratch,
                  int32_t* prim_ids_sorted,
                  int32_t* tile_bins, float* zero_buf, int64_t zero_n, int32_t* status_host,
                  hipStream_t stream);

/* ---------------- rasterization ---------------- */

/* Tiles: every raster entry point takes the tile size block_x x block_y of
 * the binning whose tile_bins it reads (ops/cubic_splatting.py:2778-2782);
 * both must be positive multiples of 16 with (block_x / 16) * (block_y / 16)
 * <= 16 (other sizes: the _any_tile entry points below).  The raster runs
 * one workgroup of two waves (16 x 8 pixels each) per 16 x 16 sub-block of
 * the image; the 2 (block_x / 16) (block_y / 16) waves
 * of a tile all walk its list, and S = ceil(W / 16) * ceil(H / 16) counts the
 * sub-blocks.
 * Scheduling (no reference counterpart; it changes no result).  Every raster
 * entry point takes, before its stream,
 *   tile_order [cs_raster_tile_order_elems(S)] (NULL: XCD-contiguous order,
 *     one workgroup per sub-block) -- an order written by
 *     cs_raster_tile_order: the launch then has one workgroup per position,
 *     workgroup b (on XCD b mod 8) rasterizes the sub-block at position
 *     (b mod 8) * cap + b / 8 (cap = cs_raster_tile_order_elems(S) / 8), and
 *     positions holding -1 do nothing; every sub-block must appear once;
 * and the forward ones also
 *   wave_cost [2S] uint32 out (NULL: not recorded; 8-byte aligned) -- each
 *     wave's duration in ticks of the 100 MHz constant clock.
 * S is at most 2^20 (16384 x 16384 pixels) for cs_raster_tile_order.
 * cs_raster_tile_order turns the costs of one launch into a heavy-first order
 * for the next ones (the backward of the same forward, the next forward of
 * the scene): long sub-blocks start first, short ones fill the tail.
 * chunked != 0 cuts the sub-blocks into eight contiguous runs of about equal
 * total cost (at most cap each) and sorts run x onto XCD x's positions (XCD x
 * keeps its part of the image, and its L2 the records of that part, and the
 * XCDs finish together); chunked == 0 sorts all of them and deals them out
 * over the XCDs in turn (balance for skewed scenes). */
size_t cs_raster_tile_order_elems(int32_t ntiles);
int cs_raster_tile_order(const uint32_t* wave_cost, int32_t ntiles, int32_t chunked,
                         int32_t* tile_order, hipStream_t stream);

/* cs_raster_tile_order from running averages (no reference counterpart): a
 * sub-block's cost is its two waves' durations summed, averaged with its
 * previous cost cost_in [S] when given (round half up), and the costs used
 * are written to cost_out [S] (or NULL) for the next call's cost_in; cost_out
 * must not be cost_in.  One launch's durations vary by about a fifth from
 * launch to launch, so the average orders the next launches better. */
int cs_raster_tile_order_averaged(const uint32_t* wave_cost, const uint32_t* cost_in,
                                  uint32_t* cost_out, int32_t ntiles, int32_t chunked,
                                  int32_t* tile_order, hipStream_t stream);

/* Tiles of any size (block_x * block_y <= 1024, the reference's
 * one-thread-per-pixel launch threads=(block_x, block_y)), for sizes the
 * 16 x 16 sub-block entry points above do not take (for example 8 x 8 or
 * 16 x 8): one workgroup per tile, one lane per pixel, every edge of every
 * list entry evaluated with the same expressions (image, final_Ts and
 * final_idx identical to the sub-block kernels' on tiles both take).  No
 * raster log, no tile order.
 * cs_rasterize_forward_any_tile replaces rasterize_cubic_fill_forward_kernel
 * (ops/cubic_splatting.py:918-1194, wrapper :2181-2305; mode 1:
 * ops/cubic_polyline_splatting.py:33-249); edges [E] edge records, prim_recs
 * [P] primitive records as for cs_rasterize_forward; out_img [H,W,3] or, with
 * out_planar, three [H,W] planes; out_planes as for cs_rasterize_forward.
 * cs_rasterize_backward_any_tile replaces rasterize_cubic_fill_backward_kernel
 * (ops/cubic_splatting.py:1197-1651, wrapper :2572-2747; mode 1:
 * ops/cubic_polyline_splatting.py:252-660): adds into v_edges [E,2,2]
 * (zeroed by the caller; fold with cs_accumulate_edge_grads or
 * cs_accumulate_edge_grads_csr), v_colors [P,3], v_opacities, v_inv_sigma2s
 * [P], v_stroke_widths [P] (mode 1) and, when not NULL, curve_contrib_rgb
 * [P,3] / curve_isect_contrib [I]. */
int cs_rasterize_forward_any_tile(int32_t mode, const int32_t* prim_ids_sorted,
                                  const int32_t* tile_bins, const void* edges,
                                  const void* prim_recs, const float* background, int32_t img_h,
                                  int32_t img_w, int32_t block_x, int32_t block_y,
                                  float* out_img, int32_t out_planar, float* out_planes,
                                  float* final_Ts, int32_t* final_idx, hipStream_t stream);
int cs_rasterize_backward_any_tile(int32_t mode, const int32_t* prim_ids_sorted,
                                   const int32_t* tile_bins, const void* edges,
                                   const void* prim_recs, const float* background, int32_t img_h,
                                   int32_t img_w, int32_t block_x, int32_t block_y,
                                   const float* final_Ts, const int32_t* final_idx,
                                   const float* v_output, int32_t v_output_planar,
                                   float* v_edges, float* v_colors, float* v_opacities,
                                   float* v_inv_sigma2s, float* v_stroke_widths,
                                   float* curve_contrib_rgb, float* curve_isect_contrib,
                                   hipStream_t stream);

/* Raster log (no reference counterpart: the reference's backward re-runs the
 * edge loop and the coverage, ops/cubic_splatting.py:1451-1530,
 * ops/cubic_polyline_splatting.py:465-545).  The forward records, for every
 * list entry g a wave of tile rows processes, what its backward needs:
 *   log_index [V * num_entries] int32 (V = 2 (block_x / 16) (block_y / 16),
 *     the waves of a tile; num_entries: the size of prim_ids_sorted, every
 *     tile_bins range lies below it), entry V g + wave (the wave's slot in
 *     its tile, 2 (16 x 16 sub-block in row-major order) + wave of the pair):
 *     the record's position in log_pool in 16-byte units, or -1 when no pixel
 *     of the wave is inside the primitive or near it (the entry contributes
 *     nothing), or -2 when the pool was full (the backward then recomputes
 *     that entry); entries the wave did not process are not written;
 *   log_pool (16-byte aligned, log_pool_bytes): unit 0 holds a uint32
 *     counter; then each wave's own region, log_entry_units units for every
 *     entry of its tile's list (V * num_entries * log_entry_units units in
 *     all, placed by the tile's list range, written without atomics); then
 *     shared blocks of CS_RASTER_LOG_BLOCK_BYTES that a wave whose records
 *     outgrow its region reserves through the counter (which the forward
 *     sets to the first shared unit and which ends at the units reserved,
 *     plus at most one failed reservation per wave).  A record is 32 bytes of
 *     lane masks (inside bits of the winding test, zero for strokes; exact
 *     bits of the live pixels whose coverage needs the exact distance; one
 *     64-bit mask per pixel row of the lanes), then one (best edge int32,
 *     coverage fp32 bits) pair per exact pixel in lane order.
 * Any pool of at least 16 * (1 + V * num_entries * log_entry_units) bytes is
 * correct (a full pool only costs backward time).  log_index NULL: no log
 * (the forward of a render no backward follows); the backward then
 * recomputes every entry. */
#define CS_RASTER_LOG_BLOCK_BYTES 2048

/* Raster records (the edges, edge_culls and prim_recs the raster entry points
 * read) from the reference's raster inputs: flattened edges_px [E, 2, 2],
 * prim_ids_sorted [I] and one edge range per intersection,
 * isect_edge_ranges [I, 2] (rasterize_cubic_fill_forward_tilelang,
 * ops/cubic_splatting.py:2181-2305, and the backward :2572-2747), colors
 * [P, 3], opacities [P], inv_sigma2s [P], fill_rules [P] (NULL: nonzero rule;
 * mode 0) or stroke_widths [P] (mode 1).  The records hold one edge range per
 * primitive, taken from its intersections: *status (device int32) is set to
 * 0, or ORs 1 when an id lies outside [0, P), 2 when two intersections of one
 * primitive carry different ranges (or a range outside [0, E]), 4 when one of
 * the num_tiles tile_bins ranges is not within [0, I]; the records and a
 * raster over them are then not meaningful (the raster kernels trust their
 * inputs).  Scratch: prim_edge_ranges [P, 2] and edge_cull_d [E] int32. */
int cs_raster_records_from_edges(int32_t mode, const float* edges_px, int32_t num_edges,
                                 const int32_t* prim_ids_sorted,
                                 const int32_t* isect_edge_ranges, int64_t num_intersects,
                                 const float* colors, const float* opacities,
                                 const float* inv_sigma2s, const int32_t* fill_rules,
                                 const float* stroke_widths, int32_t nprim,
                                 const int32_t* tile_bins, int32_t num_tiles,
                                 int32_t* prim_edge_ranges, int32_t* edge_cull_d,
                                 int32_t* status, void* edges, void* edge_culls,
                                 void* prim_recs, hipStream_t stream);

/* The (segment, t0, t1) edge records cs_rasterize_backward_de_casteljau reads,
 * from the adaptive flattening's segment_edge_offsets [nseg + 1],
 * edge_t_starts / edge_t_ends [E] (ops/cubic_splatting.py:1812-1828). */
int cs_edge_aux_from_csr(const int32_t* segment_edge_offsets, int32_t nseg,
                         const float* edge_t_starts, const float* edge_t_ends, int32_t num_edges,
                         void* edge_aux, hipStream_t stream);

/* rasterize_cubic_fill_forward_kernel (ops/cubic_splatting.py:918-1194) when
 * mode 0, rasterize_cubic_polyline_forward_kernel
 * (ops/cubic_polyline_splatting.py:33-249) when mode 1.  Tiles as above.
 * The primitive records hold each primitive's edge range, so
 * edges_per_segment is not used (>= 0; 0 for adaptive records).  out_img is
 * written as [H, W, 3] (the reference's layout), or, when out_planar != 0, as
 * three [H, W] planes (channel c at out_img + c H W).  out_planes, when not
 * NULL, receives the image once more as three [H, W] planes (the layout
 * cs_clamp_mse_ssim_loss reads with img_planar, clamping on load, so the
 * clamp(0, 1).permute(2, 0, 1) glue of gaussian_trace/render.py:1309-1310
 * needs no pass of its own).  log_counter: NULL,
 * or a device word that is zero on entry, which then counts the raster log's
 * shared blocks (the call takes no launch of its own to set up the counter in
 * the pool's first unit; the word is left at the count used). */
int cs_rasterize_forward(int32_t mode, const int32_t* prim_ids_sorted, const int32_t* tile_bins,
                         const void* edges, const void* edge_culls, const void* prim_recs,
                         const float* background, int32_t img_h, int32_t img_w,
                         int32_t block_x, int32_t block_y,
                         int32_t edges_per_segment, float* out_img, int32_t out_planar,
                         float* out_planes, float* final_Ts, int32_t* final_idx,
                         int64_t num_entries, int32_t* log_index, void* log_pool,
                         int64_t log_pool_bytes, int32_t log_entry_units,
                         uint32_t* log_counter, const int32_t* tile_order, uint32_t* wave_cost,
                         hipStream_t stream);

/* rasterize_cubic_fill_backward_kernel (ops/cubic_splatting.py:1197-1651) /
 * rasterize_cubic_polyline_backward_kernel (ops/cubic_polyline_splatting.py:252-660)
 * fused with _accumulate_edge_grads_to_cubics (ops/cubic_splatting.py:2308-2396):
 * accumulates (atomically) into zero-initialised v_cubics_px [nseg,4,2],
 * v_colors [P,3], v_opacities [P], v_inv_sigma2s [P], v_stroke_widths [P]
 * (mode 1), and optionally curve_contrib_rgb [P,3] / curve_isect_contrib [I].
 * v_output is the gradient of out_img: [H, W, 3] interleaved, or, when
 * v_output_planar != 0, three [H, W] planes (channel c at v_output + c H W;
 * the layout cs_clamp_mse_ssim_backward writes with grad_planar). */
int cs_rasterize_backward(int32_t mode, const int32_t* prim_ids_sorted, const int32_t* tile_bins,
                          const void* edges, const void* edge_culls, const void* prim_recs,
                          const float* background, int32_t img_h, int32_t img_w,
                          int32_t block_x, int32_t block_y,
                          int32_t edges_per_segment, const float* final_Ts,
                          const int32_t* final_idx, const int32_t* log_index,
                          const void* log_pool, const float* v_output,
                          int32_t v_output_planar,
                          float* v_cubics_px, float* v_colors, float* v_opacities,
                          float* v_inv_sigma2s, float* v_stroke_widths, float* curve_contrib_rgb,
                          float* curve_isect_contrib, int32_t nprim, float* prim_scratch,
                          const int32_t* tile_order, hipStream_t stream);

/* Floats of the prim_scratch buffer the backward entry points take for
 * nprim primitives (mode 0 fill, 1 stroke).  With prim_scratch (zero on
 * entry; the call leaves it zero), the per-primitive gradients (v_colors,
 * v_opacities, v_inv_sigma2s, v_stroke_widths) are first summed into 8
 * copies, one per XCD of the launch, then added into the caller's arrays:
 * the atomic additions of the many tiles a large primitive covers no longer
 * meet at one address.  NULL: direct atomic additions (nprim unused).  No
 * reference counterpart; it changes no value beyond fp32 summation order. */
size_t cs_raster_prim_scratch_elems(int32_t nprim, int32_t mode);

/* cs_rasterize_backward for records from cs_bin_prepare_de_casteljau
 * (the reference's flatten_method="de_casteljau" backward: the raster kernel
 * plus _accumulate_edge_grads_to_cubics_csr_kernel,
 * ops/cubic_splatting.py:2399-2487): each edge's gradient is folded into its
 * segment's control points with the Bernstein weights at its edge_aux
 * interval [t0, t1]. */
int cs_rasterize_backward_de_casteljau(int32_t mode, const int32_t* prim_ids_sorted,
                                       const int32_t* tile_bins, const void* edges,
                                       const void* edge_culls, const void* prim_recs,
                                       const float* background, int32_t img_h, int32_t img_w,
                                       int32_t block_x, int32_t block_y,
                                       const void* edge_aux, const float* final_Ts,
                                       const int32_t* final_idx, const int32_t* log_index,
                                       const void* log_pool, const float* v_output,
                                       int32_t v_output_planar,
                                       float* v_cubics_px, float* v_colors,
                                       float* v_opacities, float* v_inv_sigma2s,
                                       float* v_stroke_widths, float* curve_contrib_rgb,
                                       float* curve_isect_contrib, int32_t nprim,
                                       float* prim_scratch, const int32_t* tile_order,
                                       hipStream_t stream);

/* cs_rasterize_forward / cs_rasterize_backward with the same results, plus
 * evaluation counts added into eval_counts[5] (device uint64, caller-zeroed),
 * each an (edge, pixel) term of the reference's edge loop
 * (cubic_splatting.py:1095-1134) that the kernel evaluated rather than
 * proved irrelevant: [0] distance terms, [1] crossing terms evaluated with
 * the cross product, [2] crossing terms of far edges decided by the row span
 * alone; then [3] (wave, list entry) pairs processed past the primitive cull
 * and [4] exact coverage evaluations (pixels within the cull distance).
 * Measurement only (no reference counterpart): the counting instantiation is
 * slower than the plain one. */
int cs_rasterize_forward_counted(int32_t mode, const int32_t* prim_ids_sorted,
                                 const int32_t* tile_bins, const void* edges,
                                 const void* edge_culls, const void* prim_recs,
                                 const float* background, int32_t img_h, int32_t img_w,
                                 int32_t block_x, int32_t block_y,
                                 int32_t edges_per_segment, float* out_img,
                                 int32_t out_planar, float* out_planes, float* final_Ts,
                                 int32_t* final_idx, int64_t num_entries, int32_t* log_index,
                                 void* log_pool,
                                 int64_t log_pool_bytes, int32_t log_entry_units,
                                 uint32_t* log_counter, unsigned long long* eval_counts,
                                 const int32_t* tile_order,
                                 uint32_t* wave_cost, hipStream_t stream);
int cs_rasterize_backward_counted(int32_t mode, const int32_t* prim_ids_sorted,
                                  const int32_t* tile_bins, const void* edges,
                                  const void* edge_culls, const void* prim_recs,
                                  const float* background, int32_t img_h, int32_t img_w,
                                  int32_t block_x, int32_t block_y,
                                  int32_t edges_per_segment, const float* final_Ts,
                                  const int32_t* final_idx, const int32_t* log_index,
                                  const void* log_pool, const float* v_output,
                                  int32_t v_output_planar,
                                  float* v_cubics_px, float* v_colors,
                                  float* v_opacities, float* v_inv_sigma2s, float* v_stroke_widths,
                                  float* curve_contrib_rgb, float* curve_isect_contrib,
                                  unsigned long long* eval_counts, int32_t nprim,
                                  float* prim_scratch, const int32_t* tile_order,
                                  hipStream_t stream);

/* _accumulate_edge_grads_to_cubics_kernel (ops/cubic_splatting.py:2308-2396)
 * fused with the v_cubics_norm scaling (ops/cubic_splatting.py:3096-3100). */
int cs_accumulate_edge_grads(const float* v_edges, int32_t nseg, int32_t edges_per_segment,
                             int32_t img_h, int32_t img_w, float* v_cubics_px,
                             float* v_cubics_norm, hipStream_t stream);

/* _accumulate_edge_grads_to_cubics_csr_kernel (ops/cubic_splatting.py:2399-2487)
 * fused with the v_cubics_norm scaling: v_edges [E,2,2], edge_t_starts /
 * edge_t_ends [E], segment_edge_offsets [nseg + 1]; v_cubics_norm may be NULL. */
int cs_accumulate_edge_grads_csr(const float* v_edges, const float* edge_t_starts,
                                 const float* edge_t_ends, const int32_t* segment_edge_offsets,
                                 int32_t nseg, int32_t img_h, int32_t img_w, float* v_cubics_px,
                                 float* v_cubics_norm, hipStream_t stream);

/* Backward epilogue (ops/cubic_splatting.py:3096-3104): v_cubics_norm =
 * v_cubics_px * (W/2, H/2) and v_aa_widths = -2 v_inv_sigma2 / max(w^3, 1e-12)
 * with w = max(widths, 1e-4) (the clamp of ops/cubic_splatting.py:2820). */
int cs_backward_finalize(const float* v_cubics_px, int32_t nseg, int32_t img_h, int32_t img_w,
                         const float* widths, const float* v_inv_sigma2s, int32_t nprim,
                         float* v_cubics_norm, float* v_aa_widths, hipStream_t stream);

/* cs_rasterize_backward (with prim_scratch, no contribution outputs) followed
 * by cs_backward_finalize (ops/cubic_splatting.py:1197-1651, then
 * :3096-3104), with the per-XCD copies' reduction and the epilogue in one
 * launch: v_colors, v_opacities, v_inv_sigma2s, v_stroke_widths receive the
 * copies' sums as with cs_rasterize_backward, v_cubics_px the control-point
 * gradients, and v_cubics_norm [nseg,4,2] / v_aa_widths [P] what
 * cs_backward_finalize computes from them (widths: the aa widths, clamped to
 * 1e-4 inside).  For callers with nothing to run between the two (the
 * reference's process_fn hook post_backward_rasterize absent); the results
 * equal the two calls'. */
int cs_rasterize_backward_finalized(
    int32_t mode, const int32_t* prim_ids_sorted, const int32_t* tile_bins, const void* edges,
    const void* edge_culls, const void* prim_recs, const float* background, int32_t img_h,
    int32_t img_w, int32_t block_x, int32_t block_y, int32_t edges_per_segment,
    const float* final_Ts, const int32_t* final_idx, const int32_t* log_index,
    const void* log_pool, const float* v_output, int32_t v_output_planar, float* v_cubics_px,
    float* v_colors, float* v_opacities, float* v_inv_sigma2s, float* v_stroke_widths,
    int32_t nprim, float* prim_scratch, const int32_t* tile_order, int32_t nseg,
    const float* widths, float* v_cubics_norm, float* v_aa_widths, hipStream_t stream);

/* ---------------- closed rings -> cubic segments ---------------- */

/* closed_cubic_fill_segments_forward_kernel (ops/cubic_splatting.py:137-268):
 * control_points [num_curves, K, 2] (K >= 4, K even; 8-byte aligned) ->
 * out_segments [num_curves * 2 * subdiv, 4, 2] (16-byte aligned), with the
 * basis tables of _closed_fill_piecewise_basis_tensors (:81-134): basis
 * [subdiv+1, kb], deriv_basis [subdiv+1, kb-1], dt [subdiv], kb = (K+2)/2. */
int cs_closed_ring_segments(const float* control_points, int32_t num_curves, int32_t K,
                            int32_t subdiv, const float* basis, const float* deriv_basis,
                            const float* dt, float* out_segments, hipStream_t stream);

/* closed_cubic_fill_segments_backward_kernel (ops/cubic_splatting.py:271-383):
 * grad_control_points [num_curves, K, 2] (written, not accumulated; 8-byte
 * aligned) from grad_segments (16-byte aligned), deterministic (no atomics). */
int cs_closed_ring_segments_backward(const float* grad_segments, int32_t num_curves, int32_t K,
                                     int32_t subdiv, const float* basis,
                                     const float* deriv_basis, const float* dt,
                                     float* grad_control_points, hipStream_t stream);

/* ---------------- losses ---------------- */

/* Number of float partials cs_mse_forward / cs_ssim needs in `partials`, and
 * of floats in cs_ssim's `abc` maps ([3, nc, oh, ow rounded up to 4]). */
size_t cs_mse_partials_elems(int64_t n);
size_t cs_ssim_partials_elems(int32_t nc, int32_t h, int32_t w);
size_t cs_ssim_abc_elems(int32_t nc, int32_t h, int32_t w, int32_t win);

/* mse_partial_sum_kernel + reduce_sum_partial_kernel (ops/metric.py:18-163,
 * metric.py:102-131): *loss = sum((x-y)^2)/n (device scalar), two launches,
 * deterministic summation order. */
int cs_mse_forward(const float* x, const float* y, int64_t n, float* partials, float* loss,
                   hipStream_t stream);

/* No counterpart in the reference: cs_mse_forward for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc).  The partial sums go to a file-scope
 * device array of the library (256 KiB per GPU, held until the process ends;
 * its address is looked up once per device with hipGetSymbolAddress) instead
 * of a caller workspace; nothing is allocated or freed.  n is limited to
 * cs_mse_forward_noalloc_max_elems() (2^28) elements; larger n returns
 * CS_ERR_ARGS.  Every call on one GPU shares that array: calls that overlap on
 * one GPU (different streams, host threads) race and must be serialized by
 * the caller.  The result equals cs_mse_forward's bit for bit (same kernels). */
int64_t cs_mse_forward_noalloc_max_elems(void);
int cs_mse_forward_noalloc(const float* x, const float* y, int64_t n, float* loss,
                           hipStream_t stream);

/* mse_backward_diff_kernel (ops/metric.py:166-202): grad = scale (lhs - rhs)
 * over n fp32 elements (the reference's mse_backward_diff_tilelang,
 * ops/metric.py:344-360). */
int cs_mse_backward_diff(const float* lhs, const float* rhs, int64_t n, float scale, float* grad,
                         hipStream_t stream);

/* reduce_sum_partial_kernel applied until one value is left
 * (reduce_sum_1d_tilelang, ops/metric.py:363-382): *out = sum of x[0..n) in
 * fp32 (device scalar; partials of cs_reduce_sum_partials_elems(n) floats),
 * two launches, deterministic order.  n >= 1. */
size_t cs_reduce_sum_partials_elems(int64_t n);
int cs_reduce_sum_f32(const float* x, int64_t n, float* partials, float* out,
                      hipStream_t stream);

/* mse_backward_diff_kernel (ops/metric.py:166-202) with the scale
 * grad_loss * 2/n read on the device (metric.py:168 reads it on the host):
 * grad_x = s (x - y), grad_y = -s (x - y); either output may be null. */
int cs_mse_backward(const float* x, const float* y, int64_t n, const float* grad_loss,
                    float* grad_x, float* grad_y, hipStream_t stream);

/* Floats of the scratch buffer cs_ssim and cs_ssim_backward need for a
 * window wider than 15 (0 otherwise: pass NULL). */
size_t cs_ssim_scratch_elems(int32_t nc, int32_t h, int32_t w, int32_t win);

/* ssim_map_kernel (ops/metric.py:205-341) + the means of metric.py:262-273,
 * separable window `win1d` [win] (any odd win <= h, w; the 2D window is its
 * outer product), valid window.  per_map = 0: *out = mean over the SSIM map
 * of every (image, channel), then over them; per_map = 1: out[i] = the mean
 * of map i (the per-image, per-channel values of size_average=False and
 * nonnegative_ssim).  If abc != null also stores, per map pixel, dS/dmu_x,
 * dS/dE[x^2], dS/dE[xy] (cs_ssim_abc_elems floats: [3, nc, oh, ow] with rows
 * padded to a multiple of 4 floats) for cs_ssim_backward; with windows up
 * to 15 one map plane (oh rows of the padded ow) holds at most 2^30 floats
 * (CS_ERR_ARGS beyond).  x, y: [nc, h, w]; scratch: cs_ssim_scratch_elems
 * floats. */
int cs_ssim(const float* x, const float* y, int32_t nc, int32_t h, int32_t w,
            const float* win1d, int32_t win, float c1, float c2, int32_t per_map,
            float* partials, float* out, float* abc, float* scratch, hipStream_t stream);

/* Gradient of cs_ssim's output w.r.t. x (the reference has no SSIM backward):
 * grad_x = g * [W*(A) + 2 x W*(B) + y W*(C)] / count, W* the transposed (full)
 * window correlation; per_map = 0: g = *grad_out, count = nc*oh*ow; per_map =
 * 1: g = grad_out[i] for map i, count = oh*ow.  scratch as for cs_ssim. */
int cs_ssim_backward(const float* x, const float* y, int32_t nc, int32_t h, int32_t w,
                     const float* win1d, int32_t win, const float* abc, const float* grad_out,
                     int32_t per_map, float* grad_x, float* scratch, hipStream_t stream);

/* ---------------- fused training-step operations ---------------- */

/* The caller's glue between the render and the losses,
 * gaussian_trace/render.py:1309-1310: out [3, h, w] = clamp(img, lo, hi)
 * permuted from img [h, w, 3]; and its gradient, grad_img [h, w, 3] =
 * grad [3, h, w] where lo <= img <= hi, else 0 (torch's clamp gradient). */
int cs_clamp_hwc_to_nchw(const float* img, int32_t h, int32_t w, float lo, float hi, float* out,
                         hipStream_t stream);
int cs_clamp_hwc_to_nchw_backward(const float* img, const float* grad, int32_t h, int32_t w,
                                  float lo, float hi, float* grad_img, hipStream_t stream);

/* loss = MSE(x, y) + ssim_weight * (1 - SSIM(x, y)) in one call (the MSE of
 * metric.py:102-212 and the SSIM of metric.py:215-273; the SSIM kernel also
 * sums the squared differences, per tile, so the MSE equals cs_mse_forward's up
 * to fp32 summation order): out[0] = loss, out[1] = MSE, out[2] = SSIM
 * (device); `partials` holds cs_mse_ssim_partials_elems floats; abc as for
 * cs_ssim.
 * The backward writes grad_x = g (2 (x - y) / n - ssim_weight dSSIM/dx) in one
 * pass, g = *grad_loss. */
size_t cs_mse_ssim_partials_elems(int32_t nc, int32_t h, int32_t w);
int cs_mse_ssim_loss(const float* x, const float* y, int32_t nc, int32_t h, int32_t w,
                     const float* win1d, int32_t win, float c1, float c2, float ssim_weight,
                     float* partials, float* out, float* abc, hipStream_t stream);
int cs_mse_ssim_backward(const float* x, const float* y, int32_t nc, int32_t h, int32_t w,
                         const float* win1d, int32_t win, const float* abc, float ssim_weight,
                         const float* grad_loss, float* grad_x, hipStream_t stream);

/* The same loss on the renderer's image, with the caller's
 * clamp(0, 1).permute(2, 0, 1) glue (gaussian_trace/render.py:1309-1310)
 * folded in.  img is [h, w, 3], or, when img_planar != 0, three [h, w] planes
 * (cs_rasterize_forward's out_planar layout).  The forward computes the loss
 * on x = clamp(img, lo, hi): from [h, w, 3] it first writes x as [3, h, w]
 * into the caller's buffer x; planes it reads clamped in place (x unused,
 * may be NULL).  The backward reads img itself and writes grad_img directly,
 * zero where img lies outside [lo, hi] (no gradient pass through the glue):
 * [h, w, 3], or, with grad_planar != 0, three [h, w] planes (whole-line
 * writes; cs_rasterize_backward reads that layout with v_output_planar).  A
 * planar img takes grad_planar != 0.  y is the [3, h, w] target; partials /
 * abc as for cs_mse_ssim_loss with nc = 3. */
int cs_clamp_mse_ssim_loss(const float* img, int32_t img_planar, const float* y, int32_t h,
                           int32_t w, float lo, float hi, const float* win1d, int32_t win,
                           float c1, float c2, float ssim_weight, float* x, float* partials,
                           float* out, float* abc, hipStream_t stream);
int cs_clamp_mse_ssim_backward(const float* img, int32_t img_planar, const float* y, int32_t h,
                               int32_t w, float lo, float hi, const float* win1d, int32_t win,
                               const float* abc, float ssim_weight, const float* grad_loss,
                               float* grad_img, int32_t grad_planar, hipStream_t stream);

/* ---------------- optimizer ---------------- */

/* One Adam step (torch.optim.Adam as gaussian_trace/model.py:172-189 builds
 * it: per-group learning rates, amsgrad and maximize off) over up to
 * CS_ADAM_MAX_TENSORS fp32 tensors in one launch.  The arrays are host arrays
 * of ntensors entries; the pointers in them are device pointers.  Per tensor
 * k: step_sizes[k] = lr / (1 - beta1^step), bias_correction2_sqrts[k] =
 * sqrt(1 - beta2^step) (> 0), weight_decays[k] the L2 coefficient.  The
 * hyperparameters are doubles, as torch's Python floats: 1 - beta is formed in
 * double and rounded to fp32 once.  Updates params, exp_avgs and exp_avg_sqs
 * in place. */
#define CS_ADAM_MAX_TENSORS 16
int cs_adam_step(int32_t ntensors, float* const* params, const float* const* grads,
                 float* const* exp_avgs, float* const* exp_avg_sqs, const int64_t* numels,
                 const float* step_sizes, const float* bias_correction2_sqrts,
                 const float* weight_decays, double beta1, double beta2, double eps,
                 hipStream_t stream);

/* One Adan step (manbo/optim.py:70-190, adan_step_from_grad_kernel
 * ops/optim.py:8-113; the default optimizer of train.py:106) over up to
 * CS_ADAM_MAX_TENSORS fp32 tensors in one launch, updating params, exp_avgs,
 * exp_avg_sqs, exp_avg_diffs and neg_pre_grads in place.  Host arrays of
 * ntensors entries: numels; scalars [10 k .. 10 k + 9] = beta1, beta2, beta3,
 * bias_correction1, bias_correction2, sqrt(bias_correction3), lr,
 * weight_decay, eps, clip factor of tensor k (fp32, as the reference kernel
 * casts them); flags [2 k] = 1 on the first step (no previous gradient),
 * flags [2 k + 1] = no_prox.  clip: a device fp32 global-norm clip factor
 * that replaces the host ones, or NULL. */
int cs_adan_step(int32_t ntensors, float* const* params, const float* const* grads,
                 float* const* exp_avgs, float* const* exp_avg_sqs, float* const* exp_avg_diffs,
                 float* const* neg_pre_grads, const int64_t* numels, const float* scalars,
                 const int32_t* flags, const float* clip, hipStream_t stream);

/* ---------------- 2D Gaussian splats (GsRenderFunction) ---------------- */

/* project_gaussians_2d_scale_rot_forward_kernel (ops/forward2d.py:14-164):
 * means2d [n,2] in the normalized [-1,1] frame, scales2d [n,2], rotation [n]
 * (8-byte aligned [n,2] arrays) -> xys [n,2], depths [n] (zeros), radii [n],
 * conics [n,3], num_tiles_hit [n]; all zero for a Gaussian whose tile
 * rectangle is empty.  block_x * block_y <= 1024. */
int cs_gs_project_forward(const float* means2d, const float* scales2d, const float* rotation,
                          int32_t n, int32_t img_h, int32_t img_w, int32_t block_x,
                          int32_t block_y, float* xys, float* depths, int32_t* radii,
                          float* conics, int32_t* num_tiles_hit, hipStream_t stream);

/* Replaces tilelang_renderer.py:224-269 (cumsum, map_gaussian_to_intersects,
 * torch.sort, get_tile_bin_edges) up to the count: per Gaussian the tile
 * rectangle of ops/intersects.py:34-121 (tile_rects [n,4], 16-byte aligned)
 * and the raw depth bits as key; depth ranks (ties by id: the stable order of
 * the reference's sort); tile-list counts; status[0] = intersection total,
 * status[1..3] = 0.  Scratch sizes as for cs_bin_prepare.  cs_bin_finish then
 * writes gaussian_ids_sorted and tile_bins ([start, end) per tile, (0,0) when
 * empty). */
int cs_gs_bin_prepare(const float* xys, const float* conics, const int32_t* radii,
                      const float* depths, int32_t n, int32_t img_h, int32_t img_w,
                      int32_t block_x, int32_t block_y, int32_t* tile_rects, uint32_t* keys,
                      int32_t* order, uint32_t* keys_alt, int32_t* vals_alt,
                      uint32_t* radix_counts, uint32_t* scan_temp, int32_t* rank_tile_ranges,
                      uint32_t* tile_count, uint32_t* tile_scratch,
                      int32_t* status, hipStream_t stream);

/* The per-Gaussian raster records (48 bytes each, 16-byte aligned) that the
 * two raster entry points read: centre, halved conic, opacity and its alpha
 * cut, colour, conic diagonal.  No reference counterpart: the reference's
 * raster kernels gather these fields from xys / conics / colors / opacities
 * into shared memory per batch (ops/rasterize.py:92-103, :300-311). */
#define CS_GS_RECORD_BYTES 48
int cs_gs_pack_records(const float* xys, const float* conics, const float* colors,
                       const float* opacities, int32_t n, void* records, hipStream_t stream);

/* rasterize_forward_kernel (ops/rasterize.py:18-157): out_img [H,W,3],
 * final_Ts [H,W], final_idx [H,W] (index of the pixel's last contributing
 * intersection, 0 if none). */
int cs_gs_rasterize_forward(const int32_t* gaussian_ids_sorted, const int32_t* tile_bins,
                            const void* records, const float* background, int32_t img_h,
                            int32_t img_w, int32_t block_x, int32_t block_y, float* out_img,
                            float* final_Ts, int32_t* final_idx, hipStream_t stream);

/* rasterize_backward_kernel (ops/rasterize.py:160-529): ADDS into v_xy [n,2],
 * v_conic [n,3], v_rgb [n,3], v_opacity [n] and, when not NULL, contrib_rgb
 * [n,3] and isect_contrib [num_intersects] (the caller zeroes them).
 * intersect_meta_sorted NULL enables every intersection's geometry
 * gradients; v_output_alpha NULL reads as zeros. */
int cs_gs_rasterize_backward(const int32_t* gaussian_ids_sorted,
                             const int32_t* intersect_meta_sorted, const int32_t* tile_bins,
                             const void* records, const float* background, int32_t img_h,
                             int32_t img_w, int32_t block_x, int32_t block_y,
                             const float* final_Ts, const int32_t* final_idx,
                             const float* v_output, const float* v_output_alpha, float* v_xy,
                             float* v_conic, float* v_rgb, float* v_opacity, float* contrib_rgb,
                             float* isect_contrib, hipStream_t stream);

/* project_gaussians_2d_scale_rot_backward_kernel (ops/backward2d.py:8-151)
 * with the gaussian_meta scaling of tilelang_renderer.py:111-116 (meta NULL:
 * none).  v_cov2d may be NULL. */
int cs_gs_project_backward(const float* scales2d, const float* rotation, const int32_t* radii,
                           const float* conics, const float* v_xy, const float* v_conic,
                           const int32_t* gaussian_meta, int32_t n, int32_t img_h, int32_t img_w,
                           float* v_cov2d, float* v_mean2d, float* v_scale, float* v_rot,
                           hipStream_t stream);

/* map_gaussian_to_intersects{,_isotropic}_kernel (ops/intersects.py:12-226):
 * the reference's int64 (tile << 32 | depth bits) keys and Gaussian ids at
 * [cum_tiles_hit[g-1], cum_tiles_hit[g]); conics NULL selects the isotropic
 * rectangle.  Entries outside [0, num_intersects) are not written. */
int cs_gs_map_to_intersects(const float* xys, const float* conics, const float* depths,
                            const int32_t* radii, const int32_t* cum_tiles_hit, int32_t n,
                            int64_t num_intersects, int32_t tile_bound_x, int32_t tile_bound_y,
                            int32_t block_x, int32_t block_y, int64_t* isect_ids,
                            int32_t* gaussian_ids, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* CUBICSPLAT_HIP_H */
