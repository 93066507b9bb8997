"""The reference's raster building blocks with their own argument layouts:
rasterize_cubic_fill_forward_tilelang (ops/cubic_splatting.py:2181-2305) and
rasterize_cubic_fill_backward_tilelang (:2572-2747).

They take flattened edges [E, 2, 2] and one edge range per intersection
[I, 2]; the MI355X raster kernels read per-primitive records, which
cs_raster_records_from_edges builds from those inputs (each primitive's edge
range taken from its intersections, which must agree: the reference's
pipeline always passes [offs_e[pid], offs_e[pid + 1]],
_build_fill_isect_edge_ranges :1849-1860).  The forward writes no raster log,
so the backward recomputes every entry's geometry with the forward's edge
walk.  The fused path (repo_amd.splat) does not use these; they keep the
reference's intermediate API callable.
"""
from __future__ import annotations

import torch

from . import _native as N
from .splat import (
    BLOCK_X,
    BLOCK_Y,
    DEFAULT_AA_WIDTH,
    DEFAULT_CUBIC_FLATTEN_METHOD,
    DEFAULT_DISTANCE_SAMPLES,
    DEFAULT_THREADS,
    normalize_cubic_flatten_method,
)


def _f32(t):
    if t.dtype is torch.float32 and t.is_contiguous():
        return t
    return t.to(torch.float32).contiguous()


def _i32(t):
    if t.dtype is torch.int32 and t.is_contiguous():
        return t
    return t.to(torch.int32).contiguous()


def _inv_sigma2s(aa_widths, inv_sigma2s, aa_width, num_primitives, device):
    """cubic_splatting.py:2225-2257 (the same expressions on the same device)."""
    if inv_sigma2s is None:
        if aa_widths is None:
            w = torch.full((num_primitives,), float(aa_width), device=device,
                           dtype=torch.float32)
        else:
            w = aa_widths.to(device=device, dtype=torch.float32).view(-1)
            if int(w.numel()) == 1 and num_primitives > 1:
                w = w.expand(num_primitives)
            if int(w.numel()) != num_primitives:
                raise ValueError(
                    f"aa_widths size must match num_primitives ({num_primitives}), "
                    f"got {int(w.numel())}")
        w = torch.clamp(_f32(w), min=1e-4)
        return (1.0 / torch.clamp(w * w, min=1e-6)).contiguous()
    s = inv_sigma2s.to(device=device, dtype=torch.float32).view(-1)
    if int(s.numel()) == 1 and num_primitives > 1:
        s = s.expand(num_primitives)
    if int(s.numel()) != num_primitives:
        raise ValueError(
            f"inv_sigma2s size must match num_primitives ({num_primitives}), "
            f"got {int(s.numel())}")
    return _f32(s)


def _check_ranges(isect_edge_ranges, num_intersects):
    r = _i32(isect_edge_ranges)
    if r.dim() != 2 or int(r.shape[1]) != 2:
        raise ValueError(
            f"isect_edge_ranges must be [num_intersects,2], got {tuple(r.shape)}")
    if int(r.shape[0]) != num_intersects:
        raise ValueError(
            "isect_edge_ranges first dim must match num_intersects "
            f"({num_intersects}), got {int(r.shape[0])}")
    return r


def _check_block(block):
    from .splat import check_block
    check_block(int(block[0]), int(block[1]))
    return int(block[0]), int(block[1])


def is_sub_block_tile(bx, by):
    from .splat import is_sub_block_tile as f
    return f(bx, by)


def _check_pixels(name, t, shape):
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must be {list(shape)}, got {list(t.shape)}")


def raster_records(edges_px, ids, ranges, colors, opacities, inv_s2, fill_rules, tile_bins,
                   img_h, img_w, *, stroke_widths=None, block_x=BLOCK_X, block_y=BLOCK_Y):
    """(edges, edge_culls, prim_recs) for the raster entry points, built on
    the device from the reference's inputs; raises ValueError when the
    intersections of one primitive carry different edge ranges, or tile_bins
    does not hold a list range within [0, num_intersects] for each of the
    image's block_x x block_y tiles."""
    dev = edges_px.device
    T = ((img_w + block_x - 1) // block_x) * ((img_h + block_y - 1) // block_y)
    if int(tile_bins.numel()) < 2 * T:
        raise ValueError(f"tile_bins must hold [{T}, 2] ranges for a {img_h}x{img_w} image, "
                         f"got {tuple(tile_bins.shape)}")
    E = int(edges_px.shape[0])
    P = int(colors.shape[0])
    I = int(ids.numel())
    edges = torch.empty((E, N.EDGE_RECORD_FLOATS), dtype=torch.float32, device=dev)
    culls = torch.empty((E, N.EDGE_CULL_INTS), dtype=torch.int32, device=dev)
    prims = torch.empty((P, N.PRIM_RECORD_FLOATS), dtype=torch.float32, device=dev)
    scratch = torch.empty((2 * P + E + 1,), dtype=torch.int32, device=dev)
    mode = 0 if stroke_widths is None else 1
    N.call("cs_raster_records_from_edges", mode, N.ptr(edges_px), E, N.ptr(ids), N.ptr(ranges), I,
           N.ptr(colors), N.ptr(opacities), N.ptr(inv_s2), N.ptr(fill_rules),
           N.ptr(stroke_widths), P, N.ptr(tile_bins), T, N.ptr(scratch),
           scratch.data_ptr() + 8 * P, scratch.data_ptr() + 4 * (2 * P + E), N.ptr(edges),
           N.ptr(culls), N.ptr(prims), N.stream(dev))
    status = int(scratch[-1].item())
    if status & 4:
        raise ValueError(f"tile_bins must hold ranges [start, end) within [0, {I}]")
    if status & 1:
        raise ValueError(f"primitive_ids_sorted holds ids outside [0, {P})")
    if status & 2:
        raise ValueError(
            "isect_edge_ranges must hold each primitive's edge range [start, end) within "
            f"[0, {E}], the same for every intersection of the primitive")
    return edges, culls, prims


def rasterize_cubic_fill_forward_tilelang(tile_bounds, block, img_size, primitive_ids_sorted,
                                          tile_bins, cubics_px, primitive_seg_offsets, colors,
                                          opacities, fill_rules, background, *, aa_widths=None,
                                          inv_sigma2s=None, edges_px, isect_edge_ranges,
                                          aa_width=DEFAULT_AA_WIDTH,
                                          distance_samples=DEFAULT_DISTANCE_SAMPLES,
                                          map_threads=DEFAULT_THREADS):
    """cubic_splatting.py:2181-2305 -> (out_img [H,W,3], final_Ts [H,W],
    final_idx [H,W])."""
    _ = (tile_bounds, primitive_seg_offsets, distance_samples, map_threads)
    img_width, img_height, _ = img_size
    H, W = int(img_height), int(img_width)
    num_primitives = int(colors.shape[0])
    num_intersects = int(primitive_ids_sorted.shape[0])
    dev = cubics_px.device
    out_img = torch.empty((H, W, 3), dtype=torch.float32, device=dev)
    final_Ts = torch.empty((H, W), dtype=torch.float32, device=dev)
    final_idx = torch.empty((H, W), dtype=torch.int32, device=dev)
    bg = background.to(device=dev, dtype=torch.float32).contiguous().view(3)

    def empty():
        out_img.copy_(bg.view(1, 1, 3).expand(H, W, 3))
        final_Ts.fill_(1.0)
        final_idx.fill_(0)
        return out_img, final_Ts, final_idx

    if num_intersects <= 0 or num_primitives <= 0:
        return empty()
    inv_s2 = _inv_sigma2s(aa_widths, inv_sigma2s, aa_width, num_primitives, dev)
    e_px = _f32(edges_px)
    if int(e_px.shape[0]) <= 0:
        return empty()
    ranges = _check_ranges(isect_edge_ranges, num_intersects)
    bx, by = _check_block(block)
    N.require_gpu(cubics_px, "cubics_px")
    ids = _i32(primitive_ids_sorted).view(-1)
    bins = _i32(tile_bins)
    edges, culls, prims = raster_records(e_px, ids, ranges, _f32(colors),
                                         _f32(opacities).view(-1), inv_s2,
                                         _i32(fill_rules).view(-1), bins, H, W, block_x=bx,
                                         block_y=by)
    if not is_sub_block_tile(bx, by):
        N.call("cs_rasterize_forward_any_tile", 0, N.ptr(ids), N.ptr(bins), N.ptr(edges),
               N.ptr(prims), N.ptr(bg), H, W, bx, by, N.ptr(out_img), 0, None, N.ptr(final_Ts),
               N.ptr(final_idx), N.stream(dev))
        return out_img, final_Ts, final_idx
    N.call("cs_rasterize_forward", 0, N.ptr(ids), N.ptr(bins), N.ptr(edges),
           N.ptr(culls), N.ptr(prims), N.ptr(bg), H, W, bx, by, 0, N.ptr(out_img), 0, None,
           N.ptr(final_Ts),
           N.ptr(final_idx), num_intersects, None, None, 0, 0, None, None, None, N.stream(dev))
    return out_img, final_Ts, final_idx


def rasterize_cubic_fill_backward_tilelang(tile_bounds, block, img_size, primitive_ids_sorted,
                                           tile_bins, cubics_px, primitive_seg_offsets, colors,
                                           opacities, fill_rules, background, final_Ts,
                                           final_idx, v_output, *, aa_widths=None,
                                           inv_sigma2s=None, edges_px, isect_edge_ranges,
                                           segment_edge_offsets=None, edge_t_starts=None,
                                           edge_t_ends=None, aa_width=DEFAULT_AA_WIDTH,
                                           distance_samples=DEFAULT_DISTANCE_SAMPLES,
                                           flatten_method=DEFAULT_CUBIC_FLATTEN_METHOD,
                                           map_threads=DEFAULT_THREADS, curve_contrib_rgb=None,
                                           curve_isect_contrib=None):
    """cubic_splatting.py:2572-2747 -> (v_cubics_px [nseg,4,2], v_colors [P,3],
    v_opacities [P], v_inv_sigma2s [P]).  The edge gradients are folded into
    the control points inside the raster kernel with
    _accumulate_edge_grads_to_cubics' weights (:2308-2487): uniform
    t = e / (distance_samples - 1), or the de Casteljau intervals."""
    _ = (tile_bounds, primitive_seg_offsets, map_threads)
    img_width, img_height, _ = img_size
    H, W = int(img_height), int(img_width)
    num_primitives = int(colors.shape[0])
    num_segments = int(cubics_px.shape[0])
    dev = colors.device
    v_colors = torch.zeros_like(colors, dtype=torch.float32)
    v_opacities = torch.zeros_like(opacities.view(-1), dtype=torch.float32)
    v_inv_sigma2s = torch.zeros((num_primitives,), dtype=torch.float32, device=dev)
    v_cubics_px = torch.zeros_like(cubics_px, dtype=torch.float32)
    num_intersects = int(primitive_ids_sorted.numel())
    if num_intersects <= 0 or num_primitives <= 0 or num_segments <= 0:
        return v_cubics_px, v_colors, v_opacities, v_inv_sigma2s
    inv_s2 = _inv_sigma2s(aa_widths, inv_sigma2s, aa_width, num_primitives, cubics_px.device)
    e_px = _f32(edges_px)
    E = int(e_px.shape[0])
    if E <= 0:
        return v_cubics_px, v_colors, v_opacities, v_inv_sigma2s
    ranges = _check_ranges(isect_edge_ranges, int(primitive_ids_sorted.shape[0]))
    bx, by = _check_block(block)
    contrib = None
    if curve_contrib_rgb is not None:
        if curve_contrib_rgb.shape != colors.shape:
            raise ValueError("curve_contrib_rgb must match colors shape "
                             f"{tuple(colors.shape)}, got {tuple(curve_contrib_rgb.shape)}")
        contrib = curve_contrib_rgb.to(device=dev, dtype=torch.float32).contiguous()
    isect_contrib = None
    if curve_isect_contrib is not None:
        if curve_isect_contrib.ndim != 1:
            raise ValueError("curve_isect_contrib must be a 1D tensor")
        if int(curve_isect_contrib.numel()) != num_intersects:
            raise ValueError("curve_isect_contrib size must match primitive_ids_sorted")
        isect_contrib = curve_isect_contrib.to(device=dev, dtype=torch.float32).contiguous()
    method = normalize_cubic_flatten_method(flatten_method)
    ids = _i32(primitive_ids_sorted).view(-1)
    bins = _i32(tile_bins)
    _check_pixels("final_Ts", final_Ts, (H, W))
    _check_pixels("final_idx", final_idx, (H, W))
    _check_pixels("v_output", v_output, (H, W, 3))
    edges, culls, prims = raster_records(e_px, ids, ranges, _f32(colors),
                                         _f32(opacities).view(-1), inv_s2,
                                         _i32(fill_rules).view(-1), bins, H, W, block_x=bx,
                                         block_y=by)
    bg = background.to(device=dev, dtype=torch.float32).contiguous().view(3)
    v_px = v_cubics_px if (v_cubics_px.dtype is torch.float32 and v_cubics_px.is_contiguous()) \
        else torch.zeros((num_segments, 4, 2), dtype=torch.float32, device=dev)
    common = (0, N.ptr(ids), N.ptr(bins), N.ptr(edges), N.ptr(culls), N.ptr(prims), N.ptr(bg),
              H, W, bx, by)
    # No scratch copies here: direct atomic additions (nprim is then unused).
    grads = (N.ptr(v_px), N.ptr(v_colors), N.ptr(v_opacities), N.ptr(v_inv_sigma2s), None,
             N.ptr(contrib), N.ptr(isect_contrib), 0, None, None, N.stream(dev))
    fT, fi, vo = _f32(final_Ts), _i32(final_idx), _f32(v_output)
    if not is_sub_block_tile(bx, by):
        # Tiles of any size: endpoint gradients per edge, then folded into
        # the control points (cubic_splatting.py:2308-2487).
        v_edges = torch.zeros((E, 4), dtype=torch.float32, device=dev)
        N.call("cs_rasterize_backward_any_tile", 0, N.ptr(ids), N.ptr(bins), N.ptr(edges),
               N.ptr(prims), N.ptr(bg), H, W, bx, by, N.ptr(fT), N.ptr(fi), N.ptr(vo), 0,
               N.ptr(v_edges), N.ptr(v_colors), N.ptr(v_opacities), N.ptr(v_inv_sigma2s), None,
               N.ptr(contrib), N.ptr(isect_contrib), N.stream(dev))
        v_norm = torch.empty_like(v_px)
        if method == "bernstein":
            eps = max(2, int(distance_samples)) - 1
            if E != num_segments * eps:
                raise ValueError(f"v_edges size mismatch: got {E}, expected {num_segments * eps}")
            N.call("cs_accumulate_edge_grads", N.ptr(v_edges), num_segments, eps, H, W,
                   N.ptr(v_px), N.ptr(v_norm), N.stream(dev))
        else:
            if segment_edge_offsets is None or edge_t_starts is None or edge_t_ends is None:
                raise ValueError("de_casteljau flatten backward requires CSR metadata "
                                 "(segment_edge_offsets, edge_t_starts, edge_t_ends)")
            seo = _i32(segment_edge_offsets).view(-1)
            if int(seo.numel()) != num_segments + 1:
                raise ValueError(f"segment_edge_offsets size mismatch: got {int(seo.numel())}, "
                                 f"expected {num_segments + 1}")
            N.call("cs_accumulate_edge_grads_csr", N.ptr(v_edges), N.ptr(_f32(edge_t_starts)),
                   N.ptr(_f32(edge_t_ends)), N.ptr(seo), num_segments, H, W, N.ptr(v_px),
                   N.ptr(v_norm), N.stream(dev))
        if v_px is not v_cubics_px:
            v_cubics_px.copy_(v_px)
        return v_cubics_px, v_colors, v_opacities, v_inv_sigma2s
    if method == "bernstein":
        eps = max(2, int(distance_samples)) - 1
        if E != num_segments * eps:
            raise ValueError(f"v_edges size mismatch: got {E}, expected {num_segments * eps}")
        N.call("cs_rasterize_backward", *common, eps, N.ptr(fT), N.ptr(fi), None, None,
               N.ptr(vo), 0, *grads)
    else:
        if segment_edge_offsets is None or edge_t_starts is None or edge_t_ends is None:
            raise ValueError("de_casteljau flatten backward requires CSR metadata "
                             "(segment_edge_offsets, edge_t_starts, edge_t_ends)")
        seo = _i32(segment_edge_offsets).view(-1)
        if int(seo.numel()) != num_segments + 1:
            raise ValueError(f"segment_edge_offsets size mismatch: got {int(seo.numel())}, "
                             f"expected {num_segments + 1}")
        aux = torch.zeros((E, N.EDGE_AUX_INTS), dtype=torch.int32, device=dev)
        N.call("cs_edge_aux_from_csr", N.ptr(seo), num_segments, N.ptr(_f32(edge_t_starts)),
               N.ptr(_f32(edge_t_ends)), E, N.ptr(aux), N.stream(dev))
        N.call("cs_rasterize_backward_de_casteljau", *common, N.ptr(aux), N.ptr(fT), N.ptr(fi),
               None, None, N.ptr(vo), 0, *grads)
    if v_px is not v_cubics_px:
        v_cubics_px.copy_(v_px)
    # As in the reference, the contribution sums land in the caller's tensors
    # when those are float32 and contiguous on the device (else in copies).
    return v_cubics_px, v_colors, v_opacities, v_inv_sigma2s
