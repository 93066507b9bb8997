"""Reference-layout building blocks of the binning path, one HIP kernel each:
project_cubics_2d_forward_tilelang (ops/cubic_splatting.py:822-871),
map_cubic_to_intersects_tilelang (:874-915),
_primitive_tile_ranges_from_segment_tile_ranges (:2140-2178),
_build_fill_isect_edge_ranges (:1849-1860), get_tile_bin_edges_tilelang
(ops/tile_bins.py:46-60), and the flattening blocks
_flatten_cubics_to_edges (:1654-1846, both methods),
cubic_adaptive_flatness_flags_tilelang (:1918-1965),
cubic_split_half_tilelang (:2033-2068) and _accumulate_edge_grads_to_cubics
(:2490-2545).  The fused forward (repo_amd.splat) does not use them; they
keep the reference's intermediate API callable."""
from __future__ import annotations

import torch

from . import _native as N

DEFAULT_THREADS = 256


def _f32(t):
    return t.detach().to(torch.float32).contiguous()


def _i32(t):
    return t.detach().to(torch.int32).contiguous()


def project_cubics_2d_forward_tilelang(cubics_norm, stroke_widths, support_radii, img_height,
                                       img_width, tile_bounds, *, block_x=16, block_y=16,
                                       threads=DEFAULT_THREADS, aabb_pad=1.0,
                                       aniso_intersects=False):
    n = int(cubics_norm.shape[0])
    dev = cubics_norm.device
    cubics_px = torch.empty((n, 4, 2), dtype=torch.float32, device=dev)
    tile_ranges = torch.empty((n, 4), dtype=torch.int32, device=dev)
    num_tiles_hit = torch.empty((n,), dtype=torch.int32, device=dev)
    if n == 0:
        return cubics_px, tile_ranges, num_tiles_hit
    N.call("cs_project_cubics_2d_forward", N.ptr(_f32(cubics_norm)),
           N.ptr(_f32(stroke_widths).view(-1)), N.ptr(_f32(support_radii).view(-1)), n,
           int(img_height), int(img_width), int(block_x), int(block_y), float(aabb_pad),
           int(bool(aniso_intersects)), N.ptr(cubics_px), N.ptr(tile_ranges),
           N.ptr(num_tiles_hit), N.stream(dev))
    return cubics_px, tile_ranges, num_tiles_hit


def primitive_tile_ranges_from_segment_tile_ranges(segment_tile_ranges, primitive_seg_offsets,
                                                   tile_bounds):
    offs = _i32(primitive_seg_offsets).view(-1)
    P = max(0, int(offs.numel()) - 1)
    dev = segment_tile_ranges.device
    out = torch.empty((P, 4), dtype=torch.int32, device=dev)
    hit = torch.empty((P,), dtype=torch.int32, device=dev)
    if P == 0:
        return out, hit
    N.call("cs_primitive_tile_ranges", N.ptr(_i32(segment_tile_ranges)), N.ptr(offs), P,
           int(tile_bounds[0]), int(tile_bounds[1]), N.ptr(out), N.ptr(hit), N.stream(dev))
    return out, hit


def map_cubic_to_intersects_tilelang(tile_ranges, depths, cum_tiles_hit, tile_bounds, *,
                                     threads=DEFAULT_THREADS):
    dev = tile_ranges.device
    num_intersects = int(cum_tiles_hit[-1].item()) if int(cum_tiles_hit.numel()) > 0 else 0
    if num_intersects <= 0:
        return (torch.empty((0,), dtype=torch.int64, device=dev),
                torch.empty((0,), dtype=torch.int32, device=dev))
    isect_ids = torch.empty((num_intersects,), dtype=torch.int64, device=dev)
    curve_ids = torch.empty((num_intersects,), dtype=torch.int32, device=dev)
    tr = _i32(tile_ranges)
    N.call("cs_map_cubic_to_intersects", N.ptr(tr), N.ptr(_f32(depths).view(-1)),
           N.ptr(_i32(cum_tiles_hit)), int(tr.shape[0]), int(tile_bounds[0]), N.ptr(isect_ids),
           N.ptr(curve_ids), N.stream(dev))
    return isect_ids, curve_ids


def build_fill_isect_edge_ranges(primitive_ids_sorted, primitive_seg_offsets,
                                 edges_per_segment: int):
    ids = _i32(primitive_ids_sorted).view(-1)
    n = int(ids.numel())
    out = torch.empty((n, 2), dtype=torch.int32, device=ids.device)
    if n:
        N.call("cs_isect_edge_ranges", N.ptr(ids), N.ptr(_i32(primitive_seg_offsets)), n,
               int(edges_per_segment), N.ptr(out), N.stream(ids.device))
    return out


def get_tile_bin_edges_tilelang(num_intersects, isect_ids_sorted, *, num_tiles, compact=False,
                                threads=DEFAULT_THREADS):
    rows = int(num_tiles) if compact else max(int(num_tiles), int(num_intersects))
    keys = isect_ids_sorted.detach().to(torch.int64).contiguous()
    bins = torch.empty((rows, 2), dtype=torch.int32, device=keys.device)
    N.call("cs_get_tile_bin_edges", N.ptr(keys), int(num_intersects), rows, N.ptr(bins),
           N.stream(keys.device))
    return bins


# ---- flattening blocks (ops/cubic_splatting.py:1654-2068, 2399-2526) ----

DE_CASTELJAU_FLATNESS_TOL_PX = 0.5   # DEFAULT_DE_CASTELJAU_FLATNESS_TOL_PX (:18)


def cubic_adaptive_flatness_flags_tilelang(cubics, *, tol_px, force_flat=False,
                                           threads=DEFAULT_THREADS):
    """cubic_splatting.py:1918-1965 -> uint8 [n] (1 = flat within tol_px)."""
    c = _f32(cubics)
    n = int(c.shape[0])
    out = torch.empty((n,), dtype=torch.uint8, device=c.device)
    if n:
        N.call("cs_cubic_flatness_flags", N.ptr(c), n, float(tol_px), int(bool(force_flat)),
               N.ptr(out), N.stream(c.device))
    return out


def cubic_split_half_tilelang(cubics, *, threads=DEFAULT_THREADS):
    """cubic_splatting.py:2033-2068 -> (left, right) halves at t = 0.5, [n,4,2] each."""
    c = _f32(cubics)
    n = int(c.shape[0])
    halves = torch.empty((2, n, 4, 2), dtype=torch.float32, device=c.device)
    if n:
        N.call("cs_cubic_split_half", N.ptr(c), n, N.ptr(halves[0]), N.ptr(halves[1]),
               N.stream(c.device))
    return halves[0], halves[1]


def flatten_cubics_to_edges(cubics_px, primitive_seg_offsets, *, distance_samples,
                            flatten_method="bernstein"):
    """_flatten_cubics_to_edges (cubic_splatting.py:1654-1846) -> (edges_px [E,2,2],
    primitive_edge_offsets [P+1], segment_edge_offsets [nseg+1], edge_t_starts,
    edge_t_ends); the last two are None for the Bernstein flattening.  The
    adaptive branch reads its edge count back to the host to size the outputs,
    as the reference does."""
    from .splat import normalize_cubic_flatten_method
    c = _f32(cubics_px)
    offs = _i32(primitive_seg_offsets).view(-1)
    if c.dim() != 3 or tuple(c.shape[1:]) != (4, 2):
        raise ValueError(f"cubics_px must be [N,4,2], got {tuple(c.shape)}")
    if offs.dim() != 1 or int(offs.numel()) <= 0:
        raise ValueError(
            f"primitive_seg_offsets must be non-empty 1D tensor, got {tuple(offs.shape)}")
    method = normalize_cubic_flatten_method(flatten_method)
    dev = c.device
    nseg = int(c.shape[0])
    P = int(offs.numel()) - 1
    S = max(2, int(distance_samples))
    eps = S - 1
    if method == "bernstein":
        edges = torch.empty((nseg * eps, 2, 2), dtype=torch.float32, device=dev)
        if nseg:
            N.call("cs_flatten_cubics_bernstein", N.ptr(c), nseg, S, N.ptr(edges), N.stream(dev))
        prim_eo = (offs.to(torch.int64) * eps).to(torch.int32)
        seg_eo = torch.arange(0, (nseg + 1) * eps, eps, dtype=torch.int32, device=dev)
        return edges, prim_eo, seg_eo, None, None
    per_seg = int(N.lib().cs_de_casteljau_max_edges_per_segment(S))
    if per_seg <= 0 or nseg * per_seg >= 2 ** 31:
        raise ValueError(f"de_casteljau flattening of {nseg} segments with "
                         f"distance_samples={S} exceeds the supported edge count")
    cap = max(1, nseg * per_seg)
    ints = torch.empty((nseg + (nseg + 1) + (P + 1),), dtype=torch.int32, device=dev)
    leaf_counts, seg_eo, prim_eo = ints[:nseg], ints[nseg:2 * nseg + 1], ints[2 * nseg + 1:]
    scan_temp = torch.empty((int(N.lib().cs_scan_temp_elems(max(nseg, 1))),), dtype=torch.int32,
                            device=dev)
    edges = torch.empty((cap, 2, 2), dtype=torch.float32, device=dev)
    ts = torch.empty((2, cap), dtype=torch.float32, device=dev)
    N.call("cs_flatten_cubics_de_casteljau", N.ptr(c), N.ptr(offs), P, nseg, S, N.ptr(leaf_counts),
           N.ptr(scan_temp), N.ptr(seg_eo), N.ptr(prim_eo), N.ptr(edges), N.ptr(ts[0]),
           N.ptr(ts[1]), N.stream(dev))
    E = int(seg_eo[-1].item())
    return edges[:E], prim_eo, seg_eo, ts[0, :E], ts[1, :E]


def accumulate_edge_grads_to_cubics(v_edges, num_segments, *, distance_samples,
                                    flatten_method="bernstein", segment_edge_offsets=None,
                                    edge_t_starts=None, edge_t_ends=None,
                                    threads=DEFAULT_THREADS):
    """_accumulate_edge_grads_to_cubics (cubic_splatting.py:2490-2545) -> v_cubics_px
    [nseg,4,2]."""
    from .splat import normalize_cubic_flatten_method
    method = normalize_cubic_flatten_method(flatten_method)
    nseg = int(num_segments)
    ve = _f32(v_edges)
    dev = ve.device
    v_px = torch.empty((max(nseg, 0), 4, 2), dtype=torch.float32, device=dev)
    if nseg <= 0:
        return v_px
    if method == "bernstein":
        eps = max(2, int(distance_samples)) - 1
        if int(ve.shape[0]) != nseg * eps:
            raise ValueError(f"v_edges size mismatch: got {int(ve.shape[0])}, "
                             f"expected {nseg * eps}")
        N.call("cs_accumulate_edge_grads", N.ptr(ve), nseg, eps, 2, 2, N.ptr(v_px), None,
               N.stream(dev))
        return v_px
    if segment_edge_offsets is None or edge_t_starts is None or edge_t_ends is None:
        raise ValueError("de_casteljau flatten backward requires CSR metadata "
                         "(segment_edge_offsets, edge_t_starts, edge_t_ends)")
    seo = _i32(segment_edge_offsets).view(-1)
    if int(seo.numel()) != nseg + 1:
        raise ValueError(f"segment_edge_offsets size mismatch: got {int(seo.numel())}, "
                         f"expected {nseg + 1}")
    N.call("cs_accumulate_edge_grads_csr", N.ptr(ve), N.ptr(_f32(edge_t_starts)),
           N.ptr(_f32(edge_t_ends)), N.ptr(seo), nseg, 2, 2, N.ptr(v_px), None, N.stream(dev))
    return v_px
