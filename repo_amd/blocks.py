"""Reference-layout building blocks of the binning path, one HIP kernel each:
project_cubics_2d_forward_tilelang (ops/cubic_splatting.py:822-871),
map_cubic_to_intersects_tilelang (:874-915),
_primitive_tile_ranges_from_segment_tile_ranges (:2140-2178),
_build_fill_isect_edge_ranges (:1849-1860) and get_tile_bin_edges_tilelang
(ops/tile_bins.py:46-60).  The fused forward (repo_amd.splat) does not use
them; they keep the reference's intermediate API callable."""
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
