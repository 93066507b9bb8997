"""Host side of the 2D Gaussian splat path: projection, binning, raster and
their backwards, and the op-level functions of the reference's
ops/forward2d.py, ops/backward2d.py, ops/intersects.py and ops/rasterize.py.

Every device computation is a call into libcubicsplat_hip.so on torch's
current stream; there is no CPU or torch fallback.  The binning replaces the
reference's cumsum + map + torch.sort + tile-bin pass
(tilelang_renderer.py:224-269) with depth ranks and per-tile counting lists
(cs_gs_bin_prepare / cs_bin_finish), which produce the same
gaussian_ids_sorted and tile_bins; one host read of the intersection count
sizes gaussian_ids_sorted (the reference reads the same count,
tilelang_renderer.py:54-58).
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _native as N
from .splat import _give_pinned, _layout, _take_pinned

GS_RECORD_FLOATS = N.GS_RECORD_BYTES // 4


def _f32(t: torch.Tensor) -> torch.Tensor:
    return t.detach().to(torch.float32).contiguous()


def _i32(t: torch.Tensor) -> torch.Tensor:
    return t.detach().to(torch.int32).contiguous()


def tile_bounds(img_h: int, img_w: int, block_x: int, block_y: int):
    """tilelang_renderer.py:69-75."""
    return ((img_w + block_x - 1) // block_x, (img_h + block_y - 1) // block_y, 1)


def _check_block(block_x: int, block_y: int) -> None:
    if block_x <= 0 or block_y <= 0 or block_x * block_y > 1024:
        raise ValueError(
            f"block_x * block_y must be in [1, 1024] (one thread per pixel of a tile in the "
            f"reference, rasterize.py:51); got {block_x} x {block_y}")


# ----------------------------------------------------------------- projection


def project_forward(means2d, scales2d, rotation, img_h: int, img_w: int, block_x: int,
                    block_y: int):
    """forward2d.py:14-220 -> (xys, depths, radii, conics, num_tiles_hit)."""
    _check_block(block_x, block_y)
    if rotation.dim() == 2 and rotation.shape[1] == 1:
        rotation = rotation.view(-1)
    m, s, r = _f32(means2d), _f32(scales2d), _f32(rotation)
    n = int(m.shape[0])
    dev = m.device
    ints = torch.empty((2, n), dtype=torch.int32, device=dev)
    xys, depths, conics = (torch.empty((n, 2), dtype=torch.float32, device=dev),
                           torch.empty((n,), dtype=torch.float32, device=dev),
                           torch.empty((n, 3), dtype=torch.float32, device=dev))
    radii, tiles = ints[0], ints[1]
    with N.prof("gs.fwd.proj"):
        N.call("cs_gs_project_forward", N.ptr(m), N.ptr(s), N.ptr(r), n, int(img_h), int(img_w),
               int(block_x), int(block_y), N.ptr(xys), N.ptr(depths), N.ptr(radii),
               N.ptr(conics), N.ptr(tiles), N.stream(dev))
    return xys, depths, radii, conics, tiles


def project_backward(scales2d, rotation, radii, conics, v_xy, v_conic, img_h: int, img_w: int,
                     gaussian_meta: Optional[torch.Tensor] = None, with_cov2d: bool = False):
    """backward2d.py:8-212 with tilelang_renderer.py:111-116's meta scaling ->
    (v_cov2d or None, v_mean2d, v_scale, v_rot)."""
    r = _f32(rotation).view(-1)
    n = int(r.numel())
    dev = r.device
    buf = torch.empty((n * (8 if with_cov2d else 5),), dtype=torch.float32, device=dev)
    v_mean, v_scale = buf[:2 * n].view(n, 2), buf[2 * n:4 * n].view(n, 2)
    v_rot = buf[4 * n:5 * n]
    v_cov = buf[5 * n:8 * n].view(n, 3) if with_cov2d else None
    meta = None if gaussian_meta is None else _i32(gaussian_meta).view(-1)
    with N.prof("gs.bwd.proj"):
        N.call("cs_gs_project_backward", N.ptr(_f32(scales2d)), N.ptr(r), N.ptr(_i32(radii)),
               N.ptr(_f32(conics)), N.ptr(_f32(v_xy)), N.ptr(_f32(v_conic)), N.ptr(meta), n,
               int(img_h), int(img_w), N.ptr(v_cov), N.ptr(v_mean), N.ptr(v_scale), N.ptr(v_rot),
               N.stream(dev))
    return v_cov, v_mean, v_scale, v_rot


# -------------------------------------------------------------------- binning


def _gs_fields(n, T, radix_elems, scan_elems, list_elems):
    f32, i32 = torch.float32, torch.int32
    return (
        ("tile_rects", i32, (n, 4)),
        ("keys", i32, (n,)),
        ("order", i32, (n,)),
        ("keys_alt", i32, (n,)),
        ("vals_alt", i32, (n,)),
        ("radix_counts", i32, (radix_elems,)),
        ("scan_temp", i32, (scan_elems,)),
        ("rank_tile_ranges", i32, (n, 4)),
        ("tile_count", i32, (list_elems,)),
        ("tile_scratch", i32, (list_elems,)),
        ("status", i32, (4,)),
        ("tile_bins", i32, (T, 2)),
        ("records", f32, (n, GS_RECORD_FLOATS)),
        ("grad_accum", f32, (9 * n,)),
    )


class GsBinned:
    """One binning of n Gaussians: the arena's buffers as lazy views
    (tile_rects, order, tile_bins [T,2], records [n,12], grad_accum [9n] ...),
    gaussian_ids_sorted and num_intersects."""

    def __init__(self, n, img_h, img_w, block_x, block_y, arena, table):
        self.n, self.img_h, self.img_w = n, img_h, img_w
        self.block_x, self.block_y = block_x, block_y
        self.arena = arena
        self._table = table
        self._base = arena.data_ptr()
        self._views = {}
        self.gaussian_ids_sorted: Optional[torch.Tensor] = None
        self.num_intersects = 0
        self.grad_accum_clean = True

    def ptr(self, name: str) -> int:
        return self._base + self._table[name][0]

    def __getattr__(self, name):
        table = self.__dict__.get("_table")
        if table is None or name not in table:
            raise AttributeError(name)
        v = self._views.get(name)
        if v is None:
            off, dt, shape = table[name]
            n = 1
            for d in shape:
                n *= d
            v = self.arena[off:off + n * 4].view(dt).view(shape)
            self._views[name] = v
        return v


def bin_gaussians(xys, conics, radii, depths, img_h: int, img_w: int, block_x: int,
                  block_y: int) -> GsBinned:
    """gaussian_ids_sorted and tile_bins of the reference's map + stable sort
    + tile-bin pass (tilelang_renderer.py:224-269), with the backward's
    gradient accumulators cleared in the same launches.  Raises the
    reference's RuntimeError when there are no intersections."""
    _check_block(block_x, block_y)
    xy, q, rad, d = _f32(xys), _f32(conics), _i32(radii).view(-1), _f32(depths).view(-1)
    n = int(xy.shape[0])
    if n == 0:
        raise RuntimeError("No intersections generated; increase num_points or radii")
    dev = xy.device
    lib = N.lib()
    tbx, tby, _ = tile_bounds(img_h, img_w, block_x, block_y)
    T = tbx * tby
    key = ("gs", dev.index, n, img_h, img_w, block_x, block_y)
    table, nbytes = _layout(key, _gs_fields(
        n, T, int(lib.cs_radix_counts_elems(n)), int(lib.cs_scan_temp_elems(max(n, T))),
        int(lib.cs_bin_list_elems(n, img_h, img_w, block_x, block_y))))
    arena = torch.empty((nbytes,), dtype=torch.uint8, device=dev)
    b = GsBinned(n, img_h, img_w, block_x, block_y, arena, table)
    q_ = b.ptr
    st = N.stream(dev)
    with N.prof("gs.fwd.bin_prepare"):
        N.call("cs_gs_bin_prepare", N.ptr(xy), N.ptr(q), N.ptr(rad), N.ptr(d), n, int(img_h),
               int(img_w), int(block_x), int(block_y), q_("tile_rects"), q_("keys"), q_("order"),
               q_("keys_alt"), q_("vals_alt"), q_("radix_counts"), q_("scan_temp"),
               q_("rank_tile_ranges"), q_("tile_count"), q_("tile_scratch"), q_("status"), st)
    pinned = _take_pinned(dev.index if dev.index is not None else torch.cuda.current_device())
    status_host, event = pinned[0], pinned[1]
    hip = N.hip()
    N.hip_check(hip.hipMemcpyAsync(status_host.data_ptr(), q_("status"), 16,
                                   N.HIP_MEMCPY_DEVICE_TO_HOST, st), "hipMemcpyAsync")
    N.hip_check(hip.hipEventRecord(event, st), "hipEventRecord")
    N.hip_check(hip.hipEventSynchronize(event), "hipEventSynchronize")
    I = int(status_host[0])
    _give_pinned(pinned)
    if I < 0:
        raise RuntimeError(f"intersection count overflowed int32 ({I})")
    if I < 1:
        raise RuntimeError("No intersections generated; increase num_points or radii")
    ids = torch.empty((I,), dtype=torch.int32, device=dev)
    with N.prof("gs.fwd.bin_finish"):
        N.call("cs_bin_finish", q_("order"), q_("rank_tile_ranges"), n, q_("status"), I,
               int(img_h), int(img_w), int(block_x), int(block_y), q_("tile_count"),
               q_("tile_scratch"), N.ptr(ids), q_("tile_bins"),
               q_("grad_accum"), 9 * n, None, st)
    b.gaussian_ids_sorted = ids
    b.num_intersects = I
    return b


# --------------------------------------------------------------------- raster


def pack_records(xys, conics, colors, opacities, out: Optional[torch.Tensor] = None):
    """The raster's per-Gaussian records [n, 12] (cs_gs_pack_records)."""
    xy, q, c = _f32(xys), _f32(conics), _f32(colors)
    o = _f32(opacities).view(-1)
    n = int(xy.shape[0])
    if out is None:
        out = torch.empty((n, GS_RECORD_FLOATS), dtype=torch.float32, device=xy.device)
    with N.prof("gs.pack"):
        N.call("cs_gs_pack_records", N.ptr(xy), N.ptr(q), N.ptr(c), N.ptr(o), n, N.ptr(out),
               N.stream(xy.device))
    return out


def rasterize_forward(gaussian_ids_sorted, tile_bins, records, background, img_h: int,
                      img_w: int, block_x: int, block_y: int):
    """rasterize.py:18-157 -> (out_img [H,W,3], final_Ts [H,W], final_idx [H,W])."""
    _check_block(block_x, block_y)
    dev = records.device
    out = torch.empty((img_h, img_w, 3), dtype=torch.float32, device=dev)
    tid = torch.empty((2, img_h, img_w), dtype=torch.float32, device=dev)
    final_T, final_idx = tid[0], tid[1].view(torch.int32)
    with N.prof("gs.fwd.rast"):
        N.call("cs_gs_rasterize_forward", N.ptr(_i32(gaussian_ids_sorted)), N.ptr(_i32(tile_bins)),
               N.ptr(records), N.ptr(_f32(background).view(-1)), int(img_h), int(img_w),
               int(block_x), int(block_y), N.ptr(out), N.ptr(final_T), N.ptr(final_idx),
               N.stream(dev))
    return out, final_T, final_idx


def rasterize_backward(gaussian_ids_sorted, tile_bins, records, background, img_h: int,
                       img_w: int, block_x: int, block_y: int, final_Ts, final_idx, v_output,
                       v_output_alpha=None, *, intersect_meta_sorted=None, grads=None,
                       curve_contrib_rgb=None, curve_isect_contrib=None):
    """rasterize.py:160-529 -> (v_xy [n,2], v_conic [n,3], v_rgb [n,3],
    v_opacity [n]).  `grads` is a zeroed float32 buffer of 9n elements to
    accumulate into (a fresh one when None); the contribution outputs, when
    given, are contiguous float32 tensors that the kernel adds into."""
    _check_block(block_x, block_y)
    dev = records.device
    n = int(records.shape[0])
    if grads is None:
        grads = torch.zeros((9 * n,), dtype=torch.float32, device=dev)
    v_xy, v_conic = grads[:2 * n].view(n, 2), grads[2 * n:5 * n].view(n, 3)
    v_rgb, v_op = grads[5 * n:8 * n].view(n, 3), grads[8 * n:9 * n]
    meta = None if intersect_meta_sorted is None else _i32(intersect_meta_sorted).view(-1)
    va = None if v_output_alpha is None else _f32(v_output_alpha)
    with N.prof("gs.bwd.rast"):
        N.call("cs_gs_rasterize_backward", N.ptr(_i32(gaussian_ids_sorted)), N.ptr(meta),
               N.ptr(_i32(tile_bins)), N.ptr(records), N.ptr(_f32(background).view(-1)),
               int(img_h), int(img_w), int(block_x), int(block_y), N.ptr(_f32(final_Ts)),
               N.ptr(_i32(final_idx)), N.ptr(_f32(v_output)), N.ptr(va), N.ptr(v_xy),
               N.ptr(v_conic), N.ptr(v_rgb), N.ptr(v_op), N.ptr(curve_contrib_rgb),
               N.ptr(curve_isect_contrib), N.stream(dev))
    return v_xy, v_conic, v_rgb, v_op


# ------------------------------------------------------ reference-layout ops


def map_gaussian_to_intersects(num_points: int, num_intersects: int, xys, depths, radii,
                               cum_tiles_hit, tile_bounds_, *, block_x: int, block_y: int,
                               conics=None):
    """intersects.py:243-309: the reference's int64 keys and Gaussian ids."""
    dev = xys.device
    isect_ids = torch.empty((int(num_intersects),), dtype=torch.int64, device=dev)
    gaussian_ids = torch.empty((int(num_intersects),), dtype=torch.int32, device=dev)
    if conics is not None:
        if conics.ndim != 2 or conics.shape[1] != 3:
            raise ValueError("conics must be shaped (num_points, 3)")
        if conics.shape[0] != num_points:
            raise ValueError(
                f"conics num_points mismatch: expected {num_points}, got {conics.shape[0]}")
    N.call("cs_gs_map_to_intersects", N.ptr(_f32(xys)),
           None if conics is None else N.ptr(_f32(conics)), N.ptr(_f32(depths).view(-1)),
           N.ptr(_i32(radii).view(-1)), N.ptr(_i32(cum_tiles_hit).view(-1)), int(num_points),
           int(num_intersects), int(tile_bounds_[0]), int(tile_bounds_[1]), int(block_x),
           int(block_y), N.ptr(isect_ids), N.ptr(gaussian_ids), N.stream(dev))
    return isect_ids, gaussian_ids
