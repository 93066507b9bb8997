"""manbo.ops.rasterize (reference ops/rasterize.py) on MI355X."""
from __future__ import annotations

import torch

from repo_amd import gaussian as _G

BLOCK_X = 16
BLOCK_Y = 16
DEFAULT_THREADS = 256


def rasterize_forward_tilelang(tile_bounds, block, img_size, gaussian_ids_sorted, tile_bins, xys,
                               conics, colors, opacities, background):
    """rasterize.py:532-570 -> (out_img [H,W,3], final_Ts [H,W], final_idx
    [H,W]); block = (block_x, block_y, 1), img_size = (W, H, 1)."""
    block_x, block_y, _ = block
    img_w, img_h, _ = img_size
    records = _G.pack_records(xys, conics, colors, opacities)
    return _G.rasterize_forward(gaussian_ids_sorted, tile_bins, records, background, int(img_h),
                                int(img_w), int(block_x), int(block_y))


def rasterize_backward_tilelang(tile_bounds, block, img_size, gaussian_ids_sorted, tile_bins, xys,
                                conics, colors, opacities, background, final_Ts, final_idx,
                                v_output, v_output_alpha, *, intersect_meta_sorted=None,
                                curve_contrib_rgb=None, curve_isect_contrib=None):
    """rasterize.py:573-646 -> (v_xy, v_conic, v_rgb, v_opacity).  The
    contribution tensors, when given, receive the sums in place when they are
    contiguous float32 on the device (the reference's .to().contiguous() is
    then the tensor itself)."""
    block_x, block_y, _ = block
    img_w, img_h, _ = img_size
    if opacities.dim() == 1:
        opac_was_2d = False
    elif opacities.dim() == 2 and opacities.shape[1] == 1:
        opac_was_2d = True
    else:
        raise ValueError("opacities must be shape (N,) or (N,1)")
    if curve_contrib_rgb is not None:
        if curve_contrib_rgb.shape != colors.shape:
            raise ValueError("curve_contrib_rgb must match colors shape "
                             f"{tuple(colors.shape)}, got {tuple(curve_contrib_rgb.shape)}")
        curve_contrib_rgb = curve_contrib_rgb.to(device=colors.device,
                                                 dtype=torch.float32).contiguous()
    if curve_isect_contrib is not None:
        if curve_isect_contrib.ndim != 1:
            raise ValueError("curve_isect_contrib must be a 1D tensor")
        if int(curve_isect_contrib.numel()) != int(gaussian_ids_sorted.numel()):
            raise ValueError("curve_isect_contrib size must match gaussian_ids_sorted")
        curve_isect_contrib = curve_isect_contrib.to(device=colors.device,
                                                     dtype=torch.float32).contiguous()
    if intersect_meta_sorted is not None:
        if intersect_meta_sorted.ndim != 1:
            raise ValueError("intersect_meta_sorted must be a 1D tensor")
        if intersect_meta_sorted.numel() != gaussian_ids_sorted.numel():
            raise ValueError("intersect_meta_sorted size must match gaussian_ids_sorted")
    records = _G.pack_records(xys, conics, colors, opacities)
    v_xy, v_conic, v_rgb, v_opacity = _G.rasterize_backward(
        gaussian_ids_sorted, tile_bins, records, background, int(img_h), int(img_w),
        int(block_x), int(block_y), final_Ts, final_idx, v_output, v_output_alpha,
        intersect_meta_sorted=intersect_meta_sorted, curve_contrib_rgb=curve_contrib_rgb,
        curve_isect_contrib=curve_isect_contrib)
    if opac_was_2d:
        v_opacity = v_opacity.view(-1, 1)
    return v_xy, v_conic, v_rgb, v_opacity


__all__ = ["rasterize_forward_tilelang", "rasterize_backward_tilelang"]
