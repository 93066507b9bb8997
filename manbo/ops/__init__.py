"""manbo.ops (reference ops/__init__.py:48-176): the cubic-splat and 2D
Gaussian splat kernels and the Adan step; the regularization and
connected-component kernels are not part of this build."""
from .backward2d import project_gaussians_2d_scale_rot_backward_tilelang
from .cubic_polyline_splatting import render_cubic_polyline_splat_tilelang
from .cubic_splatting import (
    closed_cubic_fill_segments_tilelang,
    map_cubic_to_intersects_tilelang,
    project_cubics_2d_forward_tilelang,
    rasterize_cubic_fill_backward_tilelang,
    rasterize_cubic_fill_forward_tilelang,
    render_cubic_fill_splat_tilelang,
)
from .forward2d import project_gaussians_2d_scale_rot_forward_tilelang
from .intersects import map_gaussian_meta_to_intersects, map_gaussian_to_intersects_tilelang
from .metric import mse_backward_diff_tilelang, reduce_sum_1d_tilelang
from .optim import adan_step_from_grad_tilelang
from .rasterize import rasterize_backward_tilelang, rasterize_forward_tilelang
from .tile_bins import get_tile_bin_edges_tilelang

__all__ = [
    "project_gaussians_2d_scale_rot_forward_tilelang",
    "project_gaussians_2d_scale_rot_backward_tilelang",
    "map_gaussian_to_intersects_tilelang",
    "map_gaussian_meta_to_intersects",
    "rasterize_forward_tilelang",
    "rasterize_backward_tilelang",
    "closed_cubic_fill_segments_tilelang",
    "get_tile_bin_edges_tilelang",
    "project_cubics_2d_forward_tilelang",
    "map_cubic_to_intersects_tilelang",
    "rasterize_cubic_fill_backward_tilelang",
    "rasterize_cubic_fill_forward_tilelang",
    "render_cubic_fill_splat_tilelang",
    "render_cubic_polyline_splat_tilelang",
    "mse_backward_diff_tilelang",
    "reduce_sum_1d_tilelang",
    "adan_step_from_grad_tilelang",
]
