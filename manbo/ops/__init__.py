"""manbo.ops for the cubic-splat hot path (reference ops/__init__.py:48-176,
hot-path names only; the Gaussian, regularization, optimizer and
connected-component kernels are not part of this build)."""
from .cubic_polyline_splatting import render_cubic_polyline_splat_tilelang
from .cubic_splatting import (
    closed_cubic_fill_segments_tilelang,
    map_cubic_to_intersects_tilelang,
    project_cubics_2d_forward_tilelang,
    render_cubic_fill_splat_tilelang,
)
from .tile_bins import get_tile_bin_edges_tilelang

__all__ = [
    "closed_cubic_fill_segments_tilelang",
    "get_tile_bin_edges_tilelang",
    "project_cubics_2d_forward_tilelang",
    "map_cubic_to_intersects_tilelang",
    "render_cubic_fill_splat_tilelang",
    "render_cubic_polyline_splat_tilelang",
]
