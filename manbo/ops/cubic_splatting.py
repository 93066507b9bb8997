"""manbo.ops.cubic_splatting (reference ops/cubic_splatting.py) on MI355X:
the closed-fill splat path and its binning building blocks."""
from repo_amd.blocks import (  # noqa: F401
    DE_CASTELJAU_FLATNESS_TOL_PX as DEFAULT_DE_CASTELJAU_FLATNESS_TOL_PX,
    accumulate_edge_grads_to_cubics as _accumulate_edge_grads_to_cubics,
    build_fill_isect_edge_ranges as _build_fill_isect_edge_ranges_uniform,
    cubic_adaptive_flatness_flags_tilelang,
    cubic_split_half_tilelang,
    flatten_cubics_to_edges as _flatten_cubics_to_edges,
    map_cubic_to_intersects_tilelang,
    primitive_tile_ranges_from_segment_tile_ranges as _primitive_tile_ranges_from_segment_tile_ranges,
    project_cubics_2d_forward_tilelang,
)
from repo_amd.raster_ref import (  # noqa: F401
    rasterize_cubic_fill_backward_tilelang,
    rasterize_cubic_fill_forward_tilelang,
)
from repo_amd.rings import (  # noqa: F401
    _ClosedCubicFillSegmentsFn,
    _closed_fill_piecewise_basis_tensors,
    closed_cubic_fill_segments_tilelang,
)
from repo_amd.splat import (  # noqa: F401
    BLOCK_X,
    BLOCK_Y,
    CUBIC_FLATTEN_METHOD_BERNSTEIN,
    CUBIC_FLATTEN_METHOD_DE_CASTELJAU,
    DEFAULT_AA_WIDTH,
    DEFAULT_AABB_PAD,
    DEFAULT_CUBIC_FLATTEN_METHOD,
    DEFAULT_DISTANCE_SAMPLES,
    DEFAULT_THREADS,
    CubicFillProcessFn,
    CubicFillProcessPayload,
    CubicProcessFn,
    CubicProcessPayload,
    _CubicFillSplatFunction,
    _run_process_fn as _run_cubic_process_fn,
    normalize_cubic_flatten_method,
    render_cubic_fill_splat_tilelang,
)

__all__ = [
    "BLOCK_X",
    "BLOCK_Y",
    "DEFAULT_AA_WIDTH",
    "DEFAULT_AABB_PAD",
    "DEFAULT_DISTANCE_SAMPLES",
    "CUBIC_FLATTEN_METHOD_BERNSTEIN",
    "CUBIC_FLATTEN_METHOD_DE_CASTELJAU",
    "DEFAULT_CUBIC_FLATTEN_METHOD",
    "DEFAULT_THREADS",
    "normalize_cubic_flatten_method",
    "closed_cubic_fill_segments_tilelang",
    "map_cubic_to_intersects_tilelang",
    "project_cubics_2d_forward_tilelang",
    "rasterize_cubic_fill_backward_tilelang",
    "rasterize_cubic_fill_forward_tilelang",
    "render_cubic_fill_splat_tilelang",
]
