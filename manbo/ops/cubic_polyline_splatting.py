"""manbo.ops.cubic_polyline_splatting (reference ops/cubic_polyline_splatting.py)
on MI355X: the open-stroke splat path."""
from repo_amd.splat import (  # noqa: F401
    _CubicPolylineSplatFunction,
    render_cubic_polyline_splat_tilelang,
)

__all__ = ["render_cubic_polyline_splat_tilelang"]
