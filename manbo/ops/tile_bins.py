"""manbo.ops.tile_bins (reference ops/tile_bins.py) on MI355X."""
from repo_amd.blocks import get_tile_bin_edges_tilelang  # noqa: F401

BLOCK_X = 16
BLOCK_Y = 16
DEFAULT_THREADS = 256

__all__ = ["get_tile_bin_edges_tilelang"]
