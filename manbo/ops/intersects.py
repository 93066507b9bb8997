"""manbo.ops.intersects (reference ops/intersects.py) on MI355X."""
from __future__ import annotations

import torch

from repo_amd import gaussian as _G

BLOCK_X = 16
BLOCK_Y = 16
DEFAULT_THREADS = 256
ANISO_SIGMA_MULT = 3.0
CONIC_EPS = 1e-12


def map_gaussian_to_intersects_tilelang(
        num_points: int, num_intersects: int, xys: torch.Tensor, depths: torch.Tensor,
        radii: torch.Tensor, cum_tiles_hit: torch.Tensor, tile_bounds: tuple, *,
        block_x: int = BLOCK_X, block_y: int = BLOCK_Y, threads: int = DEFAULT_THREADS,
        conics: torch.Tensor | None = None):
    """intersects.py:243-309 -> (isect_ids int64 [I], gaussian_ids int32 [I]):
    key (tile << 32) | depth bits; the anisotropic rectangle when conics is
    given, the radius box otherwise."""
    return _G.map_gaussian_to_intersects(int(num_points), int(num_intersects), xys, depths,
                                         radii, cum_tiles_hit, tile_bounds, block_x=int(block_x),
                                         block_y=int(block_y), conics=conics)


def map_gaussian_meta_to_intersects(gaussian_meta: torch.Tensor,
                                    gaussian_ids: torch.Tensor) -> torch.Tensor:
    """intersects.py:312-325: per-Gaussian int flags in per-intersection order
    (a gather, as in the reference)."""
    if gaussian_meta.ndim != 1:
        raise ValueError("gaussian_meta must be a 1D tensor")
    if gaussian_ids.ndim != 1:
        raise ValueError("gaussian_ids must be a 1D tensor")
    if gaussian_meta.device != gaussian_ids.device:
        gaussian_meta = gaussian_meta.to(gaussian_ids.device)
    meta = gaussian_meta.to(dtype=torch.int32).contiguous()
    return torch.gather(meta, 0, gaussian_ids.to(dtype=torch.int64).contiguous())


__all__ = ["map_gaussian_to_intersects_tilelang", "map_gaussian_meta_to_intersects"]
