"""manbo.ops.forward2d (reference ops/forward2d.py) on MI355X."""
from __future__ import annotations

import torch

from repo_amd import gaussian as _G

BLOCK_X = 16
BLOCK_Y = 16
DEFAULT_THREADS = 256
ANISO_SIGMA_MULT = 3.0
CONIC_EPS = 1e-12


def project_gaussians_2d_scale_rot_forward_tilelang(
        means2d: torch.Tensor, scales2d: torch.Tensor, rotation: torch.Tensor, img_height: int,
        img_width: int, tile_bounds: tuple, *, block_x: int = BLOCK_X, block_y: int = BLOCK_Y,
        threads: int = DEFAULT_THREADS):
    """forward2d.py:167-220 -> (xys, depths, radii, conics, num_tiles_hit).
    tile_bounds and threads are accepted for API compatibility; the tile grid
    follows from the image size and block, as in the reference."""
    return _G.project_forward(means2d, scales2d, rotation, int(img_height), int(img_width),
                              int(block_x), int(block_y))


__all__ = ["project_gaussians_2d_scale_rot_forward_tilelang"]
