"""manbo.ops.backward2d (reference ops/backward2d.py) on MI355X."""
from __future__ import annotations

import torch

from repo_amd import gaussian as _G

DEFAULT_THREADS = 256


def project_gaussians_2d_scale_rot_backward_tilelang(
        means2d: torch.Tensor, scales2d: torch.Tensor, rotation: torch.Tensor, img_height: int,
        img_width: int, radii: torch.Tensor, conics: torch.Tensor, v_xy: torch.Tensor,
        v_depth: torch.Tensor, v_conic: torch.Tensor, *, threads: int = DEFAULT_THREADS):
    """backward2d.py:154-212 -> (v_cov2d, v_mean2d, v_scale, v_rot); v_rot is
    [N,1] when rotation is.  v_depth is checked for shape and otherwise
    unused, as in the reference."""
    if rotation.dim() == 1:
        rot_was_2d = False
    elif rotation.dim() == 2 and rotation.shape[1] == 1:
        rot_was_2d = True
    else:
        raise ValueError("rotation must be shape (N,) or (N,1)")
    if not (v_depth.dim() == 1 or (v_depth.dim() == 2 and v_depth.shape[1] == 1)):
        raise ValueError("v_depth must be shape (N,) or (N,1)")
    v_cov2d, v_mean2d, v_scale, v_rot = _G.project_backward(
        scales2d, rotation, radii, conics, v_xy, v_conic, int(img_height), int(img_width),
        with_cov2d=True)
    if rot_was_2d:
        v_rot = v_rot.view(-1, 1)
    return v_cov2d, v_mean2d, v_scale, v_rot


__all__ = ["project_gaussians_2d_scale_rot_backward_tilelang"]
