"""manbo.tilelang_renderer surface (reference tilelang_renderer.py:31-589).

The profiling hook works as in the reference.  The Gaussian splat kernels
behind GsRenderFunction are not part of this build (it covers the cubic
path): the names and signatures exist so that importing code keeps working,
and rendering Gaussians raises NotImplementedError."""
from __future__ import annotations

from contextlib import nullcontext
from typing import Any, Callable, ContextManager, Mapping, MutableMapping, Optional, Tuple

import torch
from torch import nn

ProfileCtxFactory = Callable[[str], ContextManager]
_PROFILE_CTX_FACTORY: Optional[ProfileCtxFactory] = None
GsProcessPayload = MutableMapping[str, Any]
GsProcessFn = Callable[[str, GsProcessPayload], Optional[Mapping[str, Any]]]


def set_gs_profile_ctx_factory(factory: Optional[ProfileCtxFactory]) -> None:
    """tilelang_renderer.py:31-33."""
    global _PROFILE_CTX_FACTORY
    _PROFILE_CTX_FACTORY = factory


def _prof(label: str):
    """tilelang_renderer.py:36-39."""
    if _PROFILE_CTX_FACTORY is None:
        return nullcontext()
    return _PROFILE_CTX_FACTORY(label)


_NOT_BUILT = ("the 2D Gaussian splat renderer (GsRenderFunction) is not part of the MI355X "
              "cubic-splat build; use manbo.ops.render_cubic_fill_splat_tilelang or "
              "render_cubic_polyline_splat_tilelang")


class GsRenderFunction(torch.autograd.Function):
    """Signature of tilelang_renderer.py:149-166."""

    @staticmethod
    def forward(ctx, means2d, scales2d, rotation, colors, opacities, img_h, img_w, block_x,
                block_y, bg, process_fn=None, profile_fwd_prefix="tilelang.fwd",
                profile_bwd_prefix="tilelang.bwd"):
        raise NotImplementedError(_NOT_BUILT)

    @staticmethod
    def backward(ctx, grad_out_img):
        raise NotImplementedError(_NOT_BUILT)


def gs_render(means2d, scales2d, rotation, colors, opacities, img_h, img_w, block_x, block_y, bg,
              process_fn: Optional[GsProcessFn] = None, *,
              profile_fwd_prefix: str = "tilelang.fwd",
              profile_bwd_prefix: str = "tilelang.bwd"):
    """tilelang_renderer.py:493-523."""
    return GsRenderFunction.apply(means2d, scales2d, rotation, colors, opacities, img_h, img_w,
                                  block_x, block_y, bg, process_fn, str(profile_fwd_prefix),
                                  str(profile_bwd_prefix))


class GsRenderModule(nn.Module):
    """tilelang_renderer.py:526-589."""

    def __init__(self, img_h: int, img_w: int, block_x: int = 16, block_y: int = 8,
                 background: Tuple[float, float, float] = (1.0, 1.0, 1.0),
                 process_fn: Optional[GsProcessFn] = None,
                 profile_fwd_prefix: str = "tilelang.fwd",
                 profile_bwd_prefix: str = "tilelang.bwd"):
        super().__init__()
        self.img_h = int(img_h)
        self.img_w = int(img_w)
        self.block_x = int(block_x)
        self.block_y = int(block_y)
        self.process_fn = process_fn
        self.profile_fwd_prefix = str(profile_fwd_prefix)
        self.profile_bwd_prefix = str(profile_bwd_prefix)
        self.register_buffer("background", torch.tensor(background, dtype=torch.float32))

    def forward(self, means2d, scales2d, rotation, colors, opacities, bg=None, process_fn=None, *,
                profile_fwd_prefix=None, profile_bwd_prefix=None):
        return gs_render(means2d, scales2d, rotation, colors, opacities, self.img_h, self.img_w,
                         self.block_x, self.block_y, self.background if bg is None else bg,
                         self.process_fn if process_fn is None else process_fn,
                         profile_fwd_prefix=(self.profile_fwd_prefix if profile_fwd_prefix is None
                                             else str(profile_fwd_prefix)),
                         profile_bwd_prefix=(self.profile_bwd_prefix if profile_bwd_prefix is None
                                             else str(profile_bwd_prefix)))


__all__ = ["GsRenderFunction", "GsRenderModule", "gs_render", "set_gs_profile_ctx_factory"]
