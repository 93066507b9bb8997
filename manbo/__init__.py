"""Drop-in replacement for the reference's ``manbo`` package, restricted to the
cubic-splat hot path (manbo/__init__.py:1-29 of the reference).  The kernels
are the MI355X HIP kernels of ``repo_amd``."""
from . import ops
from .metric import mse_loss_tilelang, psnr, ssim
from .optim import Adan
from .tilelang_renderer import (
    GsRenderFunction,
    GsRenderModule,
    gs_render,
    set_gs_profile_ctx_factory,
)

__all__ = [
    "ops",
    "mse_loss_tilelang",
    "psnr",
    "ssim",
    "Adan",
    "GsRenderFunction",
    "GsRenderModule",
    "set_gs_profile_ctx_factory",
    "gs_render",
]
