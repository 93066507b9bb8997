"""manbo.metric (reference metric.py:64-273) on MI355X."""
from repo_amd.metric import (  # noqa: F401
    _TileLangMSEFn,
    gaussian_window_1d,
    mse_loss_tilelang,
    psnr,
    ssim,
)

__all__ = ["mse_loss_tilelang", "psnr", "ssim"]
