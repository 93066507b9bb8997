"""manbo.ops.metric (reference ops/metric.py): the loss kernels live in
libcubicsplat_hip.so; the losses are reached through manbo.metric, and this
module keeps the reference's tuning constants and its two op-level wrappers
(mse_backward_diff_tilelang, reduce_sum_1d_tilelang, ops/metric.py:344-382)."""
from repo_amd.metric import (  # noqa: F401
    DEFAULT_ITEMS_PER_THREAD,
    DEFAULT_SSIM_BLOCK_H,
    DEFAULT_SSIM_BLOCK_W,
    DEFAULT_SSIM_THREADS,
    DEFAULT_THREADS,
    mse_backward_diff_tilelang,
    reduce_sum_1d_tilelang,
)
