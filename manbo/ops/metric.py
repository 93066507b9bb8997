"""manbo.ops.metric (reference ops/metric.py): the loss kernels live in
libcubicsplat_hip.so and are reached through manbo.metric; this module keeps
the reference's tuning constants for callers that import them."""
from repo_amd.metric import (  # noqa: F401
    DEFAULT_ITEMS_PER_THREAD,
    DEFAULT_SSIM_BLOCK_H,
    DEFAULT_SSIM_BLOCK_W,
    DEFAULT_SSIM_THREADS,
    DEFAULT_THREADS,
)
