"""manbo.ops.optim (reference ops/optim.py:1-172): one in-place Adan step from
an external gradient, on the cs_adan_step HIP kernel."""
from repo_amd.optim import DEFAULT_TILELANG_THREADS as DEFAULT_THREADS  # noqa: F401
from repo_amd.optim import adan_step_from_grad_tilelang  # noqa: F401
