"""MSE, SSIM and PSNR on MI355X (manbo/metric.py, manbo/ops/metric.py).

All reductions run in libcubicsplat_hip.so; the MSE backward reads its scale
on the device (the reference reads it with .item() at metric.py:168), so a
training step needs no host synchronization here.  SSIM gains a backward,
which the reference does not have (metric.py:215-273 is forward-only).
"""
from __future__ import annotations

from typing import Dict, Tuple

import torch

from . import _native as N

DEFAULT_THREADS = 256
DEFAULT_ITEMS_PER_THREAD = 8
DEFAULT_SSIM_THREADS = 64
DEFAULT_SSIM_BLOCK_H = 8
DEFAULT_SSIM_BLOCK_W = 16

_WINDOW_CACHE: Dict[Tuple[str, int, float], torch.Tensor] = {}


def _validate_pair_4d(x: torch.Tensor, y: torch.Tensor) -> None:
    """metric.py:36-44."""
    if x.shape != y.shape:
        raise ValueError(f"x and y must have the same shape, got {x.shape} and {y.shape}")
    if x.dim() != 4:
        raise ValueError(f"expected input shape [N, C, H, W], got {x.shape}")
    if min(x.shape) <= 0:
        raise ValueError(f"all dimensions must be > 0, got {x.shape}")


def _as_f32(x: torch.Tensor, name: str) -> torch.Tensor:
    """metric.py:26-33 (device check, float32, contiguous)."""
    if x.device.type != "cuda":
        raise ValueError(f"{name} must be a CUDA tensor")
    if x.dtype is torch.float32 and x.is_contiguous():
        return x.detach()
    return x.detach().to(torch.float32).contiguous()


def gaussian_window_1d(win_size: int, win_sigma: float, device) -> torch.Tensor:
    """1D factor of metric.py:47-61 (the 2D window is its outer product), fp32."""
    device = torch.device(device) if not isinstance(device, torch.device) else device
    key = (device.type, device.index, int(win_size), float(win_sigma))
    g = _WINDOW_CACHE.get(key)
    if g is None:
        coords = torch.arange(win_size, dtype=torch.float32)
        coords -= win_size // 2
        g = torch.exp(-(coords ** 2) / (2 * (win_sigma ** 2)))
        g /= g.sum()
        g = g.to(device).contiguous()
        _WINDOW_CACHE[key] = g
    return g


def mse_forward(x: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
    """Device scalar sum((x-y)^2)/n (ops/metric.py:18-163, metric.py:102-131)."""
    n = x.numel()
    dev = x.device
    partials = torch.empty((int(N.lib().cs_mse_partials_elems(n)),), dtype=torch.float32,
                           device=dev)
    loss = torch.empty((), dtype=torch.float32, device=dev)
    with N.prof("loss.mse_fwd"):
        N.call("cs_mse_forward", N.ptr(x), N.ptr(y), n, N.ptr(partials), N.ptr(loss),
               N.stream(dev))
    return loss


def mse_backward_diff_tilelang(lhs: torch.Tensor, rhs: torch.Tensor, *, scale: float,
                               threads: int = DEFAULT_THREADS) -> torch.Tensor:
    """ops/metric.py:344-360: grad = scale * (lhs - rhs) as float32, shaped
    like lhs (threads is accepted for the reference's signature)."""
    _ = threads
    N.require_gpu(lhs, "lhs")
    lhs_flat = lhs.float().contiguous().view(-1)
    rhs_flat = rhs.float().contiguous().view(-1)
    if lhs_flat.numel() != rhs_flat.numel():
        raise ValueError(f"lhs and rhs must have the same number of elements, "
                         f"got {lhs_flat.numel()} and {rhs_flat.numel()}")
    grad = torch.empty_like(lhs_flat, dtype=torch.float32)
    N.call("cs_mse_backward_diff", N.ptr(lhs_flat), N.ptr(rhs_flat), int(lhs_flat.numel()),
           float(scale), N.ptr(grad), N.stream(lhs.device))
    return grad.view(lhs.shape)


def reduce_sum_1d_tilelang(x: torch.Tensor, *, threads: int = DEFAULT_THREADS,
                           items_per_thread: int = DEFAULT_ITEMS_PER_THREAD) -> torch.Tensor:
    """ops/metric.py:363-382: the float32 sum of a 1D tensor as a 0-d device
    tensor (threads / items_per_thread are accepted for the reference's
    signature; the blocks here are fixed)."""
    _ = (threads, items_per_thread)
    N.require_gpu(x, "x")
    cur = x.contiguous().view(-1)
    n = int(cur.numel())
    if n <= 1:   # the reference's loop does not run: its first element (or IndexError)
        return cur[0]
    if cur.dtype is not torch.float32:
        cur = cur.to(torch.float32)
    out = torch.empty((), dtype=torch.float32, device=x.device)
    partials = torch.empty((int(N.lib().cs_reduce_sum_partials_elems(n)),), dtype=torch.float32,
                           device=x.device)
    N.call("cs_reduce_sum_f32", N.ptr(cur), n, N.ptr(partials), N.ptr(out), N.stream(x.device))
    return out


class _TileLangMSEFn(torch.autograd.Function):
    """metric.py:134-195 (same signature)."""

    @staticmethod
    def forward(ctx, x, y, threads, items_per_thread, tilelang_backward):
        if x.shape != y.shape:
            raise ValueError(f"x and y must have the same shape, got {x.shape} and {y.shape}")
        x32 = _as_f32(x, "x")
        y32 = _as_f32(y, "y")
        ctx.save_for_backward(x32, y32)
        ctx.x_dtype, ctx.y_dtype = x.dtype, y.dtype
        ctx.shape = x.shape
        return mse_forward(x32.view(-1), y32.view(-1))

    @staticmethod
    def backward(ctx, grad_output):
        x, y = ctx.saved_tensors
        need_x, need_y = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        if not (need_x or need_y):
            return None, None, None, None, None
        g = grad_output.detach().to(torch.float32).contiguous()
        gx = torch.empty_like(x) if need_x else None
        gy = torch.empty_like(y) if need_y else None
        with N.prof("loss.mse_bwd"):
            N.call("cs_mse_backward", N.ptr(x), N.ptr(y), x.numel(), N.ptr(g), N.ptr(gx), N.ptr(gy),
                   N.stream(x.device))
        if gx is not None:
            gx = gx.view(ctx.shape).to(ctx.x_dtype)
        if gy is not None:
            gy = gy.view(ctx.shape).to(ctx.y_dtype)
        return gx, gy, None, None, None


def mse_loss_tilelang(x, y, *, threads=DEFAULT_THREADS, items_per_thread=DEFAULT_ITEMS_PER_THREAD,
                      tilelang_backward=True):
    """metric.py:198-212."""
    return _TileLangMSEFn.apply(x, y, int(threads), int(items_per_thread),
                                int(bool(tilelang_backward)))


def psnr(x, y, *, data_range=1.0, eps=1e-12, threads=DEFAULT_THREADS,
         items_per_thread=DEFAULT_ITEMS_PER_THREAD):
    """metric.py:64-99."""
    _validate_pair_4d(x, y)
    if data_range <= 0.0:
        raise ValueError("data_range must be > 0")
    if eps < 0.0:
        raise ValueError("eps must be >= 0")
    x32 = _as_f32(x, "x").view(-1)
    y32 = _as_f32(y, "y").view(-1)
    mse = mse_forward(x32, y32)
    return 10.0 * torch.log10((data_range * data_range) / (mse + eps))


def _ssim_scratch(nc, h, w, win_size, dev):
    n = int(N.lib().cs_ssim_scratch_elems(nc, h, w, int(win_size)))
    return torch.empty((n,), dtype=torch.float32, device=dev) if n else None


def _ssim_forward(x32, y32, win_size, win_sigma, c1, c2, want_grad, per_map=False):
    """cs_ssim: the mean SSIM of every (image, channel) map (a device scalar),
    or with per_map each map's mean [n * c]; abc holds the backward's
    per-pixel partials when want_grad."""
    n, c, h, w = x32.shape
    dev = x32.device
    g = gaussian_window_1d(win_size, win_sigma, dev)
    partials = torch.empty((int(N.lib().cs_ssim_partials_elems(n * c, h, w)),),
                           dtype=torch.float32, device=dev)
    out = torch.empty((n * c,) if per_map else (), dtype=torch.float32, device=dev)
    # Per-pixel partials for the backward, [3, n*c, oh, ow rounded up to 4].
    abc = (torch.empty((int(N.lib().cs_ssim_abc_elems(n * c, h, w, int(win_size))),),
                       dtype=torch.float32, device=dev)
           if want_grad else None)
    scratch = _ssim_scratch(n * c, h, w, win_size, dev)
    with N.prof("loss.ssim_fwd"):
        N.call("cs_ssim", N.ptr(x32), N.ptr(y32), n * c, h, w, N.ptr(g), int(win_size),
               float(c1), float(c2), int(bool(per_map)), N.ptr(partials), N.ptr(out),
               N.ptr(abc), N.ptr(scratch), N.stream(dev))
    return out, abc, g


class _SSIMFn(torch.autograd.Function):
    """Mean SSIM over all (image, channel) maps, or (per_map) each map's mean
    [n * c], with a backward w.r.t. x."""

    @staticmethod
    def forward(ctx, x, y, win_size, win_sigma, c1, c2, per_map=False):
        x32 = _as_f32(x, "x")
        y32 = _as_f32(y, "y")
        out, abc, g = _ssim_forward(x32, y32, win_size, win_sigma, c1, c2,
                                    ctx.needs_input_grad[0], per_map)
        ctx.save_for_backward(x32, y32, abc if abc is not None else torch.empty(0), g)
        ctx.win_size = int(win_size)
        ctx.per_map = bool(per_map)
        ctx.x_dtype = x.dtype
        return out

    @staticmethod
    def backward(ctx, grad_output):
        x, y, abc, g = ctx.saved_tensors
        if not ctx.needs_input_grad[0]:
            return None, None, None, None, None, None, None
        n, c, h, w = x.shape
        gx = torch.empty_like(x)
        go = grad_output.detach().to(torch.float32).contiguous()
        scratch = _ssim_scratch(n * c, h, w, ctx.win_size, x.device)
        with N.prof("loss.ssim_bwd"):
            N.call("cs_ssim_backward", N.ptr(x), N.ptr(y), n * c, h, w, N.ptr(g), ctx.win_size,
                   N.ptr(abc), N.ptr(go), int(ctx.per_map), N.ptr(gx), N.ptr(scratch),
                   N.stream(x.device))
        return gx.to(ctx.x_dtype), None, None, None, None, None, None


def ssim(x, y, *, data_range=1.0, size_average=True, win_size=11, win_sigma=1.5, k1=0.01,
         k2=0.03, nonnegative_ssim=False, block_h=DEFAULT_SSIM_BLOCK_H,
         block_w=DEFAULT_SSIM_BLOCK_W, threads=DEFAULT_SSIM_THREADS):
    """metric.py:215-273, differentiable w.r.t. x in every mode (the
    reference's SSIM has no backward).  Any odd win_size up to the image
    size: windows up to 15 run the tiled kernels, wider ones a two-pass
    kernel through a scratch buffer.  size_average=False and nonnegative_ssim
    take every (image, channel) mean from one launch."""
    _validate_pair_4d(x, y)
    if data_range <= 0.0:
        raise ValueError("data_range must be > 0")
    if win_size <= 0 or win_size % 2 == 0:
        raise ValueError("win_size must be a positive odd integer")
    if win_sigma <= 0.0:
        raise ValueError("win_sigma must be > 0")
    n, c, h, w = x.shape
    if h - win_size + 1 <= 0 or w - win_size + 1 <= 0:
        raise ValueError(f"input spatial size {(h, w)} is smaller than win_size {win_size}")
    c1 = (k1 * data_range) ** 2
    c2 = (k2 * data_range) ** 2
    if size_average and not nonnegative_ssim:
        return _SSIMFn.apply(x, y, int(win_size), float(win_sigma), float(c1), float(c2))
    # metric.py:262-273: per (image, channel) means, clamped at 0 when
    # nonnegative_ssim, then averaged over channels (and images).
    per = _SSIMFn.apply(x, y, int(win_size), float(win_sigma), float(c1), float(c2),
                        True).view(n, c)
    if nonnegative_ssim:
        per = torch.relu(per)
    if size_average:
        return per.mean()
    return per.mean(1)
