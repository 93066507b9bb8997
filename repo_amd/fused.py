"""Fused operations for the training step around the renderer.

The reference's training code turns the rendered [H, W, 3] image into the
loss input with ``img.clamp(0, 1).permute(2, 0, 1).unsqueeze(0)``
(gaussian_trace/render.py:1309-1310) and, in this build's benchmark step,
combines ``mse_loss_tilelang`` (metric.py:198-212) with ``ssim``
(metric.py:215-273) as ``MSE + w * (1 - SSIM)``.  Done with torch and the
separate loss calls, that is several full passes over 33 MB images per step
(clamp, permute copy, their backward, the two loss gradients and their sum);
here each direction is one kernel:

* ``clamp_to_nchw(img)``: one pass forward, one masked pass backward;
* ``mse_ssim_loss(x, y, w)``: one call for both losses (the SSIM tiles also
  sum the squared differences; one combining workgroup) and one backward
  kernel that writes ``g * (2 (x - y) / n - w dSSIM/dx)``;
* ``clamp_mse_ssim_loss(img, y, w)``: the two above in one autograd node
  whose backward writes the [H, W, 3] image gradient directly; the
  renderer's planar image needs no clamp pass at all (the SSIM forward reads
  it clamped).

Values equal the separate calls up to fp32 summation order; the autograd
graph is shorter.
"""
from __future__ import annotations

import torch

from . import _native as N
from .metric import _as_f32, _validate_pair_4d, gaussian_window_1d


class _ClampToNCHW(torch.autograd.Function):
    @staticmethod
    def forward(ctx, img, lo, hi):
        N.require_gpu(img, "img")
        if img.dim() != 3 or img.shape[2] != 3:
            raise ValueError(f"img must be [H, W, 3], got {tuple(img.shape)}")
        x = _as_f32(img, "img")
        h, w = int(x.shape[0]), int(x.shape[1])
        out = torch.empty((1, 3, h, w), dtype=torch.float32, device=x.device)
        with N.prof("glue.clamp_nchw"):
            N.call("cs_clamp_hwc_to_nchw", N.ptr(x), h, w, float(lo), float(hi), N.ptr(out),
                   N.stream(x.device))
        ctx.save_for_backward(x)
        ctx.lo, ctx.hi = float(lo), float(hi)
        return out

    @staticmethod
    def backward(ctx, grad):
        (x,) = ctx.saved_tensors
        h, w = int(x.shape[0]), int(x.shape[1])
        g = grad.detach().to(torch.float32).contiguous()
        gi = torch.empty_like(x)
        with N.prof("glue.clamp_nchw_bwd"):
            N.call("cs_clamp_hwc_to_nchw_backward", N.ptr(x), N.ptr(g), h, w, ctx.lo, ctx.hi,
                   N.ptr(gi), N.stream(x.device))
        return gi, None, None


def clamp_to_nchw(img: torch.Tensor, lo: float = 0.0, hi: float = 1.0) -> torch.Tensor:
    """``img.clamp(lo, hi).permute(2, 0, 1).unsqueeze(0)`` as one kernel (and
    one for its gradient); returns a contiguous [1, 3, H, W] tensor."""
    return _ClampToNCHW.apply(img, lo, hi)


class _MseSsimLoss(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, y, ssim_weight, win_size, win_sigma, c1, c2):
        _validate_pair_4d(x, y)
        x32 = _as_f32(x, "x")
        y32 = _as_f32(y, "y")
        n, c, h, w = x32.shape
        dev = x32.device
        g = gaussian_window_1d(win_size, win_sigma, dev)
        partials = torch.empty((int(N.lib().cs_mse_ssim_partials_elems(n * c, h, w)),),
                               dtype=torch.float32, device=dev)
        out = torch.empty((3,), dtype=torch.float32, device=dev)
        abc = (torch.empty((int(N.lib().cs_ssim_abc_elems(n * c, h, w, int(win_size))),),
                           dtype=torch.float32, device=dev)
               if ctx.needs_input_grad[0] else None)
        with N.prof("loss.mse_ssim"):
            N.call("cs_mse_ssim_loss", N.ptr(x32), N.ptr(y32), n * c, h, w, N.ptr(g),
                   int(win_size), float(c1), float(c2), float(ssim_weight), N.ptr(partials),
                   N.ptr(out), N.ptr(abc), N.stream(dev))
        ctx.save_for_backward(x32, y32, abc if abc is not None else torch.empty(0), g)
        ctx.win_size = int(win_size)
        ctx.ssim_weight = float(ssim_weight)
        ctx.x_dtype = x.dtype
        parts = out[1:]
        ctx.mark_non_differentiable(parts)
        # No zero gradient is made for `parts` (non-differentiable).
        ctx.set_materialize_grads(False)
        return out[0], parts

    @staticmethod
    def backward(ctx, grad_loss, _grad_parts):
        x, y, abc, g = ctx.saved_tensors
        if not ctx.needs_input_grad[0] or grad_loss is None:
            return (None,) * 7
        n, c, h, w = x.shape
        gx = torch.empty_like(x)
        go = grad_loss.detach().to(torch.float32).contiguous()
        with N.prof("loss.mse_ssim_bwd"):
            N.call("cs_mse_ssim_backward", N.ptr(x), N.ptr(y), n * c, h, w, N.ptr(g),
                   ctx.win_size, N.ptr(abc), ctx.ssim_weight, N.ptr(go), N.ptr(gx),
                   N.stream(x.device))
        return gx.to(ctx.x_dtype), None, None, None, None, None, None


def _planes_of(img: torch.Tensor):
    """Three [H, W] planes holding the values of the [H, W, 3] float32 image:
    the planar copy the renderer wrote beside its image (while the image is
    unmodified), or the planes behind an [H, W, 3] view of them (strides
    (W, 1, H W)); None for any other tensor."""
    if img.dtype is not torch.float32 or img.dim() != 3 or img.shape[2] != 3:
        return None
    from .splat import planar_copy_of
    pc = planar_copy_of(img)
    if pc is not None:
        return pc
    h, w = int(img.shape[0]), int(img.shape[1])
    if img.is_contiguous() or img.stride() != (w, 1, h * w):
        return None
    return img.detach().permute(2, 0, 1)


# Element counts of the loss's work buffers per (h, w, win_size):
# (partials, abc).
_CLAMP_LOSS_SIZES: "dict[tuple, tuple]" = {}


def _clamp_loss_sizes(h, w, win_size):
    key = (h, w, win_size)
    v = _CLAMP_LOSS_SIZES.get(key)
    if v is None:
        L = N.lib()
        v = _CLAMP_LOSS_SIZES[key] = (int(L.cs_mse_ssim_partials_elems(3, h, w)),
                                      int(L.cs_ssim_abc_elems(3, h, w, win_size)))
    return v


class _ClampMseSsimLoss(torch.autograd.Function):
    @staticmethod
    def forward(ctx, img, y, lo, hi, ssim_weight, win_size, win_sigma, c1, c2):
        N.require_gpu(img, "img")
        if img.dim() != 3 or img.shape[2] != 3:
            raise ValueError(f"img must be [H, W, 3], got {tuple(img.shape)}")
        # The renderer's planar image is read in place (clamped on load);
        # any other layout as a contiguous [H, W, 3] copy.
        planes = _planes_of(img)
        x32 = planes if planes is not None else _as_f32(img, "img")
        planar = 1 if planes is not None else 0
        h, w = int(img.shape[0]), int(img.shape[1])
        if tuple(y.shape) not in ((1, 3, h, w), (3, h, w)):
            raise ValueError(f"target must be [1, 3, {h}, {w}], got {tuple(y.shape)}")
        y32 = _as_f32(y, "target")
        dev = x32.device
        g = gaussian_window_1d(win_size, win_sigma, dev)
        n_part, n_abc = _clamp_loss_sizes(h, w, int(win_size))
        if not ctx.needs_input_grad[0]:
            n_abc = 0
        # clamp(img) as NCHW (not for planes), the partial sums and the
        # backward's SSIM terms in one work buffer; the three results in a
        # buffer of their own.
        n_x = 0 if planar else 3 * h * w
        work = torch.empty((n_x + n_part + n_abc,), dtype=torch.float32, device=dev)
        out = torch.empty((3,), dtype=torch.float32, device=dev)
        wp = work.data_ptr()
        abc_p = wp + 4 * (n_x + n_part) if n_abc else None
        with N.prof("loss.clamp_mse_ssim"):
            N.call("cs_clamp_mse_ssim_loss", x32.data_ptr(), planar, N.ptr(y32), h, w, float(lo),
                   float(hi), N.ptr(g), int(win_size), float(c1), float(c2),
                   float(ssim_weight), None if planar else wp, wp + 4 * n_x, N.ptr(out), abc_p,
                   N.stream(dev))
        ctx.planar = planar
        ctx.save_for_backward(x32, y32)
        # The SSIM terms stay in `work`, which lives as long as this node (a
        # second backward through a retained graph reads them again).
        ctx.work, ctx.abc_off, ctx.g = work, (abc_p - wp) if n_abc else None, g
        ctx.lo, ctx.hi = float(lo), float(hi)
        ctx.win_size = int(win_size)
        ctx.ssim_weight = float(ssim_weight)
        ctx.x_dtype = img.dtype
        parts = out[1:]
        ctx.mark_non_differentiable(parts)
        # No zero gradient is made for `parts` (non-differentiable).
        ctx.set_materialize_grads(False)
        return out[0], parts

    @staticmethod
    def backward(ctx, grad_loss, _grad_parts):
        if not ctx.needs_input_grad[0] or grad_loss is None:
            return (None,) * 9
        x, y = ctx.saved_tensors
        h, w = (int(x.shape[1]), int(x.shape[2])) if ctx.planar else (int(x.shape[0]),
                                                                       int(x.shape[1]))
        # The image gradient is written as three [H, W] planes (whole-line
        # writes) and returned as an [H, W, 3] view of them; the renderer's
        # backward reads that layout in place (splat.image_grad_layout).
        planes = torch.empty((3, h, w), dtype=torch.float32, device=x.device)
        go = grad_loss
        if go.dtype is not torch.float32:
            go = go.to(torch.float32)
        abc_p = ctx.work.data_ptr() + ctx.abc_off
        with N.prof("loss.clamp_mse_ssim_bwd"):
            N.call("cs_clamp_mse_ssim_backward", x.data_ptr(), ctx.planar, N.ptr(y), h, w,
                   ctx.lo, ctx.hi, N.ptr(ctx.g), ctx.win_size, abc_p, ctx.ssim_weight,
                   go.data_ptr(), planes.data_ptr(), 1, N.stream(x.device))
        gi = planes.permute(1, 2, 0)
        if ctx.x_dtype is not torch.float32:
            gi = gi.to(ctx.x_dtype)
        return gi, None, None, None, None, None, None, None, None


def clamp_mse_ssim_loss(img, y, ssim_weight: float = 0.2, *, lo: float = 0.0, hi: float = 1.0,
                        win_size: int = 11, win_sigma: float = 1.5, data_range: float = 1.0,
                        k1: float = 0.01, k2: float = 0.03):
    """``mse_ssim_loss(img.clamp(lo, hi).permute(2, 0, 1).unsqueeze(0), y, ssim_weight)``
    from the renderer's [H, W, 3] image.  The renderer's planar image (an
    [H, W, 3] view of three planes) is read in place, clamped on load; another
    layout takes one clamp/layout pass first.  The SSIM forward also sums the
    MSE; the backward reads the image itself and writes the [H, W, 3]
    gradient (a view of three planes) with the clamp's mask, so the glue has
    no gradient pass.  Returns (loss, [MSE, SSIM])."""
    if win_size <= 0 or win_size % 2 == 0:
        raise ValueError("win_size must be odd")
    if data_range <= 0.0:
        raise ValueError("data_range must be > 0")
    c1 = (k1 * data_range) ** 2
    c2 = (k2 * data_range) ** 2
    return _ClampMseSsimLoss.apply(img, y, float(lo), float(hi), float(ssim_weight),
                                   int(win_size), float(win_sigma), c1, c2)


def mse_ssim_loss(x, y, ssim_weight: float = 0.2, *, win_size: int = 11, win_sigma: float = 1.5,
                  data_range: float = 1.0, k1: float = 0.01, k2: float = 0.03):
    """``mse_loss_tilelang(x, y) + ssim_weight * (1 - ssim(x, y))`` in one call.
    Returns (loss, parts) with parts = [MSE, SSIM] (device, no gradient);
    only ``loss`` is differentiable (w.r.t. x)."""
    if win_size <= 0 or win_size % 2 == 0:
        raise ValueError("win_size must be odd")
    if data_range <= 0.0:
        raise ValueError("data_range must be > 0")
    c1 = (k1 * data_range) ** 2
    c2 = (k2 * data_range) ** 2
    return _MseSsimLoss.apply(x, y, float(ssim_weight), int(win_size), float(win_sigma), c1, c2)
