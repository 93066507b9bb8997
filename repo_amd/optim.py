"""Adam and Adan with the step in one HIP launch for up to 16 parameters.

The reference optimizes its primitives with ``torch.optim.Adam`` over
per-group learning rates (gaussian_trace/model.py:172-189).  ``Adam`` here is
a drop-in for that class on fp32 device parameters: same constructor, param
groups, ``state`` entries (``step``, ``exp_avg``, ``exp_avg_sq``) and
``state_dict`` layout, so a checkpoint moves between the two.  The update is
torch's single-tensor Adam (amsgrad and maximize off); one ``cs_adam_step``
launch covers up to 16 tensors.  Optimizer step pre/post hooks (global and
per instance) run as for torch's optimizers; the profiler range torch wraps
around ``step`` is left out, since it costs more host time than the launch.

``Adan`` is the reference's own optimizer (manbo/optim.py:10-190, the default
of its training script) with the update of ops/optim.py:8-113 as one
``cs_adan_step`` launch per 16 tensors; ``adan_step_from_grad_tilelang`` is
the reference's functional single-tensor form.
"""
from __future__ import annotations

import ctypes
import math
from itertools import chain

import torch
from torch.optim import optimizer as _torch_optimizer

from . import _native as N

MAX_TENSORS_PER_LAUNCH = 16


class _LaunchArgs:
    """ctypes argument arrays for one launch of n tensors, reused across steps."""

    def __init__(self, n):
        self.n = n
        self.params = (ctypes.c_void_p * n)()
        self.grads = (ctypes.c_void_p * n)()
        self.ms = (ctypes.c_void_p * n)()
        self.vs = (ctypes.c_void_p * n)()
        self.numels = (ctypes.c_int64 * n)()
        self.step_sizes = (ctypes.c_float * n)()
        self.bc2s = (ctypes.c_float * n)()
        self.wds = (ctypes.c_float * n)()


class Adam(torch.optim.Optimizer):
    def __init__(self, params, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.0,
                 amsgrad=False, *, maximize=False, capturable=False, differentiable=False,
                 foreach=None, fused=None):
        if not 0.0 <= float(lr):
            raise ValueError(f"Invalid learning rate: {lr}")
        if not 0.0 <= float(eps):
            raise ValueError(f"Invalid epsilon value: {eps}")
        if not 0.0 <= betas[0] < 1.0:
            raise ValueError(f"Invalid beta parameter at index 0: {betas[0]}")
        if not 0.0 <= betas[1] < 1.0:
            raise ValueError(f"Invalid beta parameter at index 1: {betas[1]}")
        if not 0.0 <= weight_decay:
            raise ValueError(f"Invalid weight_decay value: {weight_decay}")
        if amsgrad or maximize or capturable or differentiable:
            raise NotImplementedError(
                "repo_amd.optim.Adam implements amsgrad=False, maximize=False, "
                "capturable=False, differentiable=False")
        defaults = dict(lr=lr, betas=betas, eps=eps, weight_decay=weight_decay, amsgrad=False,
                        maximize=False, foreach=None, capturable=False, differentiable=False,
                        fused=None)
        super().__init__(params, defaults)
        self._launch_args = {}
        self._step_views = {}

    def zero_grad(self, set_to_none: bool = True) -> None:
        """torch.optim.Optimizer.zero_grad (foreach off), without the profiler
        range it opens around the loop."""
        for group in self.param_groups:
            for p in group["params"]:
                if p.grad is not None:
                    if set_to_none:
                        p.grad = None
                    else:
                        if p.grad.grad_fn is not None:
                            p.grad.detach_()
                        else:
                            p.grad.requires_grad_(False)
                        p.grad.zero_()

    def _step_count(self, st):
        """Increments the state's CPU ``step`` tensor through a cached numpy
        view of it (the tensor stays what torch's Adam stores) and returns the
        new count."""
        t = st["step"]
        if t.device.type != "cpu" or t.requires_grad:
            t += 1
            return float(t)
        c = self._step_views.get(id(t))
        if c is None or c[0] is not t:
            if len(self._step_views) > 4 * MAX_TENSORS_PER_LAUNCH + len(self.state):
                self._step_views.clear()
            c = self._step_views[id(t)] = (t, t.numpy())
        arr = c[1]
        arr += 1
        return float(arr)

    def step(self, closure=None):
        args, kwargs = (self,), {"closure": closure} if closure is not None else {}
        if _torch_optimizer._global_optimizer_pre_hooks or self._optimizer_step_pre_hooks:
            for pre_hook in chain(_torch_optimizer._global_optimizer_pre_hooks.values(),
                                  self._optimizer_step_pre_hooks.values()):
                result = pre_hook(self, args, kwargs)
                if result is not None:
                    if isinstance(result, tuple) and len(result) == 2:
                        args, kwargs = result
                    else:
                        raise RuntimeError(
                            "optimizer step pre-hooks must return None or (args, kwargs), got "
                            f"{result}")
            closure = kwargs.get("closure", closure)
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        batches = {}
        state = self.state
        for group in self.param_groups:
            beta1, beta2 = group["betas"]
            key = (float(beta1), float(beta2), float(group["eps"]))
            lr, wd = float(group["lr"]), float(group["weight_decay"])
            for p in group["params"]:
                g = p.grad
                if g is None:
                    continue
                if g.is_sparse:
                    raise RuntimeError("Adam does not support sparse gradients")
                if p.dtype is not torch.float32 or not p.is_contiguous() or not p.is_cuda:
                    raise ValueError(
                        "repo_amd.optim.Adam needs contiguous float32 CUDA (ROCm) parameters")
                st = state[p]
                if len(st) == 0:
                    st["step"] = torch.tensor(0.0, dtype=torch.float32)
                    st["exp_avg"] = torch.zeros_like(p, memory_format=torch.preserve_format)
                    st["exp_avg_sq"] = torch.zeros_like(p, memory_format=torch.preserve_format)
                step = self._step_count(st)
                bc1 = 1.0 - beta1 ** step
                bc2 = 1.0 - beta2 ** step
                if not g.is_contiguous():
                    g = g.contiguous()
                batches.setdefault((p.device.index, key), []).append(
                    (p, g, st["exp_avg"], st["exp_avg_sq"], lr / bc1, math.sqrt(bc2), wd))
        for (dev, (beta1, beta2, eps)), items in batches.items():
            for k in range(0, len(items), MAX_TENSORS_PER_LAUNCH):
                self._launch(dev, items[k:k + MAX_TENSORS_PER_LAUNCH], beta1, beta2, eps)
        self._optimizer_step_code()
        if self._optimizer_step_post_hooks or _torch_optimizer._global_optimizer_post_hooks:
            for post_hook in chain(self._optimizer_step_post_hooks.values(),
                                   _torch_optimizer._global_optimizer_post_hooks.values()):
                post_hook(self, args, kwargs)
        return loss

    # torch's Optimizer wraps `step` of each subclass in a profiler range unless
    # the function is marked as already hooked; the hooks are called above.
    step.hooked = True

    def _launch(self, dev, items, beta1, beta2, eps):
        n = len(items)
        a = self._launch_args.get(n)
        if a is None:
            a = self._launch_args[n] = _LaunchArgs(n)
        for k, (p, g, m, v, step_size, bc2s, wd) in enumerate(items):
            a.params[k] = p.data_ptr()
            a.grads[k] = g.data_ptr()
            a.ms[k] = m.data_ptr()
            a.vs[k] = v.data_ptr()
            a.numels[k] = p.numel()
            a.step_sizes[k] = step_size
            a.bc2s[k] = bc2s
            a.wds[k] = wd
        with N.prof("optim.adam"):
            N.call("cs_adam_step", n, a.params, a.grads, a.ms, a.vs, a.numels, a.step_sizes,
                   a.bc2s, a.wds, beta1, beta2, eps, N.stream(dev))


DEFAULT_TILELANG_THREADS = 256


class _AdanLaunchArgs:
    """ctypes argument arrays for one cs_adan_step launch of n tensors."""

    def __init__(self, n):
        self.n = n
        self.params = (ctypes.c_void_p * n)()
        self.grads = (ctypes.c_void_p * n)()
        self.ms = (ctypes.c_void_p * n)()
        self.ns = (ctypes.c_void_p * n)()
        self.ds = (ctypes.c_void_p * n)()
        self.npgs = (ctypes.c_void_p * n)()
        self.numels = (ctypes.c_int64 * n)()
        self.scalars = (ctypes.c_float * (10 * n))()
        self.flags = (ctypes.c_int32 * (2 * n))()


def _adan_launch(dev, items, clip_ptr, cache=None):
    """items: (param, grad, exp_avg, exp_avg_sq, exp_avg_diff, neg_pre_grad,
    [10 scalars], first, no_prox) per tensor, at most CS_ADAM_MAX_TENSORS."""
    n = len(items)
    a = cache.get(n) if cache is not None else None
    if a is None:
        a = _AdanLaunchArgs(n)
        if cache is not None:
            cache[n] = a
    for k, (p, g, m, v, d, npg, sc, first, no_prox) in enumerate(items):
        a.params[k] = p.data_ptr()
        a.grads[k] = g.data_ptr()
        a.ms[k] = m.data_ptr()
        a.ns[k] = v.data_ptr()
        a.ds[k] = d.data_ptr()
        a.npgs[k] = npg.data_ptr()
        a.numels[k] = p.numel()
        for j in range(10):
            a.scalars[10 * k + j] = sc[j]
        a.flags[2 * k] = int(first)
        a.flags[2 * k + 1] = int(no_prox)
    with N.prof("optim.adan"):
        N.call("cs_adan_step", n, a.params, a.grads, a.ms, a.ns, a.ds, a.npgs, a.numels,
               a.scalars, a.flags, clip_ptr, N.stream(dev))


class Adan(torch.optim.Optimizer):
    """The reference's Adan (manbo/optim.py:10-190): same constructor checks,
    param groups, per-parameter state (exp_avg, exp_avg_sq, exp_avg_diff,
    neg_pre_grad) and per-group integer ``step``, with the update of
    adan_step_from_grad_kernel (ops/optim.py:8-113) run as one cs_adan_step
    launch for up to 16 tensors.  With max_grad_norm > 0 the global-norm clip
    factor clamp(max_norm / (norm + eps), max=1) is computed on the device and
    read there (the reference reads it on the host with .item()).
    tilelang_threads is accepted for the reference's signature."""

    def __init__(self, params, lr: float = 1e-3, betas=(0.98, 0.92, 0.99), eps: float = 1e-8,
                 weight_decay: float = 0.0, max_grad_norm: float = 0.0, no_prox: bool = False,
                 tilelang_threads: int = DEFAULT_TILELANG_THREADS):
        if not 0.0 <= max_grad_norm:
            raise ValueError(f"Invalid max_grad_norm: {max_grad_norm}")
        if not 0.0 <= lr:
            raise ValueError(f"Invalid learning rate: {lr}")
        if not 0.0 <= eps:
            raise ValueError(f"Invalid epsilon value: {eps}")
        if not 0.0 <= betas[0] < 1.0:
            raise ValueError(f"Invalid beta parameter at index 0: {betas[0]}")
        if not 0.0 <= betas[1] < 1.0:
            raise ValueError(f"Invalid beta parameter at index 1: {betas[1]}")
        if not 0.0 <= betas[2] < 1.0:
            raise ValueError(f"Invalid beta parameter at index 2: {betas[2]}")
        if tilelang_threads <= 0:
            raise ValueError(f"Invalid tilelang_threads: {tilelang_threads}")
        defaults = dict(lr=lr, betas=betas, eps=eps, weight_decay=weight_decay,
                        max_grad_norm=max_grad_norm, no_prox=no_prox,
                        tilelang_threads=tilelang_threads)
        super().__init__(params, defaults)
        self._launch_args = {}

    def __setstate__(self, state):
        super().__setstate__(state)
        for group in self.param_groups:
            group.setdefault("no_prox", False)
            group.setdefault("tilelang_threads", DEFAULT_TILELANG_THREADS)
        self._launch_args = {}

    @torch.no_grad()
    def restart_opt(self):
        for group in self.param_groups:
            group["step"] = 0
            for p in group["params"]:
                if not p.requires_grad:
                    continue
                state = self.state[p]
                state["exp_avg"] = torch.zeros_like(p)
                state["exp_avg_sq"] = torch.zeros_like(p)
                state["exp_avg_diff"] = torch.zeros_like(p)
                state["neg_pre_grad"] = torch.zeros_like(p)

    def _clip_factor(self):
        """Device fp32 clamp(max_norm / (||g|| + eps), max=1) over every
        gradient (manbo/optim.py:78-96), or None when clipping is off."""
        max_norm = float(self.defaults["max_grad_norm"])
        if max_norm <= 0:
            return None
        device = self.param_groups[0]["params"][0].device
        total = torch.zeros(1, device=device)
        for group in self.param_groups:
            for p in group["params"]:
                if p.grad is not None:
                    total.add_(p.grad.pow(2).sum())
        norm = torch.sqrt(total)
        eps = self.param_groups[0]["eps"]
        return torch.clamp(torch.tensor(max_norm, device=device) / (norm + eps),
                           max=1.0).to(torch.float32).contiguous()

    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        clip = self._clip_factor()
        batches = {}
        for group in self.param_groups:
            beta1, beta2, beta3 = group["betas"]
            group["step"] = group.get("step", 0) + 1
            step = int(group["step"])
            bc1 = 1.0 - beta1 ** step
            bc2 = 1.0 - beta2 ** step
            bc3_sqrt = math.sqrt(1.0 - beta3 ** step)
            no_prox = bool(group["no_prox"])
            scalars = (float(beta1), float(beta2), float(beta3), float(bc1), float(bc2),
                       float(bc3_sqrt), float(group["lr"]), float(group["weight_decay"]),
                       float(group["eps"]), 1.0)
            for p in group["params"]:
                if p.grad is None:
                    continue
                if p.dtype != torch.float32:
                    raise ValueError("Adan expects float32 params")
                if not p.is_contiguous():
                    raise ValueError("Adan expects contiguous params")
                N.require_gpu(p, "Adan parameter")
                state = self.state[p]
                if len(state) == 0:
                    state["exp_avg"] = torch.zeros_like(p)
                    state["exp_avg_sq"] = torch.zeros_like(p)
                    state["exp_avg_diff"] = torch.zeros_like(p)
                    state["neg_pre_grad"] = torch.zeros_like(p)
                bufs = (state["exp_avg"], state["exp_avg_sq"], state["exp_avg_diff"],
                        state["neg_pre_grad"])
                if any(b.dtype != torch.float32 or not b.is_contiguous() for b in bufs):
                    raise ValueError("Adan expects contiguous float32 states")
                grad = p.grad
                if not (grad.dtype == torch.float32 and grad.device == p.device
                        and grad.is_contiguous()):
                    buf = state.get("_grad_buf")
                    if buf is None or buf.shape != p.shape:
                        buf = state["_grad_buf"] = torch.empty_like(p)
                    buf.copy_(grad)
                    grad = buf
                batches.setdefault(p.device.index, []).append(
                    (p, grad, *bufs, scalars, step == 1, no_prox))
        for dev, items in batches.items():
            for k in range(0, len(items), MAX_TENSORS_PER_LAUNCH):
                _adan_launch(dev, items[k:k + MAX_TENSORS_PER_LAUNCH],
                             None if clip is None else clip.data_ptr(), self._launch_args)
        return loss


def adan_step_from_grad_tilelang(param, grad, exp_avg, exp_avg_sq, exp_avg_diff, neg_pre_grad, *,
                                 step: int, lr: float = 1e-3, betas=(0.98, 0.92, 0.99),
                                 eps: float = 1e-8, weight_decay: float = 0.0,
                                 no_prox: bool = False, clip_global_grad_norm: float = 1.0,
                                 threads: int = DEFAULT_TILELANG_THREADS) -> None:
    """ops/optim.py:116-172: one Adan step in place from an external gradient
    (threads is accepted for the reference's signature)."""
    _ = threads
    beta1, beta2, beta3 = betas
    bc1 = 1.0 - beta1 ** step
    bc2 = 1.0 - beta2 ** step
    bc3 = 1.0 - beta3 ** step
    g = grad if grad.is_contiguous() else grad.contiguous()
    scalars = (float(beta1), float(beta2), float(beta3), float(bc1), float(bc2),
               float(bc3 ** 0.5), float(lr), float(weight_decay), float(eps),
               float(clip_global_grad_norm))
    _adan_launch(param.device.index,
                 [(param, g, exp_avg, exp_avg_sq, exp_avg_diff, neg_pre_grad, scalars,
                   int(step) == 1, bool(no_prox))], None)
