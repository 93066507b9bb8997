"""Adam with the step in one HIP launch for all parameters.

The reference optimizes its primitives with ``torch.optim.Adam`` over
per-group learning rates (gaussian_trace/model.py:172-189).  ``Adam`` here is
a drop-in for that class on fp32 device parameters: same constructor, param
groups, ``state`` entries (``step``, ``exp_avg``, ``exp_avg_sq``) and
``state_dict`` layout, so a checkpoint moves between the two.  The update is
torch's single-tensor Adam (amsgrad and maximize off); one ``cs_adam_step``
launch covers up to 16 tensors.
"""
from __future__ import annotations

import ctypes
import math

import torch

from . import _native as N

MAX_TENSORS_PER_LAUNCH = 16


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

    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        batches = {}
        for group in self.param_groups:
            beta1, beta2 = group["betas"]
            key = (float(beta1), float(beta2), float(group["eps"]))
            for p in group["params"]:
                if p.grad is None:
                    continue
                if p.grad.is_sparse:
                    raise RuntimeError("Adam does not support sparse gradients")
                N.require_gpu(p, "parameter")
                if p.dtype != torch.float32 or not p.is_contiguous():
                    raise ValueError("repo_amd.optim.Adam needs contiguous float32 parameters")
                st = self.state[p]
                if len(st) == 0:
                    st["step"] = torch.tensor(0.0, dtype=torch.float32)
                    st["exp_avg"] = torch.zeros_like(p, memory_format=torch.preserve_format)
                    st["exp_avg_sq"] = torch.zeros_like(p, memory_format=torch.preserve_format)
                st["step"] += 1
                step = float(st["step"].item())
                bc1 = 1.0 - beta1 ** step
                bc2 = 1.0 - beta2 ** step
                grad = p.grad if p.grad.is_contiguous() else p.grad.contiguous()
                batches.setdefault((p.device, key), []).append(
                    (p, grad, st["exp_avg"], st["exp_avg_sq"], float(group["lr"]) / bc1,
                     math.sqrt(bc2), float(group["weight_decay"])))
        for (dev, (beta1, beta2, eps)), items in batches.items():
            for k in range(0, len(items), MAX_TENSORS_PER_LAUNCH):
                self._launch(dev, items[k:k + MAX_TENSORS_PER_LAUNCH], beta1, beta2, eps)
        return loss

    @staticmethod
    def _launch(dev, items, beta1, beta2, eps):
        n = len(items)
        vp = ctypes.c_void_p * n
        params = vp(*[t[0].data_ptr() for t in items])
        grads = vp(*[t[1].data_ptr() for t in items])
        ms = vp(*[t[2].data_ptr() for t in items])
        vs = vp(*[t[3].data_ptr() for t in items])
        numels = (ctypes.c_int64 * n)(*[t[0].numel() for t in items])
        step_sizes = (ctypes.c_float * n)(*[t[4] for t in items])
        bc2s = (ctypes.c_float * n)(*[t[5] for t in items])
        wds = (ctypes.c_float * n)(*[t[6] for t in items])
        with N.prof("optim.adam"):
            N.call("cs_adam_step", n, params, grads, ms, vs, numels, step_sizes, bc2s, wds,
                   float(beta1), float(beta2), float(eps), N.stream(dev))
