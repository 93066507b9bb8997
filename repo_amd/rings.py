"""Closed control rings -> piecewise cubic Hermite segments, the step before
the closed-fill renderer in the reference's model
(gaussian_trace/render.py:755-777): ``closed_cubic_fill_segments_tilelang``
and its autograd Function (ops/cubic_splatting.py:81-543) on the HIP kernels
``cs_closed_ring_segments`` / ``cs_closed_ring_segments_backward``."""
from __future__ import annotations

import math

import torch

from . import _native as N

DEFAULT_THREADS = 256


def _as_f32_contig(t: torch.Tensor) -> torch.Tensor:
    return t.detach().to(torch.float32).contiguous()


def _closed_fill_piecewise_basis_tensors(*, control_points_per_bezier: int, subdiv: int,
                                         device: torch.device):
    """ops/cubic_splatting.py:81-134: basis [subdiv+1, Kb], deriv_basis
    [subdiv+1, Kb-1] (Bernstein polynomials of degree Kb-1 and Kb-2 at
    t = linspace(0, 1, subdiv+1)) and dt [subdiv]."""
    kb = int(control_points_per_bezier)
    sub = int(subdiv)
    if kb < 2:
        raise ValueError(f"control_points_per_bezier must be >=2, got {kb}")
    if sub <= 0:
        raise ValueError(f"subdiv must be >0, got {sub}")
    n = sub + 1
    t = torch.linspace(0.0, 1.0, n, device=device, dtype=torch.float32)
    t_col, omt_col = t.view(n, 1), (1.0 - t).view(n, 1)
    deg = kb - 1
    idx = torch.arange(kb, device=device, dtype=torch.float32)
    comb = torch.tensor([math.comb(deg, i) for i in range(kb)], device=device,
                        dtype=torch.float32)
    basis = (comb.view(1, kb) * torch.pow(omt_col, (deg - idx).view(1, kb))
             * torch.pow(t_col, idx.view(1, kb))).contiguous()
    didx = torch.arange(kb - 1, device=device, dtype=torch.float32)
    dcomb = torch.tensor([math.comb(deg - 1, i) for i in range(kb - 1)], device=device,
                         dtype=torch.float32)
    deriv_basis = (dcomb.view(1, kb - 1) * torch.pow(omt_col, ((deg - 1) - didx).view(1, kb - 1))
                   * torch.pow(t_col, didx.view(1, kb - 1))).contiguous()
    dt = (t[1:] - t[:-1]).contiguous()
    return basis, deriv_basis, dt


# Basis tables per (device, Kb, subdiv): the reference builds them on every
# call; they only depend on these three.
_BASIS_CACHE: "dict[tuple, tuple]" = {}


def _basis(kb: int, subdiv: int, device: torch.device):
    key = (str(device), int(kb), int(subdiv))
    v = _BASIS_CACHE.get(key)
    if v is None:
        v = _BASIS_CACHE[key] = _closed_fill_piecewise_basis_tensors(
            control_points_per_bezier=kb, subdiv=subdiv, device=device)
    return v


def _check_ring_shape(k: int) -> None:
    if k < 4 or ((k - 2) % 2) != 0:
        raise ValueError(
            "closed cubic fill expects control point count K that satisfies K>=4 and "
            f"(K-2)%2==0, got K={k}")


class _ClosedCubicFillSegmentsFn(torch.autograd.Function):
    """Signature of ops/cubic_splatting.py:386-483."""

    @staticmethod
    def forward(ctx, control_points_in, basis, deriv_basis, dt, threads, subdiv):
        cp = _as_f32_contig(control_points_in)
        N.require_gpu(cp, "control_points")
        basis_f32 = _as_f32_contig(basis)
        deriv_f32 = _as_f32_contig(deriv_basis)
        dt_f32 = _as_f32_contig(dt).view(-1)
        num_curves, k = int(cp.shape[0]), int(cp.shape[1])
        _check_ring_shape(k)
        sub = int(subdiv)
        out = torch.empty((num_curves * 2 * sub, 4, 2), dtype=torch.float32, device=cp.device)
        if num_curves > 0:
            with N.prof("cubic.fwd.ring_segments"):
                N.call("cs_closed_ring_segments", N.ptr(cp), num_curves, k, sub,
                       N.ptr(basis_f32), N.ptr(deriv_f32), N.ptr(dt_f32), N.ptr(out),
                       N.stream(cp.device))
        ctx.save_for_backward(basis_f32, deriv_f32, dt_f32)
        ctx.num_curves, ctx.control_points, ctx.subdiv = num_curves, k, sub
        ctx.threads = int(threads)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        basis, deriv_basis, dt = ctx.saved_tensors
        num_curves, k, sub = ctx.num_curves, ctx.control_points, ctx.subdiv
        g = _as_f32_contig(grad_out)
        if g.data_ptr() % 16:
            g = g.clone()
        grad_cp = torch.empty((num_curves, k, 2), dtype=torch.float32, device=g.device)
        if num_curves > 0:
            with N.prof("cubic.bwd.ring_segments"):
                N.call("cs_closed_ring_segments_backward", N.ptr(g), num_curves, k, sub,
                       N.ptr(basis), N.ptr(deriv_basis), N.ptr(dt), N.ptr(grad_cp),
                       N.stream(g.device))
        return grad_cp, None, None, None, None, None


def closed_cubic_fill_segments_tilelang(control_points: torch.Tensor, *, subdiv: int = 4,
                                        threads: int = DEFAULT_THREADS):
    """ops/cubic_splatting.py:486-543: control polygons [N, K, 2] ->
    (ring_segments [N * 2 * subdiv, 4, 2], ring_offsets [N + 1] int32 with
    stride 2 * subdiv)."""
    if control_points.ndim != 3 or int(control_points.shape[-1]) != 2:
        raise ValueError(f"control_points must be [N,K,2], got {tuple(control_points.shape)}")
    if not control_points.is_cuda:
        raise ValueError("closed_cubic_fill_segments_tilelang requires CUDA tensor")
    if int(subdiv) <= 0:
        raise ValueError(f"subdiv must be >0, got {int(subdiv)}")
    num_curves, k = int(control_points.shape[0]), int(control_points.shape[1])
    _check_ring_shape(k)
    per_curve = 2 * int(subdiv)
    dev = control_points.device
    ring_offsets = torch.arange(0, (num_curves + 1) * per_curve, per_curve, dtype=torch.int32,
                                device=dev)
    if num_curves <= 0:
        return torch.empty((0, 4, 2), dtype=torch.float32, device=dev), ring_offsets
    basis, deriv_basis, dt = _basis((k + 2) // 2, int(subdiv), dev)
    segs = _ClosedCubicFillSegmentsFn.apply(control_points, basis, deriv_basis, dt, int(threads),
                                            int(subdiv))
    return segs, ring_offsets
