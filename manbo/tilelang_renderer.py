"""manbo.tilelang_renderer (reference tilelang_renderer.py:31-589): the 2D
Gaussian splat renderer GsRenderFunction / gs_render / GsRenderModule and
its profiling hook, on the HIP kernels of repo_amd/csrc/gaussian.hip (host
side in repo_amd.gaussian)."""
from __future__ import annotations

from contextlib import nullcontext
from typing import Any, Callable, ContextManager, Mapping, MutableMapping, Optional, Tuple

import torch
from torch import nn

from repo_amd import gaussian as G

ProfileCtxFactory = Callable[[str], ContextManager]
_PROFILE_CTX_FACTORY: Optional[ProfileCtxFactory] = None
GsProcessPayload = MutableMapping[str, Any]
GsProcessFn = Callable[[str, GsProcessPayload], Optional[Mapping[str, Any]]]


def set_gs_profile_ctx_factory(factory: Optional[ProfileCtxFactory]) -> None:
    """tilelang_renderer.py:31-33."""
    global _PROFILE_CTX_FACTORY
    _PROFILE_CTX_FACTORY = factory


def _prof(label: str):
    """tilelang_renderer.py:36-39."""
    if _PROFILE_CTX_FACTORY is None:
        return nullcontext()
    return _PROFILE_CTX_FACTORY(label)


def _profile_label(prefix: str, leaf: str) -> str:
    """tilelang_renderer.py:42-49."""
    base = str(prefix).strip(".")
    suffix = str(leaf).strip(".")
    if not base:
        return suffix
    if not suffix:
        return base
    return f"{base}.{suffix}"


def _tile_bounds(img_h: int, img_w: int, block_x: int, block_y: int) -> Tuple[int, int, int]:
    """tilelang_renderer.py:69-75."""
    return ((img_w + block_x - 1) // block_x, (img_h + block_y - 1) // block_y, 1)


def _normalize_gaussian_meta(gaussian_meta: Optional[torch.Tensor], *, expected_size: int,
                             device: torch.device) -> Optional[torch.Tensor]:
    """tilelang_renderer.py:78-92."""
    if gaussian_meta is None:
        return None
    meta = gaussian_meta.to(device=device, dtype=torch.int32).contiguous().view(-1)
    if meta.numel() != int(expected_size):
        raise ValueError(
            f"gaussian_meta size mismatch: expected {expected_size}, got {meta.numel()}")
    return meta


def _run_process_fn(process_fn: Optional[GsProcessFn], stage: str,
                    payload: GsProcessPayload) -> GsProcessPayload:
    """tilelang_renderer.py:136-146."""
    if process_fn is None:
        return payload
    updates = process_fn(stage, payload)
    if updates:
        payload.update(updates)
    return payload


def _require_cuda(t: torch.Tensor, name: str) -> None:
    if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
        raise ValueError(f"{name} must be a CUDA (ROCm) tensor")


class GsRenderFunction(torch.autograd.Function):
    """tilelang_renderer.py:149-490 on the MI355X kernels of
    repo_amd/csrc/gaussian.hip.  Same inputs, outputs, process_fn stages and
    payload keys; the reference's cumsum + map + sort + tile-bin pass is one
    binning (repo_amd.gaussian.bin_gaussians) with the same results, under the
    profile label "<prefix>.bins"."""

    @staticmethod
    def forward(ctx, means2d, scales2d, rotation, colors, opacities, img_h, img_w, block_x,
                block_y, bg, process_fn=None, profile_fwd_prefix="tilelang.fwd",
                profile_bwd_prefix="tilelang.bwd"):
        for t, name in ((means2d, "means2d"), (scales2d, "scales2d"), (rotation, "rotation"),
                        (colors, "colors"), (opacities, "opacities"), (bg, "bg")):
            _require_cuda(t, name)
        img_h, img_w, block_x, block_y = int(img_h), int(img_w), int(block_x), int(block_y)
        tile_bounds = _tile_bounds(img_h, img_w, block_x, block_y)
        block = (block_x, block_y, 1)
        img_size = (img_w, img_h, 1)

        with _prof(_profile_label(profile_fwd_prefix, "total")):
            with _prof(_profile_label(profile_fwd_prefix, "proj")):
                xys, depths, radii, conics, num_tiles_hit = G.project_forward(
                    means2d, scales2d, rotation, img_h, img_w, block_x, block_y)

            payload: GsProcessPayload = {
                "means2d": means2d, "scales2d": scales2d, "rotation": rotation, "xys": xys,
                "depths": depths, "radii": radii, "conics": conics,
                "num_tiles_hit": num_tiles_hit, "colors": colors, "opacities": opacities,
                "bg": bg, "img_h": img_h, "img_w": img_w, "block_x": block_x,
                "block_y": block_y, "tile_bounds": tile_bounds,
            }
            payload = _run_process_fn(process_fn, "post_project", payload)
            xys, depths, radii = payload["xys"], payload["depths"], payload["radii"]
            conics, colors = payload["conics"], payload["colors"]
            opacities, bg = payload["opacities"], payload["bg"]
            gaussian_meta = _normalize_gaussian_meta(
                payload.get("gaussian_meta"), expected_size=means2d.shape[0], device=xys.device)

            with _prof(_profile_label(profile_fwd_prefix, "bins")):
                binned = G.bin_gaussians(xys, conics, radii, depths, img_h, img_w, block_x,
                                         block_y)
                gaussian_ids_sorted = binned.gaussian_ids_sorted
                tile_bins = binned.tile_bins
                intersect_meta_sorted = None
                if gaussian_meta is not None:
                    # map_gaussian_meta_to_intersects + gather by the sort
                    # permutation (tilelang_renderer.py:254-260) = meta[ids].
                    intersect_meta_sorted = gaussian_meta[gaussian_ids_sorted.long()]

            payload = {
                "xys": xys, "conics": conics, "colors": colors, "opacities": opacities,
                "bg": bg, "gaussian_ids_sorted": gaussian_ids_sorted,
                "intersect_meta_sorted": intersect_meta_sorted, "tile_bins": tile_bins,
                "tile_bounds": tile_bounds, "block": block, "img_size": img_size,
            }
            payload = _run_process_fn(process_fn, "pre_rasterize", payload)
            xys, conics, colors = payload["xys"], payload["conics"], payload["colors"]
            opacities, bg = payload["opacities"], payload["bg"]
            gaussian_ids_sorted = payload["gaussian_ids_sorted"]
            intersect_meta_sorted = _normalize_gaussian_meta(
                payload.get("intersect_meta_sorted"),
                expected_size=gaussian_ids_sorted.shape[0], device=gaussian_ids_sorted.device)
            tile_bins = payload["tile_bins"]

            with _prof(_profile_label(profile_fwd_prefix, "rast")):
                n = int(xys.shape[0])
                records = G.pack_records(xys, conics, colors, opacities,
                                         out=binned.records if n == binned.n else None)
                out_img, final_Ts, final_idx = G.rasterize_forward(
                    gaussian_ids_sorted, tile_bins, records, bg, img_h, img_w, block_x, block_y)

        ctx.save_for_backward(means2d, scales2d, rotation, colors, opacities, xys, depths, radii,
                              conics, gaussian_ids_sorted, tile_bins, final_Ts, final_idx, bg)
        ctx.img_h, ctx.img_w = img_h, img_w
        ctx.block_x, ctx.block_y = block_x, block_y
        ctx.tile_bounds, ctx.block, ctx.img_size = tile_bounds, block, img_size
        ctx.profile_bwd_prefix = str(profile_bwd_prefix)
        ctx.gaussian_meta = gaussian_meta
        ctx.intersect_meta_sorted = intersect_meta_sorted
        ctx.process_fn = process_fn
        ctx.binned = binned
        ctx.records = records
        return out_img

    @staticmethod
    def backward(ctx, grad_out_img):
        (means2d, scales2d, rotation, colors, opacities, xys, depths, radii, conics,
         gaussian_ids_sorted, tile_bins, final_Ts, final_idx, bg) = ctx.saved_tensors
        img_h, img_w = ctx.img_h, ctx.img_w
        gaussian_meta = ctx.gaussian_meta
        intersect_meta_sorted = ctx.intersect_meta_sorted
        process_fn = ctx.process_fn
        binned = ctx.binned
        prefix = ctx.profile_bwd_prefix
        # tilelang_renderer.py:323: zeros; the kernel reads NULL as zeros, so
        # the tensor exists only for a process_fn that can see it.
        v_out_alpha = torch.zeros_like(final_Ts) if process_fn is not None else None

        with _prof(_profile_label(prefix, "total")):
            payload: GsProcessPayload = {
                "collect_curve_contrib_rgb": False, "collect_curve_isect_contrib": False,
                "num_primitives": int(colors.shape[0]), "colors": colors,
            }
            payload = _run_process_fn(process_fn, "pre_backward_rasterize", payload)
            collect_rgb = bool(payload.get("collect_curve_contrib_rgb", False))
            collect_isect = bool(payload.get("collect_curve_isect_contrib", False))
            curve_contrib_rgb = (torch.zeros_like(colors, dtype=torch.float32)
                                 if collect_rgb else None)
            curve_isect_contrib = (torch.zeros((int(gaussian_ids_sorted.numel()),),
                                               dtype=torch.float32, device=colors.device)
                                   if collect_isect else None)
            n = int(ctx.records.shape[0])
            grads = None
            if binned.grad_accum_clean and n == binned.n:
                grads = binned.grad_accum
                binned.grad_accum_clean = False
            with _prof(_profile_label(prefix, "rast")):
                v_xy, v_conic, v_rgb, v_opacity = G.rasterize_backward(
                    gaussian_ids_sorted, tile_bins, ctx.records, bg, img_h, img_w, ctx.block_x,
                    ctx.block_y, final_Ts, final_idx, grad_out_img, v_out_alpha,
                    intersect_meta_sorted=intersect_meta_sorted, grads=grads,
                    curve_contrib_rgb=curve_contrib_rgb, curve_isect_contrib=curve_isect_contrib)
            payload = {
                "v_xy": v_xy, "v_conic": v_conic, "v_rgb": v_rgb, "v_opacity": v_opacity,
                "curve_contrib_rgb": curve_contrib_rgb,
                "curve_isect_contrib": curve_isect_contrib, "xys": xys, "conics": conics,
                "colors": colors, "opacities": opacities,
                "gaussian_ids_sorted": gaussian_ids_sorted, "tile_bins": tile_bins,
                "final_Ts": final_Ts, "final_idx": final_idx, "grad_out_img": grad_out_img,
                "gaussian_meta": gaussian_meta, "intersect_meta_sorted": intersect_meta_sorted,
                "v_out_alpha": v_out_alpha,
            }
            payload = _run_process_fn(process_fn, "post_backward_rasterize", payload)
            v_xy, v_conic = payload["v_xy"], payload["v_conic"]
            v_rgb, v_opacity = payload["v_rgb"], payload["v_opacity"]
            with _prof(_profile_label(prefix, "proj")):
                _, v_mean2d, v_scales2d, v_rotation = G.project_backward(
                    scales2d, rotation, radii, conics, v_xy, v_conic, img_h, img_w,
                    gaussian_meta=gaussian_meta)

        if v_opacity is not None and v_opacity.dim() != 1:
            v_opacity = v_opacity.view(-1)
        if v_rotation is not None and v_rotation.dim() != 1:
            v_rotation = v_rotation.view(-1)
        return (v_mean2d, v_scales2d, v_rotation, v_rgb, v_opacity, None, None, None, None, None,
                None, None, None)


def gs_render(means2d, scales2d, rotation, colors, opacities, img_h, img_w, block_x, block_y, bg,
              process_fn: Optional[GsProcessFn] = None, *,
              profile_fwd_prefix: str = "tilelang.fwd",
              profile_bwd_prefix: str = "tilelang.bwd"):
    """tilelang_renderer.py:493-523."""
    return GsRenderFunction.apply(means2d, scales2d, rotation, colors, opacities, img_h, img_w,
                                  block_x, block_y, bg, process_fn, str(profile_fwd_prefix),
                                  str(profile_bwd_prefix))


class GsRenderModule(nn.Module):
    """tilelang_renderer.py:526-589."""

    def __init__(self, img_h: int, img_w: int, block_x: int = 16, block_y: int = 8,
                 background: Tuple[float, float, float] = (1.0, 1.0, 1.0),
                 process_fn: Optional[GsProcessFn] = None,
                 profile_fwd_prefix: str = "tilelang.fwd",
                 profile_bwd_prefix: str = "tilelang.bwd"):
        super().__init__()
        self.img_h = int(img_h)
        self.img_w = int(img_w)
        self.block_x = int(block_x)
        self.block_y = int(block_y)
        self.process_fn = process_fn
        self.profile_fwd_prefix = str(profile_fwd_prefix)
        self.profile_bwd_prefix = str(profile_bwd_prefix)
        self.register_buffer("background", torch.tensor(background, dtype=torch.float32))

    def forward(self, means2d, scales2d, rotation, colors, opacities, bg=None, process_fn=None, *,
                profile_fwd_prefix=None, profile_bwd_prefix=None):
        return gs_render(means2d, scales2d, rotation, colors, opacities, self.img_h, self.img_w,
                         self.block_x, self.block_y, self.background if bg is None else bg,
                         self.process_fn if process_fn is None else process_fn,
                         profile_fwd_prefix=(self.profile_fwd_prefix if profile_fwd_prefix is None
                                             else str(profile_fwd_prefix)),
                         profile_bwd_prefix=(self.profile_bwd_prefix if profile_bwd_prefix is None
                                             else str(profile_bwd_prefix)))


__all__ = ["GsRenderFunction", "GsRenderModule", "gs_render", "set_gs_profile_ctx_factory"]
