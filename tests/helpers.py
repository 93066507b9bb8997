"""Shared test helpers: run the HIP path and the oracle on the same scene."""
from __future__ import annotations

import numpy as np
import torch

from oracle import oracle as O


def scene_np(sc):
    sw = None if sc.stroke_widths is None else sc.stroke_widths.cpu().numpy()
    return dict(cubics_norm=sc.cubics_norm.cpu().numpy(), offs=sc.seg_offsets.cpu().numpy(),
                colors=sc.colors.cpu().numpy(), opacities=sc.opacities.cpu().numpy(),
                depths=sc.depths.cpu().numpy(), aa_widths=sc.aa_widths.cpu().numpy(),
                fill_rules=sc.fill_rules.cpu().numpy(), background=sc.background.cpu().numpy(),
                stroke_widths=sw, img_h=sc.img_h, img_w=sc.img_w, S=sc.S)


def oracle_forward(sc, rows=None, flatten_method="bernstein", aniso=False, workers=None):
    """The oracle's forward of scene sc; ``rows`` as for O.raster_forward, on
    ``workers`` threads (default: the usable CPUs, at most 16)."""
    d = scene_np(sc)
    return O.render_forward(d["cubics_norm"], d["offs"], d["colors"], d["opacities"], d["depths"],
                            d["img_h"], d["img_w"], d["background"], fill_rules=d["fill_rules"],
                            aa_widths=d["aa_widths"], S=d["S"], stroke_widths=d["stroke_widths"],
                            rows=rows, flatten_method=flatten_method, aniso=aniso,
                            workers=O.default_workers() if workers is None else workers)


def hip_bin(sc, device="cuda", flatten_method="bernstein", aniso=False):
    from repo_amd import splat
    s = sc.to(device)
    mode = splat.MODE_FILL if s.stroke_widths is None else splat.MODE_STROKE
    widths = torch.clamp(s.aa_widths.float(), min=1e-4).contiguous()
    return splat.bin_primitives(
        s.cubics_norm.contiguous(), s.seg_offsets.to(torch.int32).contiguous(),
        s.colors.contiguous(), s.opacities.contiguous(), s.depths.contiguous(),
        s.fill_rules.to(torch.int32).contiguous() if mode == 0 else None, widths,
        None if s.stroke_widths is None else s.stroke_widths.contiguous(), s.img_h, s.img_w,
        s.S, mode=mode, flatten_method=flatten_method, aniso=aniso), s


def grad_scale_tol(got, ref, rtol=1e-4, floor=1e-30):
    """|got - ref| <= rtol * max|ref| elementwise (scale-aware tolerance for
    sums accumulated in a different order)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    scale = max(float(np.abs(ref).max()) if ref.size else 0.0, floor)
    err = float(np.abs(got - ref).max()) if ref.size else 0.0
    return err <= rtol * scale, err / scale


def grad_elementwise_tol(got, ref, rtol=1e-4, atol_frac=1e-6):
    """|got - ref| <= rtol * |ref| + atol_frac * max|ref| for every element.
    Returns (ok, worst |got - ref| / |ref| over elements with ref != 0,
    worst |got - ref| / (rtol |ref| + atol_frac max|ref|))."""
    got = np.asarray(got, np.float64).ravel()
    ref = np.asarray(ref, np.float64).ravel()
    if ref.size == 0:
        return True, 0.0, 0.0
    scale = float(np.abs(ref).max())
    err = np.abs(got - ref)
    bound = rtol * np.abs(ref) + atol_frac * scale
    nz = ref != 0
    worst_rel = float((err[nz] / np.abs(ref[nz])).max()) if nz.any() else 0.0
    ratio = float((err / np.maximum(bound, 1e-300)).max()) if scale > 0 else float(err.max())
    return bool(np.all(err <= bound)), worst_rel, ratio


def check_grads(checks, rtol=1e-4, atol_frac=1e-6):
    """Each (name, got, ref) within rtol of max|ref| (the scale criterion) and
    within rtol |ref| + atol_frac max|ref| elementwise; prints the worst
    elementwise relative error of every tensor."""
    bad = []
    for key, got, ref in checks:
        g = got.detach().cpu().numpy() if hasattr(got, "detach") else np.asarray(got)
        ok_s, rel_s = grad_scale_tol(g, ref, rtol=rtol)
        ok_e, worst, ratio = grad_elementwise_tol(g, ref, rtol=rtol, atol_frac=atol_frac)
        print(f"  {key}: max err {rel_s:.2e} of max|ref|, worst elementwise rel {worst:.2e}, "
              f"bound ratio {ratio:.2f}", flush=True)
        if not (ok_s and ok_e):
            bad.append(f"{key}: scale err {rel_s:.3e}, elementwise bound ratio {ratio:.3f}")
    assert not bad, "; ".join(bad)


def random_v_out(h, w, seed=7):
    g = torch.Generator("cpu").manual_seed(seed)
    return torch.randn((h, w, 3), generator=g, dtype=torch.float32)
