"""The HIP path against the committed golden fixtures: binning and forward
outputs bit for bit, gradients within 1e-4 of max|ref|, MSE and SSIM within
1e-5 relative, SSIM gradient within 1e-4."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from golden import make_fixtures as G
from helpers import grad_scale_tol


def load(case):
    with np.load(G.fixture_path(case)) as z:
        return {k: z[k] for k in z.files}


def _bits(a):
    a = np.ascontiguousarray(a)
    return a.view(np.uint8)


def _render(fx, dev="cuda"):
    import manbo
    h, w, S, mode = (int(v) for v in fx["in_meta"])
    t = lambda k: torch.from_numpy(fx[f"in_{k}"]).to(dev)  # noqa: E731
    cub = t("cubics_norm").requires_grad_(True)
    col = t("colors").requires_grad_(True)
    op = t("opacities").requires_grad_(True)
    aa = t("aa_widths").requires_grad_(True)
    sw = t("stroke_widths").requires_grad_(True) if mode == 1 else None
    if mode == 1:
        img = manbo.ops.render_cubic_polyline_splat_tilelang(
            cub, t("offs"), col, op, sw, t("depths"), h, w, 16, 16, t("background"),
            aa_widths=aa, distance_samples=S)
    else:
        img = manbo.ops.render_cubic_fill_splat_tilelang(
            cub, t("offs"), col, op, t("depths"), h, w, 16, 16, t("background"),
            fill_rules=t("fill_rules"), aa_widths=aa, distance_samples=S)
    return img, dict(cub=cub, col=col, op=op, aa=aa, sw=sw), (h, w, S, mode)


@pytest.mark.gpu
@pytest.mark.parametrize("case", list(G.CASES))
def test_binning_matches_fixture(case):
    from repo_amd import splat
    fx = load(case)
    h, w, S, mode = (int(v) for v in fx["in_meta"])
    t = lambda k: torch.from_numpy(fx[f"in_{k}"]).cuda()  # noqa: E731
    b = splat.bin_primitives(
        t("cubics_norm"), t("offs"), t("colors"), t("opacities"), t("depths"),
        t("fill_rules") if mode == 0 else None, torch.clamp(t("aa_widths"), min=1e-4),
        t("stroke_widths") if mode == 1 else None, h, w, S, mode=mode)
    np.testing.assert_array_equal(b.num_tiles_hit.cpu().numpy().astype(np.int32),
                                  fx["bin_num_tiles_hit"])
    np.testing.assert_array_equal(b.primitive_ids_sorted.cpu().numpy(),
                                  fx["bin_primitive_ids_sorted"])
    np.testing.assert_array_equal(b.tile_bins.cpu().numpy(), fx["bin_tile_bins"])


@pytest.mark.gpu
@pytest.mark.parametrize("case", list(G.CASES))
def test_forward_backward_match_fixture(case):
    fx = load(case)
    img, p, (h, w, S, mode) = _render(fx)
    np.testing.assert_array_equal(_bits(img.detach().cpu().numpy()), _bits(fx["fwd_out"]))
    img.backward(torch.from_numpy(G.v_out_pattern(h, w, 1 + mode)).cuda())
    checks = [("v_cubics_norm", p["cub"]), ("v_colors", p["col"]), ("v_opacities", p["op"]),
              ("v_aa_widths", p["aa"])]
    if mode == 1:
        checks.append(("v_stroke_widths", p["sw"]))
    for key, param in checks:
        ok, rel = grad_scale_tol(param.grad.cpu().numpy(), fx[f"bwd_{key}"])
        assert ok, f"{case} {key}: max error {rel:.3e} of max|ref|"


@pytest.mark.gpu
def test_losses_match_fixture():
    import manbo
    fx = load("cfg1_fill")
    h, w = int(fx["in_meta"][0]), int(fx["in_meta"][1])
    x = np.clip(fx["fwd_out"], 0.0, 1.0).transpose(2, 0, 1)[None].copy()
    y = torch.from_numpy(G.target_pattern(x)).cuda()
    xd = torch.from_numpy(x).cuda().requires_grad_(True)
    mse = float(manbo.mse_loss_tilelang(xd, y))
    assert abs(mse - float(fx["loss_mse"])) <= 1e-5 * abs(float(fx["loss_mse"]))
    s = manbo.ssim(xd, y)
    assert abs(float(s) - float(fx["loss_ssim"])) <= 1e-5 * abs(float(fx["loss_ssim"]))
    s.backward()
    g = xd.grad.cpu().numpy().astype(np.float64)
    samples = g.reshape(-1)[G.ssim_sample_index(g.shape)]
    ok, rel = grad_scale_tol(samples, fx["ssim_grad_samples"])
    assert ok, rel
    dirs = np.array([float((g * d).sum()) for d in G.ssim_directions(g.shape)])
    ok, rel = grad_scale_tol(dirs, fx["ssim_grad_dirs"])
    assert ok, rel
