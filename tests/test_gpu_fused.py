"""Fused training-step operations (repo_amd.fused) against the separate
reference-API calls and the float64 oracle."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O


def _img(h, w, seed):
    g = torch.Generator().manual_seed(seed)
    img = torch.rand((h, w, 3), generator=g) * 1.4 - 0.2  # values below 0 and above 1
    img[0, :4] = torch.tensor([0.0, 1.0, 0.0])  # exactly on the clamp bounds
    return img


@pytest.mark.gpu
def test_clamp_to_nchw_matches_torch():
    from repo_amd import fused
    img = _img(37, 53, 1).cuda()
    a = img.clone().requires_grad_(True)
    b = img.clone().requires_grad_(True)
    out = fused.clamp_to_nchw(a)
    ref = b.clamp(0, 1).permute(2, 0, 1).unsqueeze(0).contiguous()
    assert out.shape == ref.shape and out.is_contiguous()
    assert torch.equal(out, ref)
    g = torch.randn_like(ref)
    out.backward(g)
    ref.backward(g)
    assert torch.equal(a.grad, b.grad)


@pytest.mark.gpu
@pytest.mark.parametrize("shape,weight", [((1, 3, 64, 80), 0.2), ((2, 3, 45, 61), 0.7)])
def test_mse_ssim_loss_matches_separate_calls_and_oracle(shape, weight):
    import manbo
    from repo_amd import fused
    g = torch.Generator().manual_seed(3)
    y = torch.rand(shape, generator=g)
    x = (0.6 * y + 0.4 * torch.rand(shape, generator=g)).clamp(0, 1)
    xd = x.cuda().requires_grad_(True)
    loss, parts = fused.mse_ssim_loss(xd, y.cuda(), weight)
    sep = manbo.mse_loss_tilelang(x.cuda(), y.cuda()) + weight * (1 - manbo.ssim(x.cuda(),
                                                                                 y.cuda()))
    assert abs(float(loss.detach()) - float(sep)) <= 2e-6 * abs(float(sep))
    x64 = x.double().requires_grad_(True)
    ref = ((x64 - y.double()) ** 2).mean() + weight * (1 - O.ssim_torch64(x64, y.double()))
    assert abs(float(loss) - float(ref)) <= 1e-5 * abs(float(ref))
    assert abs(float(parts[0]) - float(((x64 - y.double()) ** 2).mean())) <= 1e-5 * float(
        ((x64 - y.double()) ** 2).mean())
    (1.5 * loss).backward()
    (1.5 * ref).backward()
    got = xd.grad.cpu().double().numpy()
    want = x64.grad.numpy()
    assert np.abs(got - want).max() <= 1e-4 * np.abs(want).max()


@pytest.mark.gpu
def test_fused_step_gradients_match_unfused():
    """Render -> clamp/permute -> MSE + 0.2 (1 - SSIM) -> backward: control-point
    and colour gradients through the fused ops equal the separate-call path."""
    import manbo
    from repo_amd import fused, synth
    sc = synth.small_scene(21, P=30, h=96, w=112, rmax=40.0)
    dev = "cuda"
    target = torch.rand((1, 3, sc.img_h, sc.img_w), generator=torch.Generator().manual_seed(4))
    target = target.to(dev)
    grads = []
    for use_fused in ("hwc", True, False):
        cub = sc.cubics_norm.to(dev).requires_grad_(True)
        col = sc.colors.to(dev).requires_grad_(True)
        img = manbo.ops.render_cubic_fill_splat_tilelang(
            cub, sc.seg_offsets.to(dev), col, sc.opacities.to(dev), sc.depths.to(dev), sc.img_h,
            sc.img_w, 16, 16, sc.background.to(dev), aa_widths=sc.aa_widths.to(dev),
            distance_samples=sc.S)
        if use_fused == "hwc":
            loss, _ = fused.clamp_mse_ssim_loss(img, target, 0.2)
        elif use_fused:
            loss, _ = fused.mse_ssim_loss(fused.clamp_to_nchw(img), target, 0.2)
        else:
            x = img.clamp(0, 1).permute(2, 0, 1).unsqueeze(0).contiguous()
            loss = manbo.mse_loss_tilelang(x, target) + 0.2 * (1 - manbo.ssim(x, target))
        loss.backward()
        grads.append((float(loss), cub.grad.cpu().numpy(), col.grad.cpu().numpy()))
    (lh, ch, kh), (lf, cf, kf), (lu, cu, ku) = grads
    for l_, c_, k_ in ((lh, ch, kh), (lf, cf, kf)):
        assert abs(l_ - lu) <= 2e-6 * abs(lu)
        for a, b in ((c_, cu), (k_, ku)):
            assert np.abs(a - b).max() <= 1e-4 * np.abs(b).max()


@pytest.mark.gpu
@pytest.mark.parametrize("h,w,weight", [(64, 80, 0.2), (45, 61, 0.7), (97, 130, 0.2),
                                        (11, 11, 0.5)])
def test_clamp_mse_ssim_loss_on_hwc_image(h, w, weight):
    """The HWC-direct loss equals torch's clamp/permute glue followed by the
    separate loss calls (value within 2e-6, gradient w.r.t. the [H, W, 3]
    image within 1e-4 of float64 autograd, zero where the image lies outside
    [0, 1]); sizes cover partial last tile rows and columns and the smallest
    image a window fits."""
    import manbo
    from repo_amd import fused
    print(f"[clamp_mse_ssim] {h}x{w}", flush=True)
    img = _img(h, w, 5)
    g = torch.Generator().manual_seed(8)
    y = torch.rand((1, 3, h, w), generator=g)
    a = img.cuda().requires_grad_(True)
    loss, parts = fused.clamp_mse_ssim_loss(a, y.cuda(), weight)
    x = img.cuda().clamp(0, 1).permute(2, 0, 1).unsqueeze(0).contiguous()
    sep_mse = manbo.mse_loss_tilelang(x, y.cuda())
    sep = sep_mse + weight * (1 - manbo.ssim(x, y.cuda()))
    assert abs(float(loss.detach()) - float(sep)) <= 2e-6 * abs(float(sep))
    assert abs(float(parts[0]) - float(sep_mse)) <= 2e-6 * abs(float(sep_mse))
    i64 = img.double().requires_grad_(True)
    x64 = i64.clamp(0, 1).permute(2, 0, 1).unsqueeze(0)
    ref = ((x64 - y.double()) ** 2).mean() + weight * (1 - O.ssim_torch64(x64, y.double()))
    assert abs(float(loss) - float(ref)) <= 1e-5 * abs(float(ref))
    (0.75 * loss).backward()
    (0.75 * ref).backward()
    got = a.grad.cpu().double().numpy()
    want = i64.grad.numpy()
    assert np.abs(got - want).max() <= 1e-4 * np.abs(want).max()
    outside = ((img < 0) | (img > 1)).numpy()
    assert outside.any() and np.all(got[outside] == 0.0)


@pytest.mark.gpu
@pytest.mark.parametrize("h,w", [(512, 768), (1356, 2040)])
def test_clamp_mse_ssim_loss_at_frame_size(h, w):
    """The benchmark's loss (clamp, MSE + 0.2 (1 - SSIM) of the HWC render) at
    config 2's and config 3's frame sizes against float64 autograd of the
    separable restatement: value within 1e-5, gradient per tensor and per
    element, zero where the clamp is active."""
    from helpers import check_grads
    from repo_amd import fused
    print(f"[clamp_mse_ssim] {h}x{w}", flush=True)
    img = _img(h, w, 11)
    y = torch.rand((1, 3, h, w), generator=torch.Generator().manual_seed(12))
    a = img.cuda().requires_grad_(True)
    loss, parts = fused.clamp_mse_ssim_loss(a, y.cuda(), 0.2)
    i64 = img.double().requires_grad_(True)
    x64 = i64.clamp(0, 1).permute(2, 0, 1).unsqueeze(0)
    mse64 = ((x64 - y.double()) ** 2).mean()
    ref = mse64 + 0.2 * (1 - O.ssim64_separable(x64, y.double()))
    assert abs(float(loss) - float(ref)) <= 1e-5 * abs(float(ref))
    assert abs(float(parts[0]) - float(mse64)) <= 1e-5 * float(mse64)
    loss.backward()
    ref.backward()
    check_grads([("v_img", a.grad, i64.grad.numpy())])
    outside = ((img < 0) | (img > 1)).numpy()
    assert np.all(a.grad.cpu().numpy()[outside] == 0.0)


@pytest.mark.gpu
@pytest.mark.parametrize("h,w,lo,hi", [(64, 80, 0.0, 1.0), (45, 61, 0.1, 0.9),
                                       (1356, 2040, 0.0, 1.0)])
def test_clamp_mse_ssim_loss_planar_image_equals_hwc(h, w, lo, hi):
    """The renderer's planar image (an [H, W, 3] view of three planes), read
    clamped in place, gives bit for bit the loss, its parts and the image
    gradient of the same values in a contiguous [H, W, 3] tensor (clamped into
    a copy first); with lo > 0 the zero padding outside the image stays
    unclamped in both."""
    from repo_amd import fused
    print(f"[clamp_mse_ssim planar] {h}x{w} [{lo}, {hi}]", flush=True)
    img = _img(h, w, 21)
    y = torch.rand((1, 3, h, w), generator=torch.Generator().manual_seed(22)).cuda()
    planes = img.permute(2, 0, 1).contiguous().cuda()
    a = planes.permute(1, 2, 0).requires_grad_(True)
    b = img.cuda().contiguous().requires_grad_(True)
    assert a.stride() == (w, 1, h * w) and fused._planes_of(a) is not None
    assert fused._planes_of(b) is None and torch.equal(a, b)
    la, pa = fused.clamp_mse_ssim_loss(a, y, 0.3, lo=lo, hi=hi)
    lb, pb = fused.clamp_mse_ssim_loss(b, y, 0.3, lo=lo, hi=hi)
    assert torch.equal(la, lb) and torch.equal(pa, pb)
    la.backward()
    lb.backward()
    assert torch.equal(a.grad, b.grad)
    outside = ((img < lo) | (img > hi)).numpy()
    assert outside.any() and np.all(a.grad.cpu().numpy()[outside] == 0.0)


@pytest.mark.gpu
def test_render_image_is_contiguous_with_a_planar_copy():
    """The render returns a contiguous [H, W, 3] image, as the reference does
    (cubic_splatting.py:2207-2209), equal to the oracle's; the planar copy
    written by the same launch holds the same values, the fused loss reads it
    (same loss and gradient as on a clone of the image), and an in-place
    change of the image makes the loss read the image itself."""
    import manbo
    from repo_amd import fused, splat, synth
    sc = synth.small_scene(23, P=20, h=64, w=80, rmax=30.0)
    dev = "cuda"
    col = sc.colors.to(dev).requires_grad_(True)
    img = manbo.ops.render_cubic_fill_splat_tilelang(
        sc.cubics_norm.to(dev), sc.seg_offsets.to(dev), col,
        sc.opacities.to(dev), sc.depths.to(dev), sc.img_h, sc.img_w, 16, 16,
        sc.background.to(dev), aa_widths=sc.aa_widths.to(dev), distance_samples=sc.S)
    assert img.shape == (sc.img_h, sc.img_w, 3) and img.is_contiguous()
    assert img.view(-1, 3).shape == (sc.img_h * sc.img_w, 3)
    fw = O.render_forward(sc.cubics_norm.numpy(), sc.seg_offsets.numpy(), sc.colors.numpy(),
                          sc.opacities.numpy(), sc.depths.numpy(), sc.img_h, sc.img_w,
                          sc.background.numpy(), aa_widths=sc.aa_widths.numpy(), S=sc.S)
    np.testing.assert_array_equal(img.detach().cpu().numpy().view(np.int32),
                                  np.ascontiguousarray(fw["out"]).view(np.int32))
    planes = splat.planar_copy_of(img)
    assert planes is not None and torch.equal(planes, img.detach().permute(2, 0, 1))
    assert fused._planes_of(img) is planes
    y = torch.rand((1, 3, sc.img_h, sc.img_w), generator=torch.Generator().manual_seed(4)).cuda()
    la, pa = fused.clamp_mse_ssim_loss(img, y, 0.2)
    ga, = torch.autograd.grad(la, col, retain_graph=True)
    ref = img.detach().clone().requires_grad_(True)
    lb, pb = fused.clamp_mse_ssim_loss(ref, y, 0.2)
    assert torch.equal(la, lb) and torch.equal(pa, pb)
    lb.backward()
    gi, = torch.autograd.grad(la, img, retain_graph=True)
    assert torch.equal(gi, ref.grad)
    # in place: the copy no longer describes the image
    with torch.no_grad():
        img.mul_(0.5)
    assert splat.planar_copy_of(img) is None and fused._planes_of(img) is None
    lc, _ = fused.clamp_mse_ssim_loss(img.detach(), y, 0.2)
    ld, _ = fused.clamp_mse_ssim_loss(img.detach().clone(), y, 0.2)
    assert torch.equal(lc, ld) and not torch.equal(lc, la)
    assert ga.abs().sum() > 0


@pytest.mark.gpu
def test_clamp_mse_ssim_loss_second_backward_through_retained_graph():
    """A second backward through a retained graph reads the SSIM terms the
    forward stored, so it gives the first gradient again (the buffer lives as
    long as the graph node; allocations in between must not disturb it)."""
    from repo_amd import fused
    img = _img(70, 90, 13).cuda().requires_grad_(True)
    y = torch.rand((1, 3, 70, 90), generator=torch.Generator().manual_seed(14)).cuda()
    loss, _ = fused.clamp_mse_ssim_loss(img, y, 0.2)
    loss.backward(retain_graph=True)
    first = img.grad.clone()
    img.grad = None
    junk = [torch.full((1 << 20,), 7.0, device="cuda") for _ in range(8)]  # reuse freed blocks
    loss.backward()
    del junk
    assert torch.equal(img.grad, first)
