"""MSE / SSIM / PSNR on the GPU vs float64 restatements (metric.py:64-273).

Tolerances: losses within 1e-5 relative; gradients within 1e-4 of the largest
reference gradient (the GPU sums in fp32, the reference in float64).
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O

SHAPES = [(1, 3, 37, 53), (2, 3, 40, 50), (1, 3, 512, 768), (1, 3, 1356, 2040)]


def _pair(shape, seed):
    g = torch.Generator("cpu").manual_seed(seed)
    x = torch.rand(shape, generator=g)
    y = (x + 0.2 * torch.randn(shape, generator=g)).clamp(0, 1)
    return x, y


@pytest.mark.gpu
@pytest.mark.parametrize("shape", SHAPES)
def test_mse_forward_backward(shape):
    import manbo
    x, y = _pair(shape, 1)
    xd = x.cuda().requires_grad_(True)
    yd = y.cuda().requires_grad_(True)
    loss = manbo.mse_loss_tilelang(xd, yd)
    ref = O.mse(x.numpy(), y.numpy())
    assert abs(float(loss) - ref) <= 1e-5 * ref
    (loss * 3.0).backward()
    n = x.numel()
    s = np.float32(3.0) * np.float32(2.0 / n)
    gref = s * (x.numpy() - y.numpy())
    np.testing.assert_allclose(xd.grad.cpu().numpy(), gref, rtol=1e-6, atol=1e-12)
    np.testing.assert_array_equal(yd.grad.cpu().numpy(), -xd.grad.cpu().numpy())


@pytest.mark.gpu
def test_mse_repeated_calls_deterministic():
    import manbo
    x, y = _pair((1, 3, 64, 64), 2)
    vals = [float(manbo.mse_loss_tilelang(x.cuda(), y.cuda())) for _ in range(5)]
    assert len(set(vals)) == 1


@pytest.mark.gpu
def test_psnr():
    import manbo
    x, y = _pair((1, 3, 100, 120), 3)
    p = float(manbo.psnr(x.cuda(), y.cuda()))
    ref = 10.0 * np.log10(1.0 / (O.mse(x.numpy(), y.numpy()) + 1e-12))
    assert abs(p - ref) < 1e-4


@pytest.mark.gpu
@pytest.mark.parametrize("shape", SHAPES)
def test_ssim_forward(shape):
    import manbo
    x, y = _pair(shape, 4)
    s = float(manbo.ssim(x.cuda(), y.cuda()))
    ref = float(O.ssim64_separable(x.double(), y.double()))
    assert abs(s - ref) <= 1e-5 * abs(ref), (s, ref)
    one = float(manbo.ssim(x.cuda(), x.cuda()))
    assert abs(one - 1.0) < 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize("shape", SHAPES[2:])
def test_ssim_backward_full_frame(shape):
    """The SSIM gradient at the benchmark's frame sizes against float64
    autograd of the separable restatement, per tensor and per element."""
    import manbo
    from helpers import check_grads
    print(f"[ssim backward] {shape}", flush=True)
    x, y = _pair(shape, 9)
    xd = x.cuda().requires_grad_(True)
    s = manbo.ssim(xd, y.cuda())
    (2.0 * s).backward()
    x64 = x.double().requires_grad_(True)
    r = O.ssim64_separable(x64, y.double())
    (2.0 * r).backward()
    assert abs(float(s) - float(r)) <= 1e-5 * abs(float(r))
    check_grads([("v_x", xd.grad, x64.grad.numpy())])


@pytest.mark.gpu
@pytest.mark.parametrize("win", [7, 11])
def test_ssim_backward(win):
    import manbo
    x, y = _pair((1, 3, 96, 128), 5)
    xd = x.cuda().requires_grad_(True)
    s = manbo.ssim(xd, y.cuda(), win_size=win)
    (2.0 * s).backward()
    x64 = x.double().requires_grad_(True)
    r = O.ssim_torch64(x64, y.double(), win_size=win)
    (2.0 * r).backward()
    got = xd.grad.cpu().numpy().astype(np.float64)
    ref = x64.grad.numpy()
    err = np.abs(got - ref).max() / np.abs(ref).max()
    assert err <= 1e-4, err
    assert abs(float(s) - float(r)) <= 1e-5


@pytest.mark.gpu
def test_ssim_per_image_means():
    import manbo
    x, y = _pair((2, 3, 40, 44), 6)
    per = manbo.ssim(x.cuda(), y.cuda(), size_average=False).cpu().numpy()
    ref = [float(O.ssim_torch64(x[i:i + 1].double(), y[i:i + 1].double())) for i in range(2)]
    np.testing.assert_allclose(per, ref, rtol=1e-5)


@pytest.mark.gpu
@pytest.mark.parametrize("win,shape", [(15, (2, 3, 70, 90)), (17, (2, 3, 70, 90)),
                                       (25, (1, 3, 64, 97)), (41, (1, 2, 41, 60)),
                                       (17, (1, 3, 512, 768))])
def test_ssim_wide_windows_forward_backward(win, shape):
    """Any odd window (metric.py:231-234 accepts every odd win_size): 15 on
    the tiled kernels, wider ones on the two-pass path, down to a one-row
    SSIM map (win = h); value within 1e-5, gradient per tensor and element
    within 1e-4 of float64 autograd."""
    import manbo
    from helpers import check_grads
    print(f"[ssim wide window] win={win} {shape}", flush=True)
    x, y = _pair(shape, 20 + win)
    xd = x.cuda().requires_grad_(True)
    s = manbo.ssim(xd, y.cuda(), win_size=win, win_sigma=0.2 * win)
    (3.0 * s).backward()
    x64 = x.double().requires_grad_(True)
    r = O.ssim64_separable(x64, y.double(), win_size=win, win_sigma=0.2 * win)
    (3.0 * r).backward()
    assert abs(float(s) - float(r)) <= 1e-5 * abs(float(r)), (float(s), float(r))
    check_grads([("v_x", xd.grad, x64.grad.numpy())])


def _anticorrelated(shape, seed):
    """Pairs whose image 0 has negative per-channel SSIM (y = 1 - x) and the
    others positive, so that nonnegative_ssim's clamp acts."""
    x, y = _pair(shape, seed)
    y[0] = 1.0 - x[0]
    return x, y


@pytest.mark.gpu
@pytest.mark.parametrize("win", [11, 19])
@pytest.mark.parametrize("size_average,nonnegative", [(False, False), (False, True),
                                                      (True, True)])
def test_ssim_per_map_modes(win, size_average, nonnegative):
    """size_average=False and nonnegative_ssim (metric.py:262-273) from one
    launch over every (image, channel) map, and their gradients, against the
    float64 restatement."""
    import manbo
    from helpers import check_grads
    x, y = _anticorrelated((3, 3, 48, 60), 30 + win)
    xd = x.cuda().requires_grad_(True)
    got = manbo.ssim(xd, y.cuda(), win_size=win, size_average=size_average,
                     nonnegative_ssim=nonnegative)
    x64 = x.double().requires_grad_(True)
    ref = O.ssim64_separable(x64, y.double(), win_size=win, size_average=size_average,
                             nonnegative=nonnegative)
    assert tuple(got.shape) == tuple(ref.shape)
    np.testing.assert_allclose(got.detach().cpu().double().numpy(), ref.detach().numpy(),
                               rtol=1e-5, atol=1e-6)
    if not size_average:
        assert float(ref[0]) <= 0.0 if nonnegative else float(ref[0]) < 0.0
    wts = torch.tensor([0.5, -1.5, 2.0], dtype=torch.float64)[: got.numel()]
    (got.double().cpu().reshape(-1) * wts).sum().backward()
    (ref.reshape(-1) * wts).sum().backward()
    check_grads([("v_x", xd.grad, x64.grad.numpy())])
