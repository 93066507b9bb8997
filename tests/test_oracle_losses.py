"""Pins of the oracle's losses (oracle.mse, oracle.gaussian_window_1d,
oracle.ssim_torch64) against closed forms, an independent brute-force loop
and finite differences."""
from __future__ import annotations

import math

import numpy as np
import torch

from oracle import oracle as O


def test_gaussian_window():
    g = O.gaussian_window_1d(11, 1.5).astype(np.float64)
    assert abs(g.sum() - 1.0) < 1e-6
    np.testing.assert_allclose(g, g[::-1], rtol=0, atol=0)
    for k in range(11):
        assert abs(g[k] / g[5] - math.exp(-((k - 5) ** 2) / (2 * 1.5 ** 2))) < 1e-6
    assert int(np.argmax(g)) == 5


def test_mse_closed_form():
    x = np.full((1, 3, 8, 9), 0.75, np.float32)
    y = np.full((1, 3, 8, 9), 0.25, np.float32)
    assert O.mse(x, y) == 0.25
    r = np.random.default_rng(0).standard_normal((2, 3, 5, 7))
    assert abs(O.mse(r, 0 * r) - float(np.mean(r * r))) < 1e-15


def test_ssim_identity_and_constants():
    x = torch.rand((1, 3, 20, 23), dtype=torch.float64, generator=torch.Generator().manual_seed(1))
    assert abs(float(O.ssim_torch64(x, x)) - 1.0) < 1e-12
    a, b = 0.3, 0.8
    xa = torch.full((1, 1, 16, 16), a, dtype=torch.float64)
    yb = torch.full((1, 1, 16, 16), b, dtype=torch.float64)
    c1, c2 = 0.01 ** 2, 0.03 ** 2
    # The window is normalised in fp32 (metric.py:55-59), so its 2D sum s is
    # 1 + O(1e-7): mu = a s, E[x^2] = a^2 s, sigma^2 = a^2 (s - s^2).
    s = float(O.gaussian_window_1d(11, 1.5).astype(np.float64).sum()) ** 2
    v = s - s * s
    expect = (((2 * a * b * s * s + c1) / ((a * a + b * b) * s * s + c1))
              * ((2 * a * b * v + c2) / ((a * a + b * b) * v + c2)))
    assert abs(float(O.ssim_torch64(xa, yb)) - expect) < 1e-12
    # With an exactly normalised window this is the textbook (2ab+c1)/(a^2+b^2+c1).
    assert abs(expect - (2 * a * b + c1) / (a * a + b * b + c1)) < 1e-4


def _ssim_loops(x, y, win=11, sigma=1.5):
    """Scalar loops over the valid window positions (2D window = outer(g, g))."""
    g = O.gaussian_window_1d(win, sigma).astype(np.float64)
    h, w = x.shape
    c1, c2 = 0.01 ** 2, 0.03 ** 2
    vals = []
    for i in range(h - win + 1):
        for j in range(w - win + 1):
            mx = my = exx = eyy = exy = 0.0
            for a in range(win):
                for b in range(win):
                    k = g[a] * g[b]
                    u, v = x[i + a, j + b], y[i + a, j + b]
                    mx += k * u
                    my += k * v
                    exx += k * u * u
                    eyy += k * v * v
                    exy += k * u * v
            sx, sy, sxy = exx - mx * mx, eyy - my * my, exy - mx * my
            vals.append(((2 * mx * my + c1) / (mx * mx + my * my + c1))
                        * ((2 * sxy + c2) / (sx + sy + c2)))
    return float(np.mean(vals))


def test_ssim_brute_force_and_channel_mean():
    rng = np.random.default_rng(3)
    x = rng.random((2, 14, 15))
    y = np.clip(x + 0.2 * rng.standard_normal(x.shape), 0, 1)
    per = [_ssim_loops(x[c], y[c]) for c in range(2)]
    got = float(O.ssim_torch64(torch.from_numpy(x)[None], torch.from_numpy(y)[None]))
    assert abs(got - np.mean(per)) < 1e-12
    # Window offsets: a 7-tap window on a non-square image.
    x7, y7 = x[0, :10, :12], y[0, :10, :12]
    got7 = float(O.ssim_torch64(torch.from_numpy(x7)[None, None], torch.from_numpy(y7)[None, None],
                                win_size=7))
    assert abs(got7 - _ssim_loops(x7, y7, win=7)) < 1e-12


def test_ssim_gradient_finite_differences():
    rng = np.random.default_rng(4)
    x = torch.from_numpy(rng.random((1, 1, 13, 14)))
    y = torch.from_numpy(rng.random((1, 1, 13, 14)))
    xr = x.clone().requires_grad_(True)
    O.ssim_torch64(xr, y).backward()
    h = 1e-6
    for (i, j) in [(0, 0), (6, 7), (12, 13), (3, 10)]:
        xp, xm = x.clone(), x.clone()
        xp[0, 0, i, j] += h
        xm[0, 0, i, j] -= h
        fd = (float(O.ssim_torch64(xp, y)) - float(O.ssim_torch64(xm, y))) / (2 * h)
        assert abs(fd - float(xr.grad[0, 0, i, j])) < 1e-7


def test_separable_ssim_equals_the_2d_window():
    """ssim64_separable (two 1D passes) equals ssim_torch64 (the 2D window
    outer(g, g), itself pinned by the loops above) in value and gradient, for
    odd windows from 3 to 21 on non-square multi-image inputs; a transposed
    pass or a wrong channel split breaks the equality."""
    rng = np.random.default_rng(6)
    for win, shape in ((11, (2, 3, 30, 41)), (7, (1, 3, 19, 25)), (3, (1, 2, 9, 8)),
                       (21, (1, 3, 40, 33)), (15, (2, 1, 24, 30))):
        x = torch.from_numpy(rng.random(shape))
        y = torch.from_numpy(np.clip(x.numpy() + 0.3 * rng.standard_normal(shape), 0, 1))
        a = x.clone().requires_grad_(True)
        b = x.clone().requires_grad_(True)
        va = O.ssim_torch64(a, y, win_size=win)
        vb = O.ssim64_separable(b, y, win_size=win)
        assert abs(float(va) - float(vb)) < 1e-12, win
        va.backward()
        vb.backward()
        assert float((a.grad - b.grad).abs().max()) < 1e-12 * float(a.grad.abs().max()) + 1e-15
        per = O.ssim64_separable(x, y, win_size=win, size_average=False)
        assert per.shape == (shape[0],)
        for i in range(shape[0]):
            assert abs(float(per[i]) - float(O.ssim_torch64(x[i:i + 1], y[i:i + 1],
                                                            win_size=win))) < 1e-12


def test_separable_ssim_nonnegative_clamps_channel_means():
    """nonnegative_ssim clamps each channel's mean at zero before averaging
    (metric.py:266-268): anti-correlated channels read 0, others unchanged."""
    rng = np.random.default_rng(7)
    x = torch.from_numpy(rng.random((1, 2, 20, 20)))
    y = x.clone()
    y[:, 1] = 1.0 - x[:, 1]                       # channel 1 anti-correlated
    per_c = [float(O.ssim64_separable(x[:, k:k + 1], y[:, k:k + 1])) for k in range(2)]
    assert per_c[0] > 0.99 and per_c[1] < 0
    got = float(O.ssim64_separable(x, y, nonnegative=True))
    assert abs(got - 0.5 * per_c[0]) < 1e-12
    assert abs(float(O.ssim64_separable(x, y)) - 0.5 * (per_c[0] + per_c[1])) < 1e-12


def test_bench_cpu_ssim_equals_the_oracle():
    """The shifted-slice SSIM the CPU baseline times computes the oracle's
    SSIM (value and gradient, float64)."""
    import bench
    g = torch.Generator().manual_seed(4)
    x = torch.rand((2, 3, 40, 57), generator=g, dtype=torch.float64, requires_grad=True)
    y = torch.rand((2, 3, 40, 57), generator=g, dtype=torch.float64)
    a = bench.ssim_cpu(x, y)
    (ga,) = torch.autograd.grad(a, x)
    b = O.ssim_torch64(x, y)
    (gb,) = torch.autograd.grad(b, x)
    assert abs(float(a) - float(b)) <= 1e-12
    assert float((ga - gb).abs().max()) <= 1e-12 * float(gb.abs().max()) + 1e-15
