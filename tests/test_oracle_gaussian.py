"""Pins for the 2D Gaussian oracle (oracle/gs_oracle.c + oracle.py gs_*), the
checker of the Gaussian renderer behind GsRenderFunction
(tilelang_renderer.py:149-490).

The reference holds no tests or fixtures for this path, so every pin is
mathematical: the spec sin/cos against float64; the conic as the inverse of
R diag(s^2) R^T; radii and tile rectangles from eigenvalues and the 3-sigma
box; the tile lists against a brute-force per-tile scan; the forward
against a float64 compositor and closed-form pixels; and the whole backward
chain (raster backward + projection backward) against central differences
of a float64 forward of the same scene."""
from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import oracle as O


def _scene(seed, n=12, img_h=24, img_w=40, spread=0.9, smin=1.0, smax=4.0, omax=0.6):
    rng = np.random.default_rng(seed)
    means = rng.uniform(-spread, spread, (n, 2)).astype(np.float32)
    scales = rng.uniform(smin, smax, (n, 2)).astype(np.float32)
    rot = rng.uniform(-3.0, 3.0, n).astype(np.float32)
    colors = rng.uniform(0.0, 1.0, (n, 3)).astype(np.float32)
    opac = rng.uniform(0.2, omax, n).astype(np.float32)
    bg = np.array([0.3, 0.6, 0.9], np.float32)
    return means, scales, rot, colors, opac, bg, img_h, img_w


def test_sincosf_accuracy_and_special_values():
    x = np.concatenate([np.linspace(-100.0, 100.0, 200001), np.linspace(-1e4, 1e4, 20001),
                        [0.0, -0.0, math.pi / 4, math.pi / 2, math.pi, 1e-30]]).astype(np.float32)
    sn, cs = O.sincosf(x)
    xd = x.astype(np.float64)
    # absolute error within 1.5 ulp of 1 (2^-23) over this range
    assert np.abs(sn - np.sin(xd)).max() < 1.5 * 2.0 ** -23
    assert np.abs(cs - np.cos(xd)).max() < 1.5 * 2.0 ** -23
    s0, c0 = O.sincosf(np.array([0.0, np.nan, np.inf, -np.inf], np.float32))
    assert s0[0] == 0.0 and c0[0] == 1.0
    assert np.isnan(s0[1:]).all() and np.isnan(c0[1:]).all()


def test_projection_closed_forms():
    means, scales, rot, *_ = _scene(1, n=400, img_h=96, img_w=160, smin=0.3, smax=12.0)
    H, W, bx, by = 96, 160, 16, 8
    xys, depths, radii, conics, tiles = O.gs_project(means, scales, rot, H, W, bx, by)
    assert (depths == 0).all()
    c, s = np.cos(rot.astype(np.float64)), np.sin(rot.astype(np.float64))
    sx, sy = scales[:, 0].astype(np.float64), scales[:, 1].astype(np.float64)
    M = np.stack([np.stack([c * sx, s * sy], -1), np.stack([-s * sx, c * sy], -1)], -2)
    cov = M @ np.swapaxes(M, -1, -2)
    vis = radii > 0
    Q = np.zeros((len(rot), 2, 2))
    Q[:, 0, 0], Q[:, 0, 1], Q[:, 1, 0], Q[:, 1, 1] = (conics[:, 0], conics[:, 1], conics[:, 1],
                                                       conics[:, 2])
    eye = np.einsum("nij,njk->nik", Q[vis], cov[vis])
    assert np.abs(eye - np.eye(2)).max() < 2e-4
    # centre: the normalized [-1, 1] frame mapped to pixels
    np.testing.assert_allclose(xys[vis, 0], 0.5 * W * (means[vis, 0].astype(np.float64) + 1),
                               rtol=1e-6, atol=1e-4)
    # radius = ceil(3 sqrt(largest eigenvalue)), the eigenvalue gap floored at sqrt(0.1)
    lam = np.linalg.eigvalsh(cov)
    b = 0.5 * (lam[:, 0] + lam[:, 1])
    half_gap = np.sqrt(np.maximum(0.1, (0.5 * (lam[:, 1] - lam[:, 0])) ** 2))
    r64 = 3.0 * np.sqrt(b + half_gap)
    near_int = np.abs(r64 - np.round(r64)) < 1e-3
    ok = vis & ~near_int
    assert (radii[ok] == np.ceil(r64[ok])).all()
    # tile rectangle = tiles meeting the 3-sigma box of the covariance
    sdx, sdy = 3.0 * np.sqrt(cov[:, 0, 0]), 3.0 * np.sqrt(cov[:, 1, 1])
    cx, cy = xys[:, 0].astype(np.float64), xys[:, 1].astype(np.float64)
    tbx, tby = O.tile_bounds(H, W, bx, by)
    lo_x, hi_x = (cx - sdx) / bx, (cx + sdx) / bx + 1
    lo_y, hi_y = (cy - sdy) / by, (cy + sdy) / by + 1
    box = np.stack([np.clip(np.trunc(lo_x), 0, tbx), np.clip(np.trunc(lo_y), 0, tby),
                    np.clip(np.trunc(hi_x), 0, tbx), np.clip(np.trunc(hi_y), 0, tby)], 1)
    edge = np.stack([lo_x, lo_y, hi_x, hi_y], 1)
    near = (np.abs(edge - np.round(edge)) < 1e-3).any(1)
    rects = O.gs_rects(xys, conics, radii, bx, by, tbx, tby)
    area = (box[:, 2] - box[:, 0]) * (box[:, 3] - box[:, 1])
    ok = vis & ~near
    assert ok.sum() > 300
    assert (rects[ok] == box[ok]).all()
    assert (tiles[ok] == area[ok]).all()
    # Gaussians whose box misses the image are dropped entirely
    dropped = (radii == 0)
    assert (tiles[dropped] == 0).all() and (xys[dropped] == 0).all() and (conics[dropped] == 0).all()


def test_projection_drops_offscreen_and_degenerate():
    means = np.array([[0.0, 0.0], [5.0, 5.0], [0.0, 0.0]], np.float32)
    scales = np.array([[2.0, 3.0], [2.0, 3.0], [0.0, 3.0]], np.float32)
    rot = np.zeros(3, np.float32)
    xys, _, radii, conics, tiles = O.gs_project(means, scales, rot, 32, 32, 16, 16)
    assert radii[0] > 0 and tiles[0] > 0
    assert radii[1] == 0 and tiles[1] == 0          # centre far outside the image
    assert radii[2] == 0 and (conics[2] == 0).all()  # zero scale: det == 0


def test_tile_lists_match_brute_force():
    means, scales, rot, _, _, _, H, W = _scene(2, n=60, img_h=40, img_w=72, smin=0.5, smax=9.0)
    bx, by = 8, 16
    xys, depths, radii, conics, _ = O.gs_project(means, scales, rot, H, W, bx, by)
    rng = np.random.default_rng(7)
    depths = rng.choice(np.array([0.0, 0.5, -0.5, 2.0, -0.0], np.float32), len(depths))
    ids, bins, keys = O.gs_bin(xys, conics, radii, depths, H, W, bx, by)
    tbx, tby = O.tile_bounds(H, W, bx, by)
    rects = O.gs_rects(xys, conics, radii, bx, by, tbx, tby)
    bits = depths.view(np.uint32)
    for t in range(tbx * tby):
        tx, ty = t % tbx, t // tbx
        mine = [g for g in range(len(depths))
                if rects[g, 0] <= tx < rects[g, 2] and rects[g, 1] <= ty < rects[g, 3]]
        mine.sort(key=lambda g: (int(bits[g]), g))
        s, e = bins[t]
        if not mine:
            assert s == 0 and e == 0
        else:
            assert list(ids[s:e]) == mine, t
    assert (np.diff(keys) >= 0).all()


def _forward64(ids, bins, xys, conics, colors, opac, bg, H, W, bx, by, cap=0.999):
    """Float64 front-to-back compositing of the same lists (independent of the
    C oracle): returns out [H,W,3] and the index of the last contribution."""
    tbx = (W + bx - 1) // bx
    out = np.zeros((H, W, 3))
    last = np.zeros((H, W), np.int64)
    for i in range(H):
        for j in range(W):
            t = (i // by) * tbx + j // bx
            T, acc = 1.0, np.zeros(3)
            for e in range(bins[t, 0], bins[t, 1]):
                g = ids[e]
                d = xys[g] - np.array([j, i], np.float64)
                q = conics[g]
                sigma = 0.5 * (q[0] * d[0] ** 2 + q[2] * d[1] ** 2) + q[1] * d[0] * d[1]
                if sigma < 0:
                    continue
                a = min(cap, opac[g] * math.exp(-sigma))
                if a < 1.0 / 255.0:
                    continue
                acc += colors[g] * a * T
                T *= 1.0 - a
                last[i, j] = e
                if T <= 1e-4:
                    break
            out[i, j] = acc + T * bg
    return out, last


def test_forward_matches_float64_compositor():
    means, scales, rot, colors, opac, bg, H, W = _scene(3, n=20, omax=1.0)
    bx, by = 16, 8
    xys, depths, radii, conics, _ = O.gs_project(means, scales, rot, H, W, bx, by)
    ids, bins, _ = O.gs_bin(xys, conics, radii, depths, H, W, bx, by)
    out, fT, fi = O.gs_raster_forward(ids, bins, xys, conics, colors, opac, bg, H, W, bx, by)
    ref, last = _forward64(ids, bins, xys.astype(np.float64), conics.astype(np.float64),
                           colors.astype(np.float64), opac.astype(np.float64),
                           bg.astype(np.float64), H, W, bx, by)
    assert np.abs(out - ref).max() < 2e-5
    assert (fi == last).mean() > 0.995


def test_forward_closed_form_pixels():
    # One Gaussian centred on pixel (5, 7): its alpha there is the opacity
    # (capped at 0.999); pixels of tiles it does not reach show the background.
    H, W = 16, 48
    xys = np.array([[7.0, 5.0]], np.float32)
    conics = np.array([[0.5, 0.0, 0.5]], np.float32)
    colors = np.array([[0.2, 0.4, 0.8]], np.float32)
    bg = np.array([1.0, 0.5, 0.0], np.float32)
    radii = np.array([6], np.int32)
    for o, a in ((0.7, 0.7), (1.0, np.float32(0.999))):
        opac = np.array([o], np.float32)
        ids, bins, _ = O.gs_bin(xys, conics, radii, np.zeros(1, np.float32), H, W, 16, 16)
        out, fT, fi = O.gs_raster_forward(ids, bins, xys, conics, colors, opac, bg, H, W, 16, 16)
        np.testing.assert_allclose(out[5, 7], a * colors[0] + (1 - a) * bg, rtol=1e-6)
        assert fT[5, 7] == np.float32(1.0) - np.float32(a)
        assert (out[:, 32:] == bg).all() and (fT[:, 32:] == 1).all() and (fi[:, 32:] == 0).all()


def _cov64(scales, rot):
    c, s = np.cos(rot), np.sin(rot)
    M = np.stack([np.stack([c * scales[:, 0], s * scales[:, 1]], -1),
                  np.stack([-s * scales[:, 0], c * scales[:, 1]], -1)], -2)
    return M @ np.swapaxes(M, -1, -2)


def _chain64(params, fixed, off_base=None):
    """Float64 projection + compositing of the fixed lists, as a function of
    (means, scales, rot, colors, opac).  With off_base (the off-diagonal
    covariance at the base point), the off-diagonal entry moves twice as far
    as the parameters move it: off_base + 2 (cov_xy - off_base)."""
    means, scales, rot, colors, opac = params
    ids, bins, bg, H, W, bx, by = fixed
    cov = _cov64(scales, rot)
    if off_base is not None:
        off = off_base + 2.0 * (cov[:, 0, 1] - off_base)
        cov[:, 0, 1] = off
        cov[:, 1, 0] = off
    Q = np.linalg.inv(cov)
    conics = np.stack([Q[:, 0, 0], Q[:, 0, 1], Q[:, 1, 1]], -1)
    xys = np.stack([0.5 * W * (means[:, 0] + 1), 0.5 * H * (means[:, 1] + 1)], -1)
    return _forward64(ids, bins, xys, conics, colors, opac, bg, H, W, bx, by)


def test_backward_chain_matches_central_differences():
    """Means, colours and opacities: the reference's gradients are the exact
    derivatives.  Scales and rotation: backward2d.py:60-140 weights the
    symmetric off-diagonal gradient g12 = v01 + v10 by 2 again (2 g12
    sigma_x_10, 2 g12 theta_10), so its v_scale / v_rot are the derivatives of
    a forward whose off-diagonal covariance moves twice as far, which is what
    they are checked against here."""
    means, scales, rot, colors, opac, bg, H, W = _scene(4, n=10, img_h=20, img_w=28, spread=0.6,
                                                        smin=1.5, smax=4.0, omax=0.6)
    bx, by = 8, 8
    xys, depths, radii, conics, _ = O.gs_project(means, scales, rot, H, W, bx, by)
    assert (radii > 0).all()
    ids, bins, _ = O.gs_bin(xys, conics, radii, depths, H, W, bx, by)
    out, fT, fi = O.gs_raster_forward(ids, bins, xys, conics, colors, opac, bg, H, W, bx, by)
    v_out = np.random.default_rng(11).standard_normal((H, W, 3)).astype(np.float32)
    v_xy, v_conic, v_rgb, v_op, _, _ = O.gs_raster_backward(
        ids, bins, xys, conics, colors, opac, bg, H, W, bx, by, fT, fi, v_out)
    _, v_mean, v_scale, v_rot = O.gs_project_backward(scales, rot, radii, conics, v_xy, v_conic,
                                                      H, W)
    params = [a.astype(np.float64) for a in (means, scales, rot, colors, opac)]
    fixed = (ids, bins, bg.astype(np.float64), H, W, bx, by)
    base, last = _chain64(params, fixed)
    assert (last == fi).all(), "float64 and fp32 forwards take different decisions"
    analytic = [v_mean, v_scale, v_rot, v_rgb, v_op]
    off_base = _cov64(params[1], params[2])[:, 0, 1].copy()
    vo = v_out.astype(np.float64)
    checked = 0
    for k, (p, g) in enumerate(zip(params, analytic)):
        flat, gflat = p.reshape(-1), np.asarray(g).reshape(-1)
        ob = off_base if k in (1, 2) else None
        for idx in range(flat.size):
            h = 1e-6 * max(1.0, abs(flat[idx]))
            keep = flat[idx]
            flat[idx] = keep + h
            up, lu = _chain64(params, fixed, ob)
            flat[idx] = keep - h
            dn, ld = _chain64(params, fixed, ob)
            flat[idx] = keep
            if not ((lu == last).all() and (ld == last).all()):
                continue  # a contribution decision flips inside the step
            fd = ((up - dn) * vo).sum() / (2 * h)
            assert abs(fd - gflat[idx]) <= 2e-3 * max(1.0, abs(fd)), (k, idx, fd, gflat[idx])
            checked += 1
    assert checked >= 0.95 * sum(p.size for p in params)


def test_backward_conic_gradient_convention():
    # v_conic holds d/dq for the diagonal entries and half of it for the
    # off-diagonal one (rasterize.py:397-399); v_xy is d/d(centre).
    means, scales, rot, colors, opac, bg, H, W = _scene(5, n=6, img_h=16, img_w=16, spread=0.5)
    bx, by = 16, 16
    xys, depths, radii, conics, _ = O.gs_project(means, scales, rot, H, W, bx, by)
    ids, bins, _ = O.gs_bin(xys, conics, radii, depths, H, W, bx, by)
    _, fT, fi = O.gs_raster_forward(ids, bins, xys, conics, colors, opac, bg, H, W, bx, by)
    v_out = np.random.default_rng(3).standard_normal((H, W, 3)).astype(np.float32)
    v_xy, v_conic, *_ = O.gs_raster_backward(ids, bins, xys, conics, colors, opac, bg, H, W, bx,
                                            by, fT, fi, v_out)
    x64, q64 = xys.astype(np.float64), conics.astype(np.float64)
    args = (colors.astype(np.float64), opac.astype(np.float64), bg.astype(np.float64), H, W, bx,
            by)
    vo = v_out.astype(np.float64)
    base, last = _forward64(ids, bins, x64, q64, *args)
    for g in range(len(opac)):
        for comp, scale in ((0, 1.0), (1, 0.5), (2, 1.0)):
            h = 1e-6
            q64[g, comp] += h
            up, lu = _forward64(ids, bins, x64, q64, *args)
            q64[g, comp] -= 2 * h
            dn, ld = _forward64(ids, bins, x64, q64, *args)
            q64[g, comp] += h
            if (lu == last).all() and (ld == last).all():
                fd = ((up - dn) * vo).sum() / (2 * h)
                assert abs(scale * fd - v_conic[g, comp]) <= 2e-3 * max(1.0, abs(fd))
        for comp in range(2):
            h = 1e-6
            x64[g, comp] += h
            up, _ = _forward64(ids, bins, x64, q64, *args)
            x64[g, comp] -= 2 * h
            dn, _ = _forward64(ids, bins, x64, q64, *args)
            x64[g, comp] += h
            fd = ((up - dn) * vo).sum() / (2 * h)
            assert abs(fd - v_xy[g, comp]) <= 2e-3 * max(1.0, abs(fd))


def test_backward_meta_and_contrib_outputs():
    means, scales, rot, colors, opac, bg, H, W = _scene(6, n=8, img_h=16, img_w=24)
    bx, by = 8, 8
    xys, depths, radii, conics, _ = O.gs_project(means, scales, rot, H, W, bx, by)
    ids, bins, _ = O.gs_bin(xys, conics, radii, depths, H, W, bx, by)
    _, fT, fi = O.gs_raster_forward(ids, bins, xys, conics, colors, opac, bg, H, W, bx, by)
    v_out = np.ones((H, W, 3), np.float32)
    full = O.gs_raster_backward(ids, bins, xys, conics, colors, opac, bg, H, W, bx, by, fT, fi,
                                v_out)
    gmeta = (np.arange(len(opac)) % 2).astype(np.int32)
    cut = O.gs_raster_backward(ids, bins, xys, conics, colors, opac, bg, H, W, bx, by, fT, fi,
                               v_out, intersect_meta=gmeta[ids])
    off = gmeta == 0
    assert (cut[0][off] == 0).all() and (cut[1][off] == 0).all()
    np.testing.assert_array_equal(cut[0][~off], full[0][~off])
    for k in (2, 3, 4):
        np.testing.assert_array_equal(cut[k], full[k])
    # per-intersection contributions sum to the per-Gaussian ones
    per_g = np.zeros(len(opac))
    np.add.at(per_g, ids, full[5])
    np.testing.assert_allclose(per_g, full[4].sum(1), rtol=1e-12, atol=1e-12)
    # the background share: sum of contributions + T_final * bg = the image
    out, _, _ = O.gs_raster_forward(ids, bins, xys, conics, colors, opac, bg, H, W, bx, by)
    np.testing.assert_allclose(full[4].sum(), (out - fT[..., None] * bg).sum(), rtol=1e-5)
    # projection backward zeroes what the meta flag turns off
    _, vm, vs, vr = O.gs_project_backward(scales, rot, radii, conics, full[0], full[1], H, W,
                                          gaussian_meta=gmeta)
    assert (vm[off] == 0).all() and (vs[off] == 0).all() and (vr[off] == 0).all()
