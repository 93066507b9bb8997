"""The 2D Gaussian splat path on the GPU (repo_amd/csrc/gaussian.hip through
the C ABI, and manbo.gs_render / GsRenderFunction) against the oracle
(oracle/gs_oracle.c): projection, binning and the forward image bit-exact;
gradients within a scale-aware tolerance (float atomics sum in another
order; the backward divides by 1 - alpha with the hardware reciprocal)."""
from __future__ import annotations

from contextlib import nullcontext

import numpy as np
import pytest
import torch

from helpers import grad_scale_tol
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _scene(seed, n, img_h, img_w, spread=1.1, smin=0.5, smax=8.0, omin=0.05, omax=1.0):
    g = torch.Generator("cpu").manual_seed(seed)
    u = lambda *s: torch.rand(s, generator=g)  # noqa: E731
    means = (u(n, 2) * 2 - 1) * spread
    scales = smin + u(n, 2) * (smax - smin)
    rot = (u(n) * 2 - 1) * 4.0
    colors = u(n, 3)
    opac = omin + u(n) * (omax - omin)
    return means, scales, rot, colors, opac


def _np(*ts):
    return [t.detach().cpu().numpy() for t in ts]


CASES = {
    # name: (seed, n, H, W, block_x, block_y)
    "small_16x16": (0, 64, 40, 56, 16, 16),
    "module_default_16x8": (1, 300, 72, 100, 16, 8),
    "blocks_8x8": (2, 200, 50, 70, 8, 8),
    "odd_blocks_5x7": (3, 150, 33, 47, 5, 7),
    "blocks_32x32": (4, 400, 96, 130, 32, 32),
    "many_radix_path": (5, 20000, 128, 160, 16, 16),
}


@pytest.mark.parametrize("name", list(CASES))
def test_projection_and_binning_bit_exact(name):
    from repo_amd import gaussian as G
    seed, n, H, W, bx, by = CASES[name]
    means, scales, rot, *_ = _scene(seed, n, H, W)
    print(f"[gs proj/bin] {name} n={n} {H}x{W} block {bx}x{by}", flush=True)
    xys, depths, radii, conics, tiles = G.project_forward(means.cuda(), scales.cuda(), rot.cuda(),
                                                          H, W, bx, by)
    ref = O.gs_project(*_np(means, scales, rot), H, W, bx, by)
    for got, want in zip(_np(xys, depths, radii, conics, tiles), ref):
        np.testing.assert_array_equal(got, want)
    # non-zero depths of both signs (the key is the raw bit pattern)
    dep = torch.tensor(np.random.default_rng(seed).choice(
        np.array([0.0, 0.25, -0.25, 3.0, -0.0], np.float32), n))
    b = G.bin_gaussians(xys, conics, radii, dep.cuda(), H, W, bx, by)
    ids_ref, bins_ref, _ = O.gs_bin(ref[0], ref[3], ref[2], dep.numpy(), H, W, bx, by)
    assert b.num_intersects == len(ids_ref)
    np.testing.assert_array_equal(b.gaussian_ids_sorted.cpu().numpy(), ids_ref)
    np.testing.assert_array_equal(b.tile_bins.cpu().numpy(), bins_ref)
    assert not b.grad_accum.any()


@pytest.mark.parametrize("name", list(CASES)[:5])
def test_raster_forward_bit_exact_and_backward(name):
    from repo_amd import gaussian as G
    seed, n, H, W, bx, by = CASES[name]
    means, scales, rot, colors, opac = _scene(seed, n, H, W)
    print(f"[gs raster] {name}", flush=True)
    xys, depths, radii, conics, _ = O.gs_project(*_np(means, scales, rot), H, W, bx, by)
    ids, bins, _ = O.gs_bin(xys, conics, radii, depths, H, W, bx, by)
    bg = np.array([0.1, 0.5, 0.9], np.float32)
    c, o = colors.numpy(), opac.numpy()
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    rec = G.pack_records(dev(xys), dev(conics), dev(c), dev(o))
    out, fT, fi = G.rasterize_forward(dev(ids), dev(bins), rec, dev(bg), H, W, bx, by)
    r_out, r_T, r_i = O.gs_raster_forward(ids, bins, xys, conics, c, o, bg, H, W, bx, by)
    np.testing.assert_array_equal(out.cpu().numpy(), r_out)
    np.testing.assert_array_equal(fT.cpu().numpy(), r_T)
    np.testing.assert_array_equal(fi.cpu().numpy(), r_i)

    rng = np.random.default_rng(seed + 100)
    v_out = rng.standard_normal((H, W, 3)).astype(np.float32)
    v_alpha = rng.standard_normal((H, W)).astype(np.float32)
    meta = (rng.random(n) < 0.7).astype(np.int32)
    for va, mt in ((None, None), (v_alpha, meta[ids])):
        contrib = torch.zeros((n, 3), device="cuda")
        isect = torch.zeros((len(ids),), device="cuda")
        got = G.rasterize_backward(dev(ids), dev(bins), rec, dev(bg), H, W, bx, by, fT, fi,
                                   dev(v_out), None if va is None else dev(va),
                                   intersect_meta_sorted=None if mt is None else dev(mt),
                                   curve_contrib_rgb=contrib, curve_isect_contrib=isect)
        want = O.gs_raster_backward(ids, bins, xys, conics, c, o, bg, H, W, bx, by, r_T, r_i,
                                    v_out, v_out_alpha=va, intersect_meta=mt)
        for k, (gv, wv) in enumerate(zip(list(got) + [contrib, isect],
                                         list(want[:4]) + [want[4], want[5]])):
            ok, rel = grad_scale_tol(gv.cpu().numpy(), wv, rtol=2e-4)
            assert ok, (name, k, rel)
        if mt is not None:
            off = np.zeros(n, bool)
            off[ids[mt == 0]] = True
            on = np.zeros(n, bool)
            on[ids[mt != 0]] = True
            only_off = off & ~on
            assert (got[0].cpu().numpy()[only_off] == 0).all()


def test_project_backward_matches_oracle():
    from repo_amd import gaussian as G
    n, H, W = 3000, 90, 120
    means, scales, rot, *_ = _scene(9, n, H, W)
    xys, depths, radii, conics, _ = O.gs_project(*_np(means, scales, rot), H, W, 16, 16)
    rng = np.random.default_rng(4)
    v_xy = rng.standard_normal((n, 2)).astype(np.float32)
    v_conic = rng.standard_normal((n, 3)).astype(np.float32) * 10
    meta = (rng.random(n) < 0.5).astype(np.int32) * rng.integers(1, 3, n).astype(np.int32)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    for mt in (None, meta):
        got = G.project_backward(scales.cuda(), rot.cuda(), dev(radii), dev(conics), dev(v_xy),
                                 dev(v_conic), H, W, gaussian_meta=None if mt is None else dev(mt),
                                 with_cov2d=True)
        want = O.gs_project_backward(scales.numpy(), rot.numpy(), radii, conics, v_xy, v_conic,
                                     H, W, gaussian_meta=mt)
        for k, (gv, wv) in enumerate(zip(got, want)):
            ok, rel = grad_scale_tol(gv.cpu().numpy(), wv, rtol=1e-5)
            assert ok, (k, rel)


def test_reference_layout_map_to_intersects():
    import manbo
    n, H, W, bx, by = 500, 64, 96, 16, 8
    means, scales, rot, *_ = _scene(12, n, H, W)
    tb = ((W + bx - 1) // bx, (H + by - 1) // by, 1)
    xys, depths, radii, conics, tiles = manbo.ops.project_gaussians_2d_scale_rot_forward_tilelang(
        means.cuda(), scales.cuda(), rot.cuda(), H, W, tb, block_x=bx, block_y=by)
    dep = torch.linspace(-1, 1, n).cuda()
    cum = torch.cumsum(tiles, 0, dtype=torch.int32)
    I = int(cum[-1])
    keys, gids = manbo.ops.map_gaussian_to_intersects_tilelang(
        n, I, xys, dep, radii, cum, tb, block_x=bx, block_y=by, conics=conics)
    rects = O.gs_rects(*_np(xys, conics, radii), bx, by, tb[0], tb[1])
    rk, ri = O.gs_map_intersects(rects, dep.cpu().numpy(), tb[0])
    np.testing.assert_array_equal(keys.cpu().numpy(), rk)
    np.testing.assert_array_equal(gids.cpu().numpy(), ri)
    # isotropic variant: the radius box on both axes
    iso = np.stack([(radii.cpu().numpy() > 0).astype(np.float32)] * 3, 1) * 0
    rects_iso = O.gs_rects(xys.cpu().numpy(), iso, radii.cpu().numpy(), bx, by, tb[0], tb[1])
    area = ((rects_iso[:, 2] - rects_iso[:, 0]) * (rects_iso[:, 3] - rects_iso[:, 1]))
    cum_iso = torch.from_numpy(np.cumsum(area).astype(np.int32)).cuda()
    keys_i, gids_i = manbo.ops.map_gaussian_to_intersects_tilelang(
        n, int(area.sum()), xys, dep, radii, cum_iso, tb, block_x=bx, block_y=by)
    rk, ri = O.gs_map_intersects(rects_iso, dep.cpu().numpy(), tb[0])
    np.testing.assert_array_equal(keys_i.cpu().numpy(), rk)
    np.testing.assert_array_equal(gids_i.cpu().numpy(), ri)
    # and the tile bins of the sorted keys equal the fused binning's
    ks, order = torch.sort(keys, stable=True)
    bins = manbo.ops.get_tile_bin_edges_tilelang(I, ks, num_tiles=tb[0] * tb[1], compact=True)
    from repo_amd import gaussian as G
    b = G.bin_gaussians(xys, conics, radii, dep, H, W, bx, by)
    assert torch.equal(bins, b.tile_bins)
    assert torch.equal(gids[order], b.gaussian_ids_sorted)


def _oracle_chain(means, scales, rot, colors, opac, bg, H, W, bx, by, v_out, depths=None,
                  gmeta=None):
    xys, dep0, radii, conics, _ = O.gs_project(means, scales, rot, H, W, bx, by)
    dep = dep0 if depths is None else depths
    ids, bins, _ = O.gs_bin(xys, conics, radii, dep, H, W, bx, by)
    out, fT, fi = O.gs_raster_forward(ids, bins, xys, conics, colors, opac, bg, H, W, bx, by)
    mt = None if gmeta is None else gmeta[ids]
    v_xy, v_conic, v_rgb, v_op, contrib, isect = O.gs_raster_backward(
        ids, bins, xys, conics, colors, opac, bg, H, W, bx, by, fT, fi, v_out, intersect_meta=mt)
    _, v_mean, v_scale, v_rot = O.gs_project_backward(scales, rot, radii, conics, v_xy, v_conic,
                                                      H, W, gaussian_meta=gmeta)
    return out, (v_mean, v_scale, v_rot, v_rgb, v_op), contrib, isect


@pytest.mark.parametrize("bx,by", [(16, 16), (16, 8)])
def test_gs_render_end_to_end(bx, by):
    import manbo
    n, H, W = 500, 80, 112
    means, scales, rot, colors, opac = _scene(21, n, H, W)
    bg = torch.tensor([1.0, 1.0, 1.0])
    ins = [t.cuda().requires_grad_(True) for t in (means, scales, rot, colors, opac)]
    out = manbo.gs_render(*ins, H, W, bx, by, bg.cuda())
    v_out = np.random.default_rng(2).standard_normal((H, W, 3)).astype(np.float32)
    out.backward(torch.from_numpy(v_out).cuda())
    r_out, r_grads, _, _ = _oracle_chain(*_np(means, scales, rot, colors, opac, bg), H, W, bx, by,
                                         v_out)
    np.testing.assert_array_equal(out.detach().cpu().numpy(), r_out)
    for k, (t, want) in enumerate(zip(ins, r_grads)):
        ok, rel = grad_scale_tol(t.grad.cpu().numpy(), want, rtol=2e-4)
        assert ok, (k, rel)


def test_gs_render_process_fn_stages_depth_override_meta_and_contrib():
    import manbo
    n, H, W, bx, by = 300, 64, 80, 16, 8
    means, scales, rot, colors, opac = _scene(33, n, H, W)
    depth = torch.linspace(2.0, 0.5, n)  # reversed order: later Gaussians in front
    gmeta = (torch.arange(n) % 3 != 0).to(torch.int32)
    seen = {}
    state = {}

    def process_fn(stage, payload):
        seen[stage] = sorted(payload.keys())
        if stage == "post_project":
            return {"depths": depth.cuda(), "gaussian_meta": gmeta.cuda()}
        if stage == "pre_backward_rasterize":
            return {"collect_curve_contrib_rgb": True, "collect_curve_isect_contrib": True}
        if stage == "post_backward_rasterize":
            state["contrib"] = payload["curve_contrib_rgb"].clone()
            state["isect"] = payload["curve_isect_contrib"].clone()
        return None

    bg = torch.tensor([0.2, 0.3, 0.4])
    ins = [t.cuda().requires_grad_(True) for t in (means, scales, rot, colors, opac)]
    labels = []
    manbo.set_gs_profile_ctx_factory(lambda lab: (labels.append(lab), nullcontext())[1])
    try:
        out = manbo.gs_render(*ins, H, W, bx, by, bg.cuda(), process_fn,
                              profile_fwd_prefix="t.fwd", profile_bwd_prefix="t.bwd")
        v_out = np.random.default_rng(5).standard_normal((H, W, 3)).astype(np.float32)
        out.backward(torch.from_numpy(v_out).cuda())
    finally:
        manbo.set_gs_profile_ctx_factory(None)
    assert set(seen) == {"post_project", "pre_rasterize", "pre_backward_rasterize",
                         "post_backward_rasterize"}
    assert "gaussian_ids_sorted" in seen["pre_rasterize"]
    assert "intersect_meta_sorted" in seen["post_backward_rasterize"]
    assert "t.fwd.total" in labels and "t.fwd.rast" in labels and "t.bwd.proj" in labels
    r_out, r_grads, r_contrib, r_isect = _oracle_chain(
        *_np(means, scales, rot, colors, opac, bg), H, W, bx, by, v_out,
        depths=depth.numpy(), gmeta=gmeta.numpy())
    np.testing.assert_array_equal(out.detach().cpu().numpy(), r_out)
    for k, (t, want) in enumerate(zip(ins, r_grads)):
        ok, rel = grad_scale_tol(t.grad.cpu().numpy(), want, rtol=2e-4)
        assert ok, (k, rel)
    off = gmeta.numpy() == 0
    assert (ins[0].grad.cpu().numpy()[off] == 0).all()
    assert (ins[1].grad.cpu().numpy()[off] == 0).all()
    ok, rel = grad_scale_tol(state["contrib"].cpu().numpy(), r_contrib, rtol=2e-4)
    assert ok, rel
    ok, rel = grad_scale_tol(state["isect"].cpu().numpy(), r_isect, rtol=2e-4)
    assert ok, rel


def test_gs_render_module_and_no_intersections():
    import manbo
    from manbo.tilelang_renderer import GsRenderModule
    n, H, W = 50, 32, 48
    means, scales, rot, colors, opac = _scene(44, n, H, W)
    m = GsRenderModule(H, W).cuda()
    out = m(means.cuda(), scales.cuda(), rot.cuda(), colors.cuda(), opac.cuda())
    r_out, *_ = _oracle_chain(*_np(means, scales, rot, colors, opac), np.ones(3, np.float32), H, W,
                              16, 8, np.zeros((H, W, 3), np.float32))
    np.testing.assert_array_equal(out.cpu().numpy(), r_out)
    far = torch.full((4, 2), 50.0).cuda()
    with pytest.raises(RuntimeError, match="No intersections"):
        manbo.gs_render(far, torch.ones(4, 2).cuda(), torch.zeros(4).cuda(),
                        torch.ones(4, 3).cuda(), torch.ones(4).cuda(), H, W, 16, 16,
                        torch.ones(3).cuda())


def test_large_scene_sampled_rows_and_properties():
    """A 1024 x 1024 image of 100k Gaussians: rows sampled against the oracle,
    T in (0, 1], final indices inside each tile's range, image =
    contributions + T bg."""
    from repo_amd import gaussian as G
    n, H, W, bx, by = 100000, 1024, 1024, 16, 16
    means, scales, rot, colors, opac = _scene(55, n, H, W, spread=1.0, smin=0.5, smax=6.0)
    print("[gs large] projecting", flush=True)
    xys, depths, radii, conics, _ = G.project_forward(means.cuda(), scales.cuda(), rot.cuda(), H,
                                                      W, bx, by)
    b = G.bin_gaussians(xys, conics, radii, depths, H, W, bx, by)
    bg = torch.tensor([0.5, 0.5, 0.5]).cuda()
    rec = G.pack_records(xys, conics, colors.cuda(), opac.cuda())
    out, fT, fi = G.rasterize_forward(b.gaussian_ids_sorted, b.tile_bins, rec, bg, H, W, bx, by)
    torch.cuda.synchronize()
    T = fT.cpu().numpy()
    assert (T > 0).all() and (T <= 1).all()
    rows = (0, 16)
    mid = (496, 512)
    x_np, q_np, r_np, d_np = _np(xys, conics, radii, depths)
    ids, bins, _ = O.gs_bin(x_np, q_np, r_np, d_np, H, W, bx, by)
    np.testing.assert_array_equal(b.tile_bins.cpu().numpy(), bins)
    for r0, r1 in (rows, mid):
        r_out, r_T, r_i = O.gs_raster_forward(ids, bins, x_np, q_np, colors.numpy(),
                                              opac.numpy(), bg.cpu().numpy(), H, W, bx, by,
                                              rows=(r0, r1))
        np.testing.assert_array_equal(out[r0:r1].cpu().numpy(), r_out[r0:r1])
        np.testing.assert_array_equal(fi[r0:r1].cpu().numpy(), r_i[r0:r1])
