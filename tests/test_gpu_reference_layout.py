"""The reference's op-level wrappers that take its own layouts, on the GPU vs
the oracle: rasterize_cubic_fill_forward_tilelang /
rasterize_cubic_fill_backward_tilelang (ops/cubic_splatting.py:2181-2305,
:2572-2747) fed with the oracle's flattened edges, per-intersection edge
ranges and tile bins, and mse_backward_diff_tilelang / reduce_sum_1d_tilelang
(ops/metric.py:344-382).  Forward bit-exact; gradients per tensor and per
element within 1e-4 (fp32 atomics vs float64 sums)."""
import numpy as np
import pytest
import torch

from helpers import check_grads, random_v_out, scene_np
from oracle import oracle as O
from repo_amd import synth

SCENES = {
    "cfg1": lambda: synth.make_scene(1),
    "cfg2": lambda: synth.make_scene(2),
    "small_fill_big": lambda: synth.small_scene(3, P=40, h=100, w=130, rmax=60.0),
}


def _bits(a):
    return np.ascontiguousarray(a).view(np.int32)


def _inputs(sc, flatten_method="bernstein"):
    d = scene_np(sc)
    ob = O.bin_scene(d["cubics_norm"], d["offs"], d["depths"], d["aa_widths"], d["img_h"],
                     d["img_w"], d["S"], flatten_method=flatten_method)
    ids = ob["primitive_ids_sorted"].astype(np.int64)
    peo = ob["prim_edge_offsets"].astype(np.int64)
    ranges = np.stack([peo[ids], peo[ids + 1]], 1).astype(np.int32)
    dev = "cuda"
    t = dict(
        tile_bounds=(ob["tbx"], ob["tby"], 1), block=(16, 16, 1),
        img_size=(sc.img_w, sc.img_h, 1),
        primitive_ids_sorted=torch.from_numpy(ob["primitive_ids_sorted"]).to(dev),
        tile_bins=torch.from_numpy(ob["tile_bins"]).to(dev),
        cubics_px=torch.from_numpy(ob["cubics_px"]).to(dev),
        primitive_seg_offsets=torch.from_numpy(d["offs"]).to(dev),
        colors=torch.from_numpy(d["colors"]).to(dev),
        opacities=torch.from_numpy(d["opacities"]).to(dev),
        fill_rules=torch.from_numpy(d["fill_rules"]).to(dev),
        background=torch.from_numpy(d["background"]).to(dev),
    )
    kw = dict(edges_px=torch.from_numpy(ob["edges"]).to(dev),
              isect_edge_ranges=torch.from_numpy(ranges).to(dev),
              inv_sigma2s=torch.from_numpy(ob["inv_sigma2s"]).to(dev))
    return d, ob, t, kw


def _positional(t):
    return (t["tile_bounds"], t["block"], t["img_size"], t["primitive_ids_sorted"],
            t["tile_bins"], t["cubics_px"], t["primitive_seg_offsets"], t["colors"],
            t["opacities"], t["fill_rules"], t["background"])


@pytest.mark.gpu
@pytest.mark.parametrize("method", ["bernstein", "de_casteljau"])
@pytest.mark.parametrize("name", list(SCENES))
def test_reference_layout_raster_forward_and_backward(name, method):
    import manbo
    print(f"[reference-layout raster] {name} {method}", flush=True)
    sc = SCENES[name]()
    d, ob, t, kw = _inputs(sc, method)
    out, T, idx = manbo.ops.rasterize_cubic_fill_forward_tilelang(*_positional(t), **kw,
                                                                  distance_samples=sc.S)
    fo, fT, fi = O.raster_forward(ob, d["colors"], d["opacities"], d["background"], sc.img_h,
                                  sc.img_w, fill_rules=d["fill_rules"])
    np.testing.assert_array_equal(_bits(out.cpu().numpy()), _bits(fo))
    np.testing.assert_array_equal(_bits(T.cpu().numpy()), _bits(fT))
    np.testing.assert_array_equal(idx.cpu().numpy(), fi)
    v = random_v_out(sc.img_h, sc.img_w, seed=12)
    extra = {}
    if method == "de_casteljau":
        extra = dict(segment_edge_offsets=torch.from_numpy(ob["segment_edge_offsets"]).cuda(),
                     edge_t_starts=torch.from_numpy(ob["edge_t_starts"]).cuda(),
                     edge_t_ends=torch.from_numpy(ob["edge_t_ends"]).cuda())
    v_px, v_col, v_op, v_is2 = manbo.ops.rasterize_cubic_fill_backward_tilelang(
        *_positional(t), T, idx, v.cuda(), **kw, **extra, distance_samples=sc.S,
        flatten_method=method)
    g = O.raster_backward(ob, d["colors"], d["opacities"], d["background"], sc.img_h, sc.img_w,
                          fT, fi, v.numpy(), fill_rules=d["fill_rules"],
                          workers=O.default_workers())
    nseg = int(d["cubics_norm"].shape[0])
    if method == "de_casteljau":
        ref_px = O.accumulate_edge_grads_csr(g["v_edges"], ob["segment_edge_offsets"],
                                             ob["edge_t_starts"], ob["edge_t_ends"], nseg)
    else:
        ref_px = O.accumulate_edge_grads(g["v_edges"], nseg, sc.S)
    check_grads([("v_cubics_px", v_px, ref_px), ("v_colors", v_col, g["v_colors"]),
                 ("v_opacities", v_op, g["v_opacities"]),
                 ("v_inv_sigma2s", v_is2, g["v_inv_sigma2s"])])


@pytest.mark.gpu
def test_reference_layout_raster_widths_contrib_and_empty():
    """aa_widths instead of inv_sigma2s (the reference's own conversion), the
    contribution outputs accumulated in place, and the empty-scene returns."""
    import manbo
    sc = SCENES["cfg2"]()
    d, ob, t, kw = _inputs(sc)
    kw_w = dict(kw)
    kw_w.pop("inv_sigma2s")
    kw_w["aa_widths"] = torch.from_numpy(d["aa_widths"]).cuda()
    out_w, T, idx = manbo.ops.rasterize_cubic_fill_forward_tilelang(*_positional(t), **kw_w)
    out_s, _, _ = manbo.ops.rasterize_cubic_fill_forward_tilelang(*_positional(t), **kw)
    assert torch.equal(out_w, out_s)
    v = random_v_out(sc.img_h, sc.img_w, seed=13).cuda()
    P = sc.num_primitives
    I = int(t["primitive_ids_sorted"].numel())
    crgb = torch.zeros((P, 3), device="cuda")
    cis = torch.zeros((I,), device="cuda")
    manbo.ops.rasterize_cubic_fill_backward_tilelang(
        *_positional(t), T, idx, v, **kw, distance_samples=sc.S, curve_contrib_rgb=crgb,
        curve_isect_contrib=cis)
    assert float(crgb.abs().sum()) > 0 and float(cis.abs().sum()) > 0
    # Against the oracle's contribution statistics (cubic_splatting.py:1540-1546,
    # 1617-1638), per primitive and per list entry.
    g = O.raster_backward(ob, d["colors"], d["opacities"], d["background"], sc.img_h, sc.img_w,
                          T.cpu().numpy(), idx.cpu().numpy(), v.cpu().numpy(),
                          fill_rules=d["fill_rules"], workers=O.default_workers(), contrib=True)
    check_grads([("curve_contrib_rgb", crgb, g["contrib_rgb"]),
                 ("curve_isect_contrib", cis, g["isect_contrib"])])
    t0 = dict(t)
    t0["primitive_ids_sorted"] = t["primitive_ids_sorted"][:0]
    kw0 = dict(kw)
    kw0["isect_edge_ranges"] = kw["isect_edge_ranges"][:0]
    out0, T0, idx0 = manbo.ops.rasterize_cubic_fill_forward_tilelang(*_positional(t0), **kw0)
    assert torch.equal(out0, t["background"].view(1, 1, 3).expand_as(out0))
    assert float(T0.min()) == 1.0 and int(idx0.abs().max()) == 0
    grads = manbo.ops.rasterize_cubic_fill_backward_tilelang(*_positional(t0), T0, idx0, v, **kw0)
    assert all(float(x.abs().sum()) == 0.0 for x in grads)


@pytest.mark.gpu
def test_reference_layout_raster_rejects_inconsistent_inputs():
    """Intersections of one primitive with different edge ranges, and tile bins
    reaching past the intersection list, are refused before any raster
    launch (the raster kernels trust their inputs)."""
    import manbo
    sc = SCENES["cfg1"]()
    d, ob, t, kw = _inputs(sc)
    bad = dict(kw)
    r = kw["isect_edge_ranges"].clone()
    ids = t["primitive_ids_sorted"].cpu().numpy()
    p0 = ids[0]
    second = int(np.nonzero(ids == p0)[0][1])
    r[second, 1] -= 1
    bad["isect_edge_ranges"] = r
    with pytest.raises(ValueError, match="same for every intersection"):
        manbo.ops.rasterize_cubic_fill_forward_tilelang(*_positional(t), **bad)
    tb = dict(t)
    bins = t["tile_bins"].clone()
    bins[0, 1] = int(t["primitive_ids_sorted"].numel()) + 5
    tb["tile_bins"] = bins
    with pytest.raises(ValueError, match="tile_bins"):
        manbo.ops.rasterize_cubic_fill_forward_tilelang(*_positional(tb), **kw)
    # 8x8 tiles are taken, but these tile_bins hold 16x16 tiles' lists
    t8 = dict(t)
    t8["block"] = (8, 8, 1)
    with pytest.raises(ValueError, match="tile_bins"):
        manbo.ops.rasterize_cubic_fill_forward_tilelang(*_positional(t8), **kw)
    with pytest.raises(NotImplementedError):
        t40 = dict(t)
        t40["block"] = (40, 40, 1)
        manbo.ops.rasterize_cubic_fill_forward_tilelang(*_positional(t40), **kw)


@pytest.mark.gpu
@pytest.mark.parametrize("n", [1, 7, 4096, 4097, 1 << 20, 3 * 1356 * 2040 + 5])
def test_mse_backward_diff_and_reduce_sum(n):
    """mse_backward_diff_tilelang: scale * (lhs - rhs) in fp32, bit for bit
    (ops/metric.py:194); reduce_sum_1d_tilelang: the sum within 1e-6 of
    float64 (fp32 partial sums in a fixed order)."""
    import manbo
    g = torch.Generator().manual_seed(n % 1000)
    lhs = torch.randn((n,), generator=g)
    rhs = torch.randn((n,), generator=g)
    scale = 2.0 / 3.7
    got = manbo.ops.mse_backward_diff_tilelang(lhs.cuda().view(1, -1), rhs.cuda().view(1, -1),
                                               scale=scale)
    assert got.shape == (1, n) and got.dtype is torch.float32
    want = np.float32(scale) * (lhs.numpy() - rhs.numpy())
    np.testing.assert_array_equal(_bits(got.cpu().numpy().ravel()), _bits(want))
    x = torch.rand((n,), generator=g) - 0.25
    s = manbo.ops.reduce_sum_1d_tilelang(x.cuda())
    assert s.dim() == 0
    ref = float(x.double().sum())
    assert abs(float(s) - ref) <= 1e-6 * float(x.double().abs().sum())


@pytest.mark.gpu
def test_reduce_sum_edge_sizes():
    import manbo
    one = torch.tensor([3.25], device="cuda")
    assert float(manbo.ops.reduce_sum_1d_tilelang(one)) == 3.25
    with pytest.raises(IndexError):
        manbo.ops.reduce_sum_1d_tilelang(torch.empty((0,), device="cuda"))
