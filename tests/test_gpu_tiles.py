"""Tile sizes other than 16x16: the block_x / block_y of the reference's
render entry points (ops/cubic_splatting.py:2778-2782, exposed by its
trainer as --block-w / --block-h).  At each tile size the binning (lists and
tile_bins), the forward (image, final T, final index into the tile's list)
are bit-exact against the oracle run at the same tile size, and the
gradients are within the elementwise tolerance.  Multiples of 16 take the
16 x 16 sub-block kernels; the others (8x8, 16x8, 8x16, 24x24, 12x12, 8x4)
take the any-size kernels (a lane per pixel)."""
import numpy as np
import pytest
import torch

from helpers import check_grads, random_v_out, scene_np
from oracle import oracle as O
from repo_amd import synth

BLOCKS = [(32, 32), (16, 32), (32, 16), (64, 16), (8, 8), (16, 8), (8, 16), (24, 24), (12, 12),
          (8, 4)]
SCENES = {
    "small_fill": lambda: synth.small_scene(3, P=40, h=100, w=130, rmax=60.0),
    "small_stroke": lambda: synth.small_scene(5, P=30, h=90, w=120, rmax=40.0, stroke=True),
    "cfg2": lambda: synth.make_scene(2),
}


def _bits(a):
    return np.ascontiguousarray(a).view(np.int32)


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(SCENES))
@pytest.mark.parametrize("block", BLOCKS, ids=lambda b: f"{b[0]}x{b[1]}")
def test_tile_size_binning_forward_backward(block, name):
    from repo_amd import splat
    bx, by = block
    print(f"[tile size] {bx}x{by} {name}", flush=True)
    sc = SCENES[name]()
    s = sc.to("cuda")
    mode = splat.MODE_FILL if s.stroke_widths is None else splat.MODE_STROKE
    widths = torch.clamp(s.aa_widths.float(), min=1e-4).contiguous()
    b = splat.bin_primitives(
        s.cubics_norm.contiguous(), s.seg_offsets.to(torch.int32).contiguous(),
        s.colors.contiguous(), s.opacities.contiguous(), s.depths.contiguous(),
        s.fill_rules.to(torch.int32).contiguous() if mode == 0 else None, widths,
        None if s.stroke_widths is None else s.stroke_widths.contiguous(), s.img_h, s.img_w,
        s.S, mode=mode, block_x=bx, block_y=by)
    d = scene_np(sc)
    fw = O.render_forward(d["cubics_norm"], d["offs"], d["colors"], d["opacities"], d["depths"],
                          sc.img_h, sc.img_w, d["background"], fill_rules=d["fill_rules"],
                          aa_widths=d["aa_widths"], S=sc.S, stroke_widths=d["stroke_widths"],
                          block_x=bx, block_y=by, workers=O.default_workers())
    np.testing.assert_array_equal(b.primitive_ids_sorted.cpu().numpy(),
                                  fw["primitive_ids_sorted"])
    np.testing.assert_array_equal(b.tile_bins.cpu().numpy(), fw["tile_bins"])
    out, T, idx = splat.rasterize_forward(b, s.background)
    np.testing.assert_array_equal(_bits(out.cpu().numpy()), _bits(fw["out"]))
    np.testing.assert_array_equal(_bits(T.cpu().numpy()), _bits(fw["final_T"]))
    np.testing.assert_array_equal(idx.cpu().numpy(), fw["final_idx"])
    v = random_v_out(sc.img_h, sc.img_w, seed=17)
    v_px, v_col, v_op, v_is2, v_sw = splat.rasterize_backward(b, s.background, T, idx, v.cuda())
    g = O.render_backward(fw, v.numpy())
    checks = [("v_cubics_px", v_px, g["v_cubics_px"]), ("v_colors", v_col, g["v_colors"]),
              ("v_opacities", v_op, g["v_opacities"]),
              ("v_inv_sigma2s", v_is2, g["v_inv_sigma2s"])]
    if mode == splat.MODE_STROKE:
        checks.append(("v_stroke_widths", v_sw, g["v_stroke_widths"]))
    check_grads(checks)


@pytest.mark.gpu
@pytest.mark.parametrize("block", [(32, 32), (48, 16), (8, 8), (16, 8)],
                         ids=lambda b: f"{b[0]}x{b[1]}")
def test_tile_size_through_the_render_entry_point(block):
    """render_cubic_fill_splat_tilelang with block_x x block_y tiles, through
    autograd, against the oracle at that tile size; the same scene at 16x16
    renders the same image."""
    import manbo
    bx, by = block
    sc = synth.small_scene(11, P=25, h=80, w=96, rmax=35.0)
    dev = "cuda"
    cub = sc.cubics_norm.to(dev).requires_grad_(True)
    col = sc.colors.to(dev).requires_grad_(True)
    op = sc.opacities.to(dev).requires_grad_(True)
    aa = (sc.aa_widths.to(dev) * 1.3).requires_grad_(True)
    args = (sc.seg_offsets.to(dev), col, op, sc.depths.to(dev), sc.img_h, sc.img_w)
    img = manbo.ops.render_cubic_fill_splat_tilelang(cub, *args, bx, by, sc.background.to(dev),
                                                     aa_widths=aa, distance_samples=sc.S)
    v = random_v_out(sc.img_h, sc.img_w, seed=3)
    img.backward(v.to(dev))
    d = scene_np(sc)
    fw = O.render_forward(d["cubics_norm"], d["offs"], d["colors"], d["opacities"], d["depths"],
                          sc.img_h, sc.img_w, d["background"], aa_widths=d["aa_widths"] * 1.3,
                          S=sc.S, block_x=bx, block_y=by)
    np.testing.assert_array_equal(_bits(img.detach().cpu().numpy()), _bits(fw["out"]))
    g = O.render_backward(fw, v.numpy())
    check_grads([("cubics", cub.grad, g["v_cubics_norm"]), ("colors", col.grad, g["v_colors"]),
                 ("opacities", op.grad, g["v_opacities"]), ("aa_widths", aa.grad, g["v_aa_widths"])])
    with torch.no_grad():
        img16 = manbo.ops.render_cubic_fill_splat_tilelang(cub, *args, 16, 16,
                                                           sc.background.to(dev), aa_widths=aa,
                                                           distance_samples=sc.S)
    np.testing.assert_array_equal(_bits(img16.cpu().numpy()), _bits(img.detach().cpu().numpy()))


@pytest.mark.gpu
@pytest.mark.parametrize("method", ["bernstein", "de_casteljau"])
def test_any_tile_stroke_and_adaptive_through_the_entry_points(method):
    """The polyline entry point at 8x8 and the de Casteljau flattening at 16x8,
    through autograd, against the oracle at the same tile size, with the
    contribution outputs of a pre_backward_rasterize hook."""
    import manbo
    dev = "cuda"
    seen = {}

    def hook(stage, payload):
        seen[stage] = payload
        if stage == "pre_backward_rasterize":
            return {"collect_curve_contrib_rgb": True, "collect_curve_isect_contrib": True}
        return None

    if method == "bernstein":
        sc, (bx, by) = SCENES["small_stroke"](), (8, 8)
    else:
        sc, (bx, by) = synth.small_scene(12, P=20, h=72, w=88, rmax=30.0), (16, 8)
    s = sc.to(dev)
    cub = s.cubics_norm.clone().requires_grad_(True)
    col = s.colors.clone().requires_grad_(True)
    if sc.stroke_widths is not None:
        sw = s.stroke_widths.clone().requires_grad_(True)
        img = manbo.ops.render_cubic_polyline_splat_tilelang(
            cub, s.seg_offsets, col, s.opacities, sw, s.depths, sc.img_h, sc.img_w, bx, by,
            s.background, aa_widths=s.aa_widths, distance_samples=sc.S, process_fn=hook)
    else:
        sw = None
        img = manbo.ops.render_cubic_fill_splat_tilelang(
            cub, s.seg_offsets, col, s.opacities, s.depths, sc.img_h, sc.img_w, bx, by,
            s.background, aa_widths=s.aa_widths, distance_samples=sc.S, process_fn=hook,
            flatten_method=method)
    v = random_v_out(sc.img_h, sc.img_w, seed=23)
    img.backward(v.to(dev))
    d = scene_np(sc)
    fw = O.render_forward(d["cubics_norm"], d["offs"], d["colors"], d["opacities"], d["depths"],
                          sc.img_h, sc.img_w, d["background"], fill_rules=d["fill_rules"],
                          aa_widths=d["aa_widths"], S=sc.S, stroke_widths=d["stroke_widths"],
                          block_x=bx, block_y=by, flatten_method=method)
    np.testing.assert_array_equal(_bits(img.detach().cpu().numpy()), _bits(fw["out"]))
    g = O.render_backward(fw, v.numpy(), contrib=True)
    post = seen["post_backward_rasterize"]
    checks = [("cubics", cub.grad, g["v_cubics_norm"]), ("colors", col.grad, g["v_colors"]),
              ("curve_contrib_rgb", post["curve_contrib_rgb"], g["contrib_rgb"]),
              ("curve_isect_contrib", post["curve_isect_contrib"], g["isect_contrib"])]
    if sw is not None:
        checks.append(("stroke", sw.grad, g["v_stroke_widths"]))
    check_grads(checks)


@pytest.mark.gpu
def test_any_tile_reference_layout_entry_points():
    """rasterize_cubic_fill_forward_tilelang / _backward_tilelang with block
    (8, 8, 1) on the oracle's edges and lists: forward bit-exact, gradients
    within tolerance."""
    import manbo
    sc = synth.make_scene(2)
    d = scene_np(sc)
    ob = O.bin_scene(d["cubics_norm"], d["offs"], d["depths"], d["aa_widths"], d["img_h"],
                     d["img_w"], d["S"], block_x=8, block_y=8)
    ids = ob["primitive_ids_sorted"].astype(np.int64)
    peo = ob["prim_edge_offsets"].astype(np.int64)
    ranges = np.stack([peo[ids], peo[ids + 1]], 1).astype(np.int32)
    dev = "cuda"
    pos = ((ob["tbx"], ob["tby"], 1), (8, 8, 1), (sc.img_w, sc.img_h, 1),
           torch.from_numpy(ob["primitive_ids_sorted"]).to(dev),
           torch.from_numpy(ob["tile_bins"]).to(dev), torch.from_numpy(ob["cubics_px"]).to(dev),
           torch.from_numpy(d["offs"]).to(dev), torch.from_numpy(d["colors"]).to(dev),
           torch.from_numpy(d["opacities"]).to(dev), torch.from_numpy(d["fill_rules"]).to(dev),
           torch.from_numpy(d["background"]).to(dev))
    kw = dict(edges_px=torch.from_numpy(ob["edges"]).to(dev),
              isect_edge_ranges=torch.from_numpy(ranges).to(dev),
              inv_sigma2s=torch.from_numpy(ob["inv_sigma2s"]).to(dev))
    out, T, idx = manbo.ops.rasterize_cubic_fill_forward_tilelang(*pos, **kw,
                                                                  distance_samples=sc.S)
    fo, fT, fi = O.raster_forward(ob, d["colors"], d["opacities"], d["background"], sc.img_h,
                                  sc.img_w, fill_rules=d["fill_rules"], block_x=8, block_y=8,
                                  workers=O.default_workers())
    np.testing.assert_array_equal(_bits(out.cpu().numpy()), _bits(fo))
    np.testing.assert_array_equal(_bits(T.cpu().numpy()), _bits(fT))
    np.testing.assert_array_equal(idx.cpu().numpy(), fi)
    v = random_v_out(sc.img_h, sc.img_w, seed=29)
    v_px, v_col, v_op, v_is2 = manbo.ops.rasterize_cubic_fill_backward_tilelang(
        *pos, T, idx, v.cuda(), **kw, distance_samples=sc.S)
    g = O.raster_backward(ob, d["colors"], d["opacities"], d["background"], sc.img_h, sc.img_w,
                          fT, fi, v.numpy(), fill_rules=d["fill_rules"], block_x=8, block_y=8,
                          workers=O.default_workers())
    check_grads([("v_cubics_px", v_px, O.accumulate_edge_grads(g["v_edges"],
                                                               int(d["cubics_norm"].shape[0]),
                                                               sc.S)),
                 ("v_colors", v_col, g["v_colors"]), ("v_opacities", v_op, g["v_opacities"]),
                 ("v_inv_sigma2s", v_is2, g["v_inv_sigma2s"])])
