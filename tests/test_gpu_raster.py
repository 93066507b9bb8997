"""Rasterization on the GPU vs the oracle.

Forward (image, final T, final index) is bit-exact: the kernels and the oracle
evaluate the same fp32 expressions.  Backward per-pixel terms are identical
too; only the order of the gradient sums differs (fp32 atomics on the GPU,
float64 in the oracle), hence |got - ref| <= 1e-4 * max|ref| per tensor and
<= 1e-4 |ref| + 1e-6 max|ref| per element.
Large configurations are checked on a band of pixel rows: the oracle
rasterizes only those rows and the GPU backward receives a zero output
gradient elsewhere (a zero output gradient contributes exactly zero).
"""
import numpy as np
import pytest
import torch

from helpers import check_grads, grad_scale_tol, hip_bin, oracle_forward, random_v_out
from oracle import oracle as O
from repo_amd import splat, synth

def _far_coords_scene():
    """Rings whose inner control points of some segments lie millions of pixels
    off the image: their flattened edges reach past +-2^20 px (the crossing
    test's far-edge shortcut does not apply to them) while others stay near."""
    sc = synth.small_scene(5, P=12, h=64, w=96, rmax=30.0)
    cub = sc.cubics_norm.clone()
    half_w = sc.img_w / 2.0
    for k, x in ((1, 5.0e6), (6, -3.0e6), (13, 2.0e6), (30, 1.1e6)):
        cub[k, 1, 0] = x / half_w - 1.0
        cub[k, 2, 0] = -0.5 * x / half_w - 1.0
    sc.cubics_norm = cub
    return sc


def _tiny_width_scene():
    """aa width 1e-4 (the clamp floor): cull distance 0.25 px, hard edges."""
    sc = synth.small_scene(6, P=10, h=64, w=80, rmax=25.0)
    sc.aa_widths = torch.full_like(sc.aa_widths, 1e-4)
    return sc


CASES = {
    "far_coords": (_far_coords_scene, None),
    "tiny_width": (_tiny_width_scene, None),
    "small_fill": (lambda: synth.small_scene(0), None),
    "small_fill_big": (lambda: synth.small_scene(3, P=40, h=100, w=130, rmax=60.0), None),
    "small_stroke": (lambda: synth.small_scene(1, stroke=True), None),
    "small_stroke_big": (lambda: synth.small_scene(4, P=30, h=90, w=120, stroke=True), None),
    "cfg1": (lambda: synth.make_scene(1), None),
    "cfg2": (lambda: synth.make_scene(2), None),
    "cfg3_band": (lambda: synth.make_scene(3), (640, 688)),
    "cfg4_band": (lambda: synth.make_scene(4), (480, 544)),
    "cfg5q_band": (lambda: synth.make_scene(5, scale=0.25), (1000, 1032)),
}


def _bits(a):
    return np.ascontiguousarray(a).view(np.int32)


def _order_runs(order, n):
    """Checks a tile order's layout (8 rows of cap positions, each a run of
    sub-blocks then -1s, every sub-block once) and returns the runs."""
    from repo_amd import _native as N
    cap = int(N.lib().cs_raster_tile_order_elems(n)) // 8
    o = order.cpu().numpy()
    assert o.size == 8 * cap
    runs = []
    for row in o.reshape(8, cap):
        k = int((row >= 0).sum())
        assert (row[:k] >= 0).all() and (row[k:] == -1).all()
        runs.append(row[:k])
    assert np.array_equal(np.sort(np.concatenate(runs)), np.arange(n))
    return runs, cap


def _expected_bounds(cost, n, cap, tile=None):
    """The chunked order's run boundaries restated: with each tile's cost (the
    wave pairs summed, or `tile`) in units of 16 ticks capped at 4095, bnd[k]
    the first tile whose predecessors cost at least floor(total k / 8),
    clamped so that every run holds at most cap tiles."""
    if tile is None:
        tile = cost.reshape(-1, 2).astype(np.uint64).sum(1)
    tile = np.minimum(np.asarray(tile, dtype=np.uint64) >> np.uint64(4), np.uint64(4095))
    csum = np.concatenate([np.zeros(1, np.uint64), np.cumsum(tile, dtype=np.uint64)])
    total = int(csum[-1])
    bnd = [0]
    for k in range(1, 8):
        mark = total * k // 8
        j = int(np.searchsorted(csum, np.uint64(mark), side="left"))
        lo = max(bnd[-1], n - (8 - k) * cap)
        bnd.append(min(max(j, lo), bnd[-1] + cap))
    return bnd + [n]


def _run(name):
    make, rows = CASES[name]
    sc = make()
    b, s = hip_bin(sc)
    out, T, idx = splat.rasterize_forward(b, s.background.float().contiguous())
    fw = oracle_forward(sc, rows)
    return sc, s, b, out, T, idx, fw, rows


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(CASES))
def test_forward_bit_exact(name):
    print(f"[forward] {name}", flush=True)
    sc, s, b, out, T, idx, fw, rows = _run(name)
    r0, r1 = rows if rows else (0, sc.img_h)
    np.testing.assert_array_equal(_bits(out.cpu().numpy()[r0:r1]), _bits(fw["out"][r0:r1]))
    np.testing.assert_array_equal(_bits(T.cpu().numpy()[r0:r1]), _bits(fw["final_T"][r0:r1]))
    np.testing.assert_array_equal(idx.cpu().numpy()[r0:r1], fw["final_idx"][r0:r1])


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(CASES))
def test_backward_matches_oracle(name):
    print(f"[backward] {name}", flush=True)
    sc, s, b, out, T, idx, fw, rows = _run(name)
    v = random_v_out(sc.img_h, sc.img_w)
    if rows:
        v[: rows[0]] = 0
        v[rows[1]:] = 0
    vd = v.cuda()
    v_px, v_col, v_op, v_is2, v_sw = splat.rasterize_backward(b, s.background.float(), T, idx,
                                                              vd)
    widths = torch.clamp(s.aa_widths.float(), min=1e-4).contiguous()
    v_norm, v_aa = splat.backward_finalize(b, v_px, widths, v_is2)
    g = O.render_backward(fw, v.numpy())
    checks = [("v_colors", v_col, g["v_colors"]), ("v_opacities", v_op, g["v_opacities"]),
              ("v_inv_sigma2s", v_is2, g["v_inv_sigma2s"]),
              ("v_cubics_px", v_px, g["v_cubics_px"]),
              ("v_cubics_norm", v_norm, g["v_cubics_norm"]),
              ("v_aa_widths", v_aa, g["v_aa_widths"])]
    if v_sw is not None:
        checks.append(("v_stroke_widths", v_sw, g["v_stroke_widths"]))
    check_grads(checks)


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(CASES))
def test_backward_finalized_matches_oracle(name):
    """cs_rasterize_backward_finalized (the backward with the per-XCD copies'
    reduction and the epilogue in one launch) against the oracle, as the two
    calls it replaces."""
    print(f"[backward finalized] {name}", flush=True)
    sc, s, b, out, T, idx, fw, rows = _run(name)
    v = random_v_out(sc.img_h, sc.img_w)
    if rows:
        v[: rows[0]] = 0
        v[rows[1]:] = 0
    widths = torch.clamp(s.aa_widths.float(), min=1e-4).contiguous()
    v_norm, v_col, v_op, v_aa, v_sw = splat.rasterize_backward_finalized(
        b, s.background.float(), T, idx, v.cuda(), widths)
    g = O.render_backward(fw, v.numpy())
    checks = [("v_colors", v_col, g["v_colors"]), ("v_opacities", v_op, g["v_opacities"]),
              ("v_cubics_norm", v_norm, g["v_cubics_norm"]),
              ("v_aa_widths", v_aa, g["v_aa_widths"])]
    if v_sw is not None:
        checks.append(("v_stroke_widths", v_sw, g["v_stroke_widths"]))
    check_grads(checks)


@pytest.mark.gpu
@pytest.mark.parametrize("S", [2, 8, 16, 33])
def test_accumulate_edge_grads_block(S):
    """_accumulate_edge_grads_to_cubics (cubic_splatting.py:2308-2396) on
    random edge gradients vs the oracle's float64 sums."""
    sc = synth.small_scene(1, P=20, S=S)
    b, _ = hip_bin(sc)
    g = np.random.default_rng(S).standard_normal((b.edges.shape[0], 2, 2)).astype(np.float32)
    v_px, v_norm = splat.accumulate_edge_grads(b, torch.from_numpy(g).cuda().view(-1, 4))
    ref = O.accumulate_edge_grads(g.astype(np.float64), b.nseg, S)
    ok, rel = grad_scale_tol(v_px.cpu().numpy(), ref, rtol=1e-5)
    assert ok, rel
    ref_n = ref * np.array([0.5 * sc.img_w, 0.5 * sc.img_h])
    ok, rel = grad_scale_tol(v_norm.cpu().numpy(), ref_n, rtol=1e-5)
    assert ok, rel


@pytest.mark.gpu
@pytest.mark.parametrize("stroke", [False, True])
def test_autograd_function_end_to_end(stroke):
    """manbo.ops entry points through autograd vs the oracle forward/backward."""
    import manbo
    sc = synth.small_scene(11, P=25, h=80, w=96, rmax=35.0, stroke=stroke)
    dev = "cuda"
    cub = sc.cubics_norm.to(dev).requires_grad_(True)
    col = sc.colors.to(dev).requires_grad_(True)
    op = sc.opacities.to(dev).requires_grad_(True)
    aa = (sc.aa_widths.to(dev) * 1.3).requires_grad_(True)
    dep = sc.depths.to(dev)
    if stroke:
        sw = sc.stroke_widths.to(dev).requires_grad_(True)
        img = manbo.ops.render_cubic_polyline_splat_tilelang(
            cub, sc.seg_offsets.to(dev), col, op, sw, dep, sc.img_h, sc.img_w, 16, 16,
            sc.background.to(dev), aa_widths=aa, distance_samples=sc.S)
    else:
        img = manbo.ops.render_cubic_fill_splat_tilelang(
            cub, sc.seg_offsets.to(dev), col, op, dep, sc.img_h, sc.img_w, 16, 16,
            sc.background.to(dev), aa_widths=aa, distance_samples=sc.S)
    v = random_v_out(sc.img_h, sc.img_w, seed=3)
    img.backward(v.to(dev))
    from helpers import scene_np
    d = scene_np(sc)
    fw = O.render_forward(d["cubics_norm"], d["offs"], d["colors"], d["opacities"], d["depths"],
                          sc.img_h, sc.img_w, d["background"], aa_widths=d["aa_widths"] * 1.3,
                          S=sc.S, stroke_widths=d["stroke_widths"])
    np.testing.assert_array_equal(_bits(img.detach().cpu().numpy()), _bits(fw["out"]))
    g = O.render_backward(fw, v.numpy())
    for key, got, ref in [("cubics", cub.grad, g["v_cubics_norm"]),
                          ("colors", col.grad, g["v_colors"]),
                          ("opacities", op.grad, g["v_opacities"]),
                          ("aa_widths", aa.grad, g["v_aa_widths"])] + (
                             [("stroke", sw.grad, g["v_stroke_widths"])] if stroke else []):
        ok, rel = grad_scale_tol(got.cpu().numpy(), ref)
        assert ok, f"{key}: max error {rel:.3e} of max|ref|"


@pytest.mark.gpu
def test_process_fn_hooks_and_contrib_outputs():
    """pre/post_backward_rasterize hooks (cubic_splatting.py:3014-3094): the
    contribution outputs they request equal the oracle's (per primitive and per
    list entry, cubic_splatting.py:1540-1546, 1617-1638); a hook can replace
    the color gradient."""
    import manbo
    sc = synth.small_scene(2, P=12, h=64, w=64, rmax=25.0)
    dev = "cuda"
    seen = {}

    def hook(stage, payload):
        seen[stage] = dict(payload)
        if stage == "pre_backward_rasterize":
            return {"collect_curve_contrib_rgb": True, "collect_curve_isect_contrib": True}
        return {"v_colors": payload["v_colors"] * 2.0}

    col = sc.colors.to(dev).requires_grad_(True)
    img = manbo.ops.render_cubic_fill_splat_tilelang(
        sc.cubics_norm.to(dev), sc.seg_offsets.to(dev), col, sc.opacities.to(dev),
        sc.depths.to(dev), sc.img_h, sc.img_w, 16, 16, sc.background.to(dev),
        distance_samples=sc.S, process_fn=hook)
    img.backward(torch.ones_like(img))
    post = seen["post_backward_rasterize"]
    contrib = post["curve_contrib_rgb"]
    isect = post["curve_isect_contrib"]
    assert contrib.shape == (12, 3) and isect.shape == post["primitive_ids_sorted"].shape
    fw = oracle_forward(sc)
    g = O.render_backward(fw, np.ones((sc.img_h, sc.img_w, 3), np.float32), contrib=True)
    check_grads([("curve_contrib_rgb", contrib, g["contrib_rgb"]),
                 ("curve_isect_contrib", isect, g["isect_contrib"])])
    # the hook saw the kernel's v_colors and doubled it
    ref = post["v_colors"] * 2.0
    assert torch.allclose(col.grad, ref)


@pytest.mark.gpu
def test_empty_scenes():
    import manbo
    dev = "cuda"
    bg = torch.tensor([0.2, 0.4, 0.6], device=dev)
    empty = torch.zeros((0, 4, 2), device=dev)
    img = manbo.ops.render_cubic_fill_splat_tilelang(
        empty, torch.zeros((1,), dtype=torch.int32, device=dev), torch.zeros((0, 3), device=dev),
        torch.zeros((0,), device=dev), torch.zeros((0,), device=dev), 20, 30, 16, 16, bg)
    assert img.shape == (20, 30, 3) and torch.equal(img, bg.view(1, 1, 3).expand(20, 30, 3))
    # everything off-screen: no intersections, background, None grads
    sc = synth.small_scene(0, P=3)
    cub = (sc.cubics_norm + 10.0).to(dev).requires_grad_(True)
    img = manbo.ops.render_cubic_fill_splat_tilelang(
        cub, sc.seg_offsets.to(dev), sc.colors.to(dev), sc.opacities.to(dev),
        sc.depths.to(dev), sc.img_h, sc.img_w, 16, 16, bg, distance_samples=sc.S)
    assert torch.equal(img, bg.view(1, 1, 3).expand(sc.img_h, sc.img_w, 3))
    img.sum().backward()
    assert cub.grad is None


@pytest.mark.gpu
def test_invalid_offsets_raise():
    import manbo
    sc = synth.small_scene(0, P=3)
    dev = "cuda"
    bad = torch.tensor([0, 4, 3, 12], dtype=torch.int32, device=dev)
    with pytest.raises(ValueError):
        manbo.ops.render_cubic_fill_splat_tilelang(
            sc.cubics_norm.to(dev), bad, sc.colors.to(dev), sc.opacities.to(dev),
            sc.depths.to(dev), sc.img_h, sc.img_w, 16, 16, sc.background.to(dev),
            distance_samples=sc.S)
    short = torch.tensor([0, 4, 8, 11], dtype=torch.int32, device=dev)
    with pytest.raises(ValueError):
        manbo.ops.render_cubic_fill_splat_tilelang(
            sc.cubics_norm.to(dev), short, sc.colors.to(dev), sc.opacities.to(dev),
            sc.depths.to(dev), sc.img_h, sc.img_w, 16, 16, sc.background.to(dev),
            distance_samples=sc.S)


@pytest.mark.gpu
def test_forward_deterministic_and_bounded_cfg3():
    """Full config 3: two runs are bit-identical; T in (0,1], idx inside the
    pixel's tile range, image in [0,1] (colors and background in [0,1])."""
    sc = synth.make_scene(3)
    b, s = hip_bin(sc)
    o1, T1, i1 = splat.rasterize_forward(b, s.background)
    o2, T2, i2 = splat.rasterize_forward(b, s.background)
    assert torch.equal(o1, o2) and torch.equal(T1, T2) and torch.equal(i1, i2)
    assert float(T1.min()) > 0 and float(T1.max()) <= 1.0
    assert float(o1.min()) >= 0.0 and float(o1.max()) <= 1.0 + 1e-6


@pytest.mark.gpu
def test_all_primitives_off_screen():
    """Zero intersections: every tile is empty and the intersection list has no
    entries; the forward returns the background (twice: without and with the
    capacity hint of the previous forward) and the backward yields no grads."""
    import manbo
    print("[off-screen]", flush=True)
    sc = synth.small_scene(2, P=5).to("cuda")
    cub = sc.cubics_norm.clone()
    cub[..., 0] += 6.0
    cub.requires_grad_(True)
    for _ in range(2):
        img = manbo.ops.render_cubic_fill_splat_tilelang(
            cub, sc.seg_offsets, sc.colors, sc.opacities, sc.depths, sc.img_h, sc.img_w, 16, 16,
            sc.background, distance_samples=sc.S)
        torch.cuda.synchronize()
        assert torch.equal(img, sc.background.view(1, 1, 3).expand_as(img))
    img.sum().backward()
    assert cub.grad is None or float(cub.grad.abs().sum()) == 0.0


@pytest.mark.gpu
def test_heavy_first_tile_order_is_a_permutation_and_changes_no_result():
    """cs_raster_tile_order yields a permutation of the tiles; a forward that
    takes tiles in that order is bit-identical to the XCD-order forward, and
    the backward in that order matches within the atomics' rounding."""
    print("[tile order]", flush=True)
    sc = synth.make_scene(2)
    b, s = hip_bin(sc)
    bg = s.background.float().contiguous()
    splat._TILE_ORDERS.clear()
    every = splat.ORDER_EVERY
    splat.ORDER_EVERY = 1                              # a new order from every forward
    out0, T0, idx0 = splat.rasterize_forward(b, bg)   # first forward: makes an order
    first = b.tile_order
    order = first.clone()
    v = random_v_out(sc.img_h, sc.img_w).cuda()
    b.tile_order = None
    g0 = [t.clone() for t in splat.rasterize_backward(b, bg, T0, idx0, v)[:4]]
    n = int(b.tile_bins.shape[0])
    runs, _ = _order_runs(order, n)
    for r in runs:                                     # chunked: contiguous runs
        assert r.size == 0 or np.array_equal(np.sort(r), np.arange(r.min(), r.min() + r.size))
    out1, T1, idx1 = splat.rasterize_forward(b, bg)   # takes `order`
    assert torch.equal(out0, out1) and torch.equal(T0, T1) and torch.equal(idx0, idx1)
    assert b.tile_order is not first                   # each forward makes a new order
    _order_runs(b.tile_order, n)
    splat.ORDER_CHUNKED = False                        # the global layout is a permutation too
    try:
        splat.rasterize_forward(b, bg)
        out2, T2, idx2 = splat.rasterize_forward(b, bg)
    finally:
        splat.ORDER_CHUNKED = True
        splat.ORDER_EVERY = every
    _order_runs(b.tile_order, n)
    assert torch.equal(out0, out2) and torch.equal(idx0, idx2)
    b.grad_accum_clean = False
    g1 = splat.rasterize_backward(b, bg, T1, idx1, v)[:4]
    for a, r in zip(g1, g0):
        ok, err = grad_scale_tol(a.cpu().numpy(), r.cpu().numpy(), rtol=1e-5)
        assert ok, err
    # Between new orders, forwards reuse the last one (and their backward
    # takes it too).
    splat._TILE_ORDERS.clear()
    splat.rasterize_forward(b, bg)
    made = b.tile_order
    for _ in range(splat.ORDER_EVERY - 1):
        out3, _, _ = splat.rasterize_forward(b, bg)
        assert b.tile_order is made
        assert torch.equal(out0, out3)
    splat.rasterize_forward(b, bg)
    assert b.tile_order is not made


@pytest.mark.gpu
@pytest.mark.parametrize("chunked", [1, 0])
def test_tile_order_at_the_largest_tile_count(chunked):
    """A 16384 x 16384 image has 2^20 tiles, the most the kernels accept:
    cs_raster_tile_order takes that count and lays out every tile once (its
    visiting stride stays a bijection), with random per-wave costs; chunked,
    its eight runs are the restated cost-balanced ones."""
    from repo_amd import _native as N
    n = (16384 // 16) ** 2
    g = torch.Generator().manual_seed(5)
    cost = torch.randint(0, 1 << 20, (2 * n,), generator=g, dtype=torch.int32)
    order = torch.full((int(N.lib().cs_raster_tile_order_elems(n)),), -7, dtype=torch.int32,
                       device="cuda")
    N.call("cs_raster_tile_order", cost.cuda().data_ptr(), n, chunked, order.data_ptr(),
           N.stream(order.device))
    runs, cap = _order_runs(order, n)
    if chunked:
        bnd = _expected_bounds(cost.numpy(), n, cap)
        for x in range(8):
            assert np.array_equal(np.sort(runs[x]), np.arange(bnd[x], bnd[x + 1]))
    else:
        assert [r.size for r in runs] == [(n - x + 7) // 8 for x in range(8)]
    assert N.lib().cs_raster_tile_order_elems(1048583) == 0
    with pytest.raises(RuntimeError):
        N.call("cs_raster_tile_order", cost.cuda().data_ptr(), 1048583, chunked,
               order.data_ptr(), N.stream(order.device))


@pytest.mark.gpu
@pytest.mark.parametrize("n", [1, 7, 9, 4096, 10880])
def test_tile_order_runs_balance_cost_within_their_cap(n):
    """Chunked orders cut the tiles into eight runs of about equal cost: with
    the heavy tiles all in the first sixteenth the first runs are short and the
    cap (an eighth of the tiles and an eighth more) bounds the later ones; the
    runs equal the restated boundaries, for tile counts below 8 too."""
    from repo_amd import _native as N
    g = torch.Generator().manual_seed(n)
    cost = torch.randint(1, 50, (2 * n,), generator=g, dtype=torch.int32)
    cost[: 2 * max(1, n // 16)] *= 1000
    order = torch.full((int(N.lib().cs_raster_tile_order_elems(n)),), -7, dtype=torch.int32,
                       device="cuda")
    N.call("cs_raster_tile_order", cost.cuda().data_ptr(), n, 1, order.data_ptr(),
           N.stream(order.device))
    runs, cap = _order_runs(order, n)
    bnd = _expected_bounds(cost.numpy(), n, cap)
    assert all(bnd[x + 1] - bnd[x] <= cap for x in range(8))
    for x in range(8):
        assert np.array_equal(np.sort(runs[x]), np.arange(bnd[x], bnd[x + 1]))
    # Heavy first within a run.
    tile = cost.numpy().reshape(-1, 2).sum(1)
    for r in runs:
        if r.size > 1:
            assert tile[r[0]] >= np.median(tile[r])


@pytest.mark.gpu
def test_averaged_tile_order_costs_and_runs():
    """cs_raster_tile_order_averaged: the costs it writes are the tile's wave
    pair averaged with the previous cost (round half up), the runs are the
    restated ones of those averages, no previous cost gives the plain pair
    sums, and the same buffer for both costs is refused."""
    from repo_amd import _native as N
    n = 10880
    g = torch.Generator().manual_seed(11)
    wave = torch.randint(0, 4000, (2 * n,), generator=g, dtype=torch.int32)
    prev = torch.randint(0, 9000, (n,), generator=g, dtype=torch.int32)
    elems = int(N.lib().cs_raster_tile_order_elems(n))
    order = torch.full((elems,), -7, dtype=torch.int32, device="cuda")
    out = torch.full((n,), -1, dtype=torch.int32, device="cuda")
    wave_d, prev_d = wave.cuda(), prev.cuda()
    st = N.stream(order.device)
    pair = wave.numpy().reshape(-1, 2).astype(np.int64).sum(1)
    N.call("cs_raster_tile_order_averaged", wave_d.data_ptr(), None, out.data_ptr(), n, 1,
           order.data_ptr(), st)
    assert np.array_equal(out.cpu().numpy(), pair)
    N.call("cs_raster_tile_order_averaged", wave_d.data_ptr(), prev_d.data_ptr(),
           out.data_ptr(), n, 1, order.data_ptr(), st)
    want = (prev.numpy().astype(np.int64) + pair + 1) >> 1
    assert np.array_equal(out.cpu().numpy(), want)
    runs, cap = _order_runs(order, n)
    bnd = _expected_bounds(None, n, cap, tile=want)
    for x in range(8):
        assert np.array_equal(np.sort(runs[x]), np.arange(bnd[x], bnd[x + 1]))
        if runs[x].size > 1:
            assert want[runs[x][0]] >= np.median(want[runs[x]])
    with pytest.raises(RuntimeError):
        N.call("cs_raster_tile_order_averaged", wave_d.data_ptr(), out.data_ptr(),
               out.data_ptr(), n, 1, order.data_ptr(), st)


@pytest.mark.gpu
def test_event_timer_brackets_the_raster_launches():
    """profiling.EventTimer as the library's profile-context factory: one HIP
    event pair per watched launch, positive device times, nothing recorded for
    unwatched labels, events released by close()."""
    from repo_amd import _native, profiling
    print("[event timer]", flush=True)
    sc = synth.small_scene(3, P=8)
    b, s = hip_bin(sc)
    bg = s.background.float().contiguous()
    timer = profiling.EventTimer({"cubic.fwd.rast": "f", "cubic.bwd.rast": "b"}, reserve=2)
    _native.set_profile_ctx_factory(timer)
    try:
        for _ in range(3):   # one more than reserved: the pool grows
            out, T, idx = splat.rasterize_forward(b, bg)
        b.grad_accum_clean = False
        splat.rasterize_backward(b, bg, T, idx, random_v_out(sc.img_h, sc.img_w).cuda())
    finally:
        _native.set_profile_ctx_factory(None)
    torch.cuda.synchronize()
    assert timer.count("cubic.fwd.rast") == 3 and timer.count("cubic.bwd.rast") == 1
    assert timer.count("cubic.fwd.tile_order") == 0
    assert timer.mean_ms("cubic.fwd.rast") > 0 and timer.mean_ms("cubic.bwd.rast") > 0
    timer.close()
    assert timer.count("cubic.fwd.rast") == 0


@pytest.mark.gpu
def test_widths_below_floor_match_the_clamped_widths():
    """aa_widths under 1e-4 render as 1e-4 (the reference clamps them before
    its kernels, cubic_splatting.py:3207): bit-identical images for raw and
    pre-clamped widths; with widths that require a gradient, the clamped
    entries receive zero gradient."""
    import manbo
    print("[width floor]", flush=True)
    sc = synth.small_scene(4, P=8).to("cuda")
    raw = sc.aa_widths.clone()
    raw[::3] = 0.0
    raw[1::3] = 1e-6

    def render(w):
        return manbo.ops.render_cubic_fill_splat_tilelang(
            sc.cubics_norm, sc.seg_offsets, sc.colors, sc.opacities, sc.depths, sc.img_h,
            sc.img_w, 16, 16, sc.background, aa_widths=w, distance_samples=sc.S)

    a = render(raw)
    b = render(torch.clamp(raw, min=1e-4))
    assert torch.equal(a, b)
    wg = raw.clone().requires_grad_(True)
    img = render(wg)
    assert torch.equal(img, a)
    img.square().sum().backward()
    low = raw < 1e-4
    assert float(wg.grad[low].abs().max()) == 0.0
    assert float(wg.grad[~low].abs().max()) > 0.0


@pytest.mark.gpu
def test_count_overflow_redo_keeps_backward_consistent():
    """A forward whose intersection count exceeds the capacity hint rebuilds
    the lists and re-rasterizes into new buffers (including the raster log);
    the backward must use the second forward's log.  Small shapes set a small
    hint, shapes enlarged 30x about their centroids overflow it: the image is
    bit-identical and the gradients match (atomics order) a run without a hint."""
    import manbo
    print("[overflow redo]", flush=True)
    sc = synth.small_scene(8, P=40, h=512, w=512, rmax=8.0).to("cuda")
    P, nseg = sc.num_primitives, sc.cubics_norm.shape[0] // sc.num_primitives
    cub = sc.cubics_norm.view(P, nseg, 4, 2)
    centre = cub.mean(dim=(1, 2), keepdim=True)
    big = (centre + 30.0 * (cub - centre)).reshape(-1, 4, 2).contiguous()
    wgt = random_v_out(sc.img_h, sc.img_w).cuda()
    redo = []
    orig = splat.resolve_binned

    def spy(b):
        r = orig(b)
        redo.append(r)
        return r

    def run(c0):
        c = c0.clone().requires_grad_(True)
        col = sc.colors.clone().requires_grad_(True)
        img = manbo.ops.render_cubic_fill_splat_tilelang(
            c, sc.seg_offsets, col, sc.opacities, sc.depths, sc.img_h, sc.img_w, 16, 16,
            sc.background, distance_samples=sc.S)
        (img * wgt).sum().backward()
        return img.detach(), c.grad, col.grad

    splat._CAPACITY_HINTS.clear()
    splat.resolve_binned = spy
    try:
        run(sc.cubics_norm)
        img1, gc1, gk1 = run(big)
    finally:
        splat.resolve_binned = orig
    assert redo == [False, True], redo
    splat._CAPACITY_HINTS.clear()
    img2, gc2, gk2 = run(big)
    assert torch.equal(img1, img2)
    for a, r in ((gc1, gc2), (gk1, gk2)):
        ok, err = grad_scale_tol(a.cpu().numpy(), r.cpu().numpy(), rtol=1e-5)
        assert ok, err


LOG_CASES = ["small_fill_big", "small_stroke_big", "cfg2", "cfg4_band"]


@pytest.mark.gpu
@pytest.mark.parametrize("name", LOG_CASES)
@pytest.mark.parametrize("pool", ["none", "tiny"])
def test_backward_without_a_complete_raster_log(name, pool):
    """The backward recomputes the geometry of entries the forward did not
    record: with no log at all (pool "none", the forward of the reference-layout
    building blocks) and with a pool that runs full part way (pool "tiny": some
    entries recorded, the rest missing).  Forward bit-exact either way, and the
    gradients match the oracle as with a full log."""
    print(f"[partial log] {name} {pool}", flush=True)
    make, rows = CASES[name]
    sc = make()
    b, s = hip_bin(sc)
    bg = s.background.float().contiguous()
    if pool == "none":
        out, T, idx = splat.rasterize_forward(b, bg, log=False)
        assert b.log_index is None and b.log_pool is None
    else:
        full_out, _, _ = splat.rasterize_forward(b, bg)
        # Shared blocks for a third of the waves and no per-wave regions.
        nbytes = 16 + 2048 * max(1, (2 * b.ntiles) // 3)
        out, T, idx = splat.rasterize_forward(b, bg, log_pool_bytes_override=nbytes)
        missing = int((b.log_index == -2).sum())
        print(f"  pool {nbytes} bytes: {missing} entries not recorded", flush=True)
        assert missing > 0
        assert torch.equal(out, full_out)
    fw = oracle_forward(sc, rows)
    r0, r1 = rows if rows else (0, sc.img_h)
    np.testing.assert_array_equal(_bits(out.cpu().numpy()[r0:r1]), _bits(fw["out"][r0:r1]))
    np.testing.assert_array_equal(idx.cpu().numpy()[r0:r1], fw["final_idx"][r0:r1])
    v = random_v_out(sc.img_h, sc.img_w)
    if rows:
        v[: rows[0]] = 0
        v[rows[1]:] = 0
    b.grad_accum_clean = False
    v_px, v_col, v_op, v_is2, v_sw = splat.rasterize_backward(b, bg, T, idx, v.cuda())
    g = O.render_backward(fw, v.numpy())
    checks = [("v_colors", v_col, g["v_colors"]), ("v_opacities", v_op, g["v_opacities"]),
              ("v_inv_sigma2s", v_is2, g["v_inv_sigma2s"]),
              ("v_cubics_px", v_px, g["v_cubics_px"])]
    if v_sw is not None:
        checks.append(("v_stroke_widths", v_sw, g["v_stroke_widths"]))
    check_grads(checks)


@pytest.mark.gpu
def test_raster_log_size_follows_use():
    """The log pool holds what the forward records, not a 1056-byte record per
    (list entry, wave): at config 3 it is a small fraction of that, and the
    regions of the next forward of the scene grow when the shared blocks
    took a noticeable part of the records."""
    sc = synth.make_scene(3)
    b, s = hip_bin(sc)
    bg = s.background.float().contiguous()
    key = (b.device.index, b.mode, b.nprim, b.nseg, b.img_h, b.img_w, b.samples, b.adaptive,
           b.block_x, b.block_y)
    for k in range(3):
        splat.rasterize_forward(b, bg)
        torch.cuda.synchronize()
        cap = int(b.primitive_ids_sorted.numel())
        pool = int(b.log_pool.numel())
        first_shared = 1 + 2 * cap * b.log_units
        shared = 16 * (splat.log_pool_counter(b) - first_shared)
        print(f"[log size] forward {k}: I={b.num_intersects}, {b.log_units} units per entry, "
              f"pool {pool / 2**20:.1f} MiB, shared blocks {shared / 2**20:.2f} MiB", flush=True)
        assert pool < 2 * cap * 1056 // 4
        assert 0 <= shared and 16 * first_shared + shared <= pool
    assert splat._LOG_UNITS.get(key, splat.LOG_FIRST_UNITS_PER_ENTRY) >= b.log_units


@pytest.mark.gpu
def test_render_without_gradients_writes_no_log():
    """A render whose inputs need no gradient (evaluation, psnr) allocates no
    raster log: its peak memory stays below that of a render that records
    one by at least the log's entry index."""
    import manbo
    sc = synth.make_scene(2).to("cuda")
    args = (sc.seg_offsets, sc.colors, sc.opacities, sc.depths, sc.img_h, sc.img_w, 16, 16,
            sc.background)
    kw = dict(fill_rules=sc.fill_rules, aa_widths=sc.aa_widths, distance_samples=sc.S)

    def peak(requires_grad):
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats()
        base = torch.cuda.memory_allocated()
        cub = sc.cubics_norm.clone().requires_grad_(requires_grad)
        img = manbo.ops.render_cubic_fill_splat_tilelang(cub, *args, **kw)
        torch.cuda.synchronize()
        return torch.cuda.max_memory_allocated() - base, img

    peak(False)
    p_no, img_no = peak(False)
    p_yes, img_yes = peak(True)
    b, _ = hip_bin(synth.make_scene(2))
    I = b.num_intersects
    print(f"[no-grad log] peak {p_no} vs {p_yes} bytes (I={I})", flush=True)
    assert p_yes - p_no >= 2 * I * 4
    assert torch.equal(img_no, img_yes.detach())


@pytest.mark.gpu
@pytest.mark.parametrize("stroke", [False, True])
def test_prim_gradient_copies_left_zero_and_equal_direct_atomics(stroke):
    """The backward's per-XCD copies of the per-primitive gradients
    (prim_scratch) are zero again after the call, and the gradients equal
    those of plain atomic additions (prim_scratch NULL) up to fp32 summation
    order."""
    from repo_amd import _native as N
    sc = synth.make_scene(4, scale=0.25) if stroke else synth.make_scene(2)
    print(f"[prim copies] stroke={stroke}", flush=True)
    b, s = hip_bin(sc)
    bg = s.background.float().contiguous()
    out, T, idx = splat.rasterize_forward(b, bg)
    v = random_v_out(sc.img_h, sc.img_w, seed=5).to("cuda")
    grads = splat.rasterize_backward(b, bg, T, idx, v)
    P = b.nprim
    nv = 6 if stroke else 5
    rest = b.grad_accum[b.nseg * 8:]
    n_copies = int(N.lib().cs_raster_prim_scratch_elems(P, b.mode))
    assert int(torch.count_nonzero(rest[nv * P:nv * P + n_copies]).item()) == 0
    # The same backward with plain atomics.
    z = torch.zeros_like(b.grad_accum)
    v_px = z[: b.nseg * 8]
    r = z[b.nseg * 8:]
    N.call("cs_rasterize_backward", b.mode, N.ptr(b.primitive_ids_sorted), b.ptr("tile_bins"),
           b.ptr("edges"), b.ptr("edge_culls"), b.ptr("prim_recs"), N.ptr(bg), b.img_h, b.img_w,
           b.block_x, b.block_y, b.edges_per_segment, N.ptr(T), N.ptr(idx), N.ptr(b.log_index),
           N.ptr(b.log_pool), N.ptr(v), 0, N.ptr(v_px), N.ptr(r), r.data_ptr() + 12 * P,
           r.data_ptr() + 16 * P, r.data_ptr() + 20 * P if stroke else None, None, None, 0,
           None, N.ptr(b.tile_order), N.stream(v.device))
    torch.cuda.synchronize()
    direct = [r[: 3 * P].view(P, 3), r[3 * P: 4 * P], r[4 * P: 5 * P]] + (
        [r[5 * P: 6 * P]] if stroke else [])
    copied = [grads[1], grads[2], grads[3]] + ([grads[4]] if stroke else [])
    for got, ref in zip(copied, direct):
        ok, rel = grad_scale_tol(got.cpu().numpy(), ref.cpu().numpy(), rtol=1e-5)
        assert ok, f"max error {rel:.3e} of max|ref|"
    ok, rel = grad_scale_tol(grads[0].cpu().numpy(), v_px.view(b.nseg, 4, 2).cpu().numpy(),
                             rtol=1e-5)
    assert ok, f"v_cubics_px: max error {rel:.3e} of max|ref|"
