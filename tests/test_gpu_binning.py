"""Binning on the GPU vs the oracle: bit-exact (cubic_splatting.py:2815-2908)."""
import numpy as np
import pytest
import torch

from helpers import hip_bin, scene_np
from oracle import oracle as O
from repo_amd import synth

SCENES = {
    "small_fill": lambda: synth.small_scene(0),
    "small_fill_big": lambda: synth.small_scene(3, P=40, h=100, w=130, rmax=60.0),
    "small_stroke": lambda: synth.small_scene(1, stroke=True),
    # One tile column: no spare tile_scratch word, so the segment scan runs
    # as a launch of its own; and two row segments per tile row.
    "narrow_fill": lambda: synth.small_scene(4, P=12, h=100, w=16, rmax=20.0),
    "wide_fill": lambda: synth.small_scene(5, P=30, h=40, w=1100, rmax=60.0),
    "cfg1": lambda: synth.make_scene(1),
    "cfg2": lambda: synth.make_scene(2),
    "cfg3": lambda: synth.make_scene(3),
    "cfg4": lambda: synth.make_scene(4),
    "cfg5_quarter": lambda: synth.make_scene(5, scale=0.25),
}


def _bits(a):
    a = np.ascontiguousarray(a)
    return a.view(np.int32) if a.dtype == np.float32 else a


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(SCENES))
def test_binning_bit_exact(name):
    print(f"[binning] {name}", flush=True)
    sc = SCENES[name]()
    b, _ = hip_bin(sc)
    d = scene_np(sc)
    ob = O.bin_scene(d["cubics_norm"], d["offs"], d["depths"], d["aa_widths"], d["img_h"],
                     d["img_w"], d["S"], stroke_widths=d["stroke_widths"])
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_bits(b.cubics_px.cpu().numpy()), _bits(ob["cubics_px"]))
    np.testing.assert_array_equal(b.seg_tile_ranges.cpu().numpy(), ob["seg_tile_ranges"])
    np.testing.assert_array_equal(b.prim_tile_ranges.cpu().numpy(), ob["prim_tile_ranges"])
    np.testing.assert_array_equal(b.num_tiles_hit.cpu().numpy(), ob["num_tiles_hit"])
    np.testing.assert_array_equal(_bits(b.edges_px().cpu().numpy()), _bits(ob["edges"]))
    np.testing.assert_array_equal(_bits(b.inv_sigma2s.cpu().numpy()), _bits(ob["inv_sigma2s"]))
    assert b.num_intersects == ob["primitive_ids_sorted"].shape[0]
    np.testing.assert_array_equal(b.primitive_ids_sorted.cpu().numpy(),
                                  ob["primitive_ids_sorted"])
    np.testing.assert_array_equal(b.tile_bins.cpu().numpy(), ob["tile_bins"])


def _with_empty_primitives(sc, runs):
    """Scene sc with runs[i] primitives without segments inserted before
    primitive i (their attributes copied from primitive i)."""
    import dataclasses
    offs = sc.seg_offsets.tolist()
    P = len(offs) - 1
    new_offs, src = [0], []
    for i in range(P):
        for _ in range(runs[i]):
            new_offs.append(offs[i])
            src.append(i)
        new_offs.append(offs[i + 1])
        src.append(i)
    idx = torch.tensor(src)
    return dataclasses.replace(
        sc, seg_offsets=torch.tensor(new_offs, dtype=torch.int32), colors=sc.colors[idx],
        opacities=sc.opacities[idx], depths=sc.depths[idx] + 1e-3 * torch.arange(len(src)),
        aa_widths=sc.aa_widths[idx], fill_rules=sc.fill_rules[idx])


@pytest.mark.gpu
@pytest.mark.parametrize("runs", [(0, 1, 0, 3, 0, 0, 2, 0, 0, 1), (0, 70, 0, 0, 130, 1, 0, 64, 0, 0)])
def test_binning_bit_exact_with_primitives_without_segments(runs):
    """Primitives without segments (repeated offsets), also in runs longer
    than a wave's 64 offsets (where a segment's owner is searched on its
    own): binning bit-exact against the oracle."""
    sc = _with_empty_primitives(synth.small_scene(6, P=10, nseg=4, h=70, w=90, rmax=30.0), runs)
    print(f"[binning empty prims] P={sc.num_primitives}", flush=True)
    b, _ = hip_bin(sc)
    d = scene_np(sc)
    ob = O.bin_scene(d["cubics_norm"], d["offs"], d["depths"], d["aa_widths"], d["img_h"],
                     d["img_w"], d["S"])
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_bits(b.cubics_px.cpu().numpy()), _bits(ob["cubics_px"]))
    np.testing.assert_array_equal(b.seg_tile_ranges.cpu().numpy(), ob["seg_tile_ranges"])
    np.testing.assert_array_equal(b.prim_tile_ranges.cpu().numpy(), ob["prim_tile_ranges"])
    np.testing.assert_array_equal(_bits(b.edges_px().cpu().numpy()), _bits(ob["edges"]))
    np.testing.assert_array_equal(b.primitive_ids_sorted.cpu().numpy(),
                                  ob["primitive_ids_sorted"])
    np.testing.assert_array_equal(b.tile_bins.cpu().numpy(), ob["tile_bins"])


@pytest.mark.gpu
def test_binning_ties_stable_by_primitive_id():
    """Equal depths (the training default, depth = sigmoid(1)) order each tile
    list by primitive id (stable sort of primitive-major emission)."""
    sc = synth.small_scene(5, P=30, h=64, w=64, rmax=30.0)
    sc.depths = torch.full_like(sc.depths, 0.7310586)
    b, _ = hip_bin(sc)
    d = scene_np(sc)
    ob = O.bin_scene(d["cubics_norm"], d["offs"], d["depths"], d["aa_widths"], d["img_h"],
                     d["img_w"], d["S"])
    ids = b.primitive_ids_sorted.cpu().numpy()
    np.testing.assert_array_equal(ids, ob["primitive_ids_sorted"])
    bins = b.tile_bins.cpu().numpy()
    for s, e in bins:
        assert np.all(np.diff(ids[s:e]) > 0)


@pytest.mark.gpu
def test_reference_layout_blocks():
    """project / primitive ranges / map / tile bins with the reference's own
    layouts (int64 keys) match the oracle, and the reference's pipeline on
    those blocks (torch.sort stable) yields the fused path's lists."""
    from repo_amd import blocks
    sc = synth.make_scene(2)
    d = scene_np(sc)
    dev = "cuda"
    P = sc.num_primitives
    w, inv, support = O.prim_params(d["aa_widths"], P)
    counts = np.diff(d["offs"])
    sup_seg = np.repeat(support, counts)
    sw_seg = np.zeros(sup_seg.shape, np.float32)
    tb = (48, 32, 1)
    px, tr, nh = blocks.project_cubics_2d_forward_tilelang(
        sc.cubics_norm.to(dev), torch.from_numpy(sw_seg).to(dev),
        torch.from_numpy(sup_seg).to(dev), sc.img_h, sc.img_w, tb)
    opx, otr, onh = O.project_cubics(d["cubics_norm"], sw_seg, sup_seg, sc.img_h, sc.img_w)
    np.testing.assert_array_equal(_bits(px.cpu().numpy()), _bits(opx))
    np.testing.assert_array_equal(tr.cpu().numpy(), otr)
    np.testing.assert_array_equal(nh.cpu().numpy(), onh)
    ptr, phit = blocks.primitive_tile_ranges_from_segment_tile_ranges(
        tr, sc.seg_offsets.to(dev), tb)
    optr, ophit = O.prim_tile_ranges(otr, d["offs"], 48, 32)
    np.testing.assert_array_equal(ptr.cpu().numpy(), optr)
    np.testing.assert_array_equal(phit.cpu().numpy(), ophit)
    cum = torch.cumsum(phit, 0, dtype=torch.int32)
    keys, ids = blocks.map_cubic_to_intersects_tilelang(ptr, sc.depths.to(dev), cum, tb)
    okeys, oids = O.map_intersects(optr, d["depths"], np.cumsum(ophit), 48)
    np.testing.assert_array_equal(keys.cpu().numpy(), okeys)
    np.testing.assert_array_equal(ids.cpu().numpy(), oids)
    skeys, order = torch.sort(keys, stable=True)
    bins = blocks.get_tile_bin_edges_tilelang(int(keys.numel()), skeys, num_tiles=48 * 32,
                                              compact=True)
    b, _ = hip_bin(sc)
    np.testing.assert_array_equal(bins.cpu().numpy(), b.tile_bins.cpu().numpy())
    np.testing.assert_array_equal(ids[order].cpu().numpy(), b.primitive_ids_sorted.cpu().numpy())
    ranges = blocks.build_fill_isect_edge_ranges(b.primitive_ids_sorted, sc.seg_offsets.to(dev),
                                                 sc.S - 1)
    off_e = d["offs"].astype(np.int64) * (sc.S - 1)
    pid = b.primitive_ids_sorted.cpu().numpy()
    np.testing.assert_array_equal(ranges.cpu().numpy(), np.stack([off_e[pid], off_e[pid + 1]], 1))


@pytest.mark.gpu
@pytest.mark.parametrize("n,bits", [(0, 8), (1, 32), (2, 1), (255, 8), (1000, 32), (4096, 14),
                                    (4097, 14), (8192, 32), (16384, 32), (16385, 32), (100003, 32),
                                    (300001, 17)])
def test_radix_sort_stable(n, bits):
    from repo_amd import _native as N
    g = np.random.default_rng(n + bits)
    hi = min(1 << bits, 1 << 31) if bits < 32 else 1 << 32
    keys = g.integers(0, hi, size=n, dtype=np.uint64).astype(np.uint32)
    keys[: n // 3] = keys[0] if n else 0  # many duplicates
    vals = np.arange(n, dtype=np.int32)
    dev = "cuda"
    k = torch.from_numpy(keys.view(np.int32)).to(dev)
    v = torch.from_numpy(vals).to(dev)
    ka = torch.empty_like(k)
    va = torch.empty_like(v)
    L = N.lib()
    cnt = torch.empty((int(L.cs_radix_counts_elems(n)),), dtype=torch.int32, device=dev)
    tmp = torch.empty((int(L.cs_scan_temp_elems(int(cnt.numel()))),), dtype=torch.int32,
                      device=dev)
    N.call("cs_radix_sort_pairs_u32", N.ptr(k), N.ptr(v), N.ptr(ka), N.ptr(va), n, bits,
           N.ptr(cnt), N.ptr(tmp), N.stream())
    order = np.argsort(keys, kind="stable")
    np.testing.assert_array_equal(v.cpu().numpy(), vals[order])
    np.testing.assert_array_equal(k.cpu().numpy().view(np.uint32), keys[order])


@pytest.mark.gpu
@pytest.mark.parametrize("n", [1, 5, 4096, 4097, 32768, 32769, 1000003])
def test_exclusive_scan(n):
    from repo_amd import _native as N
    g = np.random.default_rng(n)
    x = g.integers(0, 200, size=n).astype(np.int32)
    dev = "cuda"
    xi = torch.from_numpy(x).to(dev)
    out = torch.empty_like(xi)
    tot = torch.empty((1,), dtype=torch.int32, device=dev)
    tmp = torch.empty((int(N.lib().cs_scan_temp_elems(n)),), dtype=torch.int32, device=dev)
    N.call("cs_scan_exclusive_u32", N.ptr(xi), N.ptr(out), n, N.ptr(tmp), N.ptr(tot), N.stream())
    ref = np.concatenate([[0], np.cumsum(x)[:-1]])
    np.testing.assert_array_equal(out.cpu().numpy(), ref)
    assert int(tot.item()) == int(x.sum())


@pytest.mark.gpu
@pytest.mark.parametrize("hint", [0, 1, 17, None, 10 ** 6])
def test_deferred_count_matches_synchronous(hint):
    """bin_primitives with a capacity hint builds the lists before the host
    reads the intersection count; a too-small buffer leaves every tile empty
    until resolve_binned() rebuilds at full size.  Either way the lists, and
    the raster of them, equal the synchronous path's."""
    from repo_amd import splat
    print(f"[deferred] hint={hint}", flush=True)
    sc = synth.small_scene(8, P=24, h=80, w=112, rmax=40.0)
    ref, s = hip_bin(sc)
    bg = s.background.float().contiguous()
    out_ref, T_ref, idx_ref = splat.rasterize_forward(ref, bg)
    widths = torch.clamp(s.aa_widths.float(), min=1e-4).contiguous()
    b = splat.bin_primitives(
        s.cubics_norm.contiguous(), s.seg_offsets.to(torch.int32).contiguous(),
        s.colors.contiguous(), s.opacities.contiguous(), s.depths.contiguous(),
        s.fill_rules.to(torch.int32).contiguous(), widths, None, s.img_h, s.img_w, s.S,
        capacity_hint=hint if hint is not None else ref.num_intersects)
    # The list launch writes the status words to the pinned buffer itself.
    assert b.pending is not None and b.pending.pinned[3] is not None
    out, T, idx = splat.rasterize_forward(b, bg)
    rebuilt = splat.resolve_binned(b)
    cap = hint if hint is not None else ref.num_intersects
    assert rebuilt == (cap < ref.num_intersects)
    if rebuilt:
        out, T, idx = splat.rasterize_forward(b, bg)
    assert b.num_intersects == ref.num_intersects and b.pending is None
    np.testing.assert_array_equal(b.primitive_ids_sorted.cpu().numpy(),
                                  ref.primitive_ids_sorted.cpu().numpy())
    np.testing.assert_array_equal(b.tile_bins.cpu().numpy(), ref.tile_bins.cpu().numpy())
    assert torch.equal(out, out_ref) and torch.equal(T, T_ref) and torch.equal(idx, idx_ref)


@pytest.mark.gpu
def test_deferred_count_reports_invalid_offsets():
    """The status words the list launch writes to pinned memory carry the CSR
    checks too: offsets that decrease, or that end short of the segment count,
    raise when the deferred count is read."""
    from repo_amd import splat
    sc = synth.small_scene(0, P=3)
    s = sc.to("cuda")
    widths = torch.clamp(s.aa_widths.float(), min=1e-4).contiguous()
    for offs in ([0, 4, 3, 12], [0, 4, 8, 11]):
        print(f"[deferred offsets] {offs}", flush=True)
        b = splat.bin_primitives(
            s.cubics_norm.contiguous(), torch.tensor(offs, dtype=torch.int32, device="cuda"),
            s.colors.contiguous(), s.opacities.contiguous(), s.depths.contiguous(),
            s.fill_rules.to(torch.int32).contiguous(), widths, None, s.img_h, s.img_w, s.S,
            capacity_hint=4096)
        assert b.pending is not None and b.pending.pinned[3] is not None
        with pytest.raises(ValueError, match="primitive_seg_offsets"):
            splat.resolve_binned(b)


@pytest.mark.gpu
def test_function_forward_reuses_capacity_hint_across_scene_growth():
    """Repeated renders of one scene shape: the second render grows past the
    first one's buffer hint (rebuild path), the third fits; all bit-exact."""
    import manbo
    from repo_amd import splat
    from helpers import oracle_forward
    splat._CAPACITY_HINTS.clear()
    for k, rmax in enumerate((6.0, 45.0, 44.0)):
        sc = synth.small_scene(9, P=16, h=64, w=96, rmax=rmax)
        s = sc.to("cuda")
        img = manbo.ops.render_cubic_fill_splat_tilelang(
            s.cubics_norm, s.seg_offsets, s.colors, s.opacities, s.depths, s.img_h, s.img_w,
            16, 16, s.background, aa_widths=s.aa_widths, distance_samples=s.S)
        fw = oracle_forward(sc)
        np.testing.assert_array_equal(_bits(img.cpu().numpy()), _bits(fw["out"]))
    assert len(splat._CAPACITY_HINTS) == 1


@pytest.mark.gpu
@pytest.mark.parametrize("S", [2, 3, 5, 8, 9, 16, 17, 33, 64, 65, 80])
@pytest.mark.parametrize("stroke", [False, True])
def test_flatten_sample_counts(S, stroke):
    """Every lane-group size of the lane-per-point flattening (S <= 64) and
    the per-segment kernel above it: edges, tile ranges and lists bit-exact,
    and the forward image (which depends on every edge's cull record and
    every segment record) bit-exact against the oracle."""
    from helpers import oracle_forward
    from repo_amd import splat
    print(f"[flatten S] S={S} stroke={stroke}", flush=True)
    sc = synth.small_scene(11 + S, P=7, h=56, w=72, S=S, stroke=stroke)
    b, s = hip_bin(sc)
    d = scene_np(sc)
    ob = O.bin_scene(d["cubics_norm"], d["offs"], d["depths"], d["aa_widths"], d["img_h"],
                     d["img_w"], d["S"], stroke_widths=d["stroke_widths"])
    out, T, idx = splat.rasterize_forward(b, s.background.float().contiguous())
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_bits(b.cubics_px.cpu().numpy()), _bits(ob["cubics_px"]))
    np.testing.assert_array_equal(b.seg_tile_ranges.cpu().numpy(), ob["seg_tile_ranges"])
    np.testing.assert_array_equal(_bits(b.edges_px().cpu().numpy()), _bits(ob["edges"]))
    np.testing.assert_array_equal(b.primitive_ids_sorted.cpu().numpy(),
                                  ob["primitive_ids_sorted"])
    fw = oracle_forward(sc)
    np.testing.assert_array_equal(_bits(out.cpu().numpy()), _bits(fw["out"]))
    np.testing.assert_array_equal(_bits(T.cpu().numpy()), _bits(fw["final_T"]))
    np.testing.assert_array_equal(idx.cpu().numpy(), fw["final_idx"])


def _crossing_rows_cases():
    """Edge y-ranges for the crossing-row pin: endpoints exactly on pixel-row
    centres (k + 0.5) and one ulp either side, horizontal edges, both
    directions, ranges reaching past the image and far beyond it."""
    f = np.float32
    ys = [f(3.5), f(10.5), np.nextafter(f(3.5), f(0)), np.nextafter(f(3.5), f(9)),
          np.nextafter(f(10.5), f(0)), np.nextafter(f(10.5), f(99)), f(0.5), f(-0.5), f(0.0),
          f(-40.25), f(63.5), f(64.0), f(70.75), f(1e7), f(-1e7), f(3.0e38), f(-3.0e38),
          f(17.2), f(31.999), f(32.0), f(32.5)]
    pairs = [(a, b) for a in ys for b in ys]
    rng = np.random.default_rng(11)
    pairs += [(f(a), f(b)) for a, b in rng.uniform(-20.0, 90.0, size=(2000, 2))]
    pairs += [(f(a), f(a)) for a in rng.uniform(0.0, 64.0, size=50)]
    return np.array(pairs, dtype=np.float32)


@pytest.mark.gpu
def test_edge_cull_crossing_rows_exact():
    """The crossing rows each cull record stores are exactly the pixel rows
    whose centre py = k + 0.5 the raster's crossing test counts, i.e. where
    (y0 <= py) != (y1 <= py) in fp32, and its direction bit says y0 < y1.
    The far-entry winding number relies on both (a row outside the stored
    range must have no crossing, one inside must have one).  Checked by
    brute force over every row a wave of a 64 x 96 image can hold."""
    from repo_amd import raster_ref
    from repo_amd import _native as N
    yy = _crossing_rows_cases()
    E = yy.shape[0]
    dev = "cuda"
    rng = np.random.default_rng(12)
    xs = rng.uniform(-10.0, 100.0, size=(E, 2)).astype(np.float32)
    edges_px = np.stack([np.stack([xs[:, 0], yy[:, 0]], 1), np.stack([xs[:, 1], yy[:, 1]], 1)],
                        1).astype(np.float32)                      # [E, 2, 2]
    H, W = 64, 96
    T = (W // 16) * (H // 16)
    print(f"[cull rows] E={E}", flush=True)
    _, culls, _ = raster_ref.raster_records(
        torch.tensor(edges_px, device=dev), torch.zeros((1,), dtype=torch.int32, device=dev),
        torch.tensor([[0, E]], dtype=torch.int32, device=dev),
        torch.rand((1, 3), device=dev), torch.ones((1,), device=dev),
        torch.ones((1,), device=dev), None,
        torch.zeros((T, 2), dtype=torch.int32, device=dev), H, W)
    q = culls.cpu().numpy()
    cy = q[:, 1]
    lo = (cy.astype(np.int32) << 16) >> 16
    span = cy >> 16
    hi = lo + span - 7          # crossing ranges carry the wave's row extension (8 rows - 1)
    rows = np.arange(0, H + 16, dtype=np.int64)
    py = rows.astype(np.float32) + np.float32(0.5)
    b0 = yy[:, 0:1] <= py[None, :]
    b1 = yy[:, 1:2] <= py[None, :]
    want = b0 != b1
    got = (rows[None, :] >= lo[:, None]) & (rows[None, :] <= hi[:, None])
    bad = np.argwhere(want != got)
    assert bad.size == 0, (f"{bad.shape[0]} (edge, row) mismatches; first: edge {bad[0][0]} "
                           f"y = {yy[bad[0][0]]}, row {rows[bad[0][1]]}")
    up = (q[:, 3] & 2) != 0
    np.testing.assert_array_equal(up, yy[:, 0] < yy[:, 1])
