"""Adaptive (de Casteljau) flattening on the GPU vs the oracle
(ops/cubic_splatting.py:1729-1832, 1863-2068, 2399-2487).

Edges, their segment CSR and (segment, t0, t1) records are bit-exact; the
forward raster over them is bit-exact (image, final T, final index); the
backward, which folds each edge gradient into its segment's control points
with the Bernstein weights at t0 / t1, is within 1e-4 of the oracle's float64
sums.  The standalone reference-layout blocks are bit-exact against the
oracle's restatements."""
import numpy as np
import pytest
import torch

from helpers import grad_scale_tol, hip_bin, oracle_forward, random_v_out
from oracle import oracle as O
from repo_amd import blocks, splat, synth

DC = "de_casteljau"


def _rings_big_and_small():
    """Rings whose radii span 2..300 px: leaves from 1 to the 2^D cap."""
    sc = synth.small_scene(9, P=24, h=160, w=200, rmax=300.0, S=24)
    return sc


CASES = {
    "small_fill_S8": lambda: synth.small_scene(0),
    "small_fill_S16": lambda: synth.small_scene(3, P=40, h=100, w=130, rmax=60.0, S=16),
    "small_stroke_S12": lambda: synth.small_scene(1, stroke=True, S=12),
    "radii_S24": _rings_big_and_small,
    "cfg1": lambda: synth.make_scene(1),
    "cfg2": lambda: synth.make_scene(2),
}
BANDS = {"cfg3_band": (lambda: synth.make_scene(3), (640, 688)),
         "cfg4_band": (lambda: synth.make_scene(4), (480, 544))}


def _bits(a):
    return np.ascontiguousarray(a).view(np.int32)


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(CASES))
def test_flatten_records_bit_exact(name):
    print(f"[decas records] {name}", flush=True)
    sc = CASES[name]()
    b, s = hip_bin(sc, flatten_method=DC)
    torch.cuda.synchronize()
    fw = oracle_forward(sc, rows=(0, 1), flatten_method=DC)
    seo = b.seg_edge_offsets.cpu().numpy()
    np.testing.assert_array_equal(seo, fw["segment_edge_offsets"])
    E = int(seo[-1])
    edges = b.edges[:E, :4].cpu().numpy().reshape(-1, 2, 2)
    np.testing.assert_array_equal(_bits(edges), _bits(fw["edges"]))
    aux = b.edge_aux[:E].cpu().numpy()
    seg_of = np.repeat(np.arange(b.nseg), np.diff(seo))
    np.testing.assert_array_equal(aux[:, 0], seg_of)
    np.testing.assert_array_equal(_bits(aux[:, 1].view(np.float32)), _bits(fw["edge_t_starts"]))
    np.testing.assert_array_equal(_bits(aux[:, 2].view(np.float32)), _bits(fw["edge_t_ends"]))
    # per-tile lists do not depend on the flattening
    I = b.num_intersects
    np.testing.assert_array_equal(b.primitive_ids_sorted[:I].cpu().numpy(),
                                  fw["primitive_ids_sorted"])
    np.testing.assert_array_equal(b.tile_bins.cpu().numpy(), fw["tile_bins"])


def _raster_case(name):
    if name in CASES:
        return CASES[name](), None
    make, rows = BANDS[name]
    return make(), rows


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(CASES) + list(BANDS))
def test_raster_forward_bit_exact_and_backward(name):
    print(f"[decas raster] {name}", flush=True)
    sc, rows = _raster_case(name)
    b, s = hip_bin(sc, flatten_method=DC)
    bg = s.background.float().contiguous()
    out, T, idx = splat.rasterize_forward(b, bg)
    fw = oracle_forward(sc, rows, flatten_method=DC)
    r0, r1 = rows if rows else (0, sc.img_h)
    np.testing.assert_array_equal(_bits(out.cpu().numpy()[r0:r1]), _bits(fw["out"][r0:r1]))
    np.testing.assert_array_equal(_bits(T.cpu().numpy()[r0:r1]), _bits(fw["final_T"][r0:r1]))
    np.testing.assert_array_equal(idx.cpu().numpy()[r0:r1], fw["final_idx"][r0:r1])
    v = random_v_out(sc.img_h, sc.img_w)
    if rows:
        v[:r0] = 0
        v[r1:] = 0
    v_px, v_col, v_op, v_is2, v_sw = splat.rasterize_backward(b, bg, T, idx, v.cuda())
    gb = O.render_backward(fw, v.numpy())
    checks = [("cubics_px", v_px, gb["v_cubics_px"]), ("colors", v_col, gb["v_colors"]),
              ("opacities", v_op, gb["v_opacities"]), ("inv_sigma2", v_is2, gb["v_inv_sigma2s"])]
    if v_sw is not None:
        checks.append(("stroke", v_sw, gb["v_stroke_widths"]))
    for nm, got, ref in checks:
        ok, err = grad_scale_tol(got.cpu().numpy(), ref)
        assert ok, (nm, err)


@pytest.mark.gpu
@pytest.mark.parametrize("stroke", [False, True])
def test_render_end_to_end_de_casteljau(stroke):
    """manbo entry points with flatten_method="de_casteljau": image bit-exact,
    gradients w.r.t. normalized control points, colours and widths within 1e-4."""
    import manbo
    print(f"[decas e2e] stroke={stroke}", flush=True)
    sc = synth.small_scene(12, P=16, h=96, w=112, S=16, stroke=stroke, rmax=50.0)
    s = sc.to("cuda")
    cub = s.cubics_norm.clone().requires_grad_(True)
    col = s.colors.clone().requires_grad_(True)
    aa = s.aa_widths.clone().requires_grad_(True)
    if stroke:
        sw = s.stroke_widths.clone().requires_grad_(True)
        img = manbo.ops.render_cubic_polyline_splat_tilelang(
            cub, s.seg_offsets, col, s.opacities, sw, s.depths, s.img_h, s.img_w, 16, 16,
            s.background, aa_widths=aa, distance_samples=s.S, flatten_method="DeCasteljau")
    else:
        img = manbo.ops.render_cubic_fill_splat_tilelang(
            cub, s.seg_offsets, col, s.opacities, s.depths, s.img_h, s.img_w, 16, 16,
            s.background, fill_rules=s.fill_rules, aa_widths=aa, distance_samples=s.S,
            flatten_method="de-casteljau")
    fw = oracle_forward(sc, flatten_method=DC)
    np.testing.assert_array_equal(_bits(img.detach().cpu().numpy()), _bits(fw["out"]))
    v = random_v_out(sc.img_h, sc.img_w, seed=3)
    img.backward(v.cuda())
    gb = O.render_backward(fw, v.numpy())
    checks = [("cubics", cub.grad, gb["v_cubics_norm"]), ("colors", col.grad, gb["v_colors"]),
              ("aa", aa.grad, gb["v_aa_widths"])]
    if stroke:
        checks.append(("stroke", sw.grad, gb["v_stroke_widths"]))
    for nm, got, ref in checks:
        ok, err = grad_scale_tol(got.cpu().numpy().reshape(ref.shape), ref)
        assert ok, (nm, err)


@pytest.mark.gpu
def test_reference_layout_blocks():
    print("[decas blocks]", flush=True)
    g = np.random.default_rng(21)
    cub = (g.uniform(0, 500, (1, 1, 2)) + g.normal(0, 1, (500, 4, 2)) *
           g.uniform(0.3, 150, (500, 1, 1))).astype(np.float32)
    c = torch.from_numpy(cub).cuda()
    for force in (False, True):
        flags = blocks.cubic_adaptive_flatness_flags_tilelang(c, tol_px=0.5, force_flat=force)
        np.testing.assert_array_equal(flags.cpu().numpy(), O.flatness_flags(cub, 0.5, force))
    left, right = blocks.cubic_split_half_tilelang(c)
    l_ref, r_ref = O.split_half(cub)
    np.testing.assert_array_equal(_bits(left.cpu().numpy()), _bits(l_ref))
    np.testing.assert_array_equal(_bits(right.cpu().numpy()), _bits(r_ref))
    offs = torch.tensor([0, 100, 100, 350, 500], dtype=torch.int32, device="cuda")
    for S in (2, 9, 16, 24):
        edges, peo, seo, t0, t1 = blocks.flatten_cubics_to_edges(
            c, offs, distance_samples=S, flatten_method=DC)
        e_ref, seo_ref, t0_ref, t1_ref = O.flatten_decas(cub, S)
        np.testing.assert_array_equal(seo.cpu().numpy(), seo_ref)
        np.testing.assert_array_equal(peo.cpu().numpy(), seo_ref[offs.cpu().numpy()])
        np.testing.assert_array_equal(_bits(edges.cpu().numpy()), _bits(e_ref))
        np.testing.assert_array_equal(_bits(t0.cpu().numpy()), _bits(t0_ref))
        np.testing.assert_array_equal(_bits(t1.cpu().numpy()), _bits(t1_ref))
        v_edges = g.normal(size=e_ref.shape).astype(np.float32)
        v_px = blocks.accumulate_edge_grads_to_cubics(
            torch.from_numpy(v_edges).cuda(), len(cub), distance_samples=S,
            flatten_method=DC, segment_edge_offsets=seo, edge_t_starts=t0, edge_t_ends=t1)
        ok, err = grad_scale_tol(v_px.cpu().numpy(), O.accumulate_edge_grads_csr(
            v_edges.astype(np.float64), seo_ref, t0_ref, t1_ref, len(cub)), rtol=2e-6)
        assert ok, (S, err)
    # Bernstein branch of the same block: the oracle's uniform flattening
    edges, peo, seo, t0, t1 = blocks.flatten_cubics_to_edges(c, offs, distance_samples=16)
    assert t0 is None and t1 is None
    np.testing.assert_array_equal(_bits(edges.cpu().numpy()), _bits(O.flatten(cub, 16)))
    np.testing.assert_array_equal(peo.cpu().numpy(), offs.cpu().numpy() * 15)
