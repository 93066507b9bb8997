"""Seeded random scenes through binning, the raster forward and the raster
backward, against the oracle.

Each scene draws its properties independently, so combinations that the
structured cases hold one at a time meet here. The properties are:
* canvas sides that are not multiples of 16;
* ragged segment counts, including primitives with no segments;
* closed rings, open chains filled, random cubic loops, and rings whose segment
  junctions drifted apart (as Adam moves them);
* primitives partly or wholly off the image;
* degenerate segments (all four control points equal);
* depth ties;
* both fill rules;
* widths from the clamp floor to several pixels;
* opacities up to 1 (alpha capped);
* strokes;
* sample counts S from 2 to 33;
* tile lists longer than 64 entries (every fourth scene).

Bars: the image, T and index are bit-exact. The gradients are within
1e-4 |ref| + 1e-6 max|ref| per element (the order of the fp32 sums differs
from the oracle's float64 ones).
"""
import numpy as np
import pytest
import torch

from helpers import check_grads, hip_bin, oracle_forward, random_v_out, scene_np
from oracle import oracle as O
from repo_amd import splat, synth

SEEDS = list(range(48))


def _fuzz_scene(seed):
    rng = np.random.default_rng(9000 + seed)
    big = seed % 4 == 3        # lists longer than one 64-entry chunk
    h = int(rng.integers(100, 330) if big else rng.integers(17, 140))
    w = int(rng.integers(100, 330) if big else rng.integers(17, 170))
    P = int(rng.integers(100, 260) if big else rng.integers(1, 48))
    stroke = seed % 3 == 2
    S = int(rng.choice([2, 3, 7, 8, 16, 33]))
    counts = rng.integers(1, 7, size=P)
    counts[rng.random(P) < 0.1] = 0           # primitives without segments
    kind = rng.integers(0, 4, size=P)         # 0 ring, 1 open chain, 2 random loop, 3 drifted ring
    segs = []
    for p in range(P):
        n = int(counts[p])
        if n == 0:
            continue
        cx = rng.uniform(-0.3 * w, 1.3 * w)
        cy = rng.uniform(-0.3 * h, 1.3 * h)
        r = float(np.exp(rng.uniform(np.log(0.5), np.log(0.8 * max(h, w)))))
        if stroke or kind[p] == 1:
            # An open chain: a random walk of 3 n + 1 points.
            pts = np.cumsum(rng.normal(0.0, 0.3 * r + 1.0, size=(3 * n + 1, 2)), 0)
            pts += np.array([cx, cy])
        elif kind[p] in (0, 3):
            th = np.sort(rng.uniform(0, 2 * np.pi, size=3 * n))
            pts = np.stack([cx + r * np.cos(th), cy + r * np.sin(th)], 1)
            pts = np.concatenate([pts, pts[:1]], 0)          # closes
        else:
            pts = rng.uniform([cx - r, cy - r], [cx + r, cy + r], size=(3 * n, 2))
            pts = np.concatenate([pts, pts[:1]], 0)
        cub = np.stack([pts[0:-1:3], pts[1::3], pts[2::3], pts[3::3]], 1)
        if kind[p] == 3 and not stroke:
            # A ring whose segments' shared end points moved apart, as an
            # optimizer moves them: mostly by a few ulp, sometimes by up to
            # 0.4 px (which can put the two points in different pixel cells).
            big_drift = rng.random(n) < 0.3
            amt = np.where(big_drift, 0.4, 1e-5)[:, None] * rng.uniform(-1, 1, size=(n, 2))
            cub[:, 3] += amt
        for k in range(n):
            if rng.random() < 0.08:                          # degenerate segment
                cub[k] = cub[k, 0]
                if k + 1 < n:
                    cub[k + 1, 0] = cub[k, 0]
                elif kind[p] != 1 and not stroke:
                    cub[0, 0] = cub[k, 0]
        segs.append(cub)
    cub_px = torch.tensor(np.concatenate(segs, 0) if segs else np.zeros((0, 4, 2)),
                          dtype=torch.float32)
    offs = torch.tensor(np.concatenate([[0], np.cumsum(counts)]), dtype=torch.int32)
    opac = rng.uniform(0.02, 1.0, size=P)
    opac[rng.random(P) < 0.15] = 1.0
    depths = np.round(rng.uniform(0, 1, size=P), 1)                 # ties
    aa = np.exp(rng.uniform(np.log(1e-4), np.log(4.0), size=P))
    aa[rng.random(P) < 0.1] = 1e-4
    sc = synth.Scene(
        cfg=0, img_h=h, img_w=w, S=S, cubics_norm=synth._normalize(cub_px, h, w),
        seg_offsets=offs, colors=torch.tensor(rng.uniform(0, 1, size=(P, 3)), dtype=torch.float32),
        opacities=torch.tensor(opac, dtype=torch.float32),
        depths=torch.tensor(depths, dtype=torch.float32),
        aa_widths=torch.tensor(aa, dtype=torch.float32),
        fill_rules=torch.tensor(rng.integers(0, 2, size=P), dtype=torch.int32),
        background=torch.tensor(rng.uniform(0, 1, size=3), dtype=torch.float32),
        target=torch.zeros(1, 3, h, w),
        stroke_widths=(torch.tensor(rng.uniform(0.5, 5.0, size=P), dtype=torch.float32)
                       if stroke else None))
    return sc


def _bits(a):
    return np.ascontiguousarray(a).view(np.int32)


@pytest.mark.gpu
@pytest.mark.parametrize("seed", SEEDS)
def test_random_scene_forward_bit_exact_and_backward(seed):
    sc = _fuzz_scene(seed)
    print(f"[fuzz] seed {seed}: {sc.img_h}x{sc.img_w}, P={sc.num_primitives}, S={sc.S}, "
          f"stroke={sc.stroke_widths is not None}", flush=True)
    b, s = hip_bin(sc)
    out, T, idx = splat.rasterize_forward(b, s.background.float().contiguous())
    fw = oracle_forward(sc)
    np.testing.assert_array_equal(_bits(out.cpu().numpy()), _bits(fw["out"]))
    np.testing.assert_array_equal(_bits(T.cpu().numpy()), _bits(fw["final_T"]))
    np.testing.assert_array_equal(idx.cpu().numpy(), fw["final_idx"])
    v = random_v_out(sc.img_h, sc.img_w, seed=seed)
    v_px, v_col, v_op, v_is2, v_sw = splat.rasterize_backward(b, s.background.float(), T, idx,
                                                              v.cuda())
    widths = torch.clamp(s.aa_widths.float(), min=1e-4).contiguous()
    v_norm, v_aa = splat.backward_finalize(b, v_px, widths, v_is2)
    g = O.render_backward(fw, v.numpy())
    checks = [("v_colors", v_col, g["v_colors"]), ("v_opacities", v_op, g["v_opacities"]),
              ("v_cubics_norm", v_norm, g["v_cubics_norm"]),
              ("v_aa_widths", v_aa, g["v_aa_widths"])]
    if v_sw is not None:
        checks.append(("v_stroke_widths", v_sw, g["v_stroke_widths"]))
    check_grads(checks)


BLOCKS = [(16, 16), (8, 8), (16, 8), (32, 16), (24, 24), (48, 32)]


@pytest.mark.gpu
@pytest.mark.parametrize("seed", [s for s in SEEDS if s % 3 != 2][:16])
def test_random_fill_scene_through_the_entry_point_at_any_tile_size(seed):
    """The same random fill scenes through render_cubic_fill_splat_tilelang
    with a tile size drawn per scene (multiples of 16 and others): the image
    is bit-exact against the oracle at the same tile size."""
    sc = _fuzz_scene(seed)
    bx, by = BLOCKS[seed % len(BLOCKS)]
    print(f"[fuzz entry] seed {seed}: {sc.img_h}x{sc.img_w}, P={sc.num_primitives}, "
          f"block {bx}x{by}", flush=True)
    s = sc.to("cuda")
    img = splat.render_cubic_fill_splat_tilelang(
        s.cubics_norm, s.seg_offsets, s.colors, s.opacities, s.depths, sc.img_h, sc.img_w, bx,
        by, s.background, fill_rules=s.fill_rules, aa_widths=s.aa_widths,
        distance_samples=sc.S)
    # The oracle at the same tile size: a filled open chain changes pixels
    # left of its vertices, but only in the tiles its rectangle bins it to,
    # so the image depends on the tile size (as the reference's does).
    d = scene_np(sc)
    fw = O.render_forward(d["cubics_norm"], d["offs"], d["colors"], d["opacities"], d["depths"],
                          sc.img_h, sc.img_w, d["background"], fill_rules=d["fill_rules"],
                          aa_widths=d["aa_widths"], S=sc.S, block_x=bx, block_y=by,
                          workers=O.default_workers())
    np.testing.assert_array_equal(_bits(img.detach().cpu().numpy()), _bits(fw["out"]))
