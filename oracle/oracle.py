"""CPU oracle for the CubicSplat rasterizer hot path.

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py``, always as the checker.  The product
(``repo_amd``/``manbo``) never imports it.

Floating-point stages run in ``cs_oracle.c`` (compiled by ``build()``); the
integer binning stages are numpy restatements.  Each function cites the
reference code it follows (paths relative to ``/root/reference/manbo``).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from typing import Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SRC = os.path.join(_HERE, "cs_oracle.c")
_SRC_GS = os.path.join(_HERE, "gs_oracle.c")
_SRC_DC = os.path.join(_HERE, "decas_oracle.c")
_LIB_PATH = os.path.join(_HERE, "_build", "libcs_oracle.so")
_CFLAGS = ["-O2", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math",
           "-fno-math-errno", "-mfma", "-msse4.1"]

F32_1E4 = np.float32(1e-4)
F32_1E6 = np.float32(1e-6)


def build() -> str:
    """Compile the C restatement with gcc into oracle/_build/."""
    os.makedirs(os.path.dirname(_LIB_PATH), exist_ok=True)
    tmp = _LIB_PATH + ".tmp"
    subprocess.check_call(["gcc", *_CFLAGS, "-o", tmp, _SRC, _SRC_GS, _SRC_DC, "-lm"])
    os.replace(tmp, _LIB_PATH)
    return _LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH) or any(
                os.path.getmtime(src) > os.path.getmtime(_LIB_PATH) for src in (_SRC, _SRC_GS, _SRC_DC)):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.cs_expf.restype = ctypes.c_float
        L.cs_expf.argtypes = [ctypes.c_float]
        _lib = L
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def _i32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.int32))


class _Scene(ctypes.Structure):
    _fields_ = [
        ("edges", ctypes.c_void_p), ("prim_edge_offsets", ctypes.c_void_p),
        ("colors", ctypes.c_void_p), ("opacities", ctypes.c_void_p),
        ("inv_sigma2s", ctypes.c_void_p), ("fill_rules", ctypes.c_void_p),
        ("stroke_widths", ctypes.c_void_p), ("prim_ids_sorted", ctypes.c_void_p),
        ("tile_bins", ctypes.c_void_p), ("background", ctypes.c_void_p),
        ("img_h", ctypes.c_int32), ("img_w", ctypes.c_int32),
        ("block_x", ctypes.c_int32), ("block_y", ctypes.c_int32),
        ("mode", ctypes.c_int32),
    ]


def expf(x: float) -> float:
    """The spec exp used by every coverage evaluation (cs_oracle.c:cs_expf)."""
    return float(lib().cs_expf(ctypes.c_float(x)))


def linspace01(S: int) -> np.ndarray:
    t = np.empty(S, np.float32)
    lib().orc_linspace01(ctypes.c_int32(S), _p(t))
    return t


def tile_bounds(img_h: int, img_w: int, block_x: int = 16, block_y: int = 16):
    return ((img_w + block_x - 1) // block_x, (img_h + block_y - 1) // block_y)


def project_cubics(cubics_norm, stroke_widths, support_radii, img_h, img_w,
                   block_x=16, block_y=16, aabb_pad=1.0, aniso=False):
    """cubic_splatting.py:546-747 -> (cubics_px [N,4,2], tile_ranges [N,4], num_tiles_hit [N])."""
    c = _f32(cubics_norm).reshape(-1, 4, 2)
    n = c.shape[0]
    sw = _f32(stroke_widths).reshape(n)
    sr = _f32(support_radii).reshape(n)
    px = np.empty((n, 4, 2), np.float32)
    tr = np.empty((n, 4), np.int32)
    nh = np.empty((n,), np.int32)
    lib().orc_project_cubics(_p(c), _p(sw), _p(sr), ctypes.c_int32(n), ctypes.c_int32(img_h),
                             ctypes.c_int32(img_w), ctypes.c_int32(block_x),
                             ctypes.c_int32(block_y), ctypes.c_float(aabb_pad),
                             ctypes.c_int32(int(bool(aniso))), _p(px), _p(tr), _p(nh))
    return px, tr, nh


def cubic_aabb(cubics_px) -> np.ndarray:
    """Exact unpadded AABB per pixel-space cubic (cubic_splatting.py:606-688)."""
    c = _f32(cubics_px).reshape(-1, 4, 2)
    out = np.empty((c.shape[0], 4), np.float32)
    lib().orc_cubic_aabb(_p(c), ctypes.c_int32(c.shape[0]), _p(out))
    return out


def flatten(cubics_px, S: int) -> np.ndarray:
    """cubic_splatting.py:1709-1719 -> edges [N*(S-1), 2, 2]."""
    c = _f32(cubics_px).reshape(-1, 4, 2)
    n = c.shape[0]
    S = max(2, int(S))
    e = np.empty((n * (S - 1), 2, 2), np.float32)
    lib().orc_flatten(_p(c), ctypes.c_int32(n), ctypes.c_int32(S), _p(e))
    return e


def prim_tile_ranges(seg_ranges, offs, tbx: int, tby: int):
    """cubic_splatting.py:2071-2137: union of segment tile ranges per primitive."""
    seg_ranges = _i32(seg_ranges).reshape(-1, 4)
    offs = _i32(offs)
    P = offs.shape[0] - 1
    out = np.zeros((P, 4), np.int32)
    hit = np.zeros((P,), np.int32)
    for p in range(P):
        s0, s1 = int(offs[p]), int(offs[p + 1])
        if s1 > s0:
            r = seg_ranges[s0:s1]
            mnx = min(tbx, int(r[:, 0].min()))
            mny = min(tby, int(r[:, 1].min()))
            mxx = max(0, int(r[:, 2].max()))
            mxy = max(0, int(r[:, 3].max()))
            out[p] = (mnx, mny, mxx, mxy)
            hit[p] = max(0, mxx - mnx) * max(0, mxy - mny)
    return out, hit


def depth_keys(depths) -> np.ndarray:
    """cubic_splatting.py:799-805: fp32 bits -> unsigned key ordered like the float."""
    bits = _f32(depths).view(np.int32)
    mask = (bits >> 31) | np.int32(-2147483648)
    return (bits ^ mask).view(np.uint32)


def map_intersects(prim_ranges, depths, cum, tbx: int):
    """cubic_splatting.py:750-819: primitive-major, row-major emission of
    (tile << 32 | depth_key) keys with the primitive id as value."""
    prim_ranges = _i32(prim_ranges).reshape(-1, 4)
    cum = np.asarray(cum, np.int64)
    n_total = int(cum[-1]) if cum.size else 0
    keys = np.empty(n_total, np.int64)
    ids = np.empty(n_total, np.int32)
    dk = depth_keys(depths).astype(np.int64)
    for p in range(prim_ranges.shape[0]):
        x0, y0, x1, y1 = (int(v) for v in prim_ranges[p])
        w, h = x1 - x0, y1 - y0
        if w * h <= 0:
            continue
        base = int(cum[p - 1]) if p > 0 else 0
        ty, tx = np.meshgrid(np.arange(y0, y1), np.arange(x0, x1), indexing="ij")
        tiles = (ty * tbx + tx).reshape(-1).astype(np.int64)
        keys[base:base + w * h] = (tiles << 32) | dk[p]
        ids[base:base + w * h] = p
    return keys, ids


def sort_intersects(keys, ids):
    """torch.sort(isect_ids) + gather (cubic_splatting.py:2895-2896), with the
    tie order defined as stable (emission is primitive-major)."""
    order = np.argsort(keys, kind="stable")
    return keys[order], ids[order]


def tile_bins_from_sorted(sorted_keys, num_tiles: int) -> np.ndarray:
    """tile_bins.py:10-60: [start, end) per tile, zero for empty tiles."""
    bins = np.zeros((num_tiles, 2), np.int32)
    n = sorted_keys.shape[0]
    if n == 0:
        return bins
    tiles = (sorted_keys >> 32).astype(np.int64)
    change = np.nonzero(tiles[1:] != tiles[:-1])[0] + 1
    starts = np.concatenate([[0], change])
    ends = np.concatenate([change, [n]])
    bins[tiles[starts], 0] = starts
    bins[tiles[starts], 1] = ends
    return bins


def prim_params(aa_widths, P: int):
    """cubic_splatting.py:2815-2822: widths clamp, inv_sigma2 and support radius (fp32)."""
    w = np.maximum(_f32(aa_widths).reshape(-1), F32_1E4).astype(np.float32)
    if w.size == 1 and P > 1:
        w = np.full(P, w[0], np.float32)
    inv = (np.float32(1.0) / np.maximum(w * w, F32_1E6)).astype(np.float32)
    support = (w * np.float32(3.0)).astype(np.float32)
    return w, inv, support


def bin_scene(cubics_norm, offs, depths, aa_widths, img_h, img_w, S, *, stroke_widths=None,
              block_x=16, block_y=16, aabb_pad=1.0, aniso=False, flatten_method="bernstein"):
    """Forward up to the sorted per-tile lists (cubic_splatting.py:2815-2908)."""
    offs = _i32(offs)
    P = offs.shape[0] - 1
    cn = _f32(cubics_norm).reshape(-1, 4, 2)
    nseg = cn.shape[0]
    w, inv_s2, support = prim_params(aa_widths, P)
    counts = np.maximum(offs[1:] - offs[:-1], 0)
    sup_seg = np.repeat(support, counts)
    if stroke_widths is None:
        sw_seg = np.zeros(nseg, np.float32)
    else:
        sw_seg = np.repeat(_f32(stroke_widths).reshape(-1), counts)
    tbx, tby = tile_bounds(img_h, img_w, block_x, block_y)
    cubics_px, seg_ranges, _ = project_cubics(cn, sw_seg, sup_seg, img_h, img_w, block_x,
                                              block_y, aabb_pad, aniso)
    S = max(2, int(S))
    seo = t_starts = t_ends = None
    if flatten_method == "de_casteljau":
        edges, seo, t_starts, t_ends = flatten_decas(cubics_px, S)
        prim_edge_offsets = seo[np.clip(offs, 0, nseg)].astype(np.int32)
    else:
        edges = flatten(cubics_px, S)
        prim_edge_offsets = (offs.astype(np.int64) * (S - 1)).astype(np.int32)
    prim_ranges, num_hit = prim_tile_ranges(seg_ranges, offs, tbx, tby)
    cum = np.cumsum(num_hit.astype(np.int64))
    keys, ids = map_intersects(prim_ranges, depths, cum, tbx)
    skeys, sids = sort_intersects(keys, ids)
    bins = tile_bins_from_sorted(skeys, tbx * tby)
    return dict(widths=w, inv_sigma2s=inv_s2, support=support, cubics_px=cubics_px,
                seg_tile_ranges=seg_ranges, edges=edges, prim_edge_offsets=prim_edge_offsets,
                prim_tile_ranges=prim_ranges, num_tiles_hit=num_hit, isect_ids_sorted=skeys,
                primitive_ids_sorted=sids, tile_bins=bins, S=S, tbx=tbx, tby=tby,
                flatten_method=flatten_method, segment_edge_offsets=seo, edge_t_starts=t_starts,
                edge_t_ends=t_ends)


def _scene(b, colors, opacities, fill_rules, stroke_widths, background, img_h, img_w,
           block_x, block_y, mode, keep):
    arrs = dict(edges=_f32(b["edges"]), offs=_i32(b["prim_edge_offsets"]),
                colors=_f32(colors).reshape(-1, 3), opac=_f32(opacities).reshape(-1),
                inv=_f32(b["inv_sigma2s"]),
                rules=_i32(fill_rules if fill_rules is not None else
                           np.ones(len(b["inv_sigma2s"]), np.int32)).reshape(-1),
                sw=_f32(stroke_widths if stroke_widths is not None else
                        np.zeros(len(b["inv_sigma2s"]), np.float32)).reshape(-1),
                ids=_i32(b["primitive_ids_sorted"]), bins=_i32(b["tile_bins"]),
                bg=_f32(background).reshape(3))
    keep.append(arrs)
    return _Scene(_p(arrs["edges"]).value, _p(arrs["offs"]).value, _p(arrs["colors"]).value,
                  _p(arrs["opac"]).value, _p(arrs["inv"]).value, _p(arrs["rules"]).value,
                  _p(arrs["sw"]).value, _p(arrs["ids"]).value, _p(arrs["bins"]).value,
                  _p(arrs["bg"]).value, img_h, img_w, block_x, block_y, mode)


def default_workers() -> int:
    """Threads for the banded raster: the usable CPUs, at most 16."""
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def row_bands(rows, img_h: int):
    """``rows`` as a list of disjoint [a, b) row ranges: None is the whole
    image, (a, b) one band, a list of such pairs several."""
    if rows is None:
        return [(0, int(img_h))]
    if len(rows) == 2 and not hasattr(rows[0], "__len__"):
        rows = [rows]
    out = sorted((max(0, int(a)), min(int(img_h), int(b))) for a, b in rows)
    for (a0, b0), (a1, _) in zip(out, out[1:]):
        if a1 < b0:
            raise ValueError(f"row bands overlap: {out}")
    return [(a, b) for a, b in out if b > a]


def _run_bands(fn, bands, workers: int, band_rows: int = 16) -> None:
    """fn(a, b) over every row band, cut into pieces of band_rows rows and run
    on `workers` threads (one call per band when workers is 1)."""
    workers = max(1, int(workers))
    if workers == 1:
        for a, b in bands:
            fn(a, b)
        return
    from concurrent.futures import ThreadPoolExecutor
    pieces = [(a, min(a + band_rows, b)) for r0, b in bands for a in range(r0, b, band_rows)]
    with ThreadPoolExecutor(max_workers=workers) as ex:
        for f in [ex.submit(fn, a, b) for a, b in pieces]:
            f.result()


def raster_forward(b, colors, opacities, background, img_h, img_w, *, fill_rules=None,
                   stroke_widths=None, mode=0, block_x=16, block_y=16, rows=None, workers=1):
    """Forward raster; ``rows=(r0, r1)`` restricts it to pixel rows [r0, r1)
    and a list of such pairs to those bands (other pixels are left as
    background, T=1, idx=0).  ``workers`` > 1 splits
    the rows into bands rasterized by that many threads (the C restatement
    holds no global state and ctypes releases the GIL); every pixel's result is
    the same as in one pass."""
    keep = []
    sc = _scene(b, colors, opacities, fill_rules, stroke_widths, background, img_h, img_w,
                block_x, block_y, mode, keep)
    bands = row_bands(rows, img_h)
    out = np.empty((img_h, img_w, 3), np.float32)
    out[:] = _f32(background).reshape(1, 1, 3)
    T = np.ones((img_h, img_w), np.float32)
    idx = np.zeros((img_h, img_w), np.int32)

    def band(a, b):
        lib().orc_raster_forward(ctypes.byref(sc), ctypes.c_int32(a), ctypes.c_int32(b),
                                 _p(out), _p(T), _p(idx))

    # Bands write disjoint rows of the outputs.
    _run_bands(band, bands, workers)
    return out, T, idx


def raster_backward(b, colors, opacities, background, img_h, img_w, final_T, final_idx,
                    v_out, *, fill_rules=None, stroke_widths=None, mode=0, block_x=16,
                    block_y=16, rows=None, workers=1, contrib=False):
    """Backward raster (cubic_splatting.py:1197-1651) in float64 sums; with
    ``contrib`` also the contribution statistics ``contrib_rgb`` [P,3] and
    ``isect_contrib`` [I] (cubic_splatting.py:1540-1546, 1617-1638)."""
    keep = []
    sc = _scene(b, colors, opacities, fill_rules, stroke_widths, background, img_h, img_w,
                block_x, block_y, mode, keep)
    P = len(b["inv_sigma2s"])
    E = b["edges"].shape[0]
    v_edges = np.zeros((E, 2, 2), np.float64)
    v_col = np.zeros((P, 3), np.float64)
    v_op = np.zeros(P, np.float64)
    v_is2 = np.zeros(P, np.float64)
    v_sw = np.zeros(P, np.float64)
    fT, fi, vo = _f32(final_T), _i32(final_idx), _f32(v_out)
    bands = row_bands(rows, img_h)
    acc = [v_edges, v_col, v_op, v_is2, v_sw]
    if contrib:
        acc += [np.zeros((P, 3), np.float64),
                np.zeros(b["primitive_ids_sorted"].shape[0], np.float64)]
    parts = []
    single = workers <= 1

    def band(a, b):
        # With threads, each band sums into its own float64 accumulators, which
        # are added afterwards (the sums' order differs by rounding only).
        mine = acc if single else [np.zeros_like(x) for x in acc]
        ptrs = [_p(x) for x in mine] + ([] if contrib else [None, None])
        lib().orc_raster_backward(ctypes.byref(sc), ctypes.c_int32(a), ctypes.c_int32(b),
                                  _p(fT), _p(fi), _p(vo), *ptrs)
        if mine is not acc:
            parts.append(mine)

    _run_bands(band, bands, workers)
    for part in parts:
        for x, y in zip(acc, part):
            x += y
    out = dict(v_edges=v_edges, v_colors=v_col, v_opacities=v_op, v_inv_sigma2s=v_is2,
               v_stroke_widths=v_sw)
    if contrib:
        out.update(contrib_rgb=acc[5], isect_contrib=acc[6])
    return out


def accumulate_edge_grads(v_edges, nseg: int, S: int) -> np.ndarray:
    """cubic_splatting.py:2308-2396 -> v_cubics_px [nseg,4,2] (float64 sums)."""
    ve = np.ascontiguousarray(np.asarray(v_edges, np.float64))
    out = np.zeros((nseg, 4, 2), np.float64)
    if nseg > 0:
        lib().orc_accumulate_edge_grads(_p(ve), ctypes.c_int32(nseg), ctypes.c_int32(S - 1),
                                        _p(out))
    return out


# ---- adaptive (de Casteljau) flattening, cubic_splatting.py:1729-1832, 1863-2068, 2399-2487 ----

DECAS_TOL_PX = 0.5   # DEFAULT_DE_CASTELJAU_FLATNESS_TOL_PX (cubic_splatting.py:18)


def decas_max_depth(S: int) -> int:
    """cubic_splatting.py:1733."""
    return int(lib().orc_decas_max_depth(ctypes.c_int32(int(S))))


def flatness_flags(cubics, tol=DECAS_TOL_PX, force=False) -> np.ndarray:
    """cubic_adaptive_flatness_flags_tilelang (cubic_splatting.py:1918-1965) -> uint8 [n]."""
    c = _f32(cubics).reshape(-1, 4, 2)
    out = np.zeros(c.shape[0], np.uint8)
    if c.shape[0]:
        lib().orc_flatness_flags(_p(c), ctypes.c_int32(c.shape[0]), ctypes.c_float(tol),
                                 ctypes.c_int32(int(bool(force))), _p(out))
    return out


def split_half(cubics):
    """cubic_split_half_tilelang (cubic_splatting.py:2033-2068) -> (left, right) [n,4,2]."""
    c = _f32(cubics).reshape(-1, 4, 2)
    left, right = np.empty_like(c), np.empty_like(c)
    if c.shape[0]:
        lib().orc_split_half(_p(c), ctypes.c_int32(c.shape[0]), _p(left), _p(right))
    return left, right


def flatten_decas(cubics_px, S: int):
    """_flatten_cubics_to_edges, de Casteljau branch (cubic_splatting.py:1729-1832):
    -> (edges [E,2,2], segment_edge_offsets [nseg+1], t_starts [E], t_ends [E])."""
    c = _f32(cubics_px).reshape(-1, 4, 2)
    nseg = c.shape[0]
    cap = max(1, nseg << decas_max_depth(S))
    edges = np.zeros((cap, 2, 2), np.float32)
    t0 = np.zeros(cap, np.float32)
    t1 = np.zeros(cap, np.float32)
    seo = np.zeros(nseg + 1, np.int32)
    n = lib().orc_flatten_decas(_p(c), ctypes.c_int32(nseg), ctypes.c_int32(int(S)), _p(edges),
                                _p(t0), _p(t1), _p(seo), ctypes.c_int32(cap))
    if n < 0:
        raise MemoryError("orc_flatten_decas failed")
    return edges[:n].copy(), seo, t0[:n].copy(), t1[:n].copy()


def accumulate_edge_grads_csr(v_edges, seo, t_starts, t_ends, nseg: int) -> np.ndarray:
    """_accumulate_edge_grads_to_cubics_csr_kernel (cubic_splatting.py:2399-2487)
    -> v_cubics_px [nseg,4,2] (float64 sums)."""
    ve = np.ascontiguousarray(np.asarray(v_edges, np.float64)).reshape(-1, 2, 2)
    out = np.zeros((nseg, 4, 2), np.float64)
    if nseg > 0:
        so, a, b = _i32(seo), _f32(t_starts), _f32(t_ends)
        lib().orc_accumulate_edge_grads_csr(_p(ve), _p(so), _p(a), _p(b), ctypes.c_int32(nseg),
                                            _p(out))
    return out


def render_forward(cubics_norm, offs, colors, opacities, depths, img_h, img_w, background, *,
                   fill_rules=None, aa_widths=None, aa_width=1.0, S=24, stroke_widths=None,
                   block_x=16, block_y=16, aabb_pad=1.0, aniso=False, rows=None,
                   flatten_method="bernstein", workers=1):
    """Whole forward of _CubicFillSplatFunction (cubic_splatting.py:2752-2962) or,
    with stroke_widths, _CubicPolylineSplatFunction (cubic_polyline_splatting.py:964-1173)."""
    offs = _i32(offs)
    P = offs.shape[0] - 1
    if aa_widths is None:
        aa_widths = np.full(P, aa_width, np.float32)
    mode = 0 if stroke_widths is None else 1
    b = bin_scene(cubics_norm, offs, depths, aa_widths, img_h, img_w, S,
                  stroke_widths=stroke_widths, block_x=block_x, block_y=block_y,
                  aabb_pad=aabb_pad, aniso=aniso, flatten_method=flatten_method)
    out, T, idx = raster_forward(b, colors, opacities, background, img_h, img_w,
                                 fill_rules=fill_rules, stroke_widths=stroke_widths, mode=mode,
                                 block_x=block_x, block_y=block_y, rows=rows,
                                 workers=workers)
    b.update(rows=rows, workers=workers, out=out, final_T=T, final_idx=idx, mode=mode, colors=_f32(colors),
             opacities=_f32(opacities).reshape(-1), fill_rules=fill_rules,
             stroke_widths=stroke_widths, background=_f32(background).reshape(3),
             img_h=img_h, img_w=img_w, block_x=block_x, block_y=block_y,
             nseg=_f32(cubics_norm).reshape(-1, 4, 2).shape[0])
    return b


def render_backward(fw, v_out, contrib=False):
    """_CubicFillSplatFunction.backward (cubic_splatting.py:2964-3125) in float64 sums:
    returns grads for cubics_norm, colors, opacities, aa_widths (and stroke widths);
    with ``contrib`` also contrib_rgb and isect_contrib (:3014-3094)."""
    g = raster_backward(fw, fw["colors"], fw["opacities"], fw["background"], fw["img_h"],
                        fw["img_w"], fw["final_T"], fw["final_idx"], v_out,
                        fill_rules=fw["fill_rules"], stroke_widths=fw["stroke_widths"],
                        mode=fw["mode"], block_x=fw["block_x"], block_y=fw["block_y"],
                        rows=fw.get("rows"), workers=fw.get("workers", 1), contrib=contrib)
    if fw.get("flatten_method") == "de_casteljau":
        v_px = accumulate_edge_grads_csr(g["v_edges"], fw["segment_edge_offsets"],
                                         fw["edge_t_starts"], fw["edge_t_ends"], fw["nseg"])
    else:
        v_px = accumulate_edge_grads(g["v_edges"], fw["nseg"], fw["S"])
    half_w = 0.5 * float(fw["img_w"])
    half_h = 0.5 * float(fw["img_h"])
    v_norm = v_px.copy()
    v_norm[..., 0] *= half_w
    v_norm[..., 1] *= half_h
    w = fw["widths"].astype(np.float32)
    denom = np.maximum((w * w * w).astype(np.float32), np.float32(1e-12)).astype(np.float64)
    v_aa = -2.0 * g["v_inv_sigma2s"] / denom
    g.update(v_cubics_px=v_px, v_cubics_norm=v_norm, v_aa_widths=v_aa)
    return g


# ---- losses (manbo/metric.py, manbo/ops/metric.py) in float64 ----

def mse(x, y) -> float:
    """metric.py:102-212: mean((x-y)^2)."""
    d = np.asarray(x, np.float64) - np.asarray(y, np.float64)
    return float(np.mean(d * d))


def gaussian_window_1d(win_size=11, win_sigma=1.5) -> np.ndarray:
    """metric.py:47-61 builds the 2D window as outer(g, g) of this fp32 vector."""
    coords = np.arange(win_size, dtype=np.float32) - np.float32(win_size // 2)
    g = np.exp(-(coords ** 2) / np.float32(2 * win_sigma ** 2)).astype(np.float32)
    return (g / g.sum(dtype=np.float32)).astype(np.float32)


def ssim_torch64(x, y, win_size=11, win_sigma=1.5, data_range=1.0, k1=0.01, k2=0.03):
    """metric.py:215-273 / ops/metric.py:205-341 restated with torch float64
    conv2d (valid window); returns a differentiable scalar (mean over pixels
    per channel, then over channels)."""
    import torch
    import torch.nn.functional as F
    g = torch.from_numpy(gaussian_window_1d(win_size, win_sigma).astype(np.float64))
    w2 = torch.outer(g, g)
    n, c, h, wd = x.shape
    xf = x.reshape(n * c, 1, h, wd)
    yf = y.reshape(n * c, 1, h, wd)
    k = w2.view(1, 1, win_size, win_size).to(x.dtype)
    mu1 = F.conv2d(xf, k)
    mu2 = F.conv2d(yf, k)
    ex2 = F.conv2d(xf * xf, k)
    ey2 = F.conv2d(yf * yf, k)
    exy = F.conv2d(xf * yf, k)
    c1 = (k1 * data_range) ** 2
    c2 = (k2 * data_range) ** 2
    s1 = ex2 - mu1 * mu1
    s2 = ey2 - mu2 * mu2
    s12 = exy - mu1 * mu2
    m = ((2 * mu1 * mu2 + c1) / (mu1 * mu1 + mu2 * mu2 + c1)) * ((2 * s12 + c2) / (s1 + s2 + c2))
    return m.view(n, c, -1).mean(-1).mean()


def ssim64_separable(x, y, win_size=11, win_sigma=1.5, data_range=1.0, k1=0.01, k2=0.03,
                     size_average=True, nonnegative=False):
    """The same SSIM as ssim_torch64 with the window applied as two 1D passes
    (rows, then columns): outer(g, g) * z = g_col * (g_row * z), so the value
    agrees to float64 rounding, at 2 win instead of win^2 multiply-adds per
    output (fast enough for full frames).  Returns the mean over pixels and
    channels, or with size_average=False the per-image means [N]
    (metric.py:262-273); nonnegative clamps each channel mean at 0 first."""
    import torch
    import torch.nn.functional as F
    g = torch.from_numpy(gaussian_window_1d(win_size, win_sigma).astype(np.float64)).to(x.dtype)
    n, c, h, wd = x.shape
    kr = g.view(1, 1, 1, win_size)
    kc = g.view(1, 1, win_size, 1)
    z = torch.cat([x, y, x * x, y * y, x * y], 1).reshape(n * c * 5, 1, h, wd)
    f = F.conv2d(F.conv2d(z, kr), kc).view(n, 5, c, h - win_size + 1, wd - win_size + 1)
    # The channel-major cat above stacks (x, y, x^2, y^2, xy) per image.
    f = f.view(n, 5, c, -1)
    mu1, mu2, ex2, ey2, exy = (f[:, k] for k in range(5))
    c1 = (k1 * data_range) ** 2
    c2 = (k2 * data_range) ** 2
    s1 = ex2 - mu1 * mu1
    s2 = ey2 - mu2 * mu2
    s12 = exy - mu1 * mu2
    m = ((2 * mu1 * mu2 + c1) / (mu1 * mu1 + mu2 * mu2 + c1)) * ((2 * s12 + c2) / (s1 + s2 + c2))
    per_channel = m.mean(-1)
    if nonnegative:
        per_channel = torch.relu(per_channel)
    per_image = per_channel.mean(-1)
    return per_image.mean() if size_average else per_image


# ------------------------------------------------ closed ring -> Hermite cubics


def closed_ring_basis(kb: int, subdiv: int):
    """_closed_fill_piecewise_basis_tensors (ops/cubic_splatting.py:81-134) in
    float64: Bernstein basis of degree kb-1 and of its derivative (degree
    kb-2) at t = linspace(0, 1, subdiv+1), and the sample spacing."""
    from math import comb
    t = np.linspace(0.0, 1.0, subdiv + 1)
    n = kb - 1
    basis = np.stack([comb(n, i) * (1.0 - t) ** (n - i) * t ** i for i in range(kb)], 1)
    deriv = np.stack([comb(n - 1, i) * (1.0 - t) ** (n - 1 - i) * t ** i for i in range(kb - 1)],
                     1)
    return basis, deriv, np.diff(t)


def closed_ring_segments(cp, subdiv: int, basis=None, deriv=None, dt=None) -> np.ndarray:
    """closed_cubic_fill_segments_forward_kernel (ops/cubic_splatting.py:137-268)
    in float64: control polygon [N, K, 2] (K >= 4, K even) -> [N*2*subdiv, 4, 2].
    Branch b in {0, 1} is the Bezier curve of degree kb-1 = K/2 on control
    points b*(kb-1) + i (mod K); each branch is cut at the subdiv+1 samples
    into cubic Hermite pieces: P0, P3 on the curve and P1 = P0 + d0 dt/3,
    P2 = P3 - d1 dt/3 with d the curve's derivative."""
    cp = np.asarray(cp, np.float64)
    N, K, _ = cp.shape
    kb = (K + 2) // 2
    if basis is None:
        basis, deriv, dt = closed_ring_basis(kb, subdiv)
    basis, deriv, dt = (np.asarray(a, np.float64) for a in (basis, deriv, dt))
    out = np.zeros((N, 2, subdiv, 4, 2))
    for b in range(2):
        idx = (b * (kb - 1) + np.arange(kb)) % K
        pts = cp[:, idx]                                   # [N, kb, 2]
        diffs = pts[:, 1:] - pts[:, :-1]                   # [N, kb-1, 2]
        P = np.einsum("sk,nkc->nsc", basis, pts)           # [N, S+1, 2]
        D = (kb - 1) * np.einsum("sk,nkc->nsc", deriv, diffs)
        third = (dt / 3.0)[None, :, None]
        out[:, b, :, 0] = P[:, :-1]
        out[:, b, :, 3] = P[:, 1:]
        out[:, b, :, 1] = P[:, :-1] + D[:, :-1] * third
        out[:, b, :, 2] = P[:, 1:] - D[:, 1:] * third
    return out.reshape(N * 2 * subdiv, 4, 2)


def closed_ring_segments_backward(grad, N: int, K: int, subdiv: int, basis=None, deriv=None,
                                  dt=None) -> np.ndarray:
    """closed_cubic_fill_segments_backward_kernel (ops/cubic_splatting.py:271-383)
    in float64: the transpose of the (linear) forward map applied to
    grad [N*2*subdiv, 4, 2] -> [N, K, 2]."""
    kb = (K + 2) // 2
    if basis is None:
        basis, deriv, dt = closed_ring_basis(kb, subdiv)
    basis, deriv, dt = (np.asarray(a, np.float64) for a in (basis, deriv, dt))
    g = np.asarray(grad, np.float64).reshape(N, 2, subdiv, 4, 2)
    out = np.zeros((N, K, 2))
    third = (dt / 3.0)[None, :, None]
    for b in range(2):
        idx = (b * (kb - 1) + np.arange(kb)) % K
        gP = np.zeros((N, subdiv + 1, 2))
        gD = np.zeros((N, subdiv + 1, 2))
        gP[:, :-1] += g[:, b, :, 0] + g[:, b, :, 1]
        gP[:, 1:] += g[:, b, :, 3] + g[:, b, :, 2]
        gD[:, :-1] += g[:, b, :, 1] * third
        gD[:, 1:] -= g[:, b, :, 2] * third
        gpts = np.einsum("sk,nsc->nkc", basis, gP)
        gdiff = (kb - 1) * np.einsum("sk,nsc->nkc", deriv, gD)
        gpts[:, 1:] += gdiff
        gpts[:, :-1] -= gdiff
        np.add.at(out, (slice(None), idx), gpts)
    return out


# ------------------------------------------------------------ 2D Gaussians


def sincosf(x):
    """The spec sin/cos (gs_oracle.c orc_sincosf; the GPU's spec_sincosf)."""
    x = _f32(x).reshape(-1)
    sn = np.empty_like(x)
    cs = np.empty_like(x)
    lib().orc_sincosf_n(_p(x), ctypes.c_int32(x.size), _p(sn), _p(cs))
    return sn, cs


def gs_project(means2d, scales2d, rotation, img_h: int, img_w: int, block_x: int = 16,
               block_y: int = 16):
    """forward2d.py:14-164 -> (xys [N,2], depths [N] (zeros), radii [N] int32,
    conics [N,3], num_tiles_hit [N] int32)."""
    m, s, r = _f32(means2d).reshape(-1, 2), _f32(scales2d).reshape(-1, 2), _f32(rotation).reshape(-1)
    n = m.shape[0]
    xys = np.empty((n, 2), np.float32)
    depths = np.empty(n, np.float32)
    radii = np.empty(n, np.int32)
    conics = np.empty((n, 3), np.float32)
    tiles = np.empty(n, np.int32)
    lib().orc_gs_project(_p(m), _p(s), _p(r), ctypes.c_int32(n), ctypes.c_int32(img_h),
                         ctypes.c_int32(img_w), ctypes.c_int32(block_x), ctypes.c_int32(block_y),
                         _p(xys), _p(depths), _p(radii), _p(conics), _p(tiles))
    return xys, depths, radii, conics, tiles


def gs_rects(xys, conics, radii, block_x: int, block_y: int, tbx: int, tby: int) -> np.ndarray:
    """The tile rectangle (x0, y0, x1, y1) intersects.py:34-121 emits per
    Gaussian; zeros when it emits nothing."""
    xy, q, rad = _f32(xys).reshape(-1, 2), _f32(conics).reshape(-1, 3), _i32(radii).reshape(-1)
    n = xy.shape[0]
    rects = np.empty((n, 4), np.int32)
    lib().orc_gs_rects(_p(xy), _p(q), _p(rad), ctypes.c_int32(n), ctypes.c_int32(block_x),
                       ctypes.c_int32(block_y), ctypes.c_int32(tbx), ctypes.c_int32(tby),
                       _p(rects))
    return rects


def gs_depth_keys(depths) -> np.ndarray:
    """intersects.py:107-109: the raw fp32 bits as an unsigned 32-bit key."""
    return _f32(depths).view(np.uint32)


def gs_map_intersects(rects, depths, tbx: int):
    """intersects.py:96-121: Gaussian-major, row-major emission of
    (tile << 32 | depth bits) keys with the Gaussian id as value."""
    rects = _i32(rects).reshape(-1, 4)
    area = np.maximum(rects[:, 2] - rects[:, 0], 0) * np.maximum(rects[:, 3] - rects[:, 1], 0)
    cum = np.cumsum(area.astype(np.int64))
    n_total = int(cum[-1]) if cum.size else 0
    keys = np.empty(n_total, np.int64)
    ids = np.empty(n_total, np.int32)
    dk = gs_depth_keys(depths).astype(np.int64)
    for g in np.nonzero(area > 0)[0]:
        x0, y0, x1, y1 = (int(v) for v in rects[g])
        base = int(cum[g - 1]) if g > 0 else 0
        ty, tx = np.meshgrid(np.arange(y0, y1), np.arange(x0, x1), indexing="ij")
        tiles = (ty * tbx + tx).reshape(-1).astype(np.int64)
        keys[base:base + tiles.size] = (tiles << 32) | dk[g]
        ids[base:base + tiles.size] = g
    return keys, ids


def gs_bin(xys, conics, radii, depths, img_h: int, img_w: int, block_x: int, block_y: int):
    """tilelang_renderer.py:224-269 (cumsum, map, stable sort, tile bins) ->
    (gaussian_ids_sorted, tile_bins [T,2], isect_ids_sorted)."""
    tbx, tby = tile_bounds(img_h, img_w, block_x, block_y)
    rects = gs_rects(xys, conics, radii, block_x, block_y, tbx, tby)
    keys, ids = gs_map_intersects(rects, depths, tbx)
    keys_s, ids_s = sort_intersects(keys, ids)
    return ids_s, tile_bins_from_sorted(keys_s, tbx * tby), keys_s


def gs_raster_forward(ids_sorted, tile_bins, xys, conics, colors, opacities, background,
                      img_h: int, img_w: int, block_x: int, block_y: int, rows=None):
    """rasterize.py:18-157 -> (out [H,W,3], final_T [H,W], final_idx [H,W]).
    `rows` = (row0, row1) restricts the work to those pixel rows (the other
    rows of the outputs are left zero)."""
    ids, bins = _i32(ids_sorted), _i32(tile_bins)
    xy, q, col = _f32(xys), _f32(conics), _f32(colors)
    op, bg = _f32(opacities).reshape(-1), _f32(background).reshape(-1)
    r0, r1 = (0, img_h) if rows is None else rows
    out = np.zeros((img_h, img_w, 3), np.float32)
    fT = np.zeros((img_h, img_w), np.float32)
    fi = np.zeros((img_h, img_w), np.int32)
    lib().orc_gs_raster_forward(_p(ids), _p(bins), _p(xy), _p(q), _p(col), _p(op), _p(bg),
                                ctypes.c_int32(img_h), ctypes.c_int32(img_w),
                                ctypes.c_int32(block_x), ctypes.c_int32(block_y),
                                ctypes.c_int32(r0), ctypes.c_int32(r1), _p(out), _p(fT), _p(fi))
    return out, fT, fi


def gs_raster_backward(ids_sorted, tile_bins, xys, conics, colors, opacities, background,
                       img_h: int, img_w: int, block_x: int, block_y: int, final_T, final_idx,
                       v_out, v_out_alpha=None, intersect_meta=None, rows=None):
    """rasterize.py:160-529 -> float64 (v_xy, v_conic, v_rgb, v_opacity,
    contrib_rgb, isect_contrib)."""
    ids, bins = _i32(ids_sorted), _i32(tile_bins)
    xy, q, col = _f32(xys), _f32(conics), _f32(colors)
    op, bg = _f32(opacities).reshape(-1), _f32(background).reshape(-1)
    fT, fi, vo = _f32(final_T), _i32(final_idx), _f32(v_out)
    va = None if v_out_alpha is None else _f32(v_out_alpha)
    meta = None if intersect_meta is None else _i32(intersect_meta)
    n = op.shape[0]
    r0, r1 = (0, img_h) if rows is None else rows
    v_xy, v_conic, v_rgb = np.zeros((n, 2)), np.zeros((n, 3)), np.zeros((n, 3))
    v_op, contrib, isect = np.zeros(n), np.zeros((n, 3)), np.zeros(ids.shape[0])
    lib().orc_gs_raster_backward(
        _p(ids), None if meta is None else _p(meta), _p(bins), _p(xy), _p(q), _p(col), _p(op),
        _p(bg), ctypes.c_int32(img_h), ctypes.c_int32(img_w), ctypes.c_int32(block_x),
        ctypes.c_int32(block_y), ctypes.c_int32(r0), ctypes.c_int32(r1), _p(fT), _p(fi), _p(vo),
        None if va is None else _p(va), _p(v_xy), _p(v_conic), _p(v_rgb), _p(v_op), _p(contrib),
        _p(isect))
    return v_xy, v_conic, v_rgb, v_op, contrib, isect


def gs_project_backward(scales2d, rotation, radii, conics, v_xy, v_conic, img_h: int,
                        img_w: int, gaussian_meta=None):
    """backward2d.py:8-151 (with tilelang_renderer.py:111-116's meta scaling)
    -> float64 (v_cov2d, v_mean2d, v_scale, v_rot)."""
    s, r = _f32(scales2d).reshape(-1, 2), _f32(rotation).reshape(-1)
    rad, q = _i32(radii).reshape(-1), _f32(conics).reshape(-1, 3)
    vxy = np.ascontiguousarray(np.asarray(v_xy, np.float64).reshape(-1, 2))
    vq = np.ascontiguousarray(np.asarray(v_conic, np.float64).reshape(-1, 3))
    meta = None if gaussian_meta is None else _i32(gaussian_meta).reshape(-1)
    n = r.shape[0]
    v_cov, v_mean, v_scale, v_rot = np.empty((n, 3)), np.empty((n, 2)), np.empty((n, 2)), np.empty(n)
    lib().orc_gs_project_backward(_p(s), _p(r), _p(rad), _p(q), _p(vxy), _p(vq),
                                  None if meta is None else _p(meta), ctypes.c_int32(n),
                                  ctypes.c_int32(img_h), ctypes.c_int32(img_w), _p(v_cov),
                                  _p(v_mean), _p(v_scale), _p(v_rot))
    return v_cov, v_mean, v_scale, v_rot


# ------------------------------------------------------------------ Adan


def adan_step64(p, g, m, n, d, npg, *, step, lr=1e-3, betas=(0.98, 0.92, 0.99), eps=1e-8,
                weight_decay=0.0, no_prox=False, clip=1.0):
    """adan_step_from_grad_kernel (ops/optim.py:78-110) in float64 on numpy
    arrays: returns the new (p, m, n, d, neg_pre_grad)."""
    p, g, m, n, d, npg = (np.asarray(a, np.float64) for a in (p, g, m, n, d, npg))
    b1, b2, b3 = (float(b) for b in betas)
    bc1 = 1.0 - b1 ** step
    bc2 = 1.0 - b2 ** step
    bc3_sqrt = (1.0 - b3 ** step) ** 0.5
    g = g * clip
    ngod = np.zeros_like(g) if step == 1 else npg + g
    m = m * b1 + g * (1.0 - b1)
    d = d * b2 + ngod * (1.0 - b2)
    ngod2 = ngod * b2 + g
    n = n * b3 + ngod2 * ngod2 * (1.0 - b3)
    denom = np.sqrt(n) / bc3_sqrt + eps
    step_size = lr / bc1
    step_size_diff = lr * b2 / bc2
    if no_prox:
        p = p * (1.0 - lr * weight_decay)
        p = p - step_size * m / denom
        p = p - step_size_diff * d / denom
    else:
        p = p - step_size * m / denom
        p = p - step_size_diff * d / denom
        p = p / (1.0 + lr * weight_decay)
    return p, m, n, d, -g
