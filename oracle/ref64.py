"""Float64 brute-force restatement of the cubic splat forward, differentiable
with torch.autograd.

TEST INFRASTRUCTURE ONLY (imported by tests/ to pin the fp32 oracle).

It follows the same mathematics as cubic_splatting.py:918-1194 (fill) and
cubic_polyline_splatting.py:33-249 (stroke) but is built differently on
purpose, so that a mistake in one does not hide in the other:
  * no per-tile lists: every pixel walks all primitives in (depth, id)
    order and tests tile membership against the primitive's tile rectangle;
  * the distance is a dense [edges x pixels] minimum (autograd routes the
    gradient to the minimizing edge, the reference's "best edge");
  * the inside test of a closed primitive is the winding number by angle
    summation, not by ray crossings.
"""
from __future__ import annotations

import math

import numpy as np
import torch


def winding_by_angles(poly: torch.Tensor, px: torch.Tensor, py: torch.Tensor) -> torch.Tensor:
    """Winding number of the closed polyline ``poly`` [E,2,2] around each point,
    as the rounded sum of signed subtended angles."""
    ax = poly[:, 0, 0].unsqueeze(1) - px.unsqueeze(0)
    ay = poly[:, 0, 1].unsqueeze(1) - py.unsqueeze(0)
    bx = poly[:, 1, 0].unsqueeze(1) - px.unsqueeze(0)
    by = poly[:, 1, 1].unsqueeze(1) - py.unsqueeze(0)
    ang = torch.atan2(ax * by - ay * bx, ax * bx + ay * by)
    return torch.round(ang.sum(0) / (2 * math.pi)).to(torch.int64)


def render64(edges, prim_edge_offsets, colors, opacities, inv_sigma2s, order, prim_tile_ranges,
             img_h, img_w, background, *, mode=0, fill_rules=None, stroke_widths=None,
             block=16, contrib=None):
    """Returns the [H,W,3] float64 image; ``edges``, ``colors``, ``opacities``,
    ``inv_sigma2s`` and ``stroke_widths`` may require grad.

    ``contrib``, a dict, receives each primitive's composited term: "rgb"
    [P,3] = sum over pixels of alpha * T_before * colour, and "tile" =
    {(primitive, tile id): sum over the tile's pixels of alpha * T_before *
    (r + g + b)} (what the backward's contribution statistics must equal)."""
    dev = edges.device
    jj, ii = torch.meshgrid(torch.arange(img_w, dtype=torch.float64),
                            torch.arange(img_h, dtype=torch.float64), indexing="xy")
    px = (jj + 0.5).reshape(-1)
    py = (ii + 0.5).reshape(-1)
    tx = torch.div(jj.reshape(-1).long(), block, rounding_mode="floor")
    ty = torch.div(ii.reshape(-1).long(), block, rounding_mode="floor")
    npx = px.shape[0]
    T = torch.ones(npx, dtype=torch.float64, device=dev)
    C = torch.zeros(npx, 3, dtype=torch.float64, device=dev)
    done = torch.zeros(npx, dtype=torch.bool, device=dev)
    tbx = (img_w + block - 1) // block
    if contrib is not None:
        contrib["rgb"] = np.zeros((len(order), 3), np.float64)
        contrib["tile"] = {}
    for p in [int(v) for v in order]:
        r = [int(v) for v in prim_tile_ranges[p]]
        member = (tx >= r[0]) & (tx < r[2]) & (ty >= r[1]) & (ty < r[3])
        if not bool(member.any()):
            continue
        e0, e1 = int(prim_edge_offsets[p]), int(prim_edge_offsets[p + 1])
        if e1 <= e0:
            continue
        E = edges[e0:e1]
        a = E[:, 0, :]
        v = E[:, 1, :] - a
        vv = (v * v).sum(1).clamp_min(1e-6)
        wx = px.unsqueeze(0) - a[:, 0:1]
        wy = py.unsqueeze(0) - a[:, 1:2]
        t = ((wx * v[:, 0:1] + wy * v[:, 1:2]) / vv.unsqueeze(1)).clamp(0.0, 1.0)
        dx = t * v[:, 0:1] - wx
        dy = t * v[:, 1:2] - wy
        d2 = (dx * dx + dy * dy).min(0).values
        dist = torch.sqrt(d2.clamp_min(0.0) + 0.0)
        is2 = inv_sigma2s[p].clamp_min(1e-6)
        if mode == 0:
            wn = winding_by_angles(E.detach(), px, py)
            rule = 1 if fill_rules is None else int(fill_rules[p])
            inside = (wn % 2 != 0) if rule == 0 else (wn != 0)
            sgn = torch.where(inside, -1.0, 1.0).to(torch.float64)
            logit = (sgn * dist * torch.sqrt(is2) * 2.0).clamp(-60.0, 60.0)
            cov = 1.0 / (1.0 + torch.exp(logit))
        else:
            half_sw = stroke_widths[p].clamp_min(0.0) * 0.5
            ed = (dist - half_sw).clamp_min(0.0)
            cov = torch.exp(-0.5 * ed * ed * is2)
        alpha = torch.clamp(opacities[p] * cov, max=0.999)
        use = member & (~done) & (alpha.detach() >= 1.0 / 255.0)
        a_use = torch.where(use, alpha, torch.zeros_like(alpha))
        if contrib is not None:
            w = (a_use * T).detach()
            col = colors[p].detach().double()
            contrib["rgb"][p] = (w.sum() * col).numpy()
            tid = (ty * tbx + tx)[use]
            wt = torch.bincount(tid, weights=w[use] * col.sum())
            for t in torch.nonzero(wt).reshape(-1).tolist():
                contrib["tile"][(p, t)] = float(wt[t])
        C = C + (a_use * T).unsqueeze(1) * colors[p].unsqueeze(0)
        T = T * (1.0 - a_use)
        done = done | (use & (T.detach() <= 1e-4))
    out = C + T.unsqueeze(1) * background.view(1, 3)
    return out.view(img_h, img_w, 3)


def depth_order(depths) -> np.ndarray:
    """Primitive order of the sorted lists: ascending fp32 depth, ties by id."""
    d = np.asarray(depths, np.float32).reshape(-1)
    return np.lexsort((np.arange(d.size), d))
