"""Seeded synthetic scenes for the five benchmark configurations.

The reference ships no data for this path, so inputs are generated on the CPU
with ``torch.Generator("cpu").manual_seed(1000 + cfg)`` for geometry and
``2000 + cfg`` for the target image, then moved to the device.  Geometry is
built in pixel space and normalized with ``x_n = x / (W/2) - 1`` (the inverse
of the projection at cubic_splatting.py:588-595).
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import torch

KAPPA4 = 0.5523


@dataclass
class Scene:
    cfg: int
    img_h: int
    img_w: int
    S: int
    cubics_norm: torch.Tensor          # [Nseg,4,2] f32
    seg_offsets: torch.Tensor          # [P+1] i32
    colors: torch.Tensor               # [P,3] f32
    opacities: torch.Tensor            # [P] f32
    depths: torch.Tensor               # [P] f32
    aa_widths: torch.Tensor            # [P] f32
    fill_rules: torch.Tensor           # [P] i32
    background: torch.Tensor           # [3] f32
    target: torch.Tensor               # [1,3,H,W] f32
    stroke_widths: Optional[torch.Tensor] = None  # [P] f32 (open strokes)

    @property
    def num_primitives(self) -> int:
        return int(self.seg_offsets.numel()) - 1

    def to(self, device) -> "Scene":
        kw = {k: (v.to(device) if isinstance(v, torch.Tensor) else v)
              for k, v in self.__dict__.items()}
        return Scene(**kw)


def _value_noise(g, h, w, cell=8):
    gh, gw = h // cell + 2, w // cell + 2
    lat = torch.rand((3, gh, gw), generator=g)
    ys = (torch.arange(h, dtype=torch.float32) + 0.5) / cell
    xs = (torch.arange(w, dtype=torch.float32) + 0.5) / cell
    y0 = ys.floor().long()
    x0 = xs.floor().long()
    fy = (ys - y0).view(1, -1, 1)
    fx = (xs - x0).view(1, 1, -1)
    a = lat[:, y0][:, :, x0]
    b = lat[:, y0][:, :, x0 + 1]
    c = lat[:, y0 + 1][:, :, x0]
    d = lat[:, y0 + 1][:, :, x0 + 1]
    top = a * (1 - fx) + b * fx
    bot = c * (1 - fx) + d * fx
    return (top * (1 - fy) + bot * fy).clamp(0, 1)


def make_target(cfg: int, h: int, w: int, rects: int = 0) -> torch.Tensor:
    g = torch.Generator("cpu").manual_seed(2000 + cfg)
    img = _value_noise(g, h, w)
    for _ in range(rects):
        x0 = int(torch.randint(0, w, (1,), generator=g))
        y0 = int(torch.randint(0, h, (1,), generator=g))
        rw = int(torch.randint(4, max(5, w // 6), (1,), generator=g))
        rh = int(torch.randint(4, max(5, h // 6), (1,), generator=g))
        col = torch.rand((3, 1, 1), generator=g)
        img[:, y0:y0 + rh, x0:x0 + rw] = col
    return img.unsqueeze(0).contiguous()


def _ring(g, cx, cy, r, nseg, jitter=0.15):
    """Closed ring of ``nseg`` cubics approximating a circle (kappa for 4
    segments), every control point jittered by N(0, jitter*r); segment k's
    last point is segment k+1's first point and the ring closes."""
    P = cx.shape[0]
    kap = (4.0 / 3.0) * math.tan(math.pi / (2 * nseg))
    th = torch.arange(nseg, dtype=torch.float32) * (2 * math.pi / nseg)
    ct, st = torch.cos(th).view(1, -1), torch.sin(th).view(1, -1)
    r2 = r.view(-1, 1)
    ax = cx.view(-1, 1) + r2 * ct
    ay = cy.view(-1, 1) + r2 * st
    h1x = ax - kap * r2 * st
    h1y = ay + kap * r2 * ct
    nx = torch.roll(ax, -1, 1)
    ny = torch.roll(ay, -1, 1)
    nct, nst = torch.roll(ct, -1, 1), torch.roll(st, -1, 1)
    h2x = nx + kap * r2 * nst
    h2y = ny - kap * r2 * nct
    js = jitter * r2
    ax = ax + torch.randn(ax.shape, generator=g) * js
    ay = ay + torch.randn(ay.shape, generator=g) * js
    h1x = h1x + torch.randn(h1x.shape, generator=g) * js
    h1y = h1y + torch.randn(h1y.shape, generator=g) * js
    h2x = h2x + torch.randn(h2x.shape, generator=g) * js
    h2y = h2y + torch.randn(h2y.shape, generator=g) * js
    nx = torch.roll(ax, -1, 1)
    ny = torch.roll(ay, -1, 1)
    cub = torch.stack([torch.stack([ax, ay], -1), torch.stack([h1x, h1y], -1),
                       torch.stack([h2x, h2y], -1), torch.stack([nx, ny], -1)], 2)
    return cub.reshape(P * nseg, 4, 2)


def _normalize(cub_px, h, w):
    out = cub_px.clone()
    out[..., 0] = cub_px[..., 0] / (w / 2.0) - 1.0
    out[..., 1] = cub_px[..., 1] / (h / 2.0) - 1.0
    return out.contiguous()


def _finish(cfg, g, cub_px, P, nseg, h, w, S, *, opacity=None, rects=0, stroke=None):
    colors = torch.rand((P, 3), generator=g)
    if opacity is None:
        opac = 0.5 + 0.5 * torch.rand((P,), generator=g)
    else:
        opac = torch.full((P,), float(opacity))
    depths = (torch.randperm(P, generator=g).to(torch.float32) / P).contiguous()
    offs = (torch.arange(P + 1, dtype=torch.int32) * nseg).contiguous()
    return Scene(cfg=cfg, img_h=h, img_w=w, S=S, cubics_norm=_normalize(cub_px, h, w),
                 seg_offsets=offs, colors=colors.contiguous(), opacities=opac.contiguous(),
                 depths=depths, aa_widths=torch.ones(P), fill_rules=torch.ones(P, dtype=torch.int32),
                 background=torch.ones(3), target=make_target(cfg, h, w, rects),
                 stroke_widths=stroke)


def make_scene(cfg: int, *, scale: float = 1.0) -> Scene:
    """Config ``cfg`` (1..5).  ``scale`` < 1 shrinks the primitive count (not the
    canvas) for quick tests; the benchmark uses scale=1."""
    g = torch.Generator("cpu").manual_seed(1000 + cfg)
    if cfg == 1:
        P, nseg, h, w, S = 64, 4, 128, 128, 8
        P = max(1, int(P * scale))
        anchors = torch.rand((P, nseg, 2), generator=g) * torch.tensor([w, h])
        handles = torch.rand((P, nseg, 2, 2), generator=g) * torch.tensor([w, h])
        nxt = torch.roll(anchors, -1, 1)
        cub = torch.stack([anchors, handles[:, :, 0], handles[:, :, 1], nxt], 2)
        return _finish(cfg, g, cub.reshape(P * nseg, 4, 2), P, nseg, h, w, S, opacity=0.8)
    if cfg == 2:
        P, nseg, h, w, S = 512, 4, 512, 768, 16
        P = max(1, int(P * scale))
        cx = torch.rand((P,), generator=g) * w
        cy = torch.rand((P,), generator=g) * h
        r = 5.0 + 75.0 * torch.rand((P,), generator=g)
        return _finish(cfg, g, _ring(g, cx, cy, r, nseg), P, nseg, h, w, S, rects=200)
    if cfg == 3:
        P, nseg, h, w, S = 4096, 4, 1356, 2040, 16
        P = max(1, int(P * scale))
        cx = torch.rand((P,), generator=g) * w
        cy = torch.rand((P,), generator=g) * h
        r = torch.exp(math.log(2.0) + (math.log(200.0) - math.log(2.0)) * torch.rand((P,), generator=g))
        return _finish(cfg, g, _ring(g, cx, cy, r, nseg), P, nseg, h, w, S, rects=200)
    if cfg == 4:
        P, nseg, h, w, S = 8192, 3, 1024, 1024, 16
        P = max(1, int(P * scale))
        start = torch.rand((P, 2), generator=g) * torch.tensor([w, h])
        pts = [start]
        for _ in range(3 * nseg):
            step = torch.randn((P, 2), generator=g) * 12.0
            pts.append(pts[-1] + step)
        pts = torch.stack(pts, 1)
        cub = torch.stack([pts[:, 0:-1:3], pts[:, 1::3], pts[:, 2::3], pts[:, 3::3]], 2)
        sw = (1.0 + 3.0 * torch.rand((P,), generator=g)).contiguous()
        return _finish(cfg, g, cub.reshape(P * nseg, 4, 2), P, nseg, h, w, S, stroke=sw)
    if cfg == 5:
        P, nseg, h, w, S = 16384, 6, 2048, 2048, 32
        P = max(1, int(P * scale))
        centers = torch.rand((8, 2), generator=g) * torch.tensor([w, h])
        clustered = torch.rand((P,), generator=g) < 0.7
        which = torch.randint(0, 8, (P,), generator=g)
        cpos = centers[which] + torch.randn((P, 2), generator=g) * 100.0
        upos = torch.rand((P, 2), generator=g) * torch.tensor([w, h])
        pos = torch.where(clustered.unsqueeze(1), cpos, upos)
        r = torch.exp(math.log(4.0) + (math.log(512.0) - math.log(4.0)) * torch.rand((P,), generator=g))
        return _finish(cfg, g, _ring(g, pos[:, 0], pos[:, 1], r, nseg), P, nseg, h, w, S)
    raise ValueError(f"unknown config {cfg}")


def segments_as_primitives(sc: Scene) -> Scene:
    """The same geometry with one primitive per cubic segment, as the
    reference's training model lays out open strokes
    (gaussian_trace/render.py:669-677): seg_offsets = arange(nseg + 1) and every
    per-primitive attribute repeated over its segments.  Segments of one path
    share their depth, so each path's segments tie and keep segment order."""
    counts = (sc.seg_offsets[1:] - sc.seg_offsets[:-1]).to(torch.int64)
    nseg = int(sc.cubics_norm.shape[0])

    def rep(t):
        return None if t is None else torch.repeat_interleave(t, counts, dim=0).contiguous()

    return Scene(cfg=sc.cfg, img_h=sc.img_h, img_w=sc.img_w, S=sc.S,
                 cubics_norm=sc.cubics_norm.clone(),
                 seg_offsets=torch.arange(nseg + 1, dtype=torch.int32),
                 colors=rep(sc.colors), opacities=rep(sc.opacities), depths=rep(sc.depths),
                 aa_widths=rep(sc.aa_widths), fill_rules=rep(sc.fill_rules),
                 background=sc.background.clone(), target=sc.target,
                 stroke_widths=rep(sc.stroke_widths))


def small_scene(seed: int, *, P: int = 6, nseg: int = 4, h: int = 48, w: int = 64, S: int = 8,
                stroke: bool = False, rmin: float = 3.0, rmax: float = 20.0) -> Scene:
    """Tiny random scene for brute-force parity tests."""
    g = torch.Generator("cpu").manual_seed(seed)
    if stroke:
        start = torch.rand((P, 2), generator=g) * torch.tensor([w, h])
        pts = [start]
        for _ in range(3 * nseg):
            pts.append(pts[-1] + torch.randn((P, 2), generator=g) * 6.0)
        pts = torch.stack(pts, 1)
        cub = torch.stack([pts[:, 0:-1:3], pts[:, 1::3], pts[:, 2::3], pts[:, 3::3]], 2)
        sw = (1.0 + 3.0 * torch.rand((P,), generator=g)).contiguous()
        return _finish(0, g, cub.reshape(P * nseg, 4, 2), P, nseg, h, w, S, stroke=sw)
    cx = torch.rand((P,), generator=g) * w
    cy = torch.rand((P,), generator=g) * h
    r = rmin + (rmax - rmin) * torch.rand((P,), generator=g)
    return _finish(0, g, _ring(g, cx, cy, r, nseg), P, nseg, h, w, S)
