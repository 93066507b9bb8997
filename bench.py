"""Benchmark: config 3 training step on one MI355X.

One step = render (fused binning + forward raster) of 4096 closed cubic paths
(4 segments, S=16) at 2040x1356 -> clamp(0,1) -> NCHW -> loss
MSE + 0.2 * (1 - SSIM(11, 1.5)) against the synthetic target -> backward ->
Adam on control points and colors.  Prints one JSON line (see the contract
in the repository's build notes).  --config N runs BASELINE.json's config N
instead (1-5, each with its own loss; see WORKLOADS).

python bench.py [--gpus 1] [--steps 100] [--warmup 10] [--config 3] [--no-cpu-baseline]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

SSIM_WEIGHT = 0.2
HBM_PEAK_GBS = 8000.0
# MI355X published fp32 compute peak (TFLOP/s); the vector ALUs reach it with
# packed FMAs, plain fp32 vector issue reaches half of it.
FP32_PEAK_TFLOPS = 157.3
# fp32 operations of one (pixel, edge) term of the reference's edge loop
# (cubic_splatting.py:1095-1134): distance 15 (2 sub, mul + fma, 2 clamp,
# 2 fma, mul + fma, min; fma = 2), crossing 6 (2 compares, mul + fma,
# compare).  Strokes have no crossing term.  A far edge's crossing term
# decided by its row span alone: 2 compares + 1 add.
FLOPS_DIST, FLOPS_CROSS, FLOPS_ROW = 15.0, 6.0, 3.0
FLOPS_PER_EVAL = {0: FLOPS_DIST + FLOPS_CROSS, 1: FLOPS_DIST}
RASTER_LABELS = {"cubic.fwd.rast": "raster_fwd", "cubic.bwd.rast": "raster_bwd"}
# Every stage of the step bracketed by HIP events in the sampled timed steps
# (device time of that stage's launches, on the step's own drifting scene).
STEP_LABELS = {"cubic.fwd.bin_prepare": "bin_prepare", "cubic.fwd.bin_finish": "bin_finish",
               "cubic.fwd.tile_order": "tile_order", "loss.clamp_mse_ssim": "loss_fwd",
               "loss.clamp_mse_ssim_bwd": "loss_bwd", "loss.mse_fwd": "mse_fwd",
               "loss.mse_bwd": "mse_bwd", "glue.clamp_nchw": "clamp_nchw",
               "glue.clamp_nchw_bwd": "clamp_nchw_bwd", "cubic.bwd.finalize": "finalize",
               "optim.adam": "adam", **RASTER_LABELS}
# The raster launches of every EVENT_EVERY-th timed step are bracketed by HIP
# events (two event records per launch cost the step about 4%; a sample of
# the steps gives the same mean launch time).
EVENT_EVERY = 4
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic_{kernel}_cfg{cfg}.json")


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--stage-iters", type=int, default=20)
    ap.add_argument("--copy-calibration-mib", type=int, default=0,
                    help="after the run, copy a buffer of this size three times (the "
                         "reference kernel for scaling rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    ap.add_argument("--next-rows", action="store_true",
                    help="instead of the training step, time the components either side of "
                         "the path (ring conversion, Adan, contribution outputs, the Gaussian "
                         "renderer, de Casteljau flattening) and print them as one JSON line")
    return ap.parse_args()


def make_problem(cfg):
    import torch
    from repo_amd import synth
    sc = synth.make_scene(cfg).to("cuda")
    cub = sc.cubics_norm.clone().requires_grad_(True)
    col = sc.colors.clone().requires_grad_(True)
    # Adam (gaussian_trace/model.py:185-189) as one HIP launch per step.
    from repo_amd.optim import Adam
    opt = Adam([cub, col], lr=1e-3)
    return sc, cub, col, opt


def render(sc, cub, col):
    import manbo
    if sc.stroke_widths is not None:
        return manbo.ops.render_cubic_polyline_splat_tilelang(
            cub, sc.seg_offsets, col, sc.opacities, sc.stroke_widths, sc.depths, sc.img_h,
            sc.img_w, 16, 16, sc.background, aa_widths=sc.aa_widths, distance_samples=sc.S)
    return manbo.ops.render_cubic_fill_splat_tilelang(
        cub, sc.seg_offsets, col, sc.opacities, sc.depths, sc.img_h, sc.img_w, 16, 16,
        sc.background, aa_widths=sc.aa_widths, distance_samples=sc.S)


# The configurations of BASELINE.json: workload text and SSIM weight of the
# loss (0: MSE only).
WORKLOADS = {
    1: ("64 closed cubic paths x 4 segments, S=8, 128x128, MSE", 0.0),
    2: ("512 closed cubic paths x 4 segments, S=16, 768x512, MSE+0.2*(1-SSIM 11x11 s=1.5)",
        SSIM_WEIGHT),
    3: ("4096 closed cubic paths x 4 segments, S=16, 2040x1356, "
        "MSE+0.2*(1-SSIM 11x11 s=1.5), Adam on control points+colors", SSIM_WEIGHT),
    4: ("8192 open cubic strokes x 3 segments, S=16, widths U[1,4] px, 1024x1024, MSE", 0.0),
    5: ("16384 closed cubic paths x 6 segments, S=32, 2048x2048, 70% of centres in 8 "
        "clusters, MSE+0.2*(1-SSIM 11x11 s=1.5)", SSIM_WEIGHT),
}


def loss_fn(img, target, ssim_weight):
    """clamp(0, 1) -> NCHW -> MSE + w (1 - SSIM), with the fused kernels that
    read the [H, W, 3] image in place (the same values as
    manbo.mse_loss_tilelang + manbo.ssim on
    img.clamp(0, 1).permute(2, 0, 1).unsqueeze(0)); MSE alone for w = 0."""
    import manbo
    from repo_amd import fused
    if ssim_weight == 0:
        return manbo.mse_loss_tilelang(fused.clamp_to_nchw(img), target)
    loss, _ = fused.clamp_mse_ssim_loss(img, target, ssim_weight)
    return loss


def train_step(sc, cub, col, opt, ssim_weight=SSIM_WEIGHT):
    opt.zero_grad(set_to_none=True)
    loss = loss_fn(render(sc, cub, col), sc.target, ssim_weight)
    loss.backward()
    opt.step()
    return loss


def stage_times(sc, iters):
    """Average ms of the main stages on scene ``sc`` (the step-0 scene: fresh
    control points and colours, so the figures do not drift with --steps),
    timed with HIP events on the stream the kernels are launched on (torch's
    current stream).  Every loss stage calls its kernels directly (no
    autograd in the loop), so the figures are device time of those kernels
    plus launch gaps."""
    import torch
    from repo_amd import _native as N, splat, metric
    ev = lambda: torch.cuda.Event(enable_timing=True)  # noqa: E731
    offs = sc.seg_offsets.to(torch.int32).contiguous()
    widths = torch.clamp(sc.aa_widths.float(), min=1e-4).contiguous()
    res = {}

    def timed(name, fn):
        fn()
        torch.cuda.synchronize()
        a, b = ev(), ev()
        a.record()
        for _ in range(iters):
            out = fn()
        b.record()
        torch.cuda.synchronize()
        res[name] = a.elapsed_time(b) / iters
        return out

    mode = splat.MODE_FILL if sc.stroke_widths is None else splat.MODE_STROKE
    cubd = sc.cubics_norm.contiguous()
    cold = sc.colors.contiguous()
    rules = sc.fill_rules.to(torch.int32).contiguous() if mode == 0 else None
    sw = sc.stroke_widths

    def do_bin():
        return splat.bin_primitives(cubd, offs, cold, sc.opacities, sc.depths, rules, widths, sw,
                                    sc.img_h, sc.img_w, sc.S, mode=mode)
    b = timed("binning_ms", do_bin)
    out, T, idx = timed("raster_fwd_ms", lambda: splat.rasterize_forward(b, sc.background))
    g = torch.randn_like(out)
    timed("raster_bwd_ms", lambda: splat.rasterize_backward(b, sc.background, T, idx, g))
    x = out.clamp(0, 1).permute(2, 0, 1).unsqueeze(0).contiguous()
    tgt = sc.target.contiguous()
    n = x.numel()
    stream = N.stream(x.device)
    timed("mse_fwd_ms", lambda: metric.mse_forward(x.view(-1), tgt.view(-1)))
    one = torch.ones((), dtype=torch.float32, device=x.device)
    gx = torch.empty_like(x)
    # the reference's MSE backward: gx = 2 g (x - y) / N (read x, y; write gx)
    timed("mse_bwd_ms", lambda: N.call("cs_mse_backward", N.ptr(x), N.ptr(tgt), n, N.ptr(one),
                                       N.ptr(gx), None, stream))
    timed("ssim_fwd_ms", lambda: metric._ssim_forward(x, tgt, 11, 1.5, 1e-4, 9e-4, False))
    _, abc, win = timed("ssim_fwd_grad_ms",
                        lambda: metric._ssim_forward(x, tgt, 11, 1.5, 1e-4, 9e-4, True))
    nc, h, w = 3, sc.img_h, sc.img_w
    scratch = metric._ssim_scratch(nc, h, w, 11, x.device)
    timed("ssim_bwd_ms", lambda: N.call("cs_ssim_backward", N.ptr(x), N.ptr(tgt), nc, h, w,
                                        N.ptr(win), 11, N.ptr(abc), N.ptr(one), 0, N.ptr(gx),
                                        N.ptr(scratch), stream))
    from repo_amd import fused
    timed("glue_clamp_nchw_ms", lambda: fused.clamp_to_nchw(out))
    # The step's fused loss on the renderer's image (its planar copy read in
    # place, clamped on load; MSE summed in the SSIM forward), its forward and
    # its backward kernel.
    out.requires_grad_(True)
    loss, _ = timed("loss_fused_fwd_ms",
                    lambda: fused.clamp_mse_ssim_loss(out, tgt, SSIM_WEIGHT))
    fn = loss.grad_fn
    planes = torch.empty((3, h, w), dtype=torch.float32, device=x.device)
    timed("loss_fused_bwd_ms", lambda: N.call(
        "cs_clamp_mse_ssim_backward", fn.saved_tensors[0].data_ptr(), fn.planar,
        N.ptr(fn.saved_tensors[1]), h, w, fn.lo, fn.hi, N.ptr(fn.g), fn.win_size,
        fn.work.data_ptr() + fn.abc_off, fn.ssim_weight, one.data_ptr(), planes.data_ptr(), 1,
        stream))
    res["num_intersects"] = b.num_intersects
    res["_binned"] = b
    res["_T"] = T
    res["_idx"] = idx
    return res


def opt_scene_intersects(sc, cub, col):
    """Intersection count of the scene as the timed steps left it."""
    import torch
    from repo_amd import splat
    mode = splat.MODE_FILL if sc.stroke_widths is None else splat.MODE_STROKE
    b = splat.bin_primitives(
        cub.detach().contiguous(), sc.seg_offsets.to(torch.int32).contiguous(),
        col.detach().contiguous(), sc.opacities, sc.depths,
        sc.fill_rules.to(torch.int32).contiguous() if mode == 0 else None,
        torch.clamp(sc.aa_widths.float(), min=1e-4).contiguous(), sc.stroke_widths, sc.img_h,
        sc.img_w, sc.S, mode=mode)
    return b.num_intersects


def binning_bytes(sc, n_isect):
    """Minimal HBM bytes of one binning (the algorithmic unit of its
    roofline): project 32 B read + 16 B written per segment, 16 B per
    flattened edge vertex pair written, and per intersection 12 B emitted,
    24 B for one sort pass (read + write of key and value) and 8 B of bins,
    plus 8 B of bins per tile."""
    nseg = int(sc.cubics_norm.shape[0])
    edges = nseg * (sc.S - 1)
    tiles = ((sc.img_w + 15) // 16) * ((sc.img_h + 15) // 16)
    parts = {"project": 48 * nseg, "flatten": 16 * edges, "emit": 12 * n_isect,
             "sort_one_pass": 24 * n_isect, "bins": 8 * n_isect + 8 * tiles}
    parts["total"] = sum(parts.values())
    return parts


def reference_edge_pixel_evals(b, T, idx):
    """(forward, backward) edge-pixel evaluations of the reference's kernels.
    Forward: every pixel evaluates all edges of each entry of its tile list up
    to and including the entry where it stops (T <= 1e-4), or the whole list.
    Backward: every entry with global index <= final_idx (the last entry that
    contributed)."""
    import torch
    H, W = b.img_h, b.img_w
    tbx = (W + 15) // 16
    pr = b.prim_recs.view(torch.int32)
    prim_edges = pr[:, 9] - pr[:, 8]   # the record's edge range [e0, e1)
    ent = prim_edges[b.primitive_ids_sorted.long()].to(torch.int64)
    csum = torch.zeros(ent.numel() + 1, dtype=torch.int64, device=ent.device)
    csum[1:] = torch.cumsum(ent, 0)
    ii = torch.arange(H, device=T.device).view(-1, 1).expand(H, W)
    jj = torch.arange(W, device=T.device).view(1, -1).expand(H, W)
    tile = (ii // 16) * tbx + (jj // 16)
    g0 = b.tile_bins[tile.reshape(-1), 0].long()
    g1 = b.tile_bins[tile.reshape(-1), 1].long()
    last = idx.reshape(-1).long()
    stop_f = torch.where(T.reshape(-1) <= 1e-4, last + 1, g1)
    stop_b = torch.maximum(torch.minimum(last + 1, g1), g0)
    fwd = int((csum[stop_f] - csum[g0]).sum())
    bwd = int((csum[stop_b] - csum[g0]).sum())
    return fwd, bwd


def performed_evaluations(b, bg, T, idx, v):
    """Edge terms the raster kernels evaluate (after their exact culling) in one
    forward and one backward launch on this scene: the counting entry points
    cs_rasterize_{forward,backward}_counted, run once outside the timed region.
    Returns {"raster_fwd": counts, "raster_bwd": counts} with counts =
    {dist, cross, row, entries, cover}."""
    import torch
    from repo_amd import splat
    res = {}
    for name in ("raster_fwd", "raster_bwd"):
        c = torch.zeros(5, dtype=torch.int64, device=T.device)
        if name == "raster_fwd":
            splat.rasterize_forward(b, bg, eval_counts=c)
        else:
            splat.rasterize_backward(b, bg, T, idx, v, eval_counts=c)
        d, x, r, e, cov = (int(t) for t in c.tolist())
        res[name] = {"dist": d, "cross": x, "row": r, "entries": e, "cover": cov}
    return res


def cpu_model_name():
    """The host CPU's model name (as lscpu prints it), or None."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def ssim_cpu(x, y, win_size=11, win_sigma=1.5, k1=0.01, k2=0.03):
    """SSIM of [N, C, H, W] tensors as the CPU baseline computes it: the
    separable Gaussian window as sums of shifted slices (torch's CPU conv2d
    is several times slower for 1 x 11 kernels), valid window, mean over
    pixels, channels and images (metric.py:215-273), differentiable."""
    import numpy as np
    import torch
    # The window in fp32, as the reference builds it (metric.py:47-61).
    r = np.arange(win_size, dtype=np.float32) - np.float32(win_size // 2)
    g = np.exp(-(r * r) / np.float32(2 * win_sigma ** 2)).astype(np.float32)
    g = torch.from_numpy(g / g.sum(dtype=np.float32)).to(x.dtype)
    z = torch.cat([x, y, x * x, y * y, x * y], 1)
    w = z.shape[-1] - win_size + 1
    z = sum(g[k] * z[..., k:k + w] for k in range(win_size))
    h = z.shape[-2] - win_size + 1
    z = sum(g[k] * z[..., k:k + h, :] for k in range(win_size))
    mu1, mu2, ex2, ey2, exy = z.chunk(5, 1)
    c1, c2 = k1 * k1, k2 * k2
    s1 = ex2 - mu1 * mu1
    s2 = ey2 - mu2 * mu2
    s12 = exy - mu1 * mu2
    m = ((2 * mu1 * mu2 + c1) / (mu1 * mu1 + mu2 * mu2 + c1)) * ((2 * s12 + c2) / (s1 + s2 + c2))
    return m.mean()


def cpu_train_step(sc, workers, ssim_weight):
    """One training step of scene ``sc`` on the CPU oracle: binning and the
    forward raster, clamp -> NCHW -> MSE (+ ssim_weight * (1 - SSIM) when
    ssim_weight > 0) in fp32 torch autograd (the reference's loss dtype)
    against the scene's target, the raster backward of that loss's image
    gradient, and an Adam update of control points and colors.  Returns
    per-stage seconds."""
    import numpy as np
    import torch
    from oracle import oracle as O
    t = {}
    t0 = time.perf_counter()
    fw = O.render_forward(sc.cubics_norm.numpy(), sc.seg_offsets.numpy(), sc.colors.numpy(),
                          sc.opacities.numpy(), sc.depths.numpy(), sc.img_h, sc.img_w,
                          sc.background.numpy(), fill_rules=sc.fill_rules.numpy(),
                          aa_widths=sc.aa_widths.numpy(), S=sc.S, workers=workers)
    t["forward"] = time.perf_counter() - t0
    t0 = time.perf_counter()
    img = torch.from_numpy(fw["out"]).requires_grad_(True)
    x = img.clamp(0, 1).permute(2, 0, 1).unsqueeze(0)
    y = sc.target
    loss = ((x - y) ** 2).mean()
    if ssim_weight > 0:
        loss = loss + ssim_weight * (1 - ssim_cpu(x, y))
    loss.backward()
    v = img.grad.float().numpy()
    t["loss"] = time.perf_counter() - t0
    t0 = time.perf_counter()
    g = O.render_backward(fw, v)
    t["backward"] = time.perf_counter() - t0
    t0 = time.perf_counter()
    params = [sc.cubics_norm.clone().requires_grad_(True), sc.colors.clone().requires_grad_(True)]
    params[0].grad = torch.from_numpy(np.asarray(g["v_cubics_norm"], np.float32)).view_as(params[0])
    params[1].grad = torch.from_numpy(np.asarray(g["v_colors"], np.float32)).view_as(params[1])
    torch.optim.Adam(params, lr=1e-3, foreach=False).step()
    t["adam"] = time.perf_counter() - t0
    t["step"] = sum(t.values())
    return t


def cpu_baseline(cfg):
    """The CPU oracle timed on the host's cores (threaded row bands, torch
    threads likewise): whole training steps of configs 1 (MSE) and 2
    (MSE + SSIM), one warm-up and the median of five each, then one whole
    step of the benchmarked config."""
    import statistics
    import torch
    from oracle import oracle as O
    from repo_amd import synth
    workers = O.default_workers()
    torch.set_num_threads(workers)
    others = {}
    for c, w in ((1, 0.0), (2, SSIM_WEIGHT)):
        if c == cfg:
            continue
        s = synth.make_scene(c)
        cpu_train_step(s, workers, w)
        med = statistics.median(cpu_train_step(s, workers, w)["step"] for _ in range(5))
        others[f"config{c}"] = {"value": round(1.0 / med, 3), "unit": "it/s",
                                "ms_per_step": round(1000.0 * med, 2),
                                "loss": "MSE" if w == 0 else f"MSE+{w}*(1-SSIM)"}
    st = cpu_train_step(synth.make_scene(cfg), workers, SSIM_WEIGHT)
    stages = ", ".join(f"{k} {v:.2f}s" for k, v in st.items() if k != "step")
    return {"value": round(1.0 / st["step"], 4), "unit": "it/s", "cores": workers,
            "kind": "port", "cpu_count": os.cpu_count(), "cpu_model": cpu_model_name(),
            "sample": (f"C oracle + fp32 torch losses on {workers} threads: one whole "
                       f"config{cfg} training step, nothing extrapolated ({stages}; "
                       f"{st['step']:.2f}s per step)"),
            "other_configs": others}


def load_traffic(kernel, cfg):
    """HBM bytes per launch of `kernel` measured with rocprofv3 FETCH_SIZE and
    WRITE_SIZE (the committed summary for this config), or None."""
    path = TRAFFIC_FILE.format(kernel=kernel, cfg=cfg)
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get("bytes_per_launch")


def copy_calibration(mib):
    import torch
    n = mib * (1 << 20) // 4
    src = torch.rand(n, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()


def _events_ms(fn, iters, warm=3):
    """Mean device ms of fn() over iters calls (HIP events on the current
    stream, after warm untimed calls)."""
    import torch
    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(iters):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / iters


def next_rows(iters=50):
    """Times of the components either side of the path, each on a stated
    synthetic workload (ms per call by HIP events, HBM GB/s where the bytes
    are plain): the closed-ring -> Hermite cubic conversion forward and
    backward, Adan against Adam on config 3's parameters, the cubic raster
    backward with and without the contribution outputs, the 2D Gaussian
    renderer, and config 3 rendered with de Casteljau against uniform
    flattening."""
    import torch
    import manbo
    from repo_amd import gaussian as G
    from repo_amd import optim, profiling, rings, splat, synth, _native
    rows = {}
    g = torch.Generator(device="cuda").manual_seed(7)

    # Ring conversion: train.py's cubic_fill model (K = 10 control points,
    # subdiv 4: 8 cubics per path) for config 3's 4096 paths.
    n, k = 4096, 10
    th = torch.linspace(0.0, 6.283185307179586, k + 1, device="cuda")[:k]
    cen = torch.rand((n, 1, 2), generator=g, device="cuda") * 1.6 - 0.8
    rad = torch.rand((n, 1, 1), generator=g, device="cuda") * 0.1 + 0.01
    cp = (cen + rad * torch.stack([th.cos(), th.sin()], -1)[None]).contiguous()
    cp.requires_grad_(True)
    segs, _ = rings.closed_cubic_fill_segments_tilelang(cp, subdiv=4)
    gseg = torch.randn(segs.shape, generator=g, device="cuda")
    fwd = _events_ms(lambda: rings.closed_cubic_fill_segments_tilelang(cp, subdiv=4), iters)

    def ring_fwd_bwd():
        s_, _ = rings.closed_cubic_fill_segments_tilelang(cp, subdiv=4)
        torch.autograd.grad(s_, cp, gseg)
    both = _events_ms(ring_fwd_bwd, iters)
    b_cp, b_seg = cp.numel() * 4, segs.numel() * 4
    rows["f1_rings"] = {
        "workload": f"{n} closed rings, K={k}, subdiv 4 -> {segs.shape[0]} cubics",
        "fwd_ms": round(fwd, 4), "bwd_ms": round(both - fwd, 4),
        "fwd_GBs": round((b_cp + b_seg) / fwd / 1e6, 1),
        "bwd_GBs": round((b_cp + b_seg) / max(both - fwd, 1e-6) / 1e6, 1)}

    # Optimizers on config 3's parameters (control points and colours).
    sc = synth.make_scene(3).to("cuda")
    params = [sc.cubics_norm.clone().requires_grad_(True), sc.colors.clone().requires_grad_(True)]
    for prm in params:
        prm.grad = torch.randn(prm.shape, generator=g, device="cuda") * 1e-3
    nparam = sum(prm.numel() for prm in params)
    times = {}
    for name, cls in (("adam", optim.Adam), ("adan", optim.Adan)):
        opt = cls(params, lr=1e-3)
        times[name] = _events_ms(opt.step, iters)
    rows["f2_optimizers"] = {
        "workload": f"config 3 parameters ({nparam} floats)",
        "adam_ms": round(times["adam"], 4), "adan_ms": round(times["adan"], 4),
        "adam_GBs": round(28 * nparam / times["adam"] / 1e6, 1),
        "adan_GBs": round(40 * nparam / times["adan"] / 1e6, 1)}

    # Contribution outputs: the cubic raster backward at config 3 with and
    # without curve_contrib_rgb / curve_isect_contrib.
    widths = torch.clamp(sc.aa_widths.float(), min=1e-4).contiguous()
    b = splat.bin_primitives(sc.cubics_norm.contiguous(), sc.seg_offsets.to(torch.int32).contiguous(),
                             sc.colors.contiguous(), sc.opacities, sc.depths,
                             sc.fill_rules.to(torch.int32).contiguous(), widths, None, sc.img_h,
                             sc.img_w, sc.S)
    img, T, idx = splat.rasterize_forward(b, sc.background)
    v = torch.randn(img.shape, generator=g, device="cuda") * 1e-3
    crgb = torch.zeros_like(sc.colors)
    cis = torch.zeros((b.num_intersects,), dtype=torch.float32, device="cuda")
    plain = _events_ms(lambda: splat.rasterize_backward(b, sc.background, T, idx, v), iters)
    contrib = _events_ms(lambda: splat.rasterize_backward(
        b, sc.background, T, idx, v, curve_contrib_rgb=crgb, curve_isect_contrib=cis), iters)
    rows["f2_contribution_outputs"] = {
        "workload": "config 3 raster backward (fresh zeroed accumulators per call)",
        "bwd_ms": round(plain, 4), "bwd_with_contrib_ms": round(contrib, 4)}

    # 2D Gaussian renderer: 100k Gaussians at 1024 x 1024, 16 x 16 tiles.
    ng, H, W = 100000, 1024, 1024
    u = lambda *sh: torch.rand(sh, generator=g, device="cuda")  # noqa: E731
    means, scales = u(ng, 2) * 2 - 1, 0.5 + u(ng, 2) * 5.5
    rot, colors, opac = (u(ng) * 2 - 1) * 4.0, u(ng, 3), 0.05 + u(ng) * 0.95
    bg = torch.tensor([0.5, 0.5, 0.5], device="cuda")
    proj = _events_ms(lambda: G.project_forward(means, scales, rot, H, W, 16, 16), iters)
    xys, depths, radii, conics, _ = G.project_forward(means, scales, rot, H, W, 16, 16)
    binning = _events_ms(lambda: G.bin_gaussians(xys, conics, radii, depths, H, W, 16, 16), iters)
    gb = G.bin_gaussians(xys, conics, radii, depths, H, W, 16, 16)
    rec = G.pack_records(xys, conics, colors, opac)
    rf = _events_ms(lambda: G.rasterize_forward(gb.gaussian_ids_sorted, gb.tile_bins, rec, bg, H,
                                                W, 16, 16), iters)
    out, fT, fi = G.rasterize_forward(gb.gaussian_ids_sorted, gb.tile_bins, rec, bg, H, W, 16, 16)
    vg = torch.randn(out.shape, generator=g, device="cuda") * 1e-3
    rb = _events_ms(lambda: G.rasterize_backward(gb.gaussian_ids_sorted, gb.tile_bins, rec, bg, H,
                                                 W, 16, 16, fT, fi, vg), iters)
    ins = [t.clone().requires_grad_(True) for t in (means, scales, rot, colors, opac)]

    def gs_step():
        o = manbo.gs_render(*ins, H, W, 16, 16, bg)
        o.backward(vg)
    step = _events_ms(gs_step, iters)
    rows["f3_gaussian_renderer"] = {
        "workload": f"{ng} Gaussians, {W}x{H}, 16x16 tiles, {int(gb.num_intersects)} intersections",
        "project_ms": round(proj, 4), "binning_ms": round(binning, 4),
        "raster_fwd_ms": round(rf, 4), "raster_bwd_ms": round(rb, 4),
        "render_fwd_bwd_ms": round(step, 4)}

    # de Casteljau against uniform flattening: config 3's render forward and
    # backward through the reference entry point, per-stage device times.
    cub = sc.cubics_norm.clone().requires_grad_(True)
    col = sc.colors.clone().requires_grad_(True)
    vimg = torch.randn((sc.img_h, sc.img_w, 3), generator=g, device="cuda") * 1e-3
    for method in ("bernstein", "de_casteljau"):
        def render_step():
            o = manbo.ops.render_cubic_fill_splat_tilelang(
                cub, sc.seg_offsets, col, sc.opacities, sc.depths, sc.img_h, sc.img_w, 16, 16,
                sc.background, aa_widths=sc.aa_widths, distance_samples=sc.S,
                flatten_method=method)
            o.backward(vimg)
        total = _events_ms(render_step, iters)
        timer = profiling.EventTimer(STEP_LABELS, reserve=iters + 1)
        _native.set_profile_ctx_factory(timer)
        for _ in range(iters):
            render_step()
        torch.cuda.synchronize()
        _native.set_profile_ctx_factory(None)
        stages = {STEP_LABELS[lab]: round(timer.mean_ms(lab), 4) for lab in STEP_LABELS
                  if timer.count(lab)}
        timer.close()
        rows.setdefault("f4_de_casteljau", {"workload": "config 3 render forward + backward"})
        rows["f4_de_casteljau"][method] = {"fwd_bwd_ms": round(total, 4), "stages_ms": stages}
    return rows


def main():
    args = parse()
    if args.next_rows:
        if args.gpus != 1:
            sys.exit(2)
        print(json.dumps({"next_rows": next_rows(), "n_gpus": 1, "data": "synthetic"}),
              flush=True)
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only (several GPUs would each "
                                   "own a band of tile rows; not implemented here)",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    import torch
    from repo_amd import _native, profiling
    torch.backends.cudnn.benchmark = False
    workload, ssim_weight = WORKLOADS[args.config]
    sc, cub, col, opt = make_problem(args.config)
    for _ in range(args.warmup):
        train_step(sc, cub, col, opt, ssim_weight)
    # The raster launches of every EVENT_EVERY-th timed step are bracketed by
    # HIP events on the stream they run on (torch's current stream).
    timer = profiling.EventTimer(RASTER_LABELS, reserve=args.steps // EVENT_EVERY + 1)
    _native.set_profile_ctx_factory(timer)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        timer.enabled = i % EVENT_EVERY == 0
        loss = train_step(sc, cub, col, opt, ssim_weight)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    _native.set_profile_ctx_factory(None)
    ms = 1000.0 * elapsed / max(1, args.steps)
    launch_ms = {RASTER_LABELS[k]: timer.mean_ms(k) for k in RASTER_LABELS}
    timer.close()
    # After the timed region: a few more steps with every stage bracketed by
    # HIP events (the per-stage device times of the step, not counted in value).
    n_prof = max(4, args.steps // 5)
    timer = profiling.EventTimer(STEP_LABELS, reserve=n_prof + 1)
    _native.set_profile_ctx_factory(timer)
    for _ in range(n_prof):
        train_step(sc, cub, col, opt, ssim_weight)
    torch.cuda.synchronize()
    _native.set_profile_ctx_factory(None)
    step_ms = {v: round(timer.mean_ms(k), 4) for k, v in STEP_LABELS.items()
               if timer.pairs[k]}
    timer.close()
    n_isect_end = int(opt_scene_intersects(sc, cub, col))
    from repo_amd import synth
    st = stage_times(synth.make_scene(args.config).to("cuda"), args.stage_iters)
    b, T, idx = st.pop("_binned"), st.pop("_T"), st.pop("_idx")
    evals_fwd, evals_bwd = reference_edge_pixel_evals(b, T, idx)
    performed = performed_evaluations(b, sc.background, T, idx,
                                      torch.randn((sc.img_h, sc.img_w, 3), device="cuda"))
    n_img = 3 * sc.img_h * sc.img_w
    kern = {k: round(v, 4) for k, v in st.items() if k.endswith("_ms")}
    gbs = lambda nbytes, ms_: nbytes / (ms_ * 1e-3) / 1e9  # noqa: E731
    kern["stage_scene"] = "step 0 (fresh control points and colours)"
    kern["mse_fwd_GBs"] = round(gbs(8 * n_img, st["mse_fwd_ms"]), 1)
    kern["mse_bwd_GBs"] = round(gbs(12 * n_img, st["mse_bwd_ms"]), 1)
    kern["ssim_fwd_GBs"] = round(gbs(8 * n_img, st["ssim_fwd_ms"]), 1)
    kern["ssim_bwd_GBs"] = round(gbs(12 * n_img, st["ssim_bwd_ms"]), 1)
    kern["in_step_launch_ms"] = step_ms
    kern["in_step_note"] = ("HIP-event means of each stage's launches in %d training steps "
                            "right after the timed ones (same scene as Adam moves it)" % n_prof)
    kern["reference_edge_pixel_evals"] = {"raster_fwd": evals_fwd, "raster_bwd": evals_bwd}
    kern["binning_algorithmic_bytes"] = binning_bytes(sc, st["num_intersects"])
    kern["timed_region_launch_ms"] = {k: round(v, 4) for k, v in launch_ms.items()}
    kern["performed_evaluations"] = performed
    # Dominant kernel: the longer raster launch of the timed steps.  Its
    # algorithmic work is the edge terms it evaluates (distance 15 flops,
    # crossing 6), counted by the counting instantiation on the same scene;
    # the time is the HIP-event mean of its launches in the timed steps.
    dom = max(launch_ms, key=lambda k: launch_ms[k])
    dom_ms = launch_ms[dom]
    pc = performed[dom]
    flops = pc["dist"] * FLOPS_DIST + pc["cross"] * FLOPS_CROSS + pc["row"] * FLOPS_ROW
    achieved = flops / (dom_ms * 1e-3) / 1e12
    ref_units = evals_bwd if dom == "raster_bwd" else evals_fwd
    ref_equiv = ref_units * FLOPS_PER_EVAL[b.mode] / (dom_ms * 1e-3) / 1e12
    # "bound": the raster is bound by the fp32 vector ALUs (the compute roof;
    # it issues no matrix instruction), not by HBM.
    roofline = {"bound": "valu", "compute": "fp32 vector ALU (no matrix instructions)",
                "achieved": round(achieved, 3), "peak": FP32_PEAK_TFLOPS,
                "unit": "TFLOP/s", "frac": round(achieved / FP32_PEAK_TFLOPS, 4),
                "traffic": load_traffic(dom, args.config), "kernel": dom,
                "launch_ms": round(dom_ms, 4),
                "units_per_launch": {"dist_terms": pc["dist"], "cross_terms": pc["cross"],
                                     "row_cross_terms": pc["row"]},
                "flops_per_unit": {"dist": FLOPS_DIST, "cross": FLOPS_CROSS, "row": FLOPS_ROW},
                "reference_equivalent_TFLOPs": round(ref_equiv, 2),
                "note": "fp32 vector-ALU compute roof (no matrix instructions on this path), "
                        "priced against the published fp32 peak; units are the (edge, pixel) "
                        "terms the kernel evaluates after its exact culling. "
                        "reference_equivalent_TFLOPs prices the reference kernel's full "
                        "edge loop over the same launch time"}
    line = {
        "metric": ("train it/s, 4096 closed cubics @2040x1356 fp32" if args.config == 3
                   else f"train it/s, config {args.config} fp32"),
        "value": round(1000.0 / ms, 3), "unit": "it/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": f"config{args.config}: {workload}",
                   "num_intersects": st["num_intersects"],
                   "num_intersects_after_timed_steps": n_isect_end,
                   "final_loss": float(loss)},
        "kernels": kern, "roofline": roofline,
    }
    # The CPU step of configs 4 and 5 would take minutes; their lines carry
    # no cpu_baseline.
    if not args.no_cpu_baseline and args.config in (1, 2, 3):
        line["cpu_baseline"] = cpu_baseline(args.config)
    if args.copy_calibration_mib > 0:
        copy_calibration(args.copy_calibration_mib)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
