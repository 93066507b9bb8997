"""Host side of the cubic splat path: binning, rasterization and the two
``torch.autograd.Function``s that replace the reference's
``_CubicFillSplatFunction`` (ops/cubic_splatting.py:2750-3125) and
``_CubicPolylineSplatFunction`` (ops/cubic_polyline_splatting.py:962-1338).

Every device computation is a call into libcubicsplat_hip.so on torch's
current stream; there is no CPU or torch fallback.  Buffers come from torch's
caching allocator.  One host synchronization per forward reads the
intersection count to size the per-intersection buffers (the reference makes
the same read at cubic_splatting.py:2879).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Callable, Mapping, MutableMapping, Optional

import torch

from . import _native as N

BLOCK_X = 16
BLOCK_Y = 16
DEFAULT_THREADS = 256
DEFAULT_AABB_PAD = 1.0
DEFAULT_AA_WIDTH = 1.0
DEFAULT_DISTANCE_SAMPLES = 24
CUBIC_FLATTEN_METHOD_BERNSTEIN = "bernstein"
CUBIC_FLATTEN_METHOD_DE_CASTELJAU = "de_casteljau"
DEFAULT_CUBIC_FLATTEN_METHOD = CUBIC_FLATTEN_METHOD_BERNSTEIN
_FLATTEN_ALIASES = {
    "bernstein": CUBIC_FLATTEN_METHOD_BERNSTEIN,
    "de_casteljau": CUBIC_FLATTEN_METHOD_DE_CASTELJAU,
    "decasteljau": CUBIC_FLATTEN_METHOD_DE_CASTELJAU,
    "de-casteljau": CUBIC_FLATTEN_METHOD_DE_CASTELJAU,
}

CubicProcessPayload = MutableMapping[str, Any]
CubicProcessFn = Callable[[str, CubicProcessPayload], Optional[Mapping[str, Any]]]
CubicFillProcessPayload = CubicProcessPayload
CubicFillProcessFn = CubicProcessFn

MODE_FILL = 0
MODE_STROKE = 1


def normalize_cubic_flatten_method(method: object) -> str:
    """cubic_splatting.py:67-78."""
    raw = str(method).strip().lower()
    key = _FLATTEN_ALIASES.get(raw, raw)
    if key not in {CUBIC_FLATTEN_METHOD_BERNSTEIN, CUBIC_FLATTEN_METHOD_DE_CASTELJAU}:
        raise ValueError(
            "flatten_method must be one of "
            f"{sorted(_FLATTEN_ALIASES.keys())}, got {method!r}")
    return key


def _run_process_fn(process_fn, stage, payload):
    """cubic_splatting.py:42-52."""
    if process_fn is None:
        return payload
    updates = process_fn(stage, payload)
    if updates:
        payload.update(updates)
    return payload


def _f32(t: torch.Tensor) -> torch.Tensor:
    if t.dtype is torch.float32 and t.is_contiguous():
        return t.detach()
    return t.detach().to(torch.float32).contiguous()


def image_grad_layout(v: torch.Tensor):
    """(tensor, planar) for an upstream image gradient of shape [H, W, 3]:
    the gradient itself when it is float32 and [H, W, 3]-contiguous
    (planar 0), or, when it is an [H, W, 3] view of three contiguous [H, W]
    planes (as the fused loss's backward returns it), its planes (planar 1);
    otherwise a contiguous float32 copy."""
    v = v.detach()
    if v.dtype is torch.float32 and v.dim() == 3 and v.shape[2] == 3:
        if v.is_contiguous():
            return v, 0
        h, w = int(v.shape[0]), int(v.shape[1])
        if v.stride() == (w, 1, h * w):
            return v.permute(2, 0, 1), 1
    return v.to(torch.float32).contiguous(), 0


def attach_planar_copy(img: torch.Tensor, planes: torch.Tensor) -> None:
    """Attach to the renderer's [H, W, 3] image the [3, H, W] planes its launch
    also wrote, with the image's version counter at that time."""
    img._cs_planar_copy = (planes, img._version)


def planar_copy_of(img: torch.Tensor):
    """The [3, H, W] planes the renderer wrote beside its [H, W, 3] image, or
    None (another tensor, or the image was modified in place since)."""
    pc = getattr(img, "_cs_planar_copy", None)
    if pc is None or img._version != pc[1]:
        return None
    return pc[0]


def _i32(t: torch.Tensor) -> torch.Tensor:
    if t.dtype is torch.int32 and t.is_contiguous():
        return t.detach()
    return t.detach().to(torch.int32).contiguous()


def tile_bounds(img_h: int, img_w: int, block_x: int = BLOCK_X, block_y: int = BLOCK_Y):
    return ((img_w + block_x - 1) // block_x, (img_h + block_y - 1) // block_y, 1)


def sub_blocks(img_h: int, img_w: int) -> int:
    """The raster's workgroups: 16 x 16 sub-blocks of the image."""
    return ((img_w + BLOCK_X - 1) // BLOCK_X) * ((img_h + BLOCK_Y - 1) // BLOCK_Y)


# Buffers of one binning, carved from one arena allocation: name -> (dtype,
# shape).  Shapes depend on (nseg, P, S, T, scratch sizes).
def _binning_fields(nseg, P, E, T, nsub, radix_elems, scan_elems, grad_elems, list_elems,
                    adaptive=False):
    f32, i32 = torch.float32, torch.int32
    extra = ((("seg_edge_offsets", i32, (nseg + 1,)), ("edge_aux", i32, (E, N.EDGE_AUX_INTS)),
              ("leaf_counts", i32, (nseg,))) if adaptive else ())
    return extra + (
        ("cubics_px", f32, (nseg, 4, 2)),
        ("seg_tile_ranges", i32, (nseg, 4)),
        ("seg_recs", i32, (nseg, N.SEG_RECORD_INTS)),
        ("edges", f32, (E, N.EDGE_RECORD_FLOATS)),
        ("edge_culls", i32, (E, N.EDGE_CULL_INTS)),
        ("prim_tile_ranges", i32, (P, 4)),
        ("num_tiles_hit", i32, (P,)),
        ("inv_sigma2s", f32, (P,)),
        ("prim_recs", f32, (P, N.PRIM_RECORD_FLOATS)),
        ("keys", i32, (P,)),
        ("order", i32, (P,)),
        ("keys_alt", i32, (P,)),
        ("vals_alt", i32, (P,)),
        ("radix_counts", i32, (radix_elems,)),
        ("scan_temp", i32, (scan_elems,)),
        ("rank_tile_ranges", i32, (P, 4)),
        ("tile_count", i32, (list_elems,)),
        ("tile_scratch", i32, (list_elems,)),
        ("status", i32, (4,)),
        ("tile_bins", i32, (T, 2)),
        ("wave_cost", i32, (2 * nsub,)),
        ("grad_accum", f32, (grad_elems,)),
    )


_ALIGN = 256
_LAYOUTS: "dict[tuple, tuple]" = {}


def _layout(key, fields):
    """{name: (byte offset, dtype, shape)} and the total size, cached per key."""
    lay = _LAYOUTS.get(key)
    if lay is None:
        off, table = 0, {}
        for name, dt, shape in fields:
            n = 1
            for d in shape:
                n *= int(d)
            table[name] = (off, dt, tuple(int(d) for d in shape))
            off += (n * torch.empty((), dtype=dt).element_size() + _ALIGN - 1) // _ALIGN * _ALIGN
        if len(_LAYOUTS) >= 64:
            _LAYOUTS.pop(next(iter(_LAYOUTS)))
        lay = _LAYOUTS[key] = (table, max(off, _ALIGN))
    return lay


class Binned:
    """Everything the forward produces that the backward (and tests) use.
    The binning buffers live in one arena; `ptr(name)` is a buffer's device
    address and the attribute of the same name its tensor view (made on
    first use): cubics_px [nseg,4,2], seg_tile_ranges [nseg,4], seg_recs
    [nseg,8] (cull ranges), edges [E,8] (x0 y0 x1 y1 vx vy ux uy), edge_culls
    [E,4], prim_tile_ranges [P,4], num_tiles_hit [P], inv_sigma2s [P],
    prim_recs [P,20], order [P] (depth rank -> primitive id), tile_bins [T,2],
    grad_accum (the backward's accumulators, cleared by the binning's last
    launch).  With the adaptive (de Casteljau) flattening also
    seg_edge_offsets [nseg+1] (segment -> edge CSR), edge_aux [E,4]
    (segment, t0, t1 bits) and leaf_counts [nseg]; E is then the capacity
    nseg * 2^ceil(log2(samples - 1)) and seg_edge_offsets[-1] the edge count."""

    def __init__(self, *, mode, img_h, img_w, samples, nseg, nprim, arena, table,
                 adaptive=False, ntiles=None, block_x=BLOCK_X, block_y=BLOCK_Y):
        self.mode, self.img_h, self.img_w, self.samples = mode, img_h, img_w, samples
        self.device = arena.device
        self.ntiles = int(table["tile_bins"][2][0]) if ntiles is None else int(ntiles)
        # The raster's tiles: block_x x block_y pixels, rasterized as 16 x 16
        # sub-blocks of two waves each, all of a tile's waves on its list.
        self.block_x, self.block_y = int(block_x), int(block_y)
        self.nsub = sub_blocks(img_h, img_w)
        self.waves_per_tile = 2 * (self.block_x // BLOCK_X) * (self.block_y // BLOCK_Y)
        # Tiles whose sides are not multiples of 16 take the any-size kernels
        # (a lane per pixel, no raster log, no tile order).
        self.any_tile = not is_sub_block_tile(self.block_x, self.block_y)
        self.adaptive = adaptive
        self.nseg, self.nprim = nseg, nprim
        self.num_intersects = -1
        self.arena = arena
        self._table = table
        self._base = arena.data_ptr()
        self._views = {}
        self.primitive_ids_sorted: Optional[torch.Tensor] = None
        # Heavy-first tile order from this forward's raster (for the backward).
        self.tile_order: Optional[torch.Tensor] = None
        # The forward's raster log, for the backward: the per-(list entry,
        # wave) record index and the record pool (None: no log was written;
        # the backward then recomputes every entry's geometry).
        self.log_index: Optional[torch.Tensor] = None
        self.log_pool: Optional[torch.Tensor] = None
        # Scene-shape key of the log's sizing, and the 16-byte units per list
        # entry of each wave's own log region in this forward.
        self.log_key = None
        self.log_units = 0
        self.grad_accum_clean = True
        # The last 4 words of grad_accum (zeroed with it by the binning) count
        # the raster log's shared blocks of the first forward after a binning;
        # log_ctr = (address, first shared unit) when a forward used them.
        self.log_ctr_clean = True
        self.log_ctr = None
        # Set while the intersection count has not been read on the host yet
        # (bin_primitives with a capacity hint); resolve_binned() settles it.
        self.pending: Optional["_PendingCount"] = None

    def ptr(self, name: str) -> int:
        return self._base + self._table[name][0]

    def __getattr__(self, name):
        table = self.__dict__.get("_table")
        if table is None or name not in table:
            raise AttributeError(name)
        v = self._views.get(name)
        if v is None:
            off, dt, shape = table[name]
            n = 1
            for d in shape:
                n *= d
            nbytes = n * torch.empty((), dtype=dt).element_size()
            v = self.arena[off:off + nbytes].view(dt).view(shape)
            self._views[name] = v
        return v

    @property
    def edges_per_segment(self) -> int:
        """Uniform flattening: S - 1; adaptive: 0 (edge ranges are in the records)."""
        return 0 if self.adaptive else self.samples - 1

    def num_edges(self) -> int:
        """Edge count (a host read for the adaptive flattening)."""
        if self.adaptive:
            return int(self.seg_edge_offsets[-1].item())
        return self.nseg * (self.samples - 1)

    def edges_px(self) -> torch.Tensor:
        """Edges in the reference's [E,2,2] layout."""
        return self.edges[: self.num_edges(), :4].reshape(-1, 2, 2)


@dataclass
class _PendingCount:
    # (pinned int32 [4] that receives the status words, raw hipEvent_t
    # recorded after the launch or copy that writes them, device index, the
    # buffer's device-accessible address or None)
    pinned: tuple
    capacity: int               # elements of the primitive_ids_sorted buffer
    finish: Callable[[int], torch.Tensor]  # cs_bin_finish into a new buffer of that size


# Pinned status buffers and their (raw, non-timing) events per device, reused
# across forwards.
_PINNED_POOL: "dict[int, list]" = {}


def _take_pinned(dev_index: int):
    pool = _PINNED_POOL.get(dev_index)
    if pool:
        return pool.pop()
    with torch.cuda.device(dev_index):
        host = torch.empty((4,), dtype=torch.int32, pin_memory=True)
        return (host, N.event_create(), dev_index, N.host_device_ptr(host.data_ptr()))


def _give_pinned(entry) -> None:
    pool = _PINNED_POOL.setdefault(entry[2], [])
    if len(pool) < 16:
        pool.append(entry)
    else:
        N.event_destroy(entry[1])


# Arena fields passed to cs_bin_prepare / cs_bin_finish, in argument order.
_PREP_FIELDS = ("cubics_px", "seg_tile_ranges", "seg_recs", "edges", "edge_culls",
                "prim_tile_ranges", "num_tiles_hit", "inv_sigma2s", "prim_recs", "keys", "order",
                "keys_alt", "vals_alt", "radix_counts", "scan_temp", "rank_tile_ranges",
                "tile_count", "tile_scratch", "status")
_DECAS_FIELDS = ("seg_edge_offsets", "edge_aux", "leaf_counts")


@dataclass
class _BinPlan:
    """Arena layout of one binning shape and the byte offsets of the fields
    each launch takes (computed once per shape)."""
    table: dict
    nbytes: int
    prep: tuple
    decas: tuple
    ntiles: int
    grad_n: int


_PLANS: "dict[tuple, _BinPlan]" = {}


def _bin_plan(key, lib, nseg, P, S, img_h, img_w, block_x, block_y, mode, adaptive, per_seg):
    plan = _PLANS.get(key)
    if plan is None:
        tbx, tby, _ = tile_bounds(img_h, img_w, block_x, block_y)
        T = tbx * tby
        fields = _binning_fields(nseg, P, nseg * per_seg, T, sub_blocks(img_h, img_w),
                                 int(lib.cs_radix_counts_elems(P)),
                                 int(lib.cs_scan_temp_elems(max(P, T, nseg))),
                                 _grad_accum_elems(nseg, P, mode),
                                 int(lib.cs_bin_list_elems(P, img_h, img_w, block_x, block_y)),
                                 adaptive)
        table, nbytes = _layout(key, fields)
        plan = _BinPlan(table=table, nbytes=nbytes,
                        prep=tuple(table[f][0] for f in _PREP_FIELDS),
                        decas=tuple(table[f][0] for f in _DECAS_FIELDS) if adaptive else (),
                        ntiles=T, grad_n=table["grad_accum"][2][0])
        if len(_PLANS) >= 64:
            _PLANS.pop(next(iter(_PLANS)))
        _PLANS[key] = plan
    return plan


def bin_primitives(cubics_norm, seg_offsets, colors, opacities, depths, fill_rules, widths,
                   stroke_widths, img_h, img_w, samples, *, aabb_pad=DEFAULT_AABB_PAD,
                   aniso=False, mode=MODE_FILL, block_x=BLOCK_X, block_y=BLOCK_Y,
                   capacity_hint=None, flatten_method=CUBIC_FLATTEN_METHOD_BERNSTEIN) -> Binned:
    """Project, flatten and bin (cubic_splatting.py:2815-2908).  All inputs are
    contiguous device tensors of the reference's dtypes.  Without
    capacity_hint the host reads the intersection count before the lists are
    built; with it, the lists go into a buffer of that many entries and the
    result is pending until resolve_binned()."""
    dev = cubics_norm.device
    lib = N.lib()
    nseg = int(cubics_norm.shape[0])
    P = int(seg_offsets.numel()) - 1
    S = max(2, int(samples))
    adaptive = flatten_method == CUBIC_FLATTEN_METHOD_DE_CASTELJAU
    if adaptive:
        per_seg = int(lib.cs_de_casteljau_max_edges_per_segment(S))
        if per_seg <= 0 or nseg * per_seg >= 2 ** 31:
            raise ValueError(
                f"de_casteljau flattening of {nseg} segments with distance_samples={S} "
                "exceeds the supported edge count (2^31 - 1, depth <= 24)")
    else:
        per_seg = S - 1
    key = (dev.index, mode, nseg, P, S, img_h, img_w, block_x, block_y, adaptive)
    plan = _bin_plan(key, lib, nseg, P, S, img_h, img_w, block_x, block_y, mode, adaptive,
                     per_seg)
    arena = torch.empty((plan.nbytes,), dtype=torch.uint8, device=dev)
    b = Binned(mode=mode, img_h=img_h, img_w=img_w, samples=S, nseg=nseg, nprim=P, arena=arena,
               table=plan.table, adaptive=adaptive, ntiles=plan.ntiles, block_x=block_x,
               block_y=block_y)
    base = b._base
    st = N.stream(dev)
    args = [N.ptr(cubics_norm), N.ptr(seg_offsets), N.ptr(colors), N.ptr(opacities),
            N.ptr(depths), N.ptr(fill_rules), N.ptr(widths), N.ptr(stroke_widths), nseg, P,
            img_h, img_w, block_x, block_y, S, float(aabb_pad), int(bool(aniso)), mode]
    args += [base + o for o in plan.prep]
    with N.prof("cubic.fwd.bin_prepare"):
        if adaptive:
            N.call("cs_bin_prepare_de_casteljau", *args, *[base + o for o in plan.decas], st)
        else:
            N.call("cs_bin_prepare", *args, st)
    q = b.ptr
    order_p, ranks_p, status_p = q("order"), q("rank_tile_ranges"), q("status")
    count_p, scratch_p = q("tile_count"), q("tile_scratch")
    bins_p, grad_p, grad_n = q("tile_bins"), q("grad_accum"), plan.grad_n

    def finish(capacity: int, status_dev=None) -> torch.Tensor:
        ids = torch.empty((capacity,), dtype=torch.int32, device=dev)
        with N.prof("cubic.fwd.bin_finish"):
            N.call("cs_bin_finish", order_p, ranks_p, P, status_p, capacity, img_h, img_w,
                   block_x, block_y, count_p, scratch_p, ids.data_ptr(), bins_p,
                   grad_p, grad_n, status_dev, st)
        return ids

    # The one host read of the forward (the reference reads the same count,
    # cubic_splatting.py:2879).  With a capacity hint the lists are built into
    # a buffer of that size first and the count is checked afterwards, so the
    # GPU does not idle while the host waits for it; the list launch then also
    # writes the status words to the pinned buffer (no copy of their own).
    pinned = _take_pinned(dev.index if dev.index is not None else torch.cuda.current_device())
    status_host, event, status_dev = pinned[0], pinned[1], pinned[3]
    hip = N.hip()
    pending = _PendingCount(pinned, -1, finish)
    if capacity_hint is None or status_dev is None:
        N.hip_check(hip.hipMemcpyAsync(status_host.data_ptr(), status_p, 16,
                                       N.HIP_MEMCPY_DEVICE_TO_HOST, st), "hipMemcpyAsync")
        N.hip_check(hip.hipEventRecord(event, st), "hipEventRecord")
    if capacity_hint is None:
        I = _read_count(pending, nseg)
        b.primitive_ids_sorted = finish(I)
        b.num_intersects = I
    else:
        pending.capacity = max(0, int(capacity_hint))
        if status_dev is None:
            b.primitive_ids_sorted = finish(pending.capacity)
        else:
            b.primitive_ids_sorted = finish(pending.capacity, status_dev)
            N.hip_check(hip.hipEventRecord(event, st), "hipEventRecord")
        b.pending = pending
    return b


# Words at the end of the gradient buffer for the raster log's counter (16 B).
_LOG_COUNTER_ELEMS = 4


def _grad_accum_elems(nseg: int, nprim: int, mode: int) -> int:
    """The backward's accumulators (v_cubics_px, then the per-primitive
    gradients) followed by the copies the backward sums the per-primitive
    gradients into (cs_raster_prim_scratch_elems), all zero, then the
    forward's raster-log counter word (and padding to 16 bytes)."""
    nv = 6 if mode == MODE_STROKE else 5
    return (nseg * 8 + nprim * nv + int(N.lib().cs_raster_prim_scratch_elems(nprim, mode))
            + _LOG_COUNTER_ELEMS)


def _read_count(pending: "_PendingCount", nseg: int) -> int:
    status_host, event = pending.pinned[0], pending.pinned[1]
    N.hip_check(N.hip().hipEventSynchronize(event), "hipEventSynchronize")
    I, bad, first, last = status_host.tolist()
    _give_pinned(pending.pinned)
    if bad or first != 0 or last != nseg:
        raise ValueError(
            "primitive_seg_offsets must start at 0 and end at num_segments "
            f"(got start={first}, end={last}, num_segments={nseg})"
            + ("; offsets are not non-decreasing within [0, num_segments]" if bad else ""))
    if I < 0:
        raise RuntimeError(f"intersection count overflowed int32 ({I})")
    return I


def resolve_binned(b: Binned) -> bool:
    """Reads the intersection count of a deferred bin_primitives call and sets
    num_intersects / primitive_ids_sorted.  Returns True when the lists did
    not fit the hinted buffer and were rebuilt at full size (outputs computed
    from the first build must then be computed again)."""
    pend = b.pending
    if pend is None:
        return False
    I = _read_count(pend, b.nseg)
    b.pending = None
    b.num_intersects = I
    if I <= pend.capacity:
        b.primitive_ids_sorted = b.primitive_ids_sorted[:I]
        return False
    b.primitive_ids_sorted = pend.finish(I)
    b.grad_accum_clean = True
    b.log_ctr_clean = True
    return True


def intersection_capacity(num_intersects: int) -> int:
    """Buffer size hint for the next forward of a scene whose last count was
    num_intersects: 25% headroom, rounded up to 4096."""
    want = num_intersects + num_intersects // 4 + 4096
    return (want + 4095) // 4096 * 4096


# Heavy-first tile orders (cs_raster_tile_order) per (device, stream, tile
# count): the order the last forward's wave durations gave, which the next
# forward of an image with that many tiles on that stream starts from.  Any
# permutation gives the same results, so a stale order only changes speed;
# keying by stream keeps a forward from reading an order another stream is
# still writing.
_TILE_ORDERS: "dict[tuple, torch.Tensor]" = {}
_ORDER_AGE: "dict[tuple, int]" = {}   # forwards since the order was made
# Per key, the sub-block costs the last order was made from (a running
# average over the orders, cs_raster_tile_order_averaged) and a spare buffer
# for the next ones.
_TILE_COSTS: "dict[tuple, tuple]" = {}
_MAX_ORDERS = 16
# A new heavy-first order is made from every ORDER_EVERY-th forward's wave
# durations (a tile's cost changes slowly between training steps: every 4th
# and every 8th forward gave the same raster times, and the ordering launch
# costs the step it runs in about 16 us at config 3); the forwards in between
# reuse it and record no durations.  Any order gives the same results.
ORDER_EVERY = 8
# Sort within each XCD's contiguous tile range (keeps each XCD's L2 on its own
# part of the image) rather than across all tiles.
ORDER_CHUNKED = True


# Raster-log sizing per scene shape: each wave's own region holds
# `units per entry` 16-byte units for every entry of its tile's list; records
# that do not fit go to shared blocks after the regions.  The shared blocks a
# forward used are read back without waiting (an async copy of the pool's
# counter into pinned memory, polled by the next forward of the shape), and
# grow the regions of the next forward.
_LOG_PENDING: "dict[tuple, tuple]" = {}   # key -> ((pinned [4], event, device), units,
#                                            first shared unit, pool bytes, the counter's
#                                            value for no shared block)
_LOG_UNITS: "dict[tuple, int]" = {}       # key -> units per entry of the next forward
_MAX_LOG_KEYS = 64
# Units per (list entry, wave) of the first forward of a shape (the benchmark
# scenes record about 64 bytes, i.e. 4 units, on average).
LOG_FIRST_UNITS_PER_ENTRY = 6
LOG_MAX_UNITS_PER_ENTRY = 66     # a record is at most 66 units


def _poll_log_use(key) -> None:
    pend = _LOG_PENDING.get(key)
    if pend is None:
        return
    entry, units, first_shared, pool_bytes, zero = pend
    if N.hip().hipEventQuery(entry[1]) != 0:
        return   # not reached yet (or an error the next synchronizing call reports)
    _LOG_PENDING.pop(key)
    shared_used = 16 * max(0, int(entry[0][0]) - zero)
    _give_pinned(entry)
    regions = 16 * (first_shared - 1)
    # Shared blocks beyond a twentieth of the regions: widen the regions by
    # the shared use (so the next forward records almost everything in them).
    if regions > 0 and shared_used * 20 > regions:
        grow = -(-shared_used * units // regions)
        units = min(LOG_MAX_UNITS_PER_ENTRY, units + max(1, grow))
    if len(_LOG_UNITS) >= _MAX_LOG_KEYS and key not in _LOG_UNITS:
        _LOG_UNITS.pop(next(iter(_LOG_UNITS)))
    _LOG_UNITS[key] = units


def log_layout(key, capacity: int, nsub: int, waves_per_tile: int = 2):
    """(units per entry, pool bytes) for a forward of scene shape `key` with
    `capacity` list entries and tiles of `waves_per_tile` waves: the waves'
    own regions, plus shared blocks for a quarter of them and one block per
    wave (two per 16 x 16 sub-block)."""
    _poll_log_use(key)
    units = _LOG_UNITS.get(key, LOG_FIRST_UNITS_PER_ENTRY)
    regions = 16 * waves_per_tile * capacity * units
    shared = regions // 4 + 2 * nsub * N.RASTER_LOG_BLOCK_BYTES + (1 << 20)
    return units, (16 + regions + shared + 255) // 256 * 256


# The pool's use is read back from every LOG_READ_EVERY-th forward of a shape
# (the first one included); each read is a device-to-host copy in the stream.
LOG_READ_EVERY = 4
_LOG_READ_AGE: "dict[tuple, int]" = {}


def _read_log_use_later(key, dev_index: int, src: int, zero: int, units: int,
                        first_shared: int, pool_bytes: int, st) -> None:
    """Queues a copy of the shared-block counter at device address `src`
    (whose value `zero` means none used) into pinned memory and an event after
    it, unless one for this shape is still outstanding or this forward is not
    one of every LOG_READ_EVERY."""
    if key in _LOG_PENDING:
        return
    age = _LOG_READ_AGE.get(key, LOG_READ_EVERY - 1) + 1
    if len(_LOG_READ_AGE) >= _MAX_LOG_KEYS and key not in _LOG_READ_AGE:
        _LOG_READ_AGE.pop(next(iter(_LOG_READ_AGE)))
    if age < LOG_READ_EVERY:
        _LOG_READ_AGE[key] = age
        return
    _LOG_READ_AGE[key] = 0
    entry = _take_pinned(dev_index)
    hip = N.hip()
    N.hip_check(hip.hipMemcpyAsync(entry[0].data_ptr(), src, 4,
                                   N.HIP_MEMCPY_DEVICE_TO_HOST, st), "hipMemcpyAsync")
    N.hip_check(hip.hipEventRecord(entry[1], st), "hipEventRecord")
    if len(_LOG_PENDING) >= _MAX_LOG_KEYS:
        _, old = _LOG_PENDING.popitem()
        N.hip_check(hip.hipEventSynchronize(old[0][1]), "hipEventSynchronize")
        _give_pinned(old[0])
    _LOG_PENDING[key] = (entry, units, first_shared, pool_bytes, zero)


def rasterize_forward(b: Binned, background: torch.Tensor, eval_counts=None, log: bool = True,
                      log_pool_bytes_override: Optional[int] = None):
    """(image [H,W,3], final_Ts, final_idx).  The image is a contiguous
    [H, W, 3] tensor, as the reference returns it
    (cubic_splatting.py:2207-2209); the same launch also writes it as three
    [H, W] planes, attached to it (planar_copy_of), which the fused loss reads
    in place (clamping on load) while the image is unmodified.  With
    eval_counts (int64 [5],
    zeroed, on the device) the counting instantiation runs and adds the
    evaluation counts of cs_rasterize_forward_counted into it.  With log (the
    default) it writes the raster log its backward reads (b.log_index,
    b.log_pool); without, nothing is allocated for it and a backward would
    recompute every entry (log_pool_bytes_override sets the pool size with no
    per-wave regions, for tests of a pool that runs full).  The launch takes
    tiles in the heavy-first order made from an earlier forward of this image
    size on this stream (if any); every ORDER_EVERY-th forward records its
    wave durations and makes a new order from them, which its backward
    (b.tile_order) and the following forwards take."""
    dev = b.device
    H, W = b.img_h, b.img_w
    out = torch.empty((H, W, 3), dtype=torch.float32, device=dev)
    planes = torch.empty((3, H, W), dtype=torch.float32, device=dev)
    attach_planar_copy(out, planes)
    if b.any_tile:
        return _rasterize_forward_any(b, background, planes, out, eval_counts)
    nsub, wpt = b.nsub, b.waves_per_tile
    cap = max(int(b.primitive_ids_sorted.numel()), 1)
    # final_Ts, final_idx and the log's entry index share one allocation.
    n_index = wpt * cap if log else 0
    aux = torch.empty((2 * H * W + n_index,), dtype=torch.int32, device=dev)
    final_T = aux[:H * W].view(torch.float32).view(H, W)
    final_idx = aux[H * W:2 * H * W].view(H, W)
    st = N.stream(dev)
    if log:
        key = b.log_key if b.log_key is not None else (
            dev.index, b.mode, b.nprim, b.nseg, H, W, b.samples, b.adaptive, b.block_x,
            b.block_y)
        units, pool_bytes = log_layout(key, cap, nsub, wpt)
        if log_pool_bytes_override is not None:
            units, pool_bytes = 0, max(16, int(log_pool_bytes_override) // 16 * 16)
        b.log_index = aux[2 * H * W:]
        b.log_pool = torch.empty((pool_bytes,), dtype=torch.uint8, device=dev)
        b.log_units = units
        # The first forward after a binning counts its shared blocks in the
        # gradient buffer's zeroed counter word (no set-up launch); a repeated
        # forward lets the library set up the pool's own counter.
        ctr = None
        first_shared = 1 + wpt * cap * units
        if b.log_ctr_clean and b.grad_accum is not None:
            ga = b.grad_accum
            ctr = ga.data_ptr() + 4 * (ga.numel() - _LOG_COUNTER_ELEMS)
            b.log_ctr_clean = False
        b.log_ctr = None if ctr is None else (ctr, first_shared)
        log_args = (cap, b.log_index.data_ptr(), b.log_pool.data_ptr(), pool_bytes, units, ctr)
    else:
        b.log_index = b.log_pool = None
        b.log_ctr = None
        log_args = (cap, None, None, 0, 0, None)
    # The tile order is kept apart: the next forward reads it after this
    # forward's buffers are gone.
    okey = (dev.index, st, nsub)
    prev = _TILE_ORDERS.get(okey)
    age = _ORDER_AGE.get(okey, 0) + 1
    remake = prev is None or age >= ORDER_EVERY or eval_counts is not None
    base = aux.data_ptr()
    args = (b.mode, N.ptr(b.primitive_ids_sorted), b.ptr("tile_bins"), b.ptr("edges"),
            b.ptr("edge_culls"), b.ptr("prim_recs"), N.ptr(background), H, W, b.block_x,
            b.block_y, b.edges_per_segment, out.data_ptr(), 0, planes.data_ptr(), base,
            base + 4 * H * W,
            *log_args)
    cost = b.ptr("wave_cost") if remake else None
    prev_p = None if prev is None else prev.data_ptr()
    if eval_counts is not None:
        N.call("cs_rasterize_forward_counted", *args, N.ptr(_counts_buffer(eval_counts)),
               prev_p, cost, st)
    else:
        with N.prof("cubic.fwd.rast"):
            N.call("cs_rasterize_forward", *args, prev_p, cost, st)
    if log and log_pool_bytes_override is None:
        dix = dev.index if dev.index is not None else torch.cuda.current_device()
        if b.log_ctr is not None:
            _read_log_use_later(key, dix, b.log_ctr[0], 0, units, first_shared, pool_bytes, st)
        else:
            _read_log_use_later(key, dix, b.log_pool.data_ptr(), first_shared, units,
                                first_shared, pool_bytes, st)
    if not remake:
        b.tile_order = prev
        _ORDER_AGE[okey] = age
        return out, final_T, final_idx
    order = torch.empty((int(N.lib().cs_raster_tile_order_elems(nsub)),), dtype=torch.int32,
                        device=dev)
    last, spare = _TILE_COSTS.get(okey, (None, None))
    if spare is None:
        spare = torch.empty((nsub,), dtype=torch.int32, device=dev)
    with N.prof("cubic.fwd.tile_order"):
        N.call("cs_raster_tile_order_averaged", cost, N.ptr(last), spare.data_ptr(), nsub,
               int(ORDER_CHUNKED), order.data_ptr(), st)
    b.tile_order = order
    _TILE_COSTS[okey] = (spare, last)
    _TILE_ORDERS.pop(okey, None)
    _ORDER_AGE.pop(okey, None)
    if len(_TILE_ORDERS) >= _MAX_ORDERS:
        old = next(iter(_TILE_ORDERS))
        _TILE_ORDERS.pop(old)
        _ORDER_AGE.pop(old, None)
        _TILE_COSTS.pop(old, None)
    _TILE_ORDERS[okey] = order
    _ORDER_AGE[okey] = 0
    return out, final_T, final_idx


def _rasterize_forward_any(b: Binned, background, planes, out, eval_counts):
    """rasterize_forward for tiles whose sides are not multiples of 16: the
    any-size kernel (a lane per pixel, every edge evaluated), no raster log."""
    if eval_counts is not None:
        raise ValueError("evaluation counts are measured on 16x16 sub-block tiles only")
    dev = b.device
    H, W = b.img_h, b.img_w
    aux = torch.empty((2 * H * W,), dtype=torch.int32, device=dev)
    final_T = aux[:H * W].view(torch.float32).view(H, W)
    final_idx = aux[H * W:].view(H, W)
    b.log_index = b.log_pool = None
    b.log_ctr = None
    b.tile_order = None
    with N.prof("cubic.fwd.rast"):
        N.call("cs_rasterize_forward_any_tile", b.mode, N.ptr(b.primitive_ids_sorted),
               b.ptr("tile_bins"), b.ptr("edges"), b.ptr("prim_recs"), N.ptr(background), H, W,
               b.block_x, b.block_y, out.data_ptr(), 0, planes.data_ptr(), final_T.data_ptr(),
               final_idx.data_ptr(), N.stream(dev))
    return out, final_T, final_idx


def _rasterize_backward_any(b: Binned, background, final_T, final_idx, v_output, planar, v_px,
                            v_colors, v_opac, v_is2, v_sw, curve_contrib_rgb,
                            curve_isect_contrib):
    """rasterize_backward for tiles whose sides are not multiples of 16: the
    any-size kernel adds endpoint gradients per edge, which are then folded
    into the control points (cubic_splatting.py:2308-2396, :2399-2487)."""
    dev = b.device
    E = int(b.edges.shape[0])
    v_edges = torch.zeros((E, 4), dtype=torch.float32, device=dev)
    with N.prof("cubic.bwd.rast"):
        N.call("cs_rasterize_backward_any_tile", b.mode, N.ptr(b.primitive_ids_sorted),
               b.ptr("tile_bins"), b.ptr("edges"), b.ptr("prim_recs"), N.ptr(background),
               b.img_h, b.img_w, b.block_x, b.block_y, N.ptr(final_T), N.ptr(final_idx),
               N.ptr(v_output), planar, v_edges.data_ptr(), N.ptr(v_colors), N.ptr(v_opac),
               N.ptr(v_is2), N.ptr(v_sw), N.ptr(curve_contrib_rgb), N.ptr(curve_isect_contrib),
               N.stream(dev))
    v_norm = torch.empty_like(v_px)
    if b.adaptive:
        aux = b.edge_aux.view(torch.float32)
        t0, t1 = aux[:, 1].contiguous(), aux[:, 2].contiguous()
        N.call("cs_accumulate_edge_grads_csr", v_edges.data_ptr(), N.ptr(t0), N.ptr(t1),
               b.ptr("seg_edge_offsets"), b.nseg, b.img_h, b.img_w, N.ptr(v_px), N.ptr(v_norm),
               N.stream(dev))
    else:
        N.call("cs_accumulate_edge_grads", v_edges.data_ptr(), b.nseg, b.edges_per_segment,
               b.img_h, b.img_w, N.ptr(v_px), N.ptr(v_norm), N.stream(dev))


def log_pool_counter(b: Binned) -> int:
    """The end of the shared blocks b's forward reserved in its log pool, in
    16-byte units (a host read; tests)."""
    if b.log_pool is None:
        return 0
    if b.log_ctr is not None:
        ga = b.grad_accum
        used = int(ga[ga.numel() - _LOG_COUNTER_ELEMS:].view(torch.int32)[0].item())
        return b.log_ctr[1] + used
    return int(b.log_pool[:4].view(torch.int32)[0].item())


def _counts_buffer(t):
    if t.dtype != torch.int64 or t.numel() != 5 or not t.is_contiguous():
        raise ValueError("eval_counts must be a contiguous int64 tensor of 5 elements")
    return t


def rasterize_backward(b: Binned, background, final_T, final_idx, v_output, *,
                       curve_contrib_rgb=None, curve_isect_contrib=None, eval_counts=None):
    """Returns (v_cubics_px [nseg,4,2], v_colors [P,3], v_opacities [P],
    v_inv_sigma2s [P], v_stroke_widths [P] or None), accumulated into fresh
    zero buffers (cubic_splatting.py:2572-2747).  eval_counts as for
    rasterize_forward (cs_rasterize_backward_counted)."""
    dev = b.device
    P = b.nprim
    if b.grad_accum_clean:
        zeros = b.grad_accum
        b.grad_accum_clean = False
    else:  # a second backward through the same forward
        zeros = torch.zeros((_grad_accum_elems(b.nseg, P, b.mode),), dtype=torch.float32,
                            device=dev)
    v_px = zeros[: b.nseg * 8].view(b.nseg, 4, 2)
    rest = zeros[b.nseg * 8:]
    v_colors = rest[: 3 * P].view(P, 3)
    v_opac = rest[3 * P: 4 * P]
    v_is2 = rest[4 * P: 5 * P]
    v_sw = rest[5 * P: 6 * P] if b.mode == MODE_STROKE else None
    v_output, planar = image_grad_layout(v_output)
    if b.any_tile:
        if eval_counts is not None:
            raise ValueError("evaluation counts are measured on 16x16 sub-block tiles only")
        _rasterize_backward_any(b, background, final_T, final_idx, v_output, planar, v_px,
                                v_colors, v_opac, v_is2, v_sw, curve_contrib_rgb,
                                curve_isect_contrib)
        return v_px, v_colors, v_opac, v_is2, v_sw
    nv = 6 if b.mode == MODE_STROKE else 5
    prim_scratch = N.ptr(rest[nv * P:])
    log_index, log_pool = N.ptr(b.log_index), N.ptr(b.log_pool)
    if b.adaptive:
        if eval_counts is not None:
            raise ValueError("evaluation counts are measured on the uniform flattening only")
        with N.prof("cubic.bwd.rast"):
            N.call("cs_rasterize_backward_de_casteljau", b.mode, N.ptr(b.primitive_ids_sorted),
                   b.ptr("tile_bins"), b.ptr("edges"), b.ptr("edge_culls"), b.ptr("prim_recs"),
                   N.ptr(background), b.img_h, b.img_w, b.block_x, b.block_y,
                   b.ptr("edge_aux"), N.ptr(final_T),
                   N.ptr(final_idx), log_index, log_pool, N.ptr(v_output), planar,
                   N.ptr(v_px), N.ptr(v_colors),
                   N.ptr(v_opac), N.ptr(v_is2), N.ptr(v_sw), N.ptr(curve_contrib_rgb),
                   N.ptr(curve_isect_contrib), P, prim_scratch, N.ptr(b.tile_order),
                   N.stream(dev))
        return v_px, v_colors, v_opac, v_is2, v_sw
    args = (b.mode, N.ptr(b.primitive_ids_sorted), b.ptr("tile_bins"), b.ptr("edges"),
            b.ptr("edge_culls"), b.ptr("prim_recs"), N.ptr(background), b.img_h, b.img_w,
            b.block_x, b.block_y, b.edges_per_segment, N.ptr(final_T), N.ptr(final_idx),
            log_index, log_pool,
            N.ptr(v_output), planar, N.ptr(v_px),
            N.ptr(v_colors), N.ptr(v_opac), N.ptr(v_is2), N.ptr(v_sw), N.ptr(curve_contrib_rgb),
            N.ptr(curve_isect_contrib))
    if eval_counts is not None:
        N.call("cs_rasterize_backward_counted", *args, N.ptr(_counts_buffer(eval_counts)),
               P, prim_scratch, N.ptr(b.tile_order), N.stream(dev))
    else:
        with N.prof("cubic.bwd.rast"):
            N.call("cs_rasterize_backward", *args, P, prim_scratch, N.ptr(b.tile_order),
                   N.stream(dev))
    return v_px, v_colors, v_opac, v_is2, v_sw


def rasterize_backward_finalized(b: Binned, background, final_T, final_idx, v_output, widths):
    """rasterize_backward followed by backward_finalize, with the per-XCD
    copies' reduction and the epilogue in one launch
    (cs_rasterize_backward_finalized): returns (v_cubics_norm [nseg,4,2],
    v_colors [P,3], v_opacities [P], v_aa_widths [P], v_stroke_widths [P] or
    None), the values of the two calls.  Uniform flattening and 16 x 16
    sub-block tiles (the other backward kernels keep the two calls)."""
    dev = b.device
    P = b.nprim
    if b.grad_accum_clean:
        zeros = b.grad_accum
        b.grad_accum_clean = False
    else:  # a second backward through the same forward
        zeros = torch.zeros((_grad_accum_elems(b.nseg, P, b.mode),), dtype=torch.float32,
                            device=dev)
    v_px = zeros[: b.nseg * 8]
    rest = zeros[b.nseg * 8:]
    v_colors = rest[: 3 * P].view(P, 3)
    v_opac = rest[3 * P: 4 * P]
    v_is2 = rest[4 * P: 5 * P]
    v_sw = rest[5 * P: 6 * P] if b.mode == MODE_STROKE else None
    nv = 6 if b.mode == MODE_STROKE else 5
    out = torch.empty((b.nseg * 8 + P,), dtype=torch.float32, device=dev)
    v_norm = out[: b.nseg * 8].view(b.nseg, 4, 2)
    v_aa = out[b.nseg * 8:]
    v_output, planar = image_grad_layout(v_output)
    with N.prof("cubic.bwd.rast"):
        N.call("cs_rasterize_backward_finalized", b.mode, N.ptr(b.primitive_ids_sorted),
               b.ptr("tile_bins"), b.ptr("edges"), b.ptr("edge_culls"), b.ptr("prim_recs"),
               N.ptr(background), b.img_h, b.img_w, b.block_x, b.block_y,
               b.edges_per_segment, N.ptr(final_T), N.ptr(final_idx), N.ptr(b.log_index),
               N.ptr(b.log_pool), N.ptr(v_output), planar, N.ptr(v_px), N.ptr(v_colors),
               N.ptr(v_opac), N.ptr(v_is2), N.ptr(v_sw), P, N.ptr(rest[nv * P:]),
               N.ptr(b.tile_order), b.nseg, N.ptr(widths), N.ptr(v_norm), N.ptr(v_aa),
               N.stream(dev))
    return v_norm, v_colors, v_opac, v_aa, v_sw


def accumulate_edge_grads(b: Binned, v_edges):
    """Reference building block (cubic_splatting.py:2308-2396; the CSR form
    :2399-2487 for the adaptive flattening): v_edges [E,4] -> (v_cubics_px,
    v_cubics_norm)."""
    dev = v_edges.device
    v_px = torch.empty((b.nseg, 4, 2), dtype=torch.float32, device=dev)
    v_norm = torch.empty((b.nseg, 4, 2), dtype=torch.float32, device=dev)
    if b.adaptive:
        E = b.num_edges()
        aux = b.edge_aux[:E].view(torch.float32)
        t0, t1 = aux[:, 1].contiguous(), aux[:, 2].contiguous()
        N.call("cs_accumulate_edge_grads_csr", N.ptr(v_edges), N.ptr(t0), N.ptr(t1),
               b.ptr("seg_edge_offsets"), b.nseg, b.img_h, b.img_w, N.ptr(v_px), N.ptr(v_norm),
               N.stream(dev))
    else:
        N.call("cs_accumulate_edge_grads", N.ptr(v_edges), b.nseg, b.edges_per_segment,
               b.img_h, b.img_w, N.ptr(v_px), N.ptr(v_norm), N.stream(dev))
    return v_px, v_norm


def backward_finalize(b: Binned, v_cubics_px, widths, v_inv_sigma2s):
    """(v_cubics_norm, v_aa_widths) in one launch (cubic_splatting.py:3096-3104)."""
    dev = v_cubics_px.device
    n_cp, n_w = v_cubics_px.numel(), v_inv_sigma2s.numel()
    buf = torch.empty((n_cp + n_w,), dtype=torch.float32, device=dev)
    v_norm = buf[:n_cp].view(v_cubics_px.shape)
    v_aa = buf[n_cp:]
    with N.prof("cubic.bwd.finalize"):
        N.call("cs_backward_finalize", N.ptr(v_cubics_px), b.nseg, b.img_h, b.img_w, N.ptr(widths),
               N.ptr(v_inv_sigma2s), int(widths.numel()), N.ptr(v_norm), N.ptr(v_aa), N.stream(dev))
    return v_norm, v_aa


_NONE19 = (None,) * 19

# Last intersection-buffer size per scene shape, the capacity hint of the next
# forward of that shape (bounded: the oldest entries are dropped).
_CAPACITY_HINTS: "dict[tuple, int]" = {}
_MAX_HINTS = 64


def _remember_capacity(key, num_intersects: int) -> None:
    _CAPACITY_HINTS.pop(key, None)
    if len(_CAPACITY_HINTS) >= _MAX_HINTS:
        _CAPACITY_HINTS.pop(next(iter(_CAPACITY_HINTS)))
    _CAPACITY_HINTS[key] = intersection_capacity(max(0, num_intersects))


# Largest tile of the 16 x 16 sub-block kernels: 16 sub-blocks.
MAX_SUB_BLOCKS_PER_TILE = 16
# Largest tile of the any-size kernels (a lane per pixel): the reference's
# one-thread-per-pixel launch, threads=(block_x, block_y), allows 1024.
MAX_ANY_TILE_PIXELS = 1024


def is_sub_block_tile(block_x: int, block_y: int) -> bool:
    """Tiles the 16 x 16 sub-block raster takes: positive multiples of 16 in
    both directions, at most 16 sub-blocks."""
    bx, by = int(block_x), int(block_y)
    return (bx > 0 and by > 0 and bx % BLOCK_X == 0 and by % BLOCK_Y == 0
            and (bx // BLOCK_X) * (by // BLOCK_Y) <= MAX_SUB_BLOCKS_PER_TILE)


def check_block(block_x: int, block_y: int) -> None:
    """Tiles the MI355X raster takes: multiples of 16 (up to 16 sub-blocks of
    16 x 16, the fast kernels), or any other positive size of at most 1024
    pixels (the any-size kernels, a lane per pixel as in the reference)."""
    bx, by = int(block_x), int(block_y)
    if is_sub_block_tile(bx, by):
        return
    if bx <= 0 or by <= 0 or bx * by > MAX_ANY_TILE_PIXELS:
        raise NotImplementedError(
            f"the MI355X raster takes tiles whose sides are multiples of {BLOCK_X} pixels (at "
            f"most {MAX_SUB_BLOCKS_PER_TILE} sub-blocks of {BLOCK_X}x{BLOCK_Y}) or tiles of at "
            f"most {MAX_ANY_TILE_PIXELS} pixels; got {block_x}x{block_y}")


_check_block = check_block


def _splat_forward(ctx, mode, cubics_norm, primitive_seg_offsets, colors, opacities, depths,
                   fill_rules, stroke_widths, img_h, img_w, block_x, block_y, background,
                   aabb_pad, aniso_intersects, aa_widths, distance_samples, flatten_method,
                   process_fn):
    flatten_method_norm = normalize_cubic_flatten_method(flatten_method)
    num_segments = int(cubics_norm.shape[0])
    offs = _i32(primitive_seg_offsets).view(-1)
    num_primitives = max(0, int(offs.numel()) - 1)
    dev = cubics_norm.device
    bg = background
    if bg.dtype is not torch.float32 or bg.device != dev or not bg.is_contiguous():
        bg = bg.to(device=dev, dtype=torch.float32).contiguous()
    bg = bg.view(3)
    ctx.img_h, ctx.img_w = int(img_h), int(img_w)
    if num_primitives <= 0:
        ctx.empty = True
        return bg.view(1, 1, 3).expand(int(img_h), int(img_w), 3).clone()
    _check_block(block_x, block_y)
    if int(img_h) > N.MAX_IMAGE_DIM or int(img_w) > N.MAX_IMAGE_DIM:
        raise ValueError(f"img_h and img_w must be at most {N.MAX_IMAGE_DIM} "
                         f"(got {int(img_h)}x{int(img_w)})")
    N.require_gpu(cubics_norm, "cubics_norm")
    for name, t, k in (("colors", colors, None), ("opacities", opacities, 1),
                       ("depths", depths, 1), ("fill_rules", fill_rules, 1),
                       ("stroke_widths", stroke_widths, 1)):
        if t is None:
            continue
        n = int(t.shape[0]) if k is None else int(t.reshape(-1).shape[0])
        if n != num_primitives:
            raise ValueError(
                f"{name} size must match primitive count ({num_primitives}), got {n}"
                if k is not None else
                f"colors first dim must match primitive count ({num_primitives}), got {n}")
    # The reference clamps the widths to >= 1e-4 here (cubic_splatting.py:2820);
    # every kernel that reads them applies that clamp itself.
    widths = _f32(aa_widths).view(-1)
    if int(widths.numel()) != num_primitives:
        raise ValueError(
            f"aa_widths size must match primitive count ({num_primitives}), "
            f"got {int(widths.numel())}")

    colors_c = _f32(colors)
    opac_c = _f32(opacities).view(-1)
    rules_c = _i32(fill_rules).view(-1) if fill_rules is not None else None
    sw_c = _f32(stroke_widths).view(-1) if stroke_widths is not None else None
    hint_key = (cubics_norm.device.index, mode, num_primitives, num_segments, int(img_h),
                int(img_w), int(distance_samples), flatten_method_norm, int(block_x),
                int(block_y))
    b = bin_primitives(_f32(cubics_norm), offs, colors_c, opac_c, _f32(depths).view(-1),
                       rules_c, widths, sw_c, int(img_h), int(img_w), int(distance_samples),
                       aabb_pad=float(aabb_pad), aniso=bool(aniso_intersects), mode=mode,
                       block_x=int(block_x), block_y=int(block_y),
                       capacity_hint=_CAPACITY_HINTS.get(hint_key),
                       flatten_method=flatten_method_norm)
    # With a hint the raster is enqueued before the host reads the count; if
    # the lists did not fit, they and the raster are redone at full size.
    # The raster log is written only when a backward can follow (some input
    # requires a gradient).
    log = any(ctx.needs_input_grad)
    b.log_key = hint_key
    out, final_T, final_idx = rasterize_forward(b, bg, log=log)
    if resolve_binned(b):
        out, final_T, final_idx = rasterize_forward(b, bg, log=log)
    _remember_capacity(hint_key, b.num_intersects)
    if b.num_intersects <= 0:
        ctx.empty = True
        return bg.view(1, 1, 3).expand(int(img_h), int(img_w), 3).clone()
    ctx.empty = False
    ctx.binned = b
    ctx.process_fn = process_fn
    ctx.flatten_method = flatten_method_norm
    ctx.distance_samples = int(distance_samples)
    ctx.mode = mode
    # The backward kernels read the binned copies (records, edges); the
    # inputs are kept for process_fn payloads and gradient shapes.  Tensors
    # made here are plain attributes.
    ctx.save_for_backward(colors_c, opac_c, depths, sw_c)
    ctx.cub_shape = cubics_norm.shape
    ctx.offs, ctx.widths, ctx.bg, ctx.final_T, ctx.final_idx = offs, widths, bg, final_T, final_idx
    return out


def _splat_backward(ctx, grad_out_img):
    b: Binned = ctx.binned
    colors, opacities, depths, stroke_widths = ctx.saved_tensors
    offs, widths, bg, final_T, final_idx = ctx.offs, ctx.widths, ctx.bg, ctx.final_T, ctx.final_idx
    process_fn = ctx.process_fn
    curve_contrib_rgb = curve_isect_contrib = None
    if process_fn is not None:
        pre = _run_process_fn(process_fn, "pre_backward_rasterize", {
            "collect_curve_contrib_rgb": False,
            "collect_curve_isect_contrib": False,
            "num_primitives": int(colors.shape[0]),
            "colors": colors,
        })
        if bool(pre.get("collect_curve_contrib_rgb", False)):
            curve_contrib_rgb = torch.zeros_like(colors)
        if bool(pre.get("collect_curve_isect_contrib", False)):
            curve_isect_contrib = torch.zeros((b.num_intersects,), dtype=torch.float32,
                                              device=colors.device)
    # rasterize_backward takes the gradient in either layout (no copy of a
    # planar one).  Without the hooks the epilogue runs in the backward's
    # own last launch.
    if process_fn is None and not b.any_tile and not b.adaptive:
        v_cubics_norm, v_colors, v_opac, v_aa, v_sw = rasterize_backward_finalized(
            b, bg, final_T, final_idx, grad_out_img, widths)
        depth_index = 5 if ctx.mode == MODE_STROKE else 4
        v_depths = (torch.zeros_like(depths, dtype=torch.float32)
                    if ctx.needs_input_grad[depth_index] else None)
        return v_cubics_norm.view(ctx.cub_shape), v_colors, v_opac.view_as(opacities), v_sw, \
            v_depths, v_aa
    v_cubics_px, v_colors, v_opac, v_is2, v_sw = rasterize_backward(
        b, bg, final_T, final_idx, grad_out_img, curve_contrib_rgb=curve_contrib_rgb,
        curve_isect_contrib=curve_isect_contrib)
    if process_fn is not None:
        payload = {
            "v_cubics_px": v_cubics_px,
            "v_colors": v_colors,
            "v_opacity": v_opac,
            "curve_contrib_rgb": curve_contrib_rgb,
            "curve_isect_contrib": curve_isect_contrib,
            "primitive_ids_sorted": b.primitive_ids_sorted,
            "tile_bins": b.tile_bins,
            "colors": colors,
            "opacities": opacities,
            "primitive_seg_offsets": offs,
        }
        if ctx.mode == MODE_STROKE:
            payload["v_stroke"] = v_sw
            payload["stroke_widths"] = stroke_widths
        payload = _run_process_fn(process_fn, "post_backward_rasterize", payload)
        v_cubics_px = _f32(payload["v_cubics_px"])
        v_colors = payload["v_colors"]
        v_opac = payload["v_opacity"]
        if ctx.mode == MODE_STROKE:
            v_sw = payload["v_stroke"]
    v_cubics_norm, v_aa = backward_finalize(b, v_cubics_px, widths, v_is2)
    # The reference returns zeros for the depths (cubic_splatting.py:3102).
    depth_index = 5 if ctx.mode == MODE_STROKE else 4
    v_depths = (torch.zeros_like(depths, dtype=torch.float32)
                if ctx.needs_input_grad[depth_index] else None)
    return v_cubics_norm.view(ctx.cub_shape), v_colors, v_opac.view_as(opacities), v_sw, \
        v_depths, v_aa


class _CubicFillSplatFunction(torch.autograd.Function):
    """Signature of cubic_splatting.py:2750-2773; backward returns the 19-tuple
    of cubic_splatting.py:3105-3125."""

    @staticmethod
    def forward(ctx, cubics_norm, primitive_seg_offsets, colors, opacities, depths, fill_rules,
                img_h, img_w, block_x, block_y, background, project_threads, map_threads,
                aabb_pad, aniso_intersects, aa_widths, distance_samples,
                flatten_method=DEFAULT_CUBIC_FLATTEN_METHOD, process_fn=None):
        return _splat_forward(ctx, MODE_FILL, cubics_norm, primitive_seg_offsets, colors,
                              opacities, depths, fill_rules, None, img_h, img_w, block_x,
                              block_y, background, aabb_pad, aniso_intersects, aa_widths,
                              distance_samples, flatten_method, process_fn)

    @staticmethod
    def backward(ctx, grad_out_img):
        if getattr(ctx, "empty", False):
            return _NONE19
        v_cub, v_col, v_op, _, v_dep, v_aa = _splat_backward(ctx, grad_out_img)
        return (v_cub, None, v_col, v_op, v_dep, None, None, None, None, None, None, None,
                None, None, None, v_aa, None, None, None)


class _CubicPolylineSplatFunction(torch.autograd.Function):
    """Signature of cubic_polyline_splatting.py:962-985; backward returns the
    19-tuple of cubic_polyline_splatting.py:1318-1338."""

    @staticmethod
    def forward(ctx, cubics_norm, primitive_seg_offsets, colors, opacities, stroke_widths,
                depths, img_h, img_w, block_x, block_y, background, project_threads,
                map_threads, aabb_pad, aniso_intersects, aa_widths, distance_samples,
                flatten_method=DEFAULT_CUBIC_FLATTEN_METHOD, process_fn=None):
        return _splat_forward(ctx, MODE_STROKE, cubics_norm, primitive_seg_offsets, colors,
                              opacities, depths, None, stroke_widths, img_h, img_w, block_x,
                              block_y, background, aabb_pad, aniso_intersects, aa_widths,
                              distance_samples, flatten_method, process_fn)

    @staticmethod
    def backward(ctx, grad_out_img):
        if getattr(ctx, "empty", False):
            return _NONE19
        v_cub, v_col, v_op, v_sw, v_dep, v_aa = _splat_backward(ctx, grad_out_img)
        return (v_cub, None, v_col, v_op, v_sw, v_dep, None, None, None, None, None, None,
                None, None, None, v_aa, None, None, None)


def _prim_vector(t, num_primitives, name, device, dtype, default):
    if t is None:
        return torch.full((num_primitives,), default, device=device, dtype=dtype)
    out = t.to(device=device, dtype=dtype).view(-1)
    if int(out.numel()) == 1 and num_primitives > 1:
        out = out.expand(num_primitives)
    if int(out.numel()) != num_primitives:
        raise ValueError(
            f"{name} size must match primitive count ({num_primitives}), got {int(out.numel())}")
    return out


def _aa_widths(aa_widths, num_primitives, dev, aa_width):
    """Per-primitive widths, clamped to >= 1e-4 as the reference's render
    functions do (cubic_splatting.py:3207).  Every kernel that reads a width
    applies the same floor itself (fmaxf, so a NaN width reads as the floor
    there), so the clamp is materialised only when a gradient has to flow
    through it (where it zeroes the gradient of the clamped widths)."""
    w = _prim_vector(aa_widths, num_primitives, "aa_widths", dev, torch.float32, float(aa_width))
    if w.requires_grad:
        return torch.clamp(w.contiguous(), min=1e-4)
    return w if w.is_contiguous() else w.contiguous()


def _common_checks(cubics_norm, offs, colors, opacities, depths, num_primitives,
                   stroke_widths=None):
    if int(colors.shape[0]) != num_primitives:
        raise ValueError(
            f"colors first dim must match primitive count ({num_primitives}), "
            f"got {int(colors.shape[0])}")
    if int(opacities.reshape(-1).shape[0]) != num_primitives:
        raise ValueError(
            f"opacities size must match primitive count ({num_primitives}), "
            f"got {int(opacities.reshape(-1).shape[0])}")
    if stroke_widths is not None and int(stroke_widths.reshape(-1).shape[0]) != num_primitives:
        raise ValueError(
            f"stroke_widths size must match primitive count ({num_primitives}), "
            f"got {int(stroke_widths.reshape(-1).shape[0])}")
    if int(depths.reshape(-1).shape[0]) != num_primitives:
        raise ValueError(
            f"depths size must match primitive count ({num_primitives}), "
            f"got {int(depths.reshape(-1).shape[0])}")


def render_cubic_fill_splat_tilelang(cubics_norm, primitive_seg_offsets, colors, opacities,
                                     depths, img_h, img_w, block_x, block_y, background, *,
                                     fill_rules=None, project_threads=DEFAULT_THREADS,
                                     map_threads=DEFAULT_THREADS, aabb_pad=DEFAULT_AABB_PAD,
                                     aniso_intersects=False, aa_widths=None,
                                     aa_width=DEFAULT_AA_WIDTH,
                                     distance_samples=DEFAULT_DISTANCE_SAMPLES,
                                     flatten_method=DEFAULT_CUBIC_FLATTEN_METHOD,
                                     process_fn=None):
    """cubic_splatting.py:3128-3229 -> [H, W, 3] image."""
    offs = _i32(primitive_seg_offsets).view(-1)
    num_primitives = max(0, int(offs.numel()) - 1)
    if num_primitives <= 0:
        bg = background.to(device=cubics_norm.device, dtype=torch.float32).view(1, 1, 3)
        return bg.expand(int(img_h), int(img_w), 3).clone()
    _common_checks(cubics_norm, offs, colors, opacities, depths, num_primitives)
    dev = cubics_norm.device
    # Default: nonzero rule for every primitive (cubic_splatting.py:3175-3178),
    # which the kernels apply when no rules are passed.
    rules = (None if fill_rules is None else
             _prim_vector(fill_rules, num_primitives, "fill_rules", dev, torch.int32, 1)
             .contiguous())
    widths = _aa_widths(aa_widths, num_primitives, dev, aa_width)
    return _CubicFillSplatFunction.apply(
        cubics_norm, offs.contiguous(), colors.contiguous(), opacities.reshape(-1).contiguous(),
        depths.reshape(-1).contiguous(), rules, int(img_h), int(img_w),
        int(block_x), int(block_y), background, int(project_threads), int(map_threads),
        float(aabb_pad), bool(aniso_intersects), widths, int(distance_samples),
        normalize_cubic_flatten_method(flatten_method), process_fn)


def render_cubic_polyline_splat_tilelang(cubics_norm, primitive_seg_offsets, colors, opacities,
                                         stroke_widths, depths, img_h, img_w, block_x, block_y,
                                         background, *, project_threads=DEFAULT_THREADS,
                                         map_threads=DEFAULT_THREADS,
                                         aabb_pad=DEFAULT_AABB_PAD, aniso_intersects=False,
                                         aa_widths=None, aa_width=DEFAULT_AA_WIDTH,
                                         distance_samples=DEFAULT_DISTANCE_SAMPLES,
                                         flatten_method=DEFAULT_CUBIC_FLATTEN_METHOD,
                                         process_fn=None):
    """cubic_polyline_splatting.py:1341-1432 -> [H, W, 3] image."""
    offs = _i32(primitive_seg_offsets).view(-1)
    num_primitives = max(0, int(offs.numel()) - 1)
    if num_primitives <= 0:
        bg = background.to(device=cubics_norm.device, dtype=torch.float32).view(1, 1, 3)
        return bg.expand(int(img_h), int(img_w), 3).clone()
    _common_checks(cubics_norm, offs, colors, opacities, depths, num_primitives, stroke_widths)
    dev = cubics_norm.device
    widths = _aa_widths(aa_widths, num_primitives, dev, aa_width)
    return _CubicPolylineSplatFunction.apply(
        cubics_norm, offs.contiguous(), colors.contiguous(), opacities.reshape(-1).contiguous(),
        stroke_widths.reshape(-1).contiguous(), depths.reshape(-1).contiguous(), int(img_h),
        int(img_w), int(block_x), int(block_y), background, int(project_threads),
        int(map_threads), float(aabb_pad), bool(aniso_intersects), widths,
        int(distance_samples), normalize_cubic_flatten_method(flatten_method), process_fn)
