"""ctypes binding of libcubicsplat_hip.so (declared in include/cubicsplat_hip.h).

There is no fallback: if the library is missing or a call fails, this module
raises.  torch is imported first so that the library binds to the HIP runtime
torch has already loaded (both use the soname libamdhip64.so.7).
"""
from __future__ import annotations

import ctypes
import os
import warnings
from contextlib import nullcontext
from typing import Callable, ContextManager, Optional

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libcubicsplat_hip.so")

CS_OK, CS_ERR_ARGS, CS_ERR_HIP = 0, 1, 2
EDGE_RECORD_FLOATS = 8   # 32-byte edge record (geometry)
EDGE_CULL_INTS = 4       # 16-byte edge cull record
MAX_IMAGE_DIM = 16384
SEG_RECORD_INTS = 8      # 32-byte segment record
PRIM_RECORD_FLOATS = 20  # 80-byte primitive record
RASTER_LOG_BLOCK_BYTES = 2048  # log pool reserved per wave at a time
EDGE_AUX_INTS = 4        # 16-byte (segment, t0, t1) record of the adaptive flattening

_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_F = ctypes.c_float
_D = ctypes.c_double
_SZ = ctypes.c_size_t

_SIGNATURES = {
    "cs_scan_temp_elems": (_SZ, [_I32]),
    "cs_radix_counts_elems": (_SZ, [_I32]),
    "cs_scan_exclusive_u32": (ctypes.c_int, [_P, _P, _I32, _P, _P, _P]),
    "cs_radix_sort_pairs_u32": (ctypes.c_int, [_P, _P, _P, _P, _I32, _I32, _P, _P, _P]),
    "cs_project_cubics_2d_forward": (ctypes.c_int, [_P, _P, _P, _I32, _I32, _I32, _I32, _I32, _F,
                                                    _I32, _P, _P, _P, _P]),
    "cs_primitive_tile_ranges": (ctypes.c_int, [_P, _P, _I32, _I32, _I32, _P, _P, _P]),
    "cs_map_cubic_to_intersects": (ctypes.c_int, [_P, _P, _P, _I32, _I32, _P, _P, _P]),
    "cs_get_tile_bin_edges": (ctypes.c_int, [_P, _I32, _I32, _P, _P]),
    "cs_isect_edge_ranges": (ctypes.c_int, [_P, _P, _I32, _I32, _P, _P]),
    "cs_bin_prepare": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _P, _I32, _I32, _I32, _I32,
                                      _I32, _I32, _I32, _F, _I32, _I32, _P, _P, _P, _P, _P, _P,
                                      _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P]),
    "cs_bin_list_elems": (_SZ, [_I32, _I32, _I32, _I32, _I32]),
    "cs_bin_finish": (ctypes.c_int, [_P, _P, _I32, _P, _I64, _I32, _I32, _I32, _I32, _P, _P,
                                     _P, _P, _P, _I64, _P, _P]),
    "cs_rasterize_forward": (ctypes.c_int, [_I32, _P, _P, _P, _P, _P, _P, _I32, _I32, _I32, _I32,
                                            _I32, _P, _I32, _P, _P, _P, _I64, _P, _P, _I64, _I32,
                                            _P, _P, _P, _P]),
    "cs_rasterize_backward": (ctypes.c_int, [_I32, _P, _P, _P, _P, _P, _P, _I32, _I32, _I32, _I32,
                                             _I32, _P, _P, _P, _P, _P, _I32, _P, _P, _P, _P, _P,
                                             _P, _P, _I32, _P, _P, _P]),
    "cs_raster_prim_scratch_elems": (_SZ, [_I32, _I32]),
    "cs_rasterize_forward_counted": (ctypes.c_int, [_I32, _P, _P, _P, _P, _P, _P, _I32, _I32, _I32,
                                                    _I32, _I32, _P, _I32, _P, _P, _P, _I64, _P,
                                                    _P, _I64, _I32, _P, _P, _P, _P, _P]),
    "cs_rasterize_backward_counted": (ctypes.c_int, [_I32, _P, _P, _P, _P, _P, _P, _I32, _I32,
                                                     _I32, _I32, _I32, _P, _P, _P, _P, _P, _I32,
                                                     _P, _P, _P, _P, _P, _P, _P, _P, _I32, _P, _P,
                                                     _P]),
    "cs_raster_tile_order_elems": (_SZ, [_I32]),
    "cs_raster_tile_order": (ctypes.c_int, [_P, _I32, _I32, _P, _P]),
    "cs_raster_tile_order_averaged": (ctypes.c_int, [_P, _P, _P, _I32, _I32, _P, _P]),
    "cs_rasterize_forward_any_tile": (ctypes.c_int, [_I32, _P, _P, _P, _P, _P, _I32, _I32, _I32,
                                                     _I32, _P, _I32, _P, _P, _P, _P]),
    "cs_rasterize_backward_any_tile": (ctypes.c_int, [_I32, _P, _P, _P, _P, _P, _I32, _I32, _I32,
                                                      _I32, _P, _P, _P, _I32, _P, _P, _P, _P,
                                                      _P, _P, _P, _P]),
    "cs_raster_records_from_edges": (ctypes.c_int, [_I32, _P, _I32, _P, _P, _I64, _P, _P, _P, _P,
                                                    _P, _I32, _P, _I32, _P, _P, _P, _P, _P, _P,
                                                    _P]),
    "cs_edge_aux_from_csr": (ctypes.c_int, [_P, _I32, _P, _P, _I32, _P, _P]),
    "cs_accumulate_edge_grads": (ctypes.c_int, [_P, _I32, _I32, _I32, _I32, _P, _P, _P]),
    "cs_de_casteljau_max_edges_per_segment": (_I32, [_I32]),
    "cs_bin_prepare_de_casteljau": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _P, _I32, _I32,
                                                   _I32, _I32, _I32, _I32, _I32, _F, _I32, _I32,
                                                   _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                                   _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                                   _P]),
    "cs_flatten_cubics_de_casteljau": (ctypes.c_int, [_P, _P, _I32, _I32, _I32, _P, _P, _P, _P,
                                                      _P, _P, _P, _P]),
    "cs_flatten_cubics_bernstein": (ctypes.c_int, [_P, _I32, _I32, _P, _P]),
    "cs_cubic_flatness_flags": (ctypes.c_int, [_P, _I32, _F, _I32, _P, _P]),
    "cs_cubic_split_half": (ctypes.c_int, [_P, _I32, _P, _P, _P]),
    "cs_rasterize_backward_de_casteljau": (ctypes.c_int, [_I32, _P, _P, _P, _P, _P, _P, _I32, _I32,
                                                          _I32, _I32, _P, _P, _P, _P, _P, _P,
                                                          _I32, _P, _P, _P, _P, _P, _P, _P,
                                                          _I32, _P, _P, _P]),
    "cs_accumulate_edge_grads_csr": (ctypes.c_int, [_P, _P, _P, _P, _I32, _I32, _I32, _P, _P,
                                                    _P]),
    "cs_backward_finalize": (ctypes.c_int, [_P, _I32, _I32, _I32, _P, _P, _I32, _P, _P, _P]),
    "cs_rasterize_backward_finalized": (ctypes.c_int, [_I32, _P, _P, _P, _P, _P, _P, _I32, _I32,
                                                       _I32, _I32, _I32, _P, _P, _P, _P, _P,
                                                       _I32, _P, _P, _P, _P, _P, _I32, _P, _P,
                                                       _I32, _P, _P, _P, _P]),
    "cs_mse_partials_elems": (_SZ, [_I64]),
    "cs_ssim_partials_elems": (_SZ, [_I32, _I32, _I32]),
    "cs_ssim_abc_elems": (_SZ, [_I32, _I32, _I32, _I32]),
    "cs_mse_forward": (ctypes.c_int, [_P, _P, _I64, _P, _P, _P]),
    "cs_mse_forward_noalloc_max_elems": (_I64, []),
    "cs_mse_backward_diff": (ctypes.c_int, [_P, _P, _I64, _F, _P, _P]),
    "cs_reduce_sum_partials_elems": (_SZ, [_I64]),
    "cs_reduce_sum_f32": (ctypes.c_int, [_P, _I64, _P, _P, _P]),
    "cs_mse_forward_noalloc": (ctypes.c_int, [_P, _P, _I64, _P, _P]),
    "cs_mse_backward": (ctypes.c_int, [_P, _P, _I64, _P, _P, _P, _P]),
    "cs_ssim_scratch_elems": (_SZ, [_I32, _I32, _I32, _I32]),
    "cs_ssim": (ctypes.c_int, [_P, _P, _I32, _I32, _I32, _P, _I32, _F, _F, _I32, _P, _P, _P, _P,
                               _P]),
    "cs_ssim_backward": (ctypes.c_int, [_P, _P, _I32, _I32, _I32, _P, _I32, _P, _P, _I32, _P, _P,
                                        _P]),
    "cs_clamp_hwc_to_nchw": (ctypes.c_int, [_P, _I32, _I32, _F, _F, _P, _P]),
    "cs_clamp_hwc_to_nchw_backward": (ctypes.c_int, [_P, _P, _I32, _I32, _F, _F, _P, _P]),
    "cs_mse_ssim_partials_elems": (_SZ, [_I32, _I32, _I32]),
    "cs_mse_ssim_loss": (ctypes.c_int, [_P, _P, _I32, _I32, _I32, _P, _I32, _F, _F, _F, _P, _P,
                                        _P, _P]),
    "cs_mse_ssim_backward": (ctypes.c_int, [_P, _P, _I32, _I32, _I32, _P, _I32, _P, _F, _P, _P,
                                            _P]),
    "cs_closed_ring_segments": (ctypes.c_int, [_P, _I32, _I32, _I32, _P, _P, _P, _P, _P]),
    "cs_closed_ring_segments_backward": (ctypes.c_int, [_P, _I32, _I32, _I32, _P, _P, _P, _P,
                                                        _P]),
    "cs_clamp_mse_ssim_loss": (ctypes.c_int, [_P, _I32, _P, _I32, _I32, _F, _F, _P, _I32, _F, _F,
                                              _F, _P, _P, _P, _P, _P]),
    "cs_clamp_mse_ssim_backward": (ctypes.c_int, [_P, _I32, _P, _I32, _I32, _F, _F, _P, _I32, _P,
                                                  _F, _P, _P, _I32, _P]),
    "cs_adam_step": (ctypes.c_int, [_I32, _P, _P, _P, _P, _P, _P, _P, _P, _D, _D, _D, _P]),
    "cs_adan_step": (ctypes.c_int, [_I32, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P]),
    "cs_gs_project_forward": (ctypes.c_int, [_P, _P, _P, _I32, _I32, _I32, _I32, _I32, _P, _P, _P,
                                             _P, _P, _P]),
    "cs_gs_bin_prepare": (ctypes.c_int, [_P, _P, _P, _P, _I32, _I32, _I32, _I32, _I32, _P, _P, _P,
                                         _P, _P, _P, _P, _P, _P, _P, _P, _P]),
    "cs_gs_pack_records": (ctypes.c_int, [_P, _P, _P, _P, _I32, _P, _P]),
    "cs_gs_rasterize_forward": (ctypes.c_int, [_P, _P, _P, _P, _I32, _I32, _I32, _I32, _P, _P, _P,
                                               _P]),
    "cs_gs_rasterize_backward": (ctypes.c_int, [_P, _P, _P, _P, _P, _I32, _I32, _I32, _I32, _P, _P,
                                                _P, _P, _P, _P, _P, _P, _P, _P, _P]),
    "cs_gs_project_backward": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _I32, _I32, _I32, _P, _P,
                                              _P, _P, _P]),
    "cs_gs_map_to_intersects": (ctypes.c_int, [_P, _P, _P, _P, _P, _I32, _I64, _I32, _I32, _I32,
                                               _I32, _P, _P, _P]),
}
GS_RECORD_BYTES = 48     # per-Gaussian raster record

_lib = None


def lib() -> ctypes.CDLL:
    """Load the HIP library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built; run `python -m repo_amd.build` "
                "(or __graft_entry__.build()) first")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


# HIP runtime entry points used by the host code (event timing, the one
# device->host copy of the forward), bound through the library's handle so
# they resolve to the runtime torch has loaded (same SONAME).
_HIP_SIGNATURES = {
    "hipEventCreateWithFlags": (ctypes.c_int, [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]),
    "hipEventRecord": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p]),
    "hipEventSynchronize": (ctypes.c_int, [ctypes.c_void_p]),
    "hipEventQuery": (ctypes.c_int, [ctypes.c_void_p]),
    "hipEventElapsedTime": (ctypes.c_int, [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p,
                                           ctypes.c_void_p]),
    "hipEventDestroy": (ctypes.c_int, [ctypes.c_void_p]),
    "hipMemcpyAsync": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t,
                                      ctypes.c_int, ctypes.c_void_p]),
    "hipHostGetDevicePointer": (ctypes.c_int, [ctypes.POINTER(ctypes.c_void_p), ctypes.c_void_p,
                                               ctypes.c_uint]),
    "hipGetLastError": (ctypes.c_int, []),
}
HIP_EVENT_DEFAULT = 0
HIP_EVENT_DISABLE_TIMING = 2
HIP_MEMCPY_DEVICE_TO_HOST = 2


class _HipRuntime:
    def __init__(self):
        L = ctypes.CDLL(LIB_PATH)
        lib()
        fast = _fast_module()
        for name, (res, args) in _HIP_SIGNATURES.items():
            fn = getattr(fast, name, None) if fast is not None else None
            if fn is None:
                fn = getattr(L, name)
                fn.restype, fn.argtypes = res, args
            setattr(self, name, fn)


_hip_rt = None


def hip() -> _HipRuntime:
    global _hip_rt
    if _hip_rt is None:
        _hip_rt = _HipRuntime()
    return _hip_rt


def hip_check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what} failed (HIP status {rc})")


def event_create(timing: bool = False) -> int:
    """A raw hipEvent_t (int); destroy with event_destroy."""
    h = ctypes.c_void_p()
    flags = HIP_EVENT_DEFAULT if timing else HIP_EVENT_DISABLE_TIMING
    hip_check(hip().hipEventCreateWithFlags(ctypes.byref(h), flags), "hipEventCreateWithFlags")
    return h.value


def event_elapsed_ms(a: int, b: int) -> float:
    out = ctypes.c_float()
    hip_check(hip().hipEventElapsedTime(ctypes.byref(out), a, b), "hipEventElapsedTime")
    return float(out.value)


def host_device_ptr(host_ptr: int) -> Optional[int]:
    """The device-accessible address of pinned host memory, or None where the
    runtime gives none (the caller then copies instead)."""
    d = ctypes.c_void_p()
    if hip().hipHostGetDevicePointer(ctypes.byref(d), host_ptr, 0) != 0:
        hip().hipGetLastError()  # clear it: the entry points report the last error
        return None
    return d.value or None


def event_destroy(ev: int) -> None:
    hip_check(hip().hipEventDestroy(ev), "hipEventDestroy")


def exported_symbols():
    return list(_SIGNATURES)


def ptr(t):
    """Device pointer of a tensor as an int (None -> NULL); ctypes passes ints
    for c_void_p parameters without building pointer objects."""
    if t is None:
        return None
    return t.data_ptr()


_raw_stream = torch._C._cuda_getCurrentRawStream


def stream(device=None) -> int:
    """torch's current stream on `device` (a torch.device, an index or None
    for the current device) as the raw hipStream_t."""
    if device is None:
        idx = torch.cuda.current_device()
    elif isinstance(device, int):
        idx = device
    else:
        idx = device.index if device.index is not None else torch.cuda.current_device()
    return _raw_stream(idx)


def check(rc: int, what: str) -> None:
    if rc == CS_OK:
        return
    kind = "invalid arguments" if rc == CS_ERR_ARGS else "HIP launch failure"
    raise RuntimeError(f"{what}: {kind} (status {rc})")


_FUNCS = {}
_FAST = False   # not looked up yet


def _fast_module():
    """The compiled binding of the same entry points (repo_amd/fastcall.py),
    or None when it has not been built (ctypes is used then)."""
    global _FAST
    if _FAST is False:
        try:
            from . import _cs_fast
        except ImportError:
            _cs_fast = None
        if _cs_fast is not None:
            from . import fastcall
            if _cs_fast.signature_hash() != fastcall.signature_hash():
                warnings.warn("repo_amd._cs_fast was built from other entry-point signatures; "
                              "using ctypes (run build() again)")
                _cs_fast = None
        _FAST = _cs_fast
    return _FAST


def call(name: str, *args) -> None:
    fn = _FUNCS.get(name)
    if fn is None:
        L = lib()
        fast = _fast_module()
        fn = getattr(fast, name, None) if fast is not None else None
        _FUNCS[name] = fn = fn if fn is not None else getattr(L, name)
    rc = fn(*args)
    if rc != CS_OK:
        check(rc, name)


ProfileCtxFactory = Callable[[str], ContextManager]
_PROFILE_CTX_FACTORY: Optional[ProfileCtxFactory] = None


def set_profile_ctx_factory(factory: Optional[ProfileCtxFactory]) -> None:
    """Installs a factory of context managers that wrap each library launch,
    keyed by a stage label such as "cubic.bwd.rast" (the same protocol as the
    reference's set_gs_profile_ctx_factory, tilelang_renderer.py:31-39).  The
    context is entered right before the C-ABI call and left right after it,
    so HIP events recorded on the current stream inside it bracket exactly
    that call's kernels."""
    global _PROFILE_CTX_FACTORY
    _PROFILE_CTX_FACTORY = factory


def prof(label: str):
    if _PROFILE_CTX_FACTORY is None:
        return nullcontext()
    return _PROFILE_CTX_FACTORY(label)


def require_gpu(t: torch.Tensor, name: str) -> None:
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be a CUDA (ROCm) tensor")
