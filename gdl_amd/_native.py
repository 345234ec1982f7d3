"""ctypes binding of libgeoembodied_hip.so (the C ABI declared in include/geo_api.h).

The library is loaded once per process from ``gdl_amd/lib/`` (override with the environment
variable ``GEOEMBODIED_HIP_LIB``).  There is no fallback: if the library cannot be loaded every
operation raises ``RuntimeError`` naming the path that was tried.
"""

from __future__ import annotations

import contextlib
import ctypes
import os
import threading
from pathlib import Path

import torch

_LIB_ENV = "GEOEMBODIED_HIP_LIB"
_DEFAULT = Path(__file__).resolve().parent / "lib" / "libgeoembodied_hip.so"

c_i64 = ctypes.c_int64
c_int = ctypes.c_int
c_vp = ctypes.c_void_p
c_size = ctypes.c_size_t
c_f32 = ctypes.c_float
c_i32 = ctypes.c_int32

# name -> (restype, argtypes)
_SIGNATURES = {
    "geo_last_error": (ctypes.c_char_p, []),
    "geo_build_info": (ctypes.c_char_p, []),
    "geo_abi_version": (c_int, []),
    "geo_fps_prepare": (c_int, [c_vp, c_vp, c_i64, c_i64, c_vp, c_vp, c_vp]),
    "geo_fps_prepare_uniform": (c_int, [c_vp, c_i64, c_i64, c_i64, c_vp, c_vp, c_vp, c_vp]),
    "geo_fps_guarded": (c_int, [c_vp, c_i64, c_vp, c_vp, c_i64, c_i64, c_vp, c_vp, c_vp, c_vp]),
    "geo_fps_workspace_bytes": (c_size, [c_i64, c_i64, c_i64]),
    "geo_fps": (c_int, [c_vp, c_i64, c_vp, c_vp, c_i64, c_i64, c_vp, c_vp, c_size, c_vp]),
    "geo_knn_workspace_bytes": (c_size, [c_i64, c_i64, c_i64, c_i64]),
    "geo_knn": (c_int, [c_vp, c_i64, c_vp, c_i64, c_vp, c_vp, c_i64, c_i64, c_vp, c_vp, c_vp,
                        c_size, c_vp]),
    "geo_radius_workspace_bytes": (c_size, [c_i64, c_i64, c_i64]),
    "geo_radius_count": (c_int, [c_vp, c_i64, c_vp, c_i64, c_i64, c_vp, c_f32, c_f32, c_i64,
                                 c_int, c_vp, c_vp, c_size, c_vp]),
    "geo_radius_emit": (c_int, [c_vp, c_i64, c_vp, c_i64, c_i64, c_vp, c_f32, c_f32, c_i64,
                                c_int, c_vp, c_vp, c_vp, c_vp, c_size, c_vp]),
    "geo_csr_workspace_bytes": (c_size, [c_i64, c_i64]),
    "geo_csr_build": (c_int, [c_vp, c_i64, c_i64, c_vp, c_vp, c_vp, c_vp, c_vp, c_size, c_vp]),
    "geo_csr_build_noalloc": (c_int, [c_vp, c_i64, c_i64, c_vp, c_vp, c_vp, c_vp, c_vp]),
    "geo_csr_from_row_ptr": (c_int, [c_vp, c_i64, c_vp, c_i64, c_vp, c_vp, c_vp, c_vp, c_vp]),
    "geo_spatial_graph_epilogue_dev": (c_int, [c_vp, c_i64, c_vp, c_vp, c_vp, c_i64, c_int, c_i64,
                                               c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp,
                                               c_vp]),
    "geo_spatial_graph_epilogue": (c_int, [c_vp, c_i64, c_vp, c_vp, c_vp, c_i64, c_int, c_vp, c_i64,
                                           c_i64, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp,
                                           c_vp, c_size, c_vp]),
    "geo_segment_reduce_fwd": (c_int, [c_int, c_int, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64,
                                       c_i64, c_vp, c_vp, c_int, c_vp]),
    "geo_segment_reduce_bwd": (c_int, [c_int, c_int, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp,
                                       c_vp, c_i64, c_i64, c_i64, c_vp, c_vp]),
    "geo_segment_softmax_fwd": (c_int, [c_int, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_int,
                                        c_vp, c_vp]),
    "geo_segment_softmax_bwd": (c_int, [c_int, c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_i64,
                                        c_int, c_vp, c_vp]),
    "geo_gather_weighted_sum": (c_int, [c_int, c_vp, c_i64, c_i64, c_vp, c_vp, c_i64, c_i64, c_vp,
                                        c_vp]),
    "geo_gather_weighted_sum_bwd": (c_int, [c_int, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_i64,
                                            c_i64, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp]),
    "geo_idw_weights": (c_int, [c_vp, c_vp, c_i64, c_i64, c_vp, c_vp]),
    "geo_idw_interpolate": (c_int, [c_int, c_vp, c_i64, c_i64, c_vp, c_vp, c_i64, c_i64, c_vp,
                                    c_vp, c_vp]),
    "geo_radius_count_dev": (c_int, [c_vp, c_i64, c_vp, c_i64, c_i64, c_vp, c_vp, c_i64, c_int,
                                     c_vp, c_vp, c_size, c_vp]),
    "geo_radius_count_async": (c_int, [c_vp, c_i64, c_vp, c_i64, c_i64, c_vp, c_f32, c_f32, c_vp,
                                       c_i64, c_int, c_vp, c_vp, c_vp, c_size, c_vp]),
    "geo_radius_copy_edges": (c_int, [c_vp, c_vp, c_i64, c_vp, c_vp, c_vp]),
    "geo_radius_emit_dev": (c_int, [c_vp, c_i64, c_vp, c_i64, c_i64, c_vp, c_vp, c_i64, c_int,
                                    c_vp, c_vp, c_vp, c_vp, c_size, c_vp]),
    "geo_knn_radius_stat_workspace_bytes": (c_size, [c_i64]),
    "geo_edge_geometry": (c_int, [c_vp, c_i64, c_vp, c_vp, c_i64, c_int, c_vp, c_vp, c_vp, c_vp]),
    "geo_edge_geometry_bwd": (c_int, [c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_int, c_vp, c_vp]),
    "geo_spherical_harmonics": (c_int, [c_vp, c_i64, c_int, c_int, c_vp, c_vp, c_vp, c_vp]),
    "geo_spherical_harmonics_bwd": (c_int, [c_vp, c_vp, c_i64, c_int, c_vp, c_vp]),
    "geo_graph_avg_degree_workspace_bytes": (c_size, [c_i64]),
    "geo_graph_avg_degree": (c_int, [c_vp, c_i64, c_vp, c_i64, c_i64, c_vp, c_vp, c_size, c_vp]),
    "geo_knn_radius_stat": (c_int, [c_vp, c_i64, c_i64, c_i64, c_int, ctypes.c_double, c_vp, c_vp,
                                    c_size, c_vp]),
    "geo_se3_aggregate_fwd": (c_int, [c_vp, c_vp, c_vp, c_i64, c_i32, c_i32, c_i32, c_vp, c_vp, c_vp,
                                      c_vp, c_i64, c_vp, c_vp, c_i32, c_vp, c_i32, c_vp, c_vp, c_vp,
                                      c_i32, c_vp, c_i32, c_vp, c_i32, c_vp]),
    "geo_se3_fwd_fused_lds_bytes": (c_size, [c_i32, c_i32, c_i32, c_i32, c_i32, c_i32]),
    "geo_se3_fwd_fused": (c_int, [c_vp, c_vp, c_vp, c_i64, c_i32, c_i32, c_i32, c_vp, c_vp, c_vp, c_vp,
                                  c_i64, c_vp, c_vp, c_i32, c_vp, c_i32, c_vp, c_vp, c_vp, c_i32, c_vp,
                                  c_i32, c_vp, c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_vp,
                                  c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp]),
    "geo_se3_gemm": (c_int, [c_vp, c_i64, c_i32, c_vp, c_i32, c_i32, c_i32, c_vp, c_i64, c_vp, c_vp,
                             c_vp, c_vp]),
    "geo_se3_gemm_tn_workspace_bytes": (c_size, [c_i64, c_i32, c_i32]),
    "geo_se3_gemm_tn": (c_int, [c_vp, c_i64, c_i32, c_i32, c_vp, c_i32, c_i32, c_vp, c_i32, c_vp, c_size,
                                c_vp]),
    "geo_se3_gemm_tn_split": (c_int, [c_vp, c_i64, c_i32, c_i32, c_vp, c_i32, c_i32, c_i32, c_vp, c_vp,
                                      c_vp, c_size, c_vp]),
    "geo_se3_colsum_workspace_bytes": (c_size, [c_i64, c_i32]),
    "geo_se3_colsum": (c_int, [c_vp, c_i64, c_i32, c_vp, c_vp, c_vp, c_size, c_vp]),
    "geo_se3_pack_weights": (c_int, [c_vp, c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_vp, c_vp,
                                     c_vp, c_vp, c_vp]),
    "geo_se3_grad_prep": (c_int, [c_vp, c_i64, c_i32, c_i32, c_i32, c_vp, c_vp, c_vp, c_vp]),
    "geo_se3_bwd_edge": (c_int, [c_vp, c_vp, c_vp, c_i64, c_i32, c_i32, c_i32, c_vp, c_vp, c_vp, c_vp,
                                 c_i64, c_vp, c_vp, c_i32, c_vp, c_i32, c_vp, c_vp, c_vp, c_i32, c_vp,
                                 c_i32, c_vp, c_i32, c_vp, c_vp, c_vp, c_vp]),
    "geo_radial_mlp_fwd": (c_int, [c_vp, c_i64, c_vp, c_i32, c_f32, c_vp, c_vp, c_i32, c_vp, c_vp, c_i32,
                                   c_vp, c_vp]),
    "geo_radial_mlp_bwd_workspace_bytes": (c_size, [c_i64, c_i32, c_i32, c_i32]),
    "geo_radial_mlp_bwd": (c_int, [c_vp, c_i64, c_vp, c_i32, c_f32, c_vp, c_vp, c_i32, c_vp, c_vp, c_i32,
                                   c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_size, c_vp]),
    "geo_se3_bwd_src": (c_int, [c_vp, c_i32, c_i32, c_vp, c_i32, c_i32, c_vp, c_i32, c_i32, c_i64,
                                c_vp, c_vp, c_vp, c_vp, c_i64, c_vp, c_vp, c_i32, c_vp, c_i32, c_vp,
                                c_vp, c_vp, c_i32, c_vp, c_i32, c_vp, c_i32, c_vp, c_i32, c_vp]),
    "geo_se3_bwd_edge_fused": (c_int, [c_vp, c_vp, c_i64, c_i32, c_i32, c_vp, c_vp, c_vp, c_vp, c_i64,
                                       c_vp, c_vp, c_i32, c_vp, c_i32, c_vp, c_vp, c_vp, c_i32, c_vp,
                                       c_i32, c_vp, c_i32, c_vp, c_i32, c_i32, c_i32, c_vp, c_vp,
                                       c_vp, c_vp]),
    "geo_se3_bwd_src_fused": (c_int, [c_vp, c_i32, c_i32, c_vp, c_i32, c_i32, c_i64, c_vp, c_vp, c_vp,
                                      c_vp, c_i64, c_vp, c_vp, c_i32, c_vp, c_i32, c_vp, c_vp, c_i32,
                                      c_i32, c_vp, c_i32, c_i32, c_vp, c_vp, c_i32, c_i32, c_vp,
                                      c_vp]),
}

EXPORTED = tuple(_SIGNATURES)

GEO_F32, GEO_BF16, GEO_F64 = 0, 1, 2
REDUCE_CODES = {"sum": 0, "mean": 1, "max": 2}
DTYPE_CODES = {torch.float32: GEO_F32, torch.bfloat16: GEO_BF16, torch.float64: GEO_F64}

_lock = threading.Lock()
_lib = None
_load_error: str | None = None


def library_path() -> Path:
    return Path(os.environ.get(_LIB_ENV, str(_DEFAULT)))


def _load():
    global _lib, _load_error
    with _lock:
        if _lib is not None or _load_error is not None:
            return _lib
        path = library_path()
        try:
            lib = ctypes.CDLL(str(path))
        except OSError as exc:
            _load_error = f"cannot load {path}: {exc} (build it with `python -m gdl_amd.build`)"
            return None
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


def lib():
    """The loaded library; raises RuntimeError when it is missing."""
    out = _load()
    if out is None:
        raise RuntimeError(f"geoembodied HIP library unavailable: {_load_error}")
    return out


def loaded() -> bool:
    return _load() is not None


def last_error() -> str:
    msg = lib().geo_last_error()
    return msg.decode() if msg else ""


GEO_ERR_UNSUPPORTED = 4  # include/geo_api.h: the call declined a case it does not cover


def check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what} failed (status {rc}): {last_error()}")


def build_info() -> str:
    return lib().geo_build_info().decode()


def ptr(t: torch.Tensor | None):
    return None if t is None else t.data_ptr()


def stream_of(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


_SAME_DEVICE = contextlib.nullcontext()


def on_device(device: torch.device):
    """Context making ``device`` the current HIP device for a library call: a shared no-op
    context when it already is (entering torch.cuda.device costs microseconds per call)."""
    if device.index is None or device.index == torch.cuda.current_device():
        return _SAME_DEVICE
    return torch.cuda.device(device)


def workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


_tls = threading.local()


def sync_slot(device: torch.device):
    """(pinned int64[4] host tensor, event) kept per thread and device for an op's one size sync:
    a kernel writes the sizes into the mapped pinned memory, the op records the event behind it,
    waits for the event and reads the values before returning, so consecutive calls of a thread
    never overlap on the slot and threads never share one."""
    slots = getattr(_tls, "slots", None)
    if slots is None:
        slots = _tls.slots = {}
    key = device.index if device.index is not None else torch.cuda.current_device()
    slot = slots.get(key)
    if slot is None:
        slot = slots[key] = (torch.empty(4, dtype=torch.int64, pin_memory=True), torch.cuda.Event())
    return slot
