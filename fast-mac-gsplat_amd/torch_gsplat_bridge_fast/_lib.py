"""ctypes binding of libgsplat_hip.so (the C ABI in include/gsplat_hip.h).

The library is built in-tree (``make -C fast-mac-gsplat_amd/csrc`` or
``__graft_entry__.build()``) into ``torch_gsplat_bridge_fast/lib/``.  torch is
imported first so that the library binds to the HIP runtime torch already
loaded (one runtime per process).  There is no fallback: if the library is
missing, every entry point raises.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

import torch  # noqa: F401  (must be loaded before the HIP library)

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("GSPLAT_HIP_LIB", os.path.join(_HERE, "lib", "libgsplat_hip.so"))

ABI_VERSION = 15
TILE_SIZE = 16
RECORD_FLOATS = 16
PROJECT_NOALLOC_SCRATCH_BYTES = 1 << 20   # GSPLAT_PROJECT_NOALLOC_SCRATCH_BYTES
STATUS_LOOKBACK_TIMEOUT = 1               # GSPLAT_STATUS_LOOKBACK_TIMEOUT
HANDOFF_PAIRS = 128                       # GSPLAT_HANDOFF_PAIRS
TIME_FORWARD, TIME_BACKWARD = 0, 1        # GSPLAT_TIME_FORWARD / _BACKWARD
TRACE_MAX = 1024                          # GSPLAT_TRACE_MAX

_vp = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_sz = ctypes.c_size_t


class RasterMeta(ctypes.Structure):
    """Mirror of ``gsplat_raster_meta``."""

    _fields_ = [
        ("height", _i32),
        ("width", _i32),
        ("tile_size", _i32),
        ("batch", _i32),
        ("gaussians_per_batch", _i32),
        ("alpha_threshold", ctypes.c_float),
        ("transmittance_threshold", ctypes.c_float),
        ("background", ctypes.c_float * 3),
        ("eps", ctypes.c_float),
        ("max_alpha", ctypes.c_float),
    ]


class ProjectMeta(ctypes.Structure):
    """Mirror of ``gsplat_project_meta``."""

    _fields_ = [
        ("batch", _i32),
        ("gaussians_per_batch", _i32),
        ("near_plane", ctypes.c_float),
    ]


_PM = ctypes.POINTER(RasterMeta)
_PP = ctypes.POINTER(ProjectMeta)

# name -> (restype, argtypes); every name here is declared in gsplat_hip.h.
SIGNATURES = {
    "gsplat_hip_abi_version": (ctypes.c_int, []),
    "gsplat_hip_last_error": (ctypes.c_char_p, []),
    "gsplat_hip_time_next_launch": (ctypes.c_int, [ctypes.c_int, _vp, _vp]),
    "gsplat_hip_trace_launches": (ctypes.c_int, [ctypes.POINTER(_vp), ctypes.c_int]),
    "gsplat_hip_trace_count": (ctypes.c_int, []),
    "gsplat_hip_trace_name": (ctypes.c_char_p, [ctypes.c_int]),
    "gsplat_hip_bin_count_workspace_bytes": (_sz, [_PM]),
    "gsplat_hip_bin_count": (ctypes.c_int, [_PM] + [_vp] * 4 + [_vp, _sz, _vp]),
    "gsplat_hip_bin_depth_order": (ctypes.c_int, [_PM, _vp, _vp, _vp, _sz, _vp]),
    "gsplat_hip_bin_pack": (ctypes.c_int, [_PM] + [_vp] * 7 + [_vp, _sz, _vp]),
    "gsplat_hip_pack_records": (ctypes.c_int, [_PM] + [_vp] * 5 + [_vp]),
    "gsplat_hip_bin_emit_workspace_bytes": (_sz, [_PM, _i64]),
    "gsplat_hip_bin_emit": (ctypes.c_int, [_PM, _vp, _vp, _i64, _vp, _vp, _vp, _vp, _vp, _sz, _vp, _sz, _vp]),
    "gsplat_hip_bin_workspace_bytes": (_sz, [_PM, _i64]),
    "gsplat_hip_bin": (ctypes.c_int, [_PM] + [_vp] * 5 + [_i64] + [_vp] * 7 + [_sz] + [_vp] * 5),
    "gsplat_hip_render_workspace_bytes": (_sz, [_PM, _i64]),
    "gsplat_hip_render_forward": (ctypes.c_int, [_PM] + [_vp] * 7 + [_i64, _vp, _sz, _vp]),
    "gsplat_hip_render_forward_long": (ctypes.c_int, [_PM] + [_vp] * 7 + [_i64, _vp, _sz, _vp]),
    "gsplat_hip_bin_render_forward": (
        ctypes.c_int,
        [_PM] + [_vp] * 5 + [_i64] + [_vp] * 7 + [_sz] + [_vp] * 5 + [_sz] + [_vp] * 5,
    ),
    "gsplat_hip_render_backward": (ctypes.c_int, [_PM] + [_vp] * 11 + [_i64, _vp, _sz, _vp]),
    "gsplat_hip_project_forward": (ctypes.c_int, [_PP] + [_vp] * 10 + [_vp]),
    "gsplat_hip_project_backward_workspace_bytes": (_sz, [_PP]),
    "gsplat_hip_project_backward": (ctypes.c_int, [_PP] + [_vp] * 16 + [_vp, _sz, _vp]),
    "gsplat_hip_project_backward_noalloc": (ctypes.c_int, [_PP] + [_vp] * 16 + [_vp]),
    "gsplat_hip_scan_workspace_bytes": (_sz, [_i64]),
    "gsplat_hip_exclusive_scan_i32": (ctypes.c_int, [_vp, _vp, _i64, _vp, _vp, _sz, _vp]),
    "gsplat_hip_debug_stalled_scan": (ctypes.c_int, [_vp, _vp, _i64, _i32, _i32, _vp, _vp, _sz, _vp]),
    "gsplat_hip_radix_sort_workspace_bytes": (_sz, [_i64, _i32]),
    "gsplat_hip_radix_sort_pairs_u32": (
        ctypes.c_int,
        [_vp, _vp, _vp, _vp, _i64, _i32, _i32, _i32, _vp, _vp, _sz, _vp],
    ),
}

_lib: Optional[ctypes.CDLL] = None
_load_error: Optional[str] = None


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load (once) and return the library; raises RuntimeError if absent."""
    global _lib, _load_error
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        _load_error = f"libgsplat_hip.so not found at {path}; build it with `make -C fast-mac-gsplat_amd/csrc`"
        raise RuntimeError(_load_error)
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    ver = lib.gsplat_hip_abi_version()
    if ver != ABI_VERSION:
        raise RuntimeError(f"libgsplat_hip ABI version {ver} != expected {ABI_VERSION}")
    _lib = lib
    return lib


def lib() -> ctypes.CDLL:
    return _lib if _lib is not None else load()


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().gsplat_hip_last_error()
        raise RuntimeError(f"{what} failed (status {rc}): {msg.decode() if msg else ''}")


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def make_raster_meta(height, width, batch, gpb, alpha_threshold, transmittance_threshold, background,
                     eps=1e-8, max_alpha=0.99) -> RasterMeta:
    m = RasterMeta()
    m.height = int(height)
    m.width = int(width)
    m.tile_size = TILE_SIZE
    m.batch = int(batch)
    m.gaussians_per_batch = int(gpb)
    m.alpha_threshold = float(alpha_threshold)
    m.transmittance_threshold = float(transmittance_threshold)
    for i in range(3):
        m.background[i] = float(background[i])
    m.eps = float(eps)
    m.max_alpha = float(max_alpha)
    return m


def make_project_meta(batch, gpb, near_plane) -> ProjectMeta:
    m = ProjectMeta()
    m.batch = int(batch)
    m.gaussians_per_batch = int(gpb)
    m.near_plane = float(near_plane)
    return m
