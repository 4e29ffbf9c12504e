"""ctypes binding of libpointops_hip.so (the C ABI in include/pointops_hip.h).

This is the only way the package reaches the GPU: there is no CPU or PyTorch
fallback.  Loading fails loudly when the library is missing or was built for
another architecture; every call checks the returned hipError_t.

The reference compiles Metal shaders on first use and checks the SIMD width
(_ball_query_mps.py:34-63); the equivalent gate here is that the library is
present and the device is gfx950 (checked once per device).
"""

from __future__ import annotations

import ctypes
import functools
import os
from pathlib import Path

import torch

LIB_NAME = "libpointops_hip.so"
LIB_PATH = Path(__file__).resolve().with_name(LIB_NAME)

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_f32 = ctypes.c_float
_size = ctypes.c_size_t

# name -> argument types (pointers as void*), restype int (hipError_t)
_SIGNATURES: dict[str, list] = {
    "pointops_fps_dense": [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i32, _vp],
    "pointops_fps_large": [_vp, _vp, _vp, _i64, _i64, _i64, _i32, _vp],
    "pointops_fps_large_noalloc": [_vp, _vp, _i64, _i64, _i64, _i32, _vp],
    "pointops_fps_flat": [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp],
    "pointops_knn3": [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp],
    "pointops_knn3_grid": [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp],
    "pointops_knn3_windowed": [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp],
    "pointops_knn_feat": [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _vp],
    "pointops_knn_flat": [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp],
    "pointops_ball_query_f32": [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _f32, _vp],
    "pointops_ball_query_multi_f32": [_vp, _vp, _i64, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp],
    "pointops_ball_query_f16": [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _f32, _vp],
    "pointops_radius_flat_f32": [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _f32, _i32, _vp],
    "pointops_radius_flat_f16": [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _f32, _i32, _vp],
    "pointops_ball_query_backward_f32": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64,
                                         _i64, _vp],
    "pointops_ball_query_backward_f16": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64,
                                         _i64, _vp],
    "pointops_three_nn": [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp],
    "pointops_three_interpolate": [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp],
    "pointops_three_interpolate_backward": [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp],
    "pointops_three_interpolate_backward_csr": [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64,
                                                _vp],
    "pointops_three_interpolate_csr_build": [_vp, _vp, _vp, _i64, _i64, _i64, _vp],
    "pointops_three_interpolate_backward_from_csr": [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp],
    "pointops_ball_query_pn2_f32": [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _f32, _vp],
    "pointops_ball_query_grid_f32": [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _f32, _vp],
    "pointops_ball_query_auto_f32": [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _f32, _vp],
    "pointops_nearest3_grid": [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp],
    "pointops_group_points": [_vp, _vp, _i32, _vp, _i64, _i64, _i64, _i64, _vp],
    "pointops_group_points_backward": [_vp, _i64, _vp, _i32, _vp, _vp, _i64, _i64, _i64, _i64, _vp],
    "pointops_group_points_rel": [_vp, _vp, _vp, _vp, _i32, _vp, _i64, _i64, _i64, _i64, _i64, _vp],
    "pointops_chamfer_nearest_f32": [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i32, _vp],
    "pointops_chamfer_nearest_f64": [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i32, _vp],
    "pointops_chamfer_backward_f32": [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i32, _vp],
    "pointops_chamfer_backward_f64": [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i32, _vp],
    "pointops_fps_query_pipeline_f32": [_vp, _vp, _vp, _i64, _vp, _vp, _vp, _vp, _i64, _vp, _vp,
                                        _vp, _vp, _i64, _i64, _i64, _i64, _i32, _i64, _vp, _vp],
}
_SIZE_QUERIES: dict[str, list] = {
    "pointops_fps_dense_scratch_bytes": [_i64, _i64],
    "pointops_fps_query_pipeline_workspace_bytes": [_i64, _i64, _i64, _i64],
    "pointops_fps_large_workspace_bytes": [_i64, _i64],
    "pointops_fps_flat_scratch_bytes": [_i64, _i64],
    "pointops_knn3_grid_workspace_bytes": [_i64, _i64, _i64],
    "pointops_knn3_windowed_workspace_bytes": [_i64, _i64, _i64],
    "pointops_three_interpolate_backward_workspace_bytes": [_i64, _i64, _i64],
    "pointops_ball_query_grid_workspace_bytes": [_i64, _i64, _i64],
    "pointops_ball_query_backward_workspace_bytes": [_i64, _i64],
    "pointops_ball_query_auto_workspace_bytes": [_i64, _i64, _i64],
    "pointops_group_points_backward_workspace_bytes": [_i64, _i64, _i64, _i64],
}


@functools.lru_cache(maxsize=1)
def library() -> ctypes.CDLL:
    """Load the native library (once).  Raises if it has not been built."""
    path = Path(os.environ.get("POINTOPS_HIP_LIB", LIB_PATH))
    if not path.exists():
        raise RuntimeError(
            f"mps_pointops native library not found at {path}; build it with "
            "`python mps-pointops_amd/build.py` (hipcc, gfx950)"
        )
    lib = ctypes.CDLL(str(path))
    for name, args in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = ctypes.c_int
    for name, args in _SIZE_QUERIES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = _size
    lib.pointops_abi_version.restype = ctypes.c_int
    lib.pointops_device_supported.argtypes = [ctypes.c_int]
    lib.pointops_device_supported.restype = ctypes.c_int
    if lib.pointops_abi_version() != 1:
        raise RuntimeError(f"{path.name} has an unexpected ABI version")
    return lib


@functools.lru_cache(maxsize=None)
def _check_device(index: int) -> None:
    if not library().pointops_device_supported(index):
        name = torch.cuda.get_device_properties(index).gcnArchName
        raise RuntimeError(
            f"mps_pointops kernels are built for gfx950 (MI355X); cuda:{index} is {name}"
        )


@functools.lru_cache(maxsize=1)
def _hip_error_string():
    try:
        hip = ctypes.CDLL("libamdhip64.so")
        hip.hipGetErrorString.argtypes = [ctypes.c_int]
        hip.hipGetErrorString.restype = ctypes.c_char_p
        return hip.hipGetErrorString
    except OSError:
        return None


def require_device(device: torch.device) -> int:
    """Index of a usable ROCm device, after the one-time capability check."""
    if device.type != "cuda":
        raise ValueError(
            f"mps_pointops runs on ROCm GPU tensors (device='cuda'); got {device.type}"
        )
    index = device.index if device.index is not None else torch.cuda.current_device()
    _check_device(index)
    return index


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def call(name: str, *args) -> None:
    status = getattr(library(), name)(*args)
    if status != 0:
        getter = _hip_error_string()
        text = getter(status).decode() if getter is not None else f"hipError {status}"
        raise RuntimeError(f"{name} failed: {text}")


def size_query(name: str, *args) -> int:
    return int(getattr(library(), name)(*args))
