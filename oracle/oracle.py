"""numpy front end of the CPU oracle (pointops_oracle.c).

TEST INFRASTRUCTURE ONLY.  Only tests/, ``__graft_entry__.smoke()`` and
bench.py's ``cpu_baseline`` leg import this module, and only as the checker.
The shipped package (mps-pointops_amd/mps_pointops) never imports it.

Every function restates /root/reference/mps_pointops arithmetic bit for bit
(see the C file for the file:line each follows).  How each one is pinned:

* ``fps``: the reference's known answers (tests/test_fps.py:46-48 duplicates,
  tests/test_compat.py:96-118 skip radius, tests/test_flat.py:20-29 and
  README.md:82-93), the Metal selections recorded in
  docs/parity/pointnet2-segmentation-mps-safe.npz (four FPS calls), and an
  independent numpy recomputation of the max-min property per step.
* ``knn3`` / ``knn_feat`` / ``knn_flat``: the exact lexsort oracle of
  tests/test_knn.py:15-23 and the scalar loop of tests/test_feature_knn.py:16-35
  re-implemented in numpy, plus the reference's tie/non-finite known answers.
* ``ball_query`` / ``radius_flat``: the reference's known answers
  (tests/test_ball_query_api.py, tests/test_ball_query_mps.py, test_flat.py,
  test_flat_ragged_mps.py), the four Metal ball-query selections in the
  segmentation fixture, and brute force in numpy float32.
* ``three_nn`` / ``three_interpolate``: tests/test_pointnet2.py known answers,
  docs/parity/pointnet2-{mps-safe,cuda}.json (inputs rebuilt from
  tools/pointnet2parity.py:125-171), numpy stable argsort, and the four Metal
  three_nn selections in the segmentation fixture.
* ``chamfer_nearest``: tests/test_chamfer.py / test_chamfer_nd.py known
  answers and a numpy argmin brute force.
* ``group_points`` / ``group_points_backward`` / ``group_points_rel``: the
  known answer of tests/test_compat.py:134-137 (gradient of a gather with a
  repeated index), the element identities of tests/test_compat.py:121-131,
  numpy fancy indexing and ``np.add.at``, and the invariant that a centre
  grouped with itself is 0 in the relative channels.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "liboracle.so"
_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_i64p = ctypes.POINTER(ctypes.c_int64)
_i32p = ctypes.POINTER(ctypes.c_int32)
_i64 = ctypes.c_int64


def build(force: bool = False) -> Path:
    """Compile liboracle.so with the committed Makefile."""
    if force or not _LIB_PATH.exists():
        subprocess.run(["make", "-s", "-C", str(_HERE), "-B" if force else "liboracle.so"],
                       check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        lib = ctypes.CDLL(str(_LIB_PATH))
        lib.oracle_fps.argtypes = [_f32p, _i64, _i64, _i64, _i64, ctypes.c_int, _i64p]
        lib.oracle_fps_flat.argtypes = [_f32p, _i64p, _i64p, _i64p, _i64, _i64p]
        lib.oracle_knn3.argtypes = [_f32p, _f32p, _i64, _i64, _i64, _i64, _f32p, _i64p]
        lib.oracle_knn_feat.argtypes = [_f32p, _f32p, _i64, _i64, _i64, _i64, _i64, _f32p, _i64p]
        lib.oracle_knn_flat.argtypes = [_f32p, _f32p, _i64p, _i64p, _i64, _i64, _i64, _i64, _i64p]
        lib.oracle_ball_query.argtypes = [_f32p, _f32p, _i64p, _i64p, _i64, _i64, _i64, _i64,
                                          ctypes.c_float, _f32p, _i64p]
        lib.oracle_radius_flat.argtypes = [_f32p, _f32p, _i64p, _i64p, _i64, _i64, _i64,
                                           ctypes.c_float, ctypes.c_int, _i64p]
        lib.oracle_three_nn.argtypes = [_f32p, _f32p, _i64, _i64, _i64, _f32p, _i32p]
        lib.oracle_three_interpolate.argtypes = [_f32p, _i64p, _f32p, _i64, _i64, _i64, _i64, _f32p]
        lib.oracle_group_points.argtypes = [_f32p, _i64p, _i64, _i64, _i64, _i64, _f32p]
        lib.oracle_group_points_backward.argtypes = [_f32p, _i64p, _i64, _i64, _i64, _i64, _f32p]
        lib.oracle_group_points_rel.argtypes = [_f32p, _f32p, _f32p, _i64p, _i64, _i64, _i64, _i64,
                                                _i64, _f32p]
        lib.oracle_three_interpolate_backward.argtypes = [_f32p, _i64p, _f32p, _i64, _i64, _i64,
                                                          _i64, _f64p]
        lib.oracle_chamfer_nearest_f32.argtypes = [_f32p, _f32p, _i64p, _i64p, _i64, _i64, _i64,
                                                   _i64, ctypes.c_int, _f32p, _i64p]
        lib.oracle_chamfer_nearest_f64.argtypes = [_f64p, _f64p, _i64p, _i64p, _i64, _i64, _i64,
                                                   _i64, ctypes.c_int, _f64p, _i64p]
        _lib = lib
    return _lib


def _arr(x, dtype) -> np.ndarray:
    if hasattr(x, "detach"):  # torch tensor
        x = x.detach().cpu().numpy()
    return np.ascontiguousarray(np.asarray(x), dtype=dtype)


def _p(a: np.ndarray, ptype):
    return a.ctypes.data_as(ptype)


def f32(value: float) -> float:
    """Round a Python float to binary32."""
    return float(np.float32(value))


# ---------------------------------------------------------------- radius rules

def ball_radius_sq(radius: float) -> float:
    """fl32(fl32(r) * fl32(r)), _ball_query_mps.py:111-119 (inf on overflow)."""
    r32 = np.float32(radius)
    with np.errstate(over="ignore"):
        return float(np.float32(np.float64(r32) * np.float64(r32)))


def torch_cluster_radius_sq(radius: float) -> float:
    """fl32(r * r in double), _flat_search_mps.py:66-76 (inf on overflow)."""
    with np.errstate(over="ignore"):
        return float(np.float32(float(radius) * float(radius)))


# ------------------------------------------------------------------ functions

def fps(xyz, npoint: int, start_idx: int = 0, skip_near_origin: bool = False) -> np.ndarray:
    x = _arr(xyz, np.float32)
    B, N, _ = x.shape
    out = np.zeros((B, npoint), np.int64)
    if B and npoint:
        _load().oracle_fps(_p(x, _f32p), B, N, npoint, start_idx, int(skip_near_origin),
                           _p(out, _i64p))
    return out


def fps_flat(x, ptr, out_ptr, starts) -> np.ndarray:
    xa = _arr(x, np.float32)
    pa, oa, sa = _arr(ptr, np.int64), _arr(out_ptr, np.int64), _arr(starts, np.int64)
    out = np.zeros(int(oa[-1]), np.int64)
    if len(pa) > 1 and out.size:
        _load().oracle_fps_flat(_p(xa, _f32p), _p(pa, _i64p), _p(oa, _i64p), _p(sa, _i64p),
                                len(pa) - 1, _p(out, _i64p))
    return out


def knn3(query, ref, k: int) -> tuple[np.ndarray, np.ndarray]:
    q, r = _arr(query, np.float32), _arr(ref, np.float32)
    B, M, _ = q.shape
    N = r.shape[1]
    dist = np.zeros((B, M, k), np.float32)
    idx = np.zeros((B, M, k), np.int64)
    if B and M and k:
        _load().oracle_knn3(_p(q, _f32p), _p(r, _f32p), B, M, N, k, _p(dist, _f32p),
                            _p(idx, _i64p))
    return dist, idx


def knn_feat(query, ref, k: int) -> tuple[np.ndarray, np.ndarray]:
    q, r = _arr(query, np.float32), _arr(ref, np.float32)
    B, M, D = q.shape
    N = r.shape[1]
    dist = np.zeros((B, M, k), np.float32)
    idx = np.zeros((B, M, k), np.int64)
    if B and M and k:
        _load().oracle_knn_feat(_p(q, _f32p), _p(r, _f32p), B, M, N, D, k, _p(dist, _f32p),
                                _p(idx, _i64p))
    return dist, idx


def knn(query, ref, k: int) -> tuple[np.ndarray, np.ndarray]:
    """ops.knn semantics: the 3-D kernel for D == 3, else the feature kernel."""
    D = _arr(query, np.float32).shape[-1]
    return knn3(query, ref, k) if D == 3 else knn_feat(query, ref, k)


def knn_flat(x, y, ptr_x, ptr_y, k: int) -> np.ndarray:
    xa, ya = _arr(x, np.float32), _arr(y, np.float32)
    px, py = _arr(ptr_x, np.int64), _arr(ptr_y, np.int64)
    Q, D = ya.shape
    out = np.full((Q, k), -1, np.int64)
    if Q and k:
        _load().oracle_knn_flat(_p(ya, _f32p), _p(xa, _f32p), _p(py, _i64p), _p(px, _i64p),
                                Q, len(px) - 1, D, k, _p(out, _i64p))
    return out


def ball_query(query, ref, radius: float, k: int, query_lengths=None, point_lengths=None):
    """(dist2 (B,Q,K) f32, idx (B,Q,K) int64).  float16 inputs are widened
    exactly to float32 first, as the native f16 kernel does."""
    q, p = _arr(query, np.float32), _arr(ref, np.float32)
    B, Q, _ = q.shape
    P = p.shape[1]
    ql = _arr(query_lengths if query_lengths is not None else [Q] * B, np.int64)
    pl = _arr(point_lengths if point_lengths is not None else [P] * B, np.int64)
    dist = np.zeros((B, Q, k), np.float32)
    idx = np.full((B, Q, k), -1, np.int64)
    if B and Q and k:
        _load().oracle_ball_query(_p(q, _f32p), _p(p, _f32p), _p(ql, _i64p), _p(pl, _i64p),
                                  B, Q, P, k, ball_radius_sq(radius), _p(dist, _f32p),
                                  _p(idx, _i64p))
    return dist, idx


def radius_flat(x, y, ptr_x, ptr_y, r: float, k: int, ignore_same_index: bool = False):
    xa, ya = _arr(x, np.float32), _arr(y, np.float32)
    px, py = _arr(ptr_x, np.int64), _arr(ptr_y, np.int64)
    Q = ya.shape[0]
    out = np.full((Q, k), -1, np.int64)
    r2 = torch_cluster_radius_sq(r) if np.float32(r) != 0 else 0.0
    if Q and k:
        _load().oracle_radius_flat(_p(ya, _f32p), _p(xa, _f32p), _p(py, _i64p), _p(px, _i64p),
                                   Q, len(px) - 1, k, r2, int(ignore_same_index), _p(out, _i64p))
    return out


def three_nn(unknown, known) -> tuple[np.ndarray, np.ndarray]:
    u, kn = _arr(unknown, np.float32), _arr(known, np.float32)
    B, N, _ = u.shape
    M = kn.shape[1]
    dist = np.zeros((B, N, 3), np.float32)
    idx = np.zeros((B, N, 3), np.int32)
    if B and N:
        _load().oracle_three_nn(_p(u, _f32p), _p(kn, _f32p), B, N, M, _p(dist, _f32p),
                                _p(idx, _i32p))
    return dist, idx


def three_interpolate(features, indices, weights) -> np.ndarray:
    f = _arr(features, np.float32)
    ix, w = _arr(indices, np.int64), _arr(weights, np.float32)
    B, C, M = f.shape
    N = ix.shape[1]
    out = np.zeros((B, C, N), np.float32)
    if out.size:
        _load().oracle_three_interpolate(_p(f, _f32p), _p(ix, _i64p), _p(w, _f32p), B, C, M, N,
                                         _p(out, _f32p))
    return out


def three_interpolate_backward(grad_out, indices, weights, M: int) -> np.ndarray:
    g = _arr(grad_out, np.float32)
    ix, w = _arr(indices, np.int64), _arr(weights, np.float32)
    B, C, N = g.shape
    out = np.zeros((B, C, M), np.float64)
    if B and C and M:
        _load().oracle_three_interpolate_backward(_p(g, _f32p), _p(ix, _i64p), _p(w, _f32p),
                                                  B, C, M, N, _p(out, _f64p))
    return out


def group_points(features, idx) -> np.ndarray:
    """(B,C,N) features gathered at (B,P) indices -> (B,C,P)."""
    f, ix = _arr(features, np.float32), _arr(idx, np.int64)
    B, C, N = f.shape
    P = ix.shape[1]
    out = np.zeros((B, C, P), np.float32)
    if out.size:
        _load().oracle_group_points(_p(f, _f32p), _p(ix, _i64p), B, C, N, P, _p(out, _f32p))
    return out


def group_points_backward(grad_out, idx, N: int) -> np.ndarray:
    """Scatter-add of (B,C,P) gradients into (B,C,N), float32, p ascending."""
    g, ix = _arr(grad_out, np.float32), _arr(idx, np.int64)
    B, C, P = g.shape
    out = np.zeros((B, C, N), np.float32)
    if out.size:
        _load().oracle_group_points_backward(_p(g, _f32p), _p(ix, _i64p), B, C, N, P,
                                             _p(out, _f32p))
    return out


def group_points_rel(xyz, centres, features, idx) -> np.ndarray:
    """(B,N,3), (B,M,3), (B,C,N) or None, (B,M,S) -> (B,3+C,M,S)."""
    x, c, ix = _arr(xyz, np.float32), _arr(centres, np.float32), _arr(idx, np.int64)
    B, N, _ = x.shape
    _, M, S = ix.shape
    f = np.zeros((B, 0, N), np.float32) if features is None else _arr(features, np.float32)
    C = f.shape[1]
    out = np.zeros((B, 3 + C, M, S), np.float32)
    if out.size:
        _load().oracle_group_points_rel(_p(x, _f32p), _p(c, _f32p), _p(f, _f32p), _p(ix, _i64p),
                                        B, C, N, M, S, _p(out, _f32p))
    return out


def chamfer_nearest(query, ref, query_lengths=None, ref_lengths=None, norm: int = 2):
    """(distance (B,Q), index (B,Q) int64) with the first-minimum rule."""
    is64 = str(getattr(query, "dtype", "")).endswith("float64")
    dt = np.float64 if is64 else np.float32
    q, r = _arr(query, dt), _arr(ref, dt)
    B, Q, D = q.shape
    R = r.shape[1]
    ql = _arr(query_lengths if query_lengths is not None else [Q] * B, np.int64)
    rl = _arr(ref_lengths if ref_lengths is not None else [R] * B, np.int64)
    dist = np.zeros((B, Q), dt)
    idx = np.full((B, Q), -1, np.int64)
    if B and Q:
        fn = _load().oracle_chamfer_nearest_f64 if is64 else _load().oracle_chamfer_nearest_f32
        pt = _f64p if is64 else _f32p
        fn(_p(q, pt), _p(r, pt), _p(ql, _i64p), _p(rl, _i64p), B, Q, R, D, norm,
           _p(dist, pt), _p(idx, _i64p))
    return dist, idx


def threads() -> int:
    """OpenMP threads the oracle uses (OMP_NUM_THREADS or all cores)."""
    return int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
