"""Dense FPS, kNN and ball query on ROCm (signatures of
/root/reference/mps_pointops/ops.py).

Tensors must live on a ROCm device (``device='cuda'``); every call enqueues a
hand-written gfx950 kernel through libpointops_hip.so on the current stream.
Validation order, error types and messages follow the reference.
"""

from __future__ import annotations

import ctypes
from typing import Literal

import torch
from torch import Tensor

from . import _native
from ._ball_query import _checked_radius_and_k, ball_query as _native_ball_query

# Largest cloud the large-cloud FPS path takes, the reference's index range
# (ops.py:108-109): fewer than 2**32 points (clouds above 2**21 points use the
# streaming persistent kernel).
_FPS_LARGE_MAX_N = (1 << 32) - 1
# One cloud with at least this many points uses the all-CU persistent kernel
# under strategy="auto"; smaller clouds fit one workgroup's registers and LDS.
_FPS_MULTIGROUP_MIN_N = 65_536
# Same limit as the reference kernel (ops.py:30).
_KNN_MAX_K = 256
# 3-D kNN with at most this many neighbours, at least this many references
# per cloud and at least this many query-reference pairs in all uses the grid
# search (same results as brute force); below them the brute-force kernel is
# faster than building the grid.
_KNN_GRID_MAX_K = 32
_KNN_GRID_MIN_N = 32_768
_KNN_GRID_MIN_PAIRS = 1 << 26
# 3-D kNN with at most 32 neighbours over clouds of 2048 to 8192 references
# (and at most 16384 queries per cloud) first sorts each cloud by Morton cell
# and starts every query from a limit set by its neighbours in that order
# (pointops_knn3_windowed): same results, about 15% faster at config 2's
# shape; below 2048 references the extra launch does not pay.
_KNN_WINDOW_MAX_K = 32
_KNN_WINDOW_MIN_N = 2048
_KNN_WINDOW_MAX_N = 8192
_KNN_WINDOW_MAX_M = 16384


def _check_large_status(workspace: Tensor) -> None:
    """Raise if the persistent kernel gave up waiting for a workgroup's record
    (its first 4 workspace bytes are then non-zero and the unwritten output
    slots hold -1).  Reading the word synchronises with the stream once per
    large-cloud call; the reference's host loop has no such sync, but a
    partial result must not pass silently.  Skipped during graph capture,
    where the -1 slots remain the signal."""
    if torch.cuda.is_current_stream_capturing():
        return
    if int(workspace[:4].view(torch.int32).item()) != 0:
        raise RuntimeError(
            "furthest_point_sample: the large-cloud kernel stopped waiting for a workgroup "
            "(its cooperative launch did not run all workgroups together); the output is "
            "incomplete"
        )


def furthest_point_sample(
    xyz: Tensor,
    npoint: int,
    start_idx: int = 0,
    skip_near_origin: bool = False,
    *,
    strategy: Literal["auto", "single", "multigroup"] = "auto",
) -> Tensor:
    """Farthest point sampling (ops.py:53-141).

    Sampling starts at ``start_idx``; ties go to the smaller index; once every
    point has been sampled, the remaining slots repeat index 0.  With
    ``skip_near_origin`` points with x^2 + y^2 + z^2 <= 1e-3 are never picked
    (only the start index can be one).

    ``strategy``: ``single`` runs one workgroup per cloud; ``multigroup`` runs
    one persistent launch over every CU for a single cloud (B must be 1);
    ``auto`` picks ``multigroup`` for one cloud of at least 65,536 points.

    Returns:
        (B, npoint) int64 indices into ``xyz``.
    """
    if xyz.dim() != 3 or xyz.shape[-1] != 3:
        raise ValueError(f"xyz must have shape (B, N, 3), got {tuple(xyz.shape)}")
    if strategy not in ("auto", "single", "multigroup"):
        raise ValueError(f"strategy must be auto, single, or multigroup, got {strategy!r}")
    B, N, _ = xyz.shape
    if npoint < 0:
        raise ValueError(f"npoint must be >= 0, got {npoint}")
    if npoint > 0 and N == 0:
        raise ValueError("cannot sample from an empty point cloud")
    if npoint > 0 and not 0 <= start_idx < N:
        raise IndexError(f"start_idx {start_idx} is out of range for {N} points")
    _native.require_device(xyz.device)
    if xyz.dtype != torch.float32:
        raise TypeError(f"xyz must be float32 on ROCm, got {xyz.dtype}")
    if strategy == "multigroup" and B > 1 and npoint > 1:
        raise ValueError("multigroup FPS requires batch size 1; use auto or single for batches")
    use_large = B == 1 and npoint > 1 and (
        strategy == "multigroup" or (strategy == "auto" and N >= _FPS_MULTIGROUP_MIN_N)
    )
    if use_large and N > _FPS_LARGE_MAX_N:
        raise ValueError("multigroup FPS requires fewer than 2**32 points")
    out = torch.empty((B, npoint), dtype=torch.long, device=xyz.device)
    if B == 0 or npoint == 0:
        return out
    xyz = xyz.contiguous()
    stream = _native.stream(xyz.device)
    if use_large:
        size = _native.size_query("pointops_fps_large_workspace_bytes", N, npoint)
        workspace = torch.zeros(size, dtype=torch.uint8, device=xyz.device)
        _native.call("pointops_fps_large", xyz.data_ptr(), out.data_ptr(), workspace.data_ptr(),
                     N, npoint, start_idx, int(skip_near_origin), stream)
        _check_large_status(workspace)
        return out
    size = _native.size_query("pointops_fps_dense_scratch_bytes", B, N)
    scratch = torch.empty(size, dtype=torch.uint8, device=xyz.device) if size else None
    _native.call("pointops_fps_dense", xyz.data_ptr(), out.data_ptr(), _native.ptr(scratch),
                 B, N, npoint, start_idx, int(skip_near_origin), stream)
    return out


def knn(query: Tensor, ref: Tensor, k: int) -> tuple[Tensor, Tensor]:
    """Exact brute-force k nearest neighbours (ops.py:144-205).

    Neighbours are sorted by float32 squared distance, then by index.  D = 3
    uses the coordinate kernel; other D accumulate dimensions in order.
    ``k`` can be at most 256.  Selection has no coordinate gradients.

    Returns:
        dist: (B, M, k) Euclidean distances, ascending.
        idx: (B, M, k) int64 indices into ``ref``.
    """
    if query.dim() != 3 or query.shape[-1] < 1:
        raise ValueError(f"query must have shape (B, M, D) with D >= 1, got {tuple(query.shape)}")
    if ref.dim() != 3 or ref.shape[-1] != query.shape[-1]:
        raise ValueError(f"ref must have shape (B, N, {query.shape[-1]}), got {tuple(ref.shape)}")
    if query.device != ref.device:
        raise ValueError(f"query and ref are on different devices: {query.device} and {ref.device}")
    if query.shape[0] != ref.shape[0]:
        raise ValueError(f"batch sizes differ: {query.shape[0]} and {ref.shape[0]}")
    B, M, D = query.shape
    N = ref.shape[1]
    if not 0 <= k <= N:
        raise ValueError(f"k must be in [0, {N}], got {k}")
    _native.require_device(query.device)
    if query.dtype != torch.float32 or ref.dtype != torch.float32:
        raise TypeError(f"query and ref must be float32 on ROCm, got {query.dtype} and {ref.dtype}")
    if k > _KNN_MAX_K:
        raise ValueError(f"k must be at most {_KNN_MAX_K} on ROCm, got {k}")
    if M >= 2**31 or N >= 2**31 - 64 or D >= 2**31:
        raise ValueError("M, N, and D must each be below 2**31 for the native kNN kernel")
    dist = torch.empty(B, M, k, dtype=torch.float32, device=query.device)
    idx = torch.empty(B, M, k, dtype=torch.long, device=query.device)
    if B == 0 or M == 0 or k == 0:
        return dist, idx
    query, ref = query.contiguous(), ref.contiguous()
    stream = _native.stream(query.device)
    if (D == 3 and k <= _KNN_GRID_MAX_K and N >= _KNN_GRID_MIN_N and B <= 65_535
            and B * M * N >= _KNN_GRID_MIN_PAIRS):
        size = _native.size_query("pointops_knn3_grid_workspace_bytes", B, M, N)
        workspace = torch.empty(size, dtype=torch.uint8, device=query.device)
        _native.call("pointops_knn3_grid", query.data_ptr(), ref.data_ptr(), dist.data_ptr(),
                     idx.data_ptr(), workspace.data_ptr(), B, M, N, k, stream)
    elif (D == 3 and k <= _KNN_WINDOW_MAX_K and _KNN_WINDOW_MIN_N <= N <= _KNN_WINDOW_MAX_N
          and M <= _KNN_WINDOW_MAX_M):
        size = _native.size_query("pointops_knn3_windowed_workspace_bytes", B, M, N)
        workspace = torch.empty(size, dtype=torch.uint8, device=query.device)
        _native.call("pointops_knn3_windowed", query.data_ptr(), ref.data_ptr(), dist.data_ptr(),
                     idx.data_ptr(), workspace.data_ptr(), B, M, N, k, stream)
    elif D == 3:
        _native.call("pointops_knn3", query.data_ptr(), ref.data_ptr(), dist.data_ptr(),
                     idx.data_ptr(), B, M, N, k, stream)
    else:
        _native.call("pointops_knn_feat", query.data_ptr(), ref.data_ptr(), dist.data_ptr(),
                     idx.data_ptr(), B, M, N, D, k, stream)
    return dist, idx


def ball_query(query: Tensor, ref: Tensor, radius: float, K: int) -> tuple[Tensor, Tensor]:
    """First-K radius search with squared distances and -1 padded indices
    (ops.py:208-227).  Shapes (B, M, 3), (B, N, 3) -> (B, M, K); float32 or
    float16 inputs; coordinate gradients flow through the squared distances.
    """
    _checked_radius_and_k(radius, K)
    if query.dim() != 3 or ref.dim() != 3 or query.shape[-1] != 3 or ref.shape[-1] != 3:
        raise ValueError("query and ref must have shapes (B, M, 3) and (B, N, 3)")
    if query.shape[0] != ref.shape[0]:
        raise ValueError("query and ref must have the same batch size")
    if query.device != ref.device:
        raise ValueError(f"query and ref are on different devices: {query.device} and {ref.device}")
    result = _native_ball_query(query, ref, radius=radius, k=K)
    return result.distances, result.indices


def ball_query_multi(query: Tensor, ref: Tensor, radii, nsamples) -> list[tuple[Tensor, Tensor]]:
    """Ball queries of several radii around the same queries in one scan:
    ``[ball_query(query, ref, r, k) for r, k in zip(radii, nsamples)]``, the
    same tensors bit for bit (ops.py:208-227 per radius), each pair's
    distance computed once for up to four radii.  float32 (B, M, 3) and
    (B, N, 3), at most 8 radii, B <= 65535; no autograd (the distances do
    not require grad)."""
    radii, nsamples = list(radii), list(nsamples)
    if len(radii) != len(nsamples) or len(radii) > 8:
        raise ValueError("radii and nsamples must have the same length, at most 8")
    if query.dim() != 3 or ref.dim() != 3 or query.shape[-1] != 3 or ref.shape[-1] != 3:
        raise ValueError("query and ref must have shapes (B, M, 3) and (B, N, 3)")
    if query.shape[0] != ref.shape[0]:
        raise ValueError("query and ref must have the same batch size")
    if query.device != ref.device:
        raise ValueError(f"query and ref are on different devices: {query.device} and {ref.device}")
    if query.dtype != torch.float32 or ref.dtype != torch.float32:
        raise TypeError("ball_query_multi takes float32 coordinates")
    radii_sq = [_checked_radius_and_k(r, k)[1] for r, k in zip(radii, nsamples)]
    B, M, _ = query.shape
    N = ref.shape[1]
    if B > 65_535:
        raise ValueError(f"ball_query_multi takes at most 65535 clouds, got {B}")
    _native.require_device(query.device)
    q, r = query.detach().contiguous(), ref.detach().contiguous()
    dev = q.device
    outs = [(torch.empty(B, M, k, dtype=torch.float32, device=dev),
             torch.empty(B, M, k, dtype=torch.long, device=dev)) for k in nsamples]
    n = len(radii)
    c_radii = (ctypes.c_float * max(n, 1))(*radii_sq)
    c_ks = (ctypes.c_int64 * max(n, 1))(*nsamples)
    c_idx = (ctypes.c_void_p * max(n, 1))(*[i.data_ptr() for _, i in outs])
    c_d2 = (ctypes.c_void_p * max(n, 1))(*[d.data_ptr() for d, _ in outs])
    with torch.cuda.device(dev):
        _native.call("pointops_ball_query_multi_f32", q.data_ptr(), r.data_ptr(), n, c_radii,
                     c_ks, c_idx, c_d2, B, M, N, _native.stream(dev))
    return outs


# Streams beside the caller's stream for fps_ball_knn, one per (device,
# caller stream), default priority: calls issued from different streams keep
# independent query queues.
_SIDE_STREAMS: dict[tuple[int, int], torch.cuda.Stream] = {}
_PIPELINE_MAX_N = 8192


def fps_ball_knn(
    xyz: Tensor,
    npoint: int,
    radii: tuple[float, ...] | list[float],
    nsamples: tuple[int, ...] | list[int],
    knn_k: int,
    start_idx: int = 0,
    skip_near_origin: bool = False,
    *,
    chunk: int = 128,
    check: bool = False,
) -> tuple[Tensor, Tensor, list[tuple[Tensor, Tensor]], tuple[Tensor, Tensor]]:
    """A multi-scale set-abstraction front end in one call: samples =
    ``furthest_point_sample(xyz, npoint, start_idx, skip_near_origin)``,
    centres = ``xyz.gather(1, samples)``, then ``ball_query(centres, xyz, r,
    k)`` for each ``(r, k)`` of ``zip(radii, nsamples)`` and ``knn(centres,
    xyz, knn_k)`` -- the same tensors, bit for bit, as those calls
    (ops.py:53-227 of the reference run them one after another).

    The ball queries of each ``chunk`` of centres start as soon as FPS has
    sampled it in every cloud, on the CUs FPS leaves free (FPS uses one per
    cloud), and kNN runs once after the last chunk, on a side stream that
    the library joins back to the current one before returning (128:
    0.475 ms per call at B=32, N=4096, npoint 1024, three radii and kNN16,
    against 0.557 ms for the separate calls; 96: 0.479, 192: 0.488, 256:
    0.484: a smaller last chunk leaves less after FPS).  Each call has
    its own workspace, so calls may overlap (queued back to back, or issued
    from several streams or host threads).

    A chunk whose wait for its samples gives up (a bounded poll, several
    seconds; ``POINTOPS_PIPELINE_SPIN_LIMIT`` sets the number of polls) and
    every later chunk of the call get NaN centres, so their ball-query rows
    are (0, -1) and their kNN rows (inf, 2**32 - 1); ``samples`` stay
    exact.  ``check=True`` reads the call's status word (one host
    synchronisation) and raises RuntimeError in that case.  float32
    (B, N, 3) clouds with ``1 <= npoint <= N <= 8192``, ``knn_k <= 32``, at
    most 8 radii.

    Returns ``(samples, centres, [(ball_dists, ball_idx) per radius],
    (knn_dists, knn_idx))``.
    """
    if xyz.dim() != 3 or xyz.shape[-1] != 3:
        raise ValueError(f"xyz must have shape (B, N, 3), got {tuple(xyz.shape)}")
    if len(radii) != len(nsamples) or len(radii) > 8:
        raise ValueError("radii and nsamples must have the same length, at most 8")
    B, N, _ = xyz.shape
    if not 1 <= npoint <= N or N > _PIPELINE_MAX_N:
        raise ValueError(f"need 1 <= npoint <= N <= {_PIPELINE_MAX_N}, got npoint={npoint}, N={N}")
    if not 0 <= start_idx < N:
        raise ValueError(f"start_idx must be in [0, {N}), got {start_idx}")
    if not 0 <= knn_k <= min(N, 32):
        raise ValueError(f"knn_k must be in [0, {min(N, 32)}], got {knn_k}")
    if not 1 <= B <= 65_535 or chunk < 1:
        raise ValueError("need 1 <= B <= 65535 and chunk >= 1")
    radii_sq = [_checked_radius_and_k(r, k)[1] for r, k in zip(radii, nsamples)]
    device = _native.require_device(xyz.device)
    if xyz.dtype != torch.float32:
        raise TypeError(f"xyz must be float32 on ROCm, got {xyz.dtype}")
    xyz = xyz.contiguous()
    dev = xyz.device
    samples = torch.empty(B, npoint, dtype=torch.long, device=dev)
    centres = torch.empty(B, npoint, 3, dtype=torch.float32, device=dev)
    balls = [(torch.empty(B, npoint, k, dtype=torch.float32, device=dev),
              torch.empty(B, npoint, k, dtype=torch.long, device=dev)) for k in nsamples]
    knn_out = (torch.empty(B, npoint, knn_k, dtype=torch.float32, device=dev),
               torch.empty(B, npoint, knn_k, dtype=torch.long, device=dev))
    size = _native.size_query("pointops_fps_query_pipeline_workspace_bytes", B, N, npoint, chunk)
    # The call's progress words, kNN workspace and (last 4 bytes) status
    # word; the library clears what must start at zero on the current stream.
    workspace = torch.empty(size + 4, dtype=torch.uint8, device=dev)
    status = workspace[-4:]
    current = torch.cuda.current_stream(dev)
    side = _SIDE_STREAMS.get((device, current.cuda_stream))
    if side is None:
        side = torch.cuda.Stream(dev)
        if side.cuda_stream == current.cuda_stream:  # the pool handed back the caller's stream
            side = torch.cuda.Stream(dev)
        _SIDE_STREAMS[(device, current.cuda_stream)] = side
    n = len(radii)
    c_radii = (ctypes.c_float * max(n, 1))(*radii_sq)
    c_ks = (ctypes.c_int64 * max(n, 1))(*nsamples)
    c_idx = (ctypes.c_void_p * max(n, 1))(*[i.data_ptr() for _, i in balls])
    c_d2 = (ctypes.c_void_p * max(n, 1))(*[d.data_ptr() for d, _ in balls])
    with torch.cuda.device(dev):
        _native.call("pointops_fps_query_pipeline_f32", xyz.data_ptr(), samples.data_ptr(),
                     centres.data_ptr(), n, c_radii, c_ks, c_idx, c_d2, knn_k,
                     knn_out[0].data_ptr(), knn_out[1].data_ptr(), workspace.data_ptr(),
                     status.data_ptr(), B, N, npoint, start_idx, int(skip_near_origin), chunk,
                     current.cuda_stream, side.cuda_stream)
    # The library has joined the side stream back to `current`, so every
    # tensor above (allocated on `current`) is safe to free or reuse there.
    if check and int(status.view(torch.int32).item()) != 0:
        raise RuntimeError("fps_ball_knn: a chunk's wait for its samples gave up")
    return samples, centres, balls, knn_out
