"""Dense first-K radius search on ROCm (the MI355X counterpart of the
reference's _ball_query_mps.py).

Radius/K rules, lengths handling, autograd and error behaviour follow
/root/reference/mps_pointops/_ball_query_mps.py:73-273.  The neighbour test is
reference.py's: fl32((dx^2 + dy^2) + dz^2) < fl32(fl32(r)^2), computed by the
hand-written gfx950 kernel pointops_ball_query_{f32,f16}.
"""

from __future__ import annotations

import math
import struct
from typing import NamedTuple

import torch

from . import _native

_MIN_SUPPORTED_RADIUS_F32 = 2.0**-112


class BallQueryResult(NamedTuple):
    """Squared distances and indices, both shaped ``(B, Q, K)``."""

    distances: torch.Tensor
    indices: torch.Tensor


def _lengths_or_full(
    lengths: torch.Tensor | None, *, batch: int, count: int, device: torch.device, name: str
) -> torch.Tensor | None:
    """_ball_query_mps.py:73-84 (one host sync when lengths are given).

    ``None`` stays ``None``: the kernel then treats every row as valid, which
    saves two fill launches per call."""
    if lengths is None:
        return None
    if not isinstance(lengths, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor or None")
    if lengths.shape != (batch,) or lengths.dtype != torch.int64 or lengths.device != device:
        raise ValueError(f"{name} must have shape ({batch},), int64 dtype and device {device}")
    if torch.any((lengths < 0) | (lengths > count)).item():
        raise ValueError(f"{name} values must lie in [0, {count}]")
    return lengths.contiguous()


def _checked_radius_and_k(radius: float, k: int) -> tuple[float, float]:
    """Validate ``radius`` and ``k`` (_ball_query_mps.py:87-119).

    Returns ``(radius_f32, radius_squared)``: the radius rounded to float32 and
    fl32(fl32(radius) * fl32(radius)) (inf when that overflows).
    """
    if not isinstance(k, int) or isinstance(k, bool) or k < 0 or k > (1 << 63) - 1:
        raise ValueError("k must be a non-negative integer")
    if not isinstance(radius, (int, float)) or isinstance(radius, bool):
        raise ValueError("radius must be a finite non-negative number")
    try:
        radius = float(radius)
    except OverflowError as exc:
        raise ValueError("radius must be a finite non-negative number") from exc
    if not math.isfinite(radius) or radius < 0:
        raise ValueError("radius must be a finite non-negative number")
    try:
        radius_f32 = struct.unpack("f", struct.pack("f", radius))[0]
    except OverflowError as exc:
        raise ValueError("radius must fit in float32") from exc
    if not math.isfinite(radius_f32) or (radius > 0 and radius_f32 < _MIN_SUPPORTED_RADIUS_F32):
        raise ValueError("positive radius must round to a normal float32 value at least 2**-112")
    # Two binary32 operands multiply exactly in binary64; packing rounds once.
    radius_squared = float(radius_f32) * float(radius_f32)
    try:
        radius_squared = struct.unpack("f", struct.pack("f", radius_squared))[0]
    except OverflowError:
        radius_squared = math.inf
    return radius_f32, radius_squared


# Without lengths, float32 clouds of at least this many points, at most this
# many neighbours and at least this many query-point pairs in all go to
# pointops_ball_query_auto_f32, which chooses on the device between the grid
# search and the index-order scan (the same results): the grid scans the
# cells around each query (about 6.4 lambda points for lambda points per
# ball), the index-order scan stops after about N K / lambda points, so the
# grid is taken while lambda < sqrt(N K / 6.4), lambda estimated from each
# cloud's bounding box.  No host synchronisation is involved.
_GRID_MIN_POINTS = 32_768
_GRID_MAX_K = 64
_GRID_MIN_PAIRS = 1 << 26


def _launch(queries, points, query_lengths, point_lengths, radius_sq, k):
    batch, query_count, _ = queries.shape
    point_count = points.shape[1]
    device = queries.device
    indices = torch.empty((batch, query_count, k), device=device, dtype=torch.int64)
    distances = torch.empty((batch, query_count, k), device=device, dtype=torch.float32)
    if (indices.numel() and query_lengths is None and point_lengths is None
            and queries.dtype == torch.float32 and k <= _GRID_MAX_K
            and point_count >= _GRID_MIN_POINTS and batch <= 65_535
            and batch * query_count * point_count >= _GRID_MIN_PAIRS):
        size = _native.size_query("pointops_ball_query_auto_workspace_bytes", batch,
                                  query_count, point_count)
        workspace = torch.empty(size, dtype=torch.uint8, device=device)
        _native.call("pointops_ball_query_auto_f32", queries.data_ptr(), points.data_ptr(),
                     indices.data_ptr(), distances.data_ptr(), workspace.data_ptr(), batch,
                     query_count, point_count, k, radius_sq, _native.stream(device))
        return distances, indices
    if indices.numel():
        name = ("pointops_ball_query_f32" if queries.dtype == torch.float32
                else "pointops_ball_query_f16")
        _native.call(
            name, queries.data_ptr(), points.data_ptr(), _native.ptr(query_lengths),
            _native.ptr(point_lengths), indices.data_ptr(), distances.data_ptr(),
            batch, query_count, point_count, k, radius_sq, _native.stream(device),
        )
    return distances, indices


class _BallQuery(torch.autograd.Function):
    """Native forward and backward (_ball_query_mps.py:122-203 defines the
    gradients).  The backward (pointops_ball_query_backward_*) sums each
    query's slot contributions 2 g (q - p) in slot order and each point's in
    row order with a fixed grouping, so its bits do not vary between runs."""

    @staticmethod
    def forward(ctx, queries, points, query_lengths, point_lengths, radius_sq, k):
        distances, indices = _launch(queries, points, query_lengths, point_lengths, radius_sq, k)
        ctx.save_for_backward(queries, points, indices)
        ctx.mark_non_differentiable(indices)
        return distances, indices

    @staticmethod
    def backward(ctx, grad_distances, grad_indices):
        want_q, want_p = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        if grad_distances is None or not (want_q or want_p):
            return None, None, None, None, None, None
        queries, points, indices = ctx.saved_tensors
        batch, query_count, k = indices.shape
        device = queries.device
        grad_q = (torch.empty((batch, query_count, 3), dtype=torch.float32, device=device)
                  if want_q else None)
        grad_p = (torch.empty(points.shape, dtype=torch.float32, device=device)
                  if want_p else None)
        size = _native.size_query("pointops_ball_query_backward_workspace_bytes", batch,
                                  query_count)
        workspace = torch.empty(size, dtype=torch.uint8, device=device) if size else None
        name = ("pointops_ball_query_backward_f32" if queries.dtype == torch.float32
                else "pointops_ball_query_backward_f16")
        _native.call(name, queries.data_ptr(), points.data_ptr(), indices.data_ptr(),
                     grad_distances.float().contiguous().data_ptr(), _native.ptr(grad_q),
                     _native.ptr(grad_p), _native.ptr(workspace), batch, query_count,
                     points.shape[1], k, _native.stream(device))
        if grad_q is not None:
            grad_q = grad_q.to(queries.dtype)
        if grad_p is not None:
            grad_p = grad_p.to(points.dtype)
        return grad_q, grad_p, None, None, None, None


def ball_query(
    queries: torch.Tensor,
    points: torch.Tensor,
    *,
    radius: float,
    k: int,
    query_lengths: torch.Tensor | None = None,
    point_lengths: torch.Tensor | None = None,
) -> BallQueryResult:
    """Find the first ``k`` points strictly inside each radius.

    ``queries`` and ``points`` are float32 or float16 ROCm tensors with shapes
    ``(B,Q,3)`` and ``(B,P,3)``.  The output is ordered by input point index,
    not distance.  Missing neighbours use index ``-1`` and squared distance
    ``0``.  Non-finite coordinates never match.  Gradients of valid squared
    distances propagate to both coordinate tensors; indices are
    non-differentiable.  Supplying lengths checks their bounds with one
    device-to-host synchronisation.  Signature and errors follow
    _ball_query_mps.py:206-273.
    """
    if not isinstance(queries, torch.Tensor) or not isinstance(points, torch.Tensor):
        raise TypeError("queries and points must be torch.Tensor values")
    if queries.ndim != 3 or points.ndim != 3 or queries.shape[-1] != 3 or points.shape[-1] != 3:
        raise ValueError("queries and points must have shapes (B, Q, 3) and (B, P, 3)")
    if queries.shape[0] != points.shape[0]:
        raise ValueError("queries and points must have the same batch size")
    if queries.device.type != "cuda" or points.device != queries.device:
        raise ValueError("queries and points must be on the same ROCm (cuda) device")
    if queries.dtype not in (torch.float32, torch.float16) or points.dtype != queries.dtype:
        raise TypeError("queries and points must have the same float32 or float16 dtype")
    _, radius_squared = _checked_radius_and_k(radius, k)

    batch, query_count, _ = queries.shape
    point_count = points.shape[1]
    if batch * query_count * k > (1 << 63) - 1:
        raise ValueError("output element count exceeds int64 indexing")
    if point_count > (1 << 31) - 128:
        raise ValueError("point count exceeds the native kernel's 32-bit index range")
    _native.require_device(queries.device)
    query_lengths = _lengths_or_full(
        query_lengths, batch=batch, count=query_count, device=queries.device, name="query_lengths"
    )
    point_lengths = _lengths_or_full(
        point_lengths, batch=batch, count=point_count, device=queries.device, name="point_lengths"
    )
    distances, indices = _BallQuery.apply(
        queries.contiguous(), points.contiguous(), query_lengths, point_lengths,
        radius_squared, k,
    )
    return BallQueryResult(distances=distances, indices=indices)
