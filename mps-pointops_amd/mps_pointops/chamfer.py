"""Bidirectional L1 or squared-L2 Chamfer loss on ROCm.

The signature, PyTorch3D reduction conventions, exception types and
messages are those of /root/reference/mps_pointops/chamfer.py:342-488; the
code is this package's own.  Each direction is one native nearest search
(``pointops_chamfer_nearest_*``, or the grid search for large squared-L2
clouds) whose indices also serve the normal loss, and one native
selected-pair backward (``pointops_chamfer_backward_*``).  Weights, point
and batch reductions and the normal term are PyTorch ops on the device.
Coordinates may have any positive dimension (float32 or float64); the
normal loss is 3-D.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Literal

import torch
import torch.nn.functional as F
from torch import Tensor
from torch.autograd.function import once_differentiable

from . import _native

PointReduction = Literal["mean", "sum", "max"] | None
BatchReduction = Literal["mean", "sum"] | None


# ------------------------------------------------------------ nearest search

_GRID_MIN_REFS = 8192
_GRID_MIN_QUERIES = 4096
_GRID_MIN_PAIRS = 1 << 26


def _grid_eligible(query: Tensor, ref: Tensor, norm: int, full: bool) -> bool:
    """The grid search serves squared-L2 3-D float32 clouds without lengths
    that are large enough for its build to pay."""
    batch, query_count, dimension = query.shape
    ref_count = ref.shape[1]
    limit = (1 << 31) - 64  # the entry point's index range and launch size
    return (full and norm == 2 and dimension == 3 and query.dtype == torch.float32
            and ref_count >= _GRID_MIN_REFS and query_count >= _GRID_MIN_QUERIES
            and batch <= 65535 and batch * query_count * ref_count >= _GRID_MIN_PAIRS
            and query_count < limit and ref_count < limit
            and batch * ((query_count + 63) // 64) < limit)


def _nearest_grid(query: Tensor, ref: Tensor) -> tuple[Tensor, Tensor]:
    """pointops_nearest3_grid: the grid search, and a linear scan inside the
    same call for queries whose nearest reference is several cells away.
    Results equal the scan kernel's everywhere."""
    batch, query_count, _ = query.shape
    ref_count = ref.shape[1]
    query = query.contiguous()
    ref = ref.contiguous()
    distances = torch.empty((batch, query_count), device=query.device, dtype=query.dtype)
    indices = torch.empty((batch, query_count), device=query.device, dtype=torch.int64)
    size = _native.size_query("pointops_knn3_grid_workspace_bytes", batch, query_count, ref_count)
    workspace = torch.empty(size, dtype=torch.uint8, device=query.device)
    _native.call("pointops_nearest3_grid", query.data_ptr(), ref.data_ptr(), distances.data_ptr(),
                 indices.data_ptr(), workspace.data_ptr(), batch, query_count, ref_count,
                 _native.stream(query.device))
    return distances, indices


def _nearest_scan(query: Tensor, ref: Tensor, query_lengths: Tensor, ref_lengths: Tensor,
                  norm: int) -> tuple[Tensor, Tensor]:
    """pointops_chamfer_nearest_{f32,f64}: a linear scan per query."""
    batch, query_count, dimension = query.shape
    ref_count = ref.shape[1]
    if ref_count >= 2**31:
        raise ValueError("native Chamfer requires fewer than 2**31 reference points")
    distances = torch.empty((batch, query_count), device=query.device, dtype=query.dtype)
    indices = torch.empty((batch, query_count), device=query.device, dtype=torch.int64)
    if distances.numel():
        entry = ("pointops_chamfer_nearest_f64" if query.dtype == torch.float64
                 else "pointops_chamfer_nearest_f32")
        _native.call(entry, query.contiguous().data_ptr(), ref.contiguous().data_ptr(),
                     query_lengths.contiguous().data_ptr(), ref_lengths.contiguous().data_ptr(),
                     distances.data_ptr(), indices.data_ptr(), batch, query_count, ref_count,
                     dimension, norm, _native.stream(query.device))
    return distances, indices


@torch.no_grad()
def _nearest_device(query: Tensor, ref: Tensor, query_lengths: Tensor, ref_lengths: Tensor,
                    norm: int = 2, full: bool = False) -> tuple[Tensor, Tensor]:
    """Distance (squared L2 or L1) and first-minimum index per query row;
    rows beyond the query lengths, and rows of an empty reference cloud, are
    (0, -1) (chamfer.py:122-158).  ``full``: no lengths were given."""
    if _grid_eligible(query, ref, norm, full):
        return _nearest_grid(query, ref)
    return _nearest_scan(query, ref, query_lengths, ref_lengths, norm)


# The reference's name for the native nearest search (used by its tests).
_nearest_mps = _nearest_device


class _NativeNearest(torch.autograd.Function):
    """Forward: the native nearest search, returning (distance, index) with
    the index non-differentiable.  Backward: d distance / d query is
    2 (q - r) for squared L2 and sign(q - r) with -1 at 0 for L1
    (PyTorch3D's subgradient); the reference point gets the negative
    (chamfer.py:215-294)."""

    @staticmethod
    def forward(ctx, query, ref, query_lengths, ref_lengths, norm, full):
        distances, indices = _nearest_device(query, ref, query_lengths, ref_lengths, norm, full)
        ctx.save_for_backward(query, ref, indices)
        ctx.norm = norm
        ctx.mark_non_differentiable(indices)
        return distances, indices

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_distances, _grad_indices):
        query, ref, indices = ctx.saved_tensors
        none = (None,) * 4
        if grad_distances is None:
            return (None, None, *none)
        if indices.numel() == 0 or ref.shape[1] == 0:
            return (torch.zeros_like(query), torch.zeros_like(ref), *none)
        query = query.contiguous()
        ref = ref.contiguous()
        grad_query = torch.empty_like(query)
        grad_ref = torch.zeros_like(ref, memory_format=torch.contiguous_format)
        batch, query_count, dimension = query.shape
        entry = ("pointops_chamfer_backward_f64" if query.dtype == torch.float64
                 else "pointops_chamfer_backward_f32")
        _native.call(entry, query.data_ptr(), ref.data_ptr(), indices.data_ptr(),
                     grad_distances.contiguous().to(query.dtype).data_ptr(),
                     grad_query.data_ptr(), grad_ref.data_ptr(), batch, query_count, ref.shape[1],
                     dimension, ctx.norm, _native.stream(query.device))
        return (grad_query, grad_ref, *none)


# ------------------------------------------------------------------ inputs


@dataclass
class _Cloud:
    """One side of the loss: padded points, per-cloud lengths, optional
    normals."""

    points: Tensor
    lengths: Tensor
    normals: Tensor | None

    def valid(self) -> Tensor:
        """(B, P) mask of the rows below each cloud's length."""
        rows = torch.arange(self.points.shape[1], device=self.points.device)
        return rows[None, :] < self.lengths[:, None]


def _unpack(points, lengths, normals, name: str):
    """A tensor passes through; a PyTorch3D ``Pointclouds`` replaces the
    explicit lengths and normals (chamfer.py:32-48).  PyTorch3D is optional."""
    if isinstance(points, Tensor):
        return points, lengths, normals
    try:
        from pytorch3d.structures import Pointclouds
    except ImportError as exc:
        raise TypeError(
            f"{name} must be a tensor, or a PyTorch3D Pointclouds object "
            "(install PyTorch3D for Pointclouds inputs)"
        ) from exc
    if not isinstance(points, Pointclouds):
        raise TypeError(f"{name} must be a tensor or a PyTorch3D Pointclouds object")
    return points.points_padded(), points.num_points_per_cloud(), points.normals_padded()


def _lengths_for(points: Tensor, value: Tensor | None, name: str) -> Tensor:
    batch, capacity, _ = points.shape
    if value is None:
        return torch.full((batch,), capacity, dtype=torch.long, device=points.device)
    if value.shape != (batch,) or value.dtype != torch.long or value.device != points.device:
        raise ValueError(f"{name} must be an int64 tensor of shape ({batch},) on {points.device}")
    if bool(((value < 0) | (value > capacity)).any().item()):
        raise ValueError(f"{name} must lie in [0, {capacity}]")
    return value


def _check_coordinates(x: Tensor, y: Tensor) -> None:
    if x.ndim != 3 or y.ndim != 3 or x.shape[-1] < 1 or y.shape[-1] != x.shape[-1]:
        raise ValueError("x and y must have shapes (B, P, D) and (B, Q, D) with D >= 1")
    if x.shape[0] != y.shape[0]:
        raise ValueError("x and y must have the same batch size")
    if x.device != y.device or x.dtype != y.dtype:
        raise ValueError("x and y must have the same device and dtype")
    if x.dtype not in (torch.float32, torch.float64):
        raise TypeError("Chamfer inputs must be float32 or float64")
    _native.require_device(x.device)


def _check_finite(cloud: _Cloud, name: str) -> None:
    """Rows inside a cloud's length must be finite (one host read)."""
    bad = cloud.valid() & ~torch.isfinite(cloud.points).all(dim=-1)
    if bool(bad.any().item()):
        raise ValueError(f"valid {name} coordinates must be finite")


def _check_normals(points: Tensor, normals: Tensor | None, name: str) -> None:
    if normals is None:
        return
    if not isinstance(normals, Tensor) or normals.shape != points.shape:
        raise ValueError(f"{name} must have the same (B, P, 3) shape as its points")
    if normals.device != points.device or normals.dtype != points.dtype:
        raise ValueError(f"{name} must match its points' device and dtype")


def _check_weights(weights: Tensor, x: Tensor) -> None:
    if weights.shape != (x.shape[0],) or weights.device != x.device or weights.dtype != x.dtype:
        raise ValueError("weights must match the batch size, input device, and input dtype")
    if bool((~torch.isfinite(weights) | (weights < 0)).any().item()):
        raise ValueError("weights must be finite and nonnegative")


# ------------------------------------------------------------------- terms


def _normal_term(query: _Cloud, ref: _Cloud, index: Tensor, abs_cosine: bool) -> Tensor:
    """1 - |cos| (or 1 - cos) between each valid query normal and the normal
    of its nearest reference; 0 on padding rows, and the reference normal
    counts as zero for an empty reference cloud (PyTorch3D's knn_gather).
    Padding is cleared before the cosine so that arbitrary padded values
    cannot send NaN into the gradients (chamfer.py:60-76)."""
    valid = query.valid()
    keep = valid[..., None]
    picked = ref.normals.gather(1, index.clamp_min(0)[..., None].expand(-1, -1, 3))
    picked = picked.where(keep & (ref.lengths > 0)[:, None, None], 0.0)
    own = query.normals.where(keep, 0.0)
    cosine = F.cosine_similarity(own, picked, dim=2, eps=1e-6)
    term = 1 - (cosine.abs() if abs_cosine else cosine)
    return term.where(valid, 0.0)


def _point_reduce(values: Tensor, lengths: Tensor, mode: PointReduction) -> Tensor:
    """Per-cloud reduction of (B, P) terms: mean over each cloud's own
    length (at least 1), sum, max (0 for P = 0), or none."""
    if mode is None:
        return values
    if mode == "max":
        if values.shape[1] == 0:
            return values.new_zeros((values.shape[0],))
        return values.max(dim=1).values
    total = values.sum(dim=1)
    return total / lengths.clamp(min=1) if mode == "mean" else total


def _merge(first: Tensor, second: Tensor, mode: PointReduction):
    """The two directions combined: kept apart without a point reduction,
    the larger under "max", else added."""
    if mode is None:
        return first, second
    if mode == "max":
        return torch.maximum(first, second)
    return first + second


def _batch_reduce(value: Tensor, mode: BatchReduction, weights: Tensor | None) -> Tensor:
    """Sum over clouds, divided for "mean" by the batch size (at least 1) or,
    with weights, by their total (1 when it is 0)."""
    if mode is None:
        return value
    total = value.sum()
    if mode == "sum":
        return total
    if weights is None:
        return total / max(value.shape[0], 1)
    weight_total = weights.sum()
    return total / torch.where(weight_total > 0, weight_total, torch.ones_like(weight_total))


def _zero_weight_result(x: _Cloud, y: _Cloud, weights: Tensor, single_directional: bool,
                        point_reduction: PointReduction, batch_reduction: BatchReduction):
    """PyTorch3D's return when every weight is 0 (chamfer.py:397-424): each
    direction is a (B, B) block of zeros, weights[:, None] times the sum of
    the cloud's valid coordinates times 0, so gradients reach the inputs
    (as zeros); the normal result mirrors the loss (None under a
    bidirectional "max"), and a batch reduction is a plain sum."""
    def anchor(cloud: _Cloud) -> Tensor:
        kept = cloud.points.masked_fill(~cloud.valid()[..., None], 0.0)
        return torch.outer(weights, kept.sum(dim=(1, 2))) * 0

    if single_directional:
        loss = normals = anchor(x)
    else:
        loss = _merge(anchor(x), anchor(y), point_reduction)
        normals = None if point_reduction == "max" else loss
    if batch_reduction is not None:
        loss = loss.sum()
        normals = None if normals is None else normals.sum()
    return loss, normals


# -------------------------------------------------------------------- API


def chamfer_distance(
    x,
    y,
    x_lengths: Tensor | None = None,
    y_lengths: Tensor | None = None,
    x_normals: Tensor | None = None,
    y_normals: Tensor | None = None,
    weights: Tensor | None = None,
    batch_reduction: BatchReduction = "mean",
    point_reduction: PointReduction = "mean",
    norm: int = 2,
    single_directional: bool = False,
    abs_cosine: bool = True,
):
    """L1 or squared-L2 Chamfer loss with PyTorch3D conventions
    (chamfer.py:342-488).

    Coordinates are ``(B, P, D)`` with ``D >= 1`` (PyTorch3D ``Pointclouds``
    accepted).  Normals need ``D == 3`` and are returned when both clouds
    have them.  ``point_reduction=None`` returns the padded per-point
    distances (a pair, or one tensor when ``single_directional``) and
    requires ``batch_reduction=None``.  On a distance tie the lowest
    reference index is the neighbour.  Validation reads device scalars.
    Returns ``(loss, normal_loss)``.
    """
    if norm not in (1, 2):
        raise ValueError("Support for 1 or 2 norm.")
    if batch_reduction not in (None, "mean", "sum"):
        raise ValueError("batch_reduction must be None, 'mean', or 'sum'")
    if point_reduction not in (None, "mean", "sum", "max"):
        raise ValueError("point_reduction must be None, 'mean', 'sum', or 'max'")
    if point_reduction is None and batch_reduction is not None:
        raise ValueError("batch_reduction must be None when point_reduction is None")
    no_max_with_normals = 'Normals must be None if point_reduction is "max"'
    if point_reduction == "max" and (x_normals is not None or y_normals is not None):
        raise ValueError(no_max_with_normals)
    x_points, x_lengths, x_normals = _unpack(x, x_lengths, x_normals, "x")
    y_points, y_lengths, y_normals = _unpack(y, y_lengths, y_normals, "y")
    _check_coordinates(x_points, y_points)
    cx = _Cloud(x_points, _lengths_for(x_points, x_lengths, "x_lengths"), x_normals)
    cy = _Cloud(y_points, _lengths_for(y_points, y_lengths, "y_lengths"), y_normals)
    _check_finite(cx, "x")
    _check_finite(cy, "y")
    full = x_lengths is None and y_lengths is None  # every row of every cloud is valid
    if x_points.shape[-1] != 3 and (x_normals is not None or y_normals is not None):
        raise NotImplementedError("normal loss currently requires D == 3")
    _check_normals(x_points, x_normals, "x_normals")
    _check_normals(y_points, y_normals, "y_normals")
    if point_reduction == "max" and (x_normals is not None or y_normals is not None):
        raise ValueError(no_max_with_normals)
    with_normals = x_normals is not None and y_normals is not None
    if weights is not None:
        _check_weights(weights, x_points)
        if bool((weights == 0).all().item()):
            return _zero_weight_result(cx, cy, weights, single_directional, point_reduction,
                                       batch_reduction)

    directions = [(cx, cy)] if single_directional else [(cx, cy), (cy, cx)]
    losses, normal_losses = [], []
    for query, ref in directions:
        distance, index = _NativeNearest.apply(query.points, ref.points, query.lengths,
                                               ref.lengths, norm, full)
        normal = _normal_term(query, ref, index, abs_cosine) if with_normals else None
        if weights is not None:
            distance = distance * weights[:, None]
            normal = None if normal is None else normal * weights[:, None]
        losses.append(_point_reduce(distance, query.lengths, point_reduction))
        if normal is not None:
            normal_losses.append(_point_reduce(normal, query.lengths, point_reduction))

    if single_directional:
        loss = losses[0]
        normal_loss = normal_losses[0] if normal_losses else None
    else:
        loss = _merge(losses[0], losses[1], point_reduction)
        normal_loss = _merge(*normal_losses, point_reduction) if normal_losses else None
    if batch_reduction is not None:
        loss = _batch_reduce(loss, batch_reduction, weights)
        if normal_loss is not None:
            normal_loss = _batch_reduce(normal_loss, batch_reduction, weights)
    return loss, normal_loss
