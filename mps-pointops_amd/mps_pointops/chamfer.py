"""Bidirectional L1 or squared-L2 Chamfer loss on ROCm (signatures, reductions
and autograd contract of /root/reference/mps_pointops/chamfer.py).

The nearest-neighbour search (forward) and the selected-pair gradient
(backward) run in the native gfx950 kernels; reductions, weights and normal
losses are PyTorch ops on the same device.  Tensor coordinates may have any
positive dimension (float32 or float64); normal loss remains 3-D.
"""

from __future__ import annotations

from typing import Literal

import torch
import torch.nn.functional as F
from torch import Tensor
from torch.autograd.function import once_differentiable

from . import _native

PointReduction = Literal["mean", "sum", "max"] | None
BatchReduction = Literal["mean", "sum"] | None


def _unpack_cloud(points, lengths, normals, name: str):
    """PyTorch3D Pointclouds input precedence without a hard dependency
    (chamfer.py:32-48)."""
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


def _validate_normals(points: Tensor, normals: Tensor | None, name: str) -> None:
    if normals is None:
        return
    if not isinstance(normals, Tensor) or normals.shape != points.shape:
        raise ValueError(f"{name} must have the same (B, P, 3) shape as its points")
    if normals.device != points.device or normals.dtype != points.dtype:
        raise ValueError(f"{name} must match its points' device and dtype")


def _normal_loss(query_normals, ref_normals, index, query_lengths, ref_lengths, abs_cosine):
    """chamfer.py:60-76: knn_gather returns zero for an empty reference cloud."""
    valid = torch.arange(index.shape[1], device=index.device)[None] < query_lengths[:, None]
    safe_index = index.clamp_min(0)
    selected = ref_normals.gather(1, safe_index.unsqueeze(-1).expand(-1, -1, 3))
    selected = torch.where((ref_lengths > 0)[:, None, None], selected, torch.zeros_like(selected))
    query = torch.where(valid.unsqueeze(-1), query_normals, torch.zeros_like(query_normals))
    selected = torch.where(valid.unsqueeze(-1), selected, torch.zeros_like(selected))
    cosine = F.cosine_similarity(query, selected, dim=2, eps=1e-6)
    loss = 1 - (cosine.abs() if abs_cosine else cosine)
    return torch.where(valid, loss, torch.zeros_like(loss))


def _lengths(points: Tensor, value: Tensor | None, name: str) -> Tensor:
    batch, maximum, _ = points.shape
    if value is None:
        return torch.full((batch,), maximum, dtype=torch.long, device=points.device)
    if value.shape != (batch,) or value.dtype != torch.long or value.device != points.device:
        raise ValueError(f"{name} must be an int64 tensor of shape ({batch},) on {points.device}")
    if bool(((value < 0) | (value > maximum)).any().item()):
        raise ValueError(f"{name} must lie in [0, {maximum}]")
    return value


def _validate_clouds(x, y, x_lengths, y_lengths) -> tuple[Tensor, Tensor]:
    """chamfer.py:92-110 (two host syncs: lengths and finiteness)."""
    if x.ndim != 3 or y.ndim != 3 or x.shape[-1] < 1 or y.shape[-1] != x.shape[-1]:
        raise ValueError("x and y must have shapes (B, P, D) and (B, Q, D) with D >= 1")
    if x.shape[0] != y.shape[0]:
        raise ValueError("x and y must have the same batch size")
    if x.device != y.device or x.dtype != y.dtype:
        raise ValueError("x and y must have the same device and dtype")
    if x.dtype not in (torch.float32, torch.float64):
        raise TypeError("Chamfer inputs must be float32 or float64")
    _native.require_device(x.device)
    lx = _lengths(x, x_lengths, "x_lengths")
    ly = _lengths(y, y_lengths, "y_lengths")
    for points, lengths, name in ((x, lx, "x"), (y, ly, "y")):
        valid = torch.arange(points.shape[1], device=points.device)[None] < lengths[:, None]
        if bool((valid & ~torch.isfinite(points).all(dim=-1)).any().item()):
            raise ValueError(f"valid {name} coordinates must be finite")
    return lx, ly


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


@torch.no_grad()
def _nearest_device(query: Tensor, ref: Tensor, query_lengths: Tensor, ref_lengths: Tensor,
                    norm: int = 2, full: bool = False) -> tuple[Tensor, Tensor]:
    """Distance and first-minimum index from the native kernels (the
    counterpart of chamfer.py:122-158); ``full``: no lengths were given."""
    if _grid_eligible(query, ref, norm, full):
        return _nearest_grid(query, ref)
    return _nearest_scan(query, ref, query_lengths, ref_lengths, norm)


def _nearest_scan(query: Tensor, ref: Tensor, query_lengths: Tensor, ref_lengths: Tensor,
                  norm: int) -> tuple[Tensor, Tensor]:
    batch, query_count, dimension = query.shape
    ref_count = ref.shape[1]
    if ref_count >= 2**31:
        raise ValueError("native Chamfer requires fewer than 2**31 reference points")
    distances = torch.empty((batch, query_count), device=query.device, dtype=query.dtype)
    indices = torch.empty((batch, query_count), device=query.device, dtype=torch.int64)
    if distances.numel():
        name = ("pointops_chamfer_nearest_f64" if query.dtype == torch.float64
                else "pointops_chamfer_nearest_f32")
        _native.call(name, query.contiguous().data_ptr(), ref.contiguous().data_ptr(),
                     query_lengths.contiguous().data_ptr(), ref_lengths.contiguous().data_ptr(),
                     distances.data_ptr(), indices.data_ptr(), batch, query_count, ref_count,
                     dimension, norm, _native.stream(query.device))
    return distances, indices


# Name used by the reference's tests for the native nearest search.
_nearest_mps = _nearest_device


def _nearest_indices(query, ref, query_lengths, ref_lengths, norm: int = 2,
                     full: bool = False) -> Tensor:
    """First-minimum indices under the requested distance (chamfer.py:161-212)."""
    return _nearest_device(query, ref, query_lengths, ref_lengths, norm, full)[1]


class _NativeNearest(torch.autograd.Function):
    """Native forward and selected-pair backward for squared L2 (norm 2) or L1
    (norm 1): chamfer.py:215-294."""

    @staticmethod
    def forward(ctx, query, ref, query_lengths, ref_lengths, norm, full=False):
        distances, indices = _nearest_device(query, ref, query_lengths, ref_lengths, norm, full)
        ctx.save_for_backward(query, ref, indices)
        ctx.norm = norm
        return distances

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_distances):
        if grad_distances is None:
            return None, None, None, None, None, None
        query, ref, indices = ctx.saved_tensors
        if not indices.numel() or ref.shape[1] == 0:
            return torch.zeros_like(query), torch.zeros_like(ref), None, None, None, None
        query = query.contiguous()
        ref = ref.contiguous()
        grad_query = torch.empty_like(query)
        grad_ref = torch.zeros_like(ref, memory_format=torch.contiguous_format)
        batch, query_count, dimension = query.shape
        name = ("pointops_chamfer_backward_f64" if query.dtype == torch.float64
                else "pointops_chamfer_backward_f32")
        _native.call(name, query.data_ptr(), ref.data_ptr(), indices.data_ptr(),
                     grad_distances.contiguous().to(query.dtype).data_ptr(),
                     grad_query.data_ptr(), grad_ref.data_ptr(), batch, query_count, ref.shape[1],
                     dimension, ctx.norm, _native.stream(query.device))
        return grad_query, grad_ref, None, None, None, None


def _reduce_points(dist: Tensor, lengths: Tensor, mode: PointReduction) -> Tensor:
    if mode is None:
        return dist
    if mode == "max":
        return dist.max(dim=1).values if dist.shape[1] else dist.new_zeros((dist.shape[0],))
    result = dist.sum(dim=1)
    return result / lengths.clamp(min=1) if mode == "mean" else result


def _zero_weight_anchor(points: Tensor, lengths: Tensor, weights: Tensor) -> Tensor:
    """Graph-connected zeros with upstream's (B, B) broadcast shape."""
    valid = torch.arange(points.shape[1], device=points.device)[None] < lengths[:, None]
    selected = torch.where(valid.unsqueeze(-1), points, torch.zeros_like(points))
    per_cloud = selected.sum(dim=(1, 2))
    return (weights[:, None] * per_cloud[None, :]) * 0


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
    """L1 or squared-L2 Chamfer loss with PyTorch3D reduction conventions
    (chamfer.py:342-488).

    Coordinates have shape ``(B, P, D)`` with ``D >= 1``.  Normals are
    supported for ``D == 3`` only and returned when both clouds provide them.
    With ``point_reduction=None``, ``loss`` is a pair of padded per-point
    distance tensors (one if ``single_directional``) and batch reduction must
    also be None.  Nearest indices use the lowest reference index on a
    rounded-distance tie.  Input validation reads device scalars.
    """
    if norm not in (1, 2):
        raise ValueError("Support for 1 or 2 norm.")
    if batch_reduction not in (None, "mean", "sum"):
        raise ValueError("batch_reduction must be None, 'mean', or 'sum'")
    if point_reduction not in (None, "mean", "sum", "max"):
        raise ValueError("point_reduction must be None, 'mean', 'sum', or 'max'")
    if point_reduction is None and batch_reduction is not None:
        raise ValueError("batch_reduction must be None when point_reduction is None")
    if point_reduction == "max" and (x_normals is not None or y_normals is not None):
        raise ValueError('Normals must be None if point_reduction is "max"')
    x, x_lengths, x_normals = _unpack_cloud(x, x_lengths, x_normals, "x")
    y, y_lengths, y_normals = _unpack_cloud(y, y_lengths, y_normals, "y")
    lx, ly = _validate_clouds(x, y, x_lengths, y_lengths)
    full = x_lengths is None and y_lengths is None  # every point of every cloud is valid
    if x.shape[-1] != 3 and (x_normals is not None or y_normals is not None):
        raise NotImplementedError("normal loss currently requires D == 3")
    _validate_normals(x, x_normals, "x_normals")
    _validate_normals(y, y_normals, "y_normals")
    if point_reduction == "max" and (x_normals is not None or y_normals is not None):
        raise ValueError('Normals must be None if point_reduction is "max"')
    return_normals = x_normals is not None and y_normals is not None
    if weights is not None:
        if weights.shape != (x.shape[0],) or weights.device != x.device or weights.dtype != x.dtype:
            raise ValueError("weights must match the batch size, input device, and input dtype")
        if bool((~torch.isfinite(weights) | (weights < 0)).any().item()):
            raise ValueError("weights must be finite and nonnegative")
        # PyTorch3D's all-zero-weight branch (chamfer.py:397-424).
        if bool((weights == 0).all().item()):
            zero_x = _zero_weight_anchor(x, lx, weights)
            if single_directional:
                zero_loss = zero_x
                zero_normals = zero_x
            else:
                zero_y = _zero_weight_anchor(y, ly, weights)
                if point_reduction == "max":
                    zero_loss = torch.maximum(zero_x, zero_y)
                    zero_normals = None
                elif point_reduction is None:
                    zero_loss = (zero_x, zero_y)
                    zero_normals = (zero_x, zero_y)
                else:
                    zero_loss = zero_x + zero_y
                    zero_normals = zero_x + zero_y
            if batch_reduction is not None:
                zero_loss = zero_loss.sum()
                if zero_normals is not None:
                    zero_normals = zero_normals.sum()
            return zero_loss, zero_normals

    dx = _NativeNearest.apply(x, y, lx, ly, norm, full)
    nx = None
    if return_normals:
        ix = _nearest_indices(x, y, lx, ly, norm, full)
        nx = _normal_loss(x_normals, y_normals, ix, lx, ly, abs_cosine)
    if weights is not None:
        dx = dx * weights[:, None]
        if nx is not None:
            nx = nx * weights[:, None]
    rx = _reduce_points(dx, lx, point_reduction)
    rnx = _reduce_points(nx, lx, point_reduction) if nx is not None else None
    if single_directional:
        loss = rx
        normal_loss = rnx
    else:
        dy = _NativeNearest.apply(y, x, ly, lx, norm, full)
        ny = None
        if return_normals:
            iy = _nearest_indices(y, x, ly, lx, norm, full)
            ny = _normal_loss(y_normals, x_normals, iy, ly, lx, abs_cosine)
        if weights is not None:
            dy = dy * weights[:, None]
            if ny is not None:
                ny = ny * weights[:, None]
        ry = _reduce_points(dy, ly, point_reduction)
        rny = _reduce_points(ny, ly, point_reduction) if ny is not None else None
        loss = (rx, ry) if point_reduction is None else (
            torch.maximum(rx, ry) if point_reduction == "max" else rx + ry
        )
        normal_loss = (rnx, rny) if point_reduction is None and rnx is not None and rny is not None else (
            rnx + rny if rnx is not None and rny is not None else None
        )

    if batch_reduction is not None:
        loss = loss.sum()
        if normal_loss is not None:
            normal_loss = normal_loss.sum()
        if batch_reduction == "mean":
            if weights is None:
                denominator = max(x.shape[0], 1)
            else:
                total_weight = weights.sum()
                denominator = torch.where(total_weight > 0, total_weight,
                                          torch.ones_like(total_weight))
            loss = loss / denominator
            if normal_loss is not None:
                normal_loss = normal_loss / denominator
    return loss, normal_loss
