"""Pointcept v1.2.1 Point Transformer V1 ``pointops`` shim on the native
kernels (pointcept.py of the reference).

Flat point rows with inclusive cumulative offsets per batch (for example
``[4, 9]``).  Sampling and neighbour search run one ragged launch for all
batches (``pointops_fps_flat``, ``pointops_knn_flat``) instead of a loop over
batches; the rest is tensor glue with the reference's padding contract: a
missing neighbour is index ``-1`` with distance ``1e5``, including
candidates whose squared distance is not strictly below ``1e10`` (the
upstream CUDA heap's ceiling), non-finite ones and empty reference batches.
Neighbour selection carries no coordinate gradient; grouping propagates
feature and relative-coordinate gradients; interpolation propagates feature
gradients with fixed distance weights.  Coordinates and features are float32
ROCm (``device='cuda'``) tensors.
"""

from __future__ import annotations

import torch
from torch import Tensor

from . import _native, flat

_PAD_SQUARED_DISTANCE = 1e10  # strict ceiling of the upstream CUDA heap
_PAD_DISTANCE = 100_000.0     # sqrt(1e10), the upstream unfilled distance
_MAX_NSAMPLE = 256            # the native kNN's K limit (ops.py:30)


def _points(value, name: str) -> None:
    if not isinstance(value, Tensor) or value.ndim != 2 or value.shape[1] != 3:
        raise ValueError(f"{name} must be a tensor of shape (N, 3)")
    if value.dtype != torch.float32:
        raise ValueError(f"{name} must be float32")


def _bounds(offset, rows: int | None, device: torch.device, name: str) -> list[int]:
    """Pointcept's inclusive per-batch ends (e.g. ``[4, 9]``) as the row
    bounds ``[0, 4, 9]``, read to the host once; ``rows`` (when given) must
    be the last end (pointcept.py:47-58)."""
    if (not isinstance(offset, Tensor) or offset.ndim != 1
            or offset.dtype not in (torch.int32, torch.int64)):
        raise ValueError(f"{name} must be a one-dimensional int32/int64 tensor")
    if offset.device != device:
        raise ValueError(f"{name} must be on {device}")
    bounds = [0, *offset.tolist()]
    if rows is not None and bounds[-1] != rows:
        raise ValueError(f"{name} must end at its point count ({rows})")
    if any(hi < lo for lo, hi in zip(bounds, bounds[1:])):
        raise ValueError(f"{name} must be nondecreasing and nonnegative")
    return bounds


def _pairs(xyz, offset, new_xyz, new_offset) -> tuple[Tensor, list[int], list[int]]:
    """Reference and query rows with their bounds; without new_xyz /
    new_offset the points query themselves (pointcept.py:61-77)."""
    _points(xyz, "xyz")
    if (new_xyz is None) != (new_offset is None):
        raise ValueError("new_xyz and new_offset must be provided together")
    if new_xyz is None:
        new_xyz, new_offset = xyz, offset
    _points(new_xyz, "new_xyz")
    if xyz.device != new_xyz.device:
        raise ValueError("xyz and new_xyz must be on the same device")
    ref_bounds = _bounds(offset, len(xyz), xyz.device, "offset")
    query_bounds = _bounds(new_offset, len(new_xyz), xyz.device, "new_offset")
    if len(ref_bounds) != len(query_bounds):
        raise ValueError("offset and new_offset must have the same batch count")
    return new_xyz, ref_bounds, query_bounds


def _gather_rows(table: Tensor, idx: Tensor) -> Tensor:
    """(M, K, C) rows of an (N, C) table at (M, K) indices, zeros where the
    index is -1 (their gradient is masked out as well)."""
    rows = table.index_select(0, idx.reshape(-1).long().clamp_min(0))
    rows = rows.view(*idx.shape, table.shape[1])
    return rows.where((idx >= 0)[..., None], 0.0)


def farthest_point_sampling(xyz: Tensor, offset: Tensor, new_offset: Tensor) -> Tensor:
    """Global int32 FPS indices, starting at each batch's first point
    (pointcept.py:80-104): one ragged launch for every batch."""
    _points(xyz, "xyz")
    source = _bounds(offset, len(xyz), xyz.device, "offset")
    target = _bounds(new_offset, None, xyz.device, "new_offset")
    if len(source) != len(target):
        raise ValueError("offset and new_offset must have the same batch count")
    lengths = [hi - lo for lo, hi in zip(source, source[1:])]
    for n, lo, hi in zip(lengths, target, target[1:]):
        if hi - lo > n:
            raise ValueError("a batch requests more FPS samples than input points")
    if target[-1] == 0:
        return torch.empty(0, dtype=torch.int32, device=xyz.device)
    _native.require_device(xyz.device)
    x = xyz.detach().contiguous()
    ptr = torch.tensor(source, dtype=torch.long, device=x.device)
    out_ptr = torch.tensor(target, dtype=torch.long, device=x.device)
    starts = torch.zeros(len(lengths), dtype=torch.long, device=x.device)
    out = torch.empty(target[-1], dtype=torch.long, device=x.device)
    max_len = max(lengths)
    size = _native.size_query("pointops_fps_flat_scratch_bytes", len(x), max_len)
    scratch = torch.empty(size, dtype=torch.uint8, device=x.device) if size else None
    _native.call("pointops_fps_flat", x.data_ptr(), ptr.data_ptr(), out_ptr.data_ptr(),
                 starts.data_ptr(), out.data_ptr(), _native.ptr(scratch), len(lengths), len(x),
                 max_len, _native.stream(x.device))
    return out.to(torch.int32)


def knn_query(nsample: int, xyz: Tensor, offset: Tensor, new_xyz: Tensor | None = None,
              new_offset: Tensor | None = None) -> tuple[Tensor, Tensor]:
    """Global int32 neighbours and float32 Euclidean distances, (M, nsample)
    (pointcept.py:107-172); ties to the smaller global index."""
    if isinstance(nsample, bool) or not isinstance(nsample, int) or nsample < 0:
        raise ValueError("nsample must be a nonnegative integer")
    new_xyz, source, target = _pairs(xyz, offset, new_xyz, new_offset)
    if nsample > _MAX_NSAMPLE:
        raise ValueError(f"ROCm kNN supports at most {_MAX_NSAMPLE} neighbors")
    M = len(new_xyz)
    if M == 0 or nsample == 0:
        return (torch.empty((M, nsample), dtype=torch.int32, device=xyz.device),
                torch.empty((M, nsample), dtype=torch.float32, device=xyz.device))
    _native.require_device(xyz.device)
    with torch.no_grad():
        x, y = xyz.detach().contiguous(), new_xyz.detach().contiguous()
        if len(x) == 0:
            return (torch.full((M, nsample), -1, dtype=torch.int32, device=x.device),
                    torch.full((M, nsample), _PAD_DISTANCE, dtype=torch.float32, device=x.device))
        ptr_x = torch.tensor(source, dtype=torch.long, device=x.device)
        ptr_y = torch.tensor(target, dtype=torch.long, device=x.device)
        idx = flat.knn_indices(x, y, ptr_x, ptr_y, nsample)
        # The ceiling is applied to the squared distance recomputed from the
        # selected coordinates, in the kernels' order ((dx^2 + dy^2) + dz^2).
        valid = idx >= 0
        delta = y[:, None, :] - x[torch.where(valid, idx, 0)]
        squared = delta[..., 0] * delta[..., 0]
        squared = squared + delta[..., 1] * delta[..., 1]
        squared = squared + delta[..., 2] * delta[..., 2]
        valid = valid & (squared < _PAD_SQUARED_DISTANCE)
        dist = torch.where(valid, torch.sqrt(squared), _PAD_DISTANCE)
        return torch.where(valid, idx, -1).to(torch.int32), dist


def grouping(idx: Tensor, feat: Tensor, xyz: Tensor, new_xyz: Tensor | None = None,
             with_xyz: bool = False) -> Tensor:
    """(N, C) features gathered to (M, K, C), zeros for -1; with ``with_xyz``
    the neighbours' positions relative to their query come first, (M, K,
    3+C) (pointcept.py:175-210).  Gradients reach ``feat`` and, through the
    relative positions, ``xyz`` and ``new_xyz``; padded slots carry none."""
    _points(xyz, "xyz")
    _check_features(feat, xyz)
    if not isinstance(idx, Tensor) or idx.ndim != 2 or idx.dtype not in (torch.int32, torch.int64):
        raise ValueError("idx must be a two-dimensional int32/int64 tensor")
    if idx.device != xyz.device:
        raise ValueError("idx must be on the xyz device")
    if bool(((idx < -1) | (idx >= len(xyz))).any().item()):
        raise ValueError("idx contains an out-of-range point index")
    grouped = _gather_rows(feat, idx)
    if not with_xyz:
        return grouped
    centres = xyz if new_xyz is None else new_xyz
    _points(centres, "new_xyz")
    if centres.device != xyz.device or len(centres) != len(idx):
        raise ValueError("new_xyz must have one row per idx row on the xyz device")
    relative = (_gather_rows(xyz, idx) - centres[:, None, :]).where((idx >= 0)[..., None], 0.0)
    return torch.cat((relative, grouped), dim=-1)


def knn_query_and_group(feat: Tensor, xyz: Tensor, offset: Tensor | None = None,
                        new_xyz: Tensor | None = None, new_offset: Tensor | None = None,
                        idx: Tensor | None = None, nsample: int | None = None,
                        with_xyz: bool = False) -> tuple[Tensor, Tensor]:
    """kNN when ``idx`` is absent, then grouping (pointcept.py:213-225)."""
    if idx is None:
        if offset is None or nsample is None:
            raise ValueError("offset and nsample are required when idx is absent")
        idx, _ = knn_query(nsample, xyz, offset, new_xyz, new_offset)
    return grouping(idx, feat, xyz, new_xyz, with_xyz), idx


def interpolation(xyz: Tensor, new_xyz: Tensor, feat: Tensor, offset: Tensor,
                  new_offset: Tensor, k: int = 3) -> Tensor:
    """Inverse-distance interpolation of (N, C) features to the new points
    over their ``k`` nearest (pointcept.py:228-253): weights 1 / (d + 1e-8)
    normalised per query (the sum floored at 1e-20), 0 for -1 neighbours,
    so a query of an empty reference batch gets 0; the weights are
    constants for autograd."""
    _check_features(feat, xyz)
    idx, dist = knn_query(k, xyz, offset, new_xyz, new_offset)
    inverse = (1.0 / (dist + 1e-8)).where(idx >= 0, 0.0)
    weight = inverse / inverse.sum(dim=1, keepdim=True).clamp_min(1e-20)
    return (_gather_rows(feat, idx) * weight[..., None]).sum(dim=1)


def _check_features(feat, xyz: Tensor) -> None:
    if not isinstance(feat, Tensor) or feat.ndim != 2 or len(feat) != len(xyz):
        raise ValueError("feat must have shape (N, C) matching xyz")
    if feat.dtype != torch.float32 or feat.device != xyz.device:
        raise ValueError("feat must be float32 on the xyz device")


__all__ = ["farthest_point_sampling", "knn_query", "grouping", "knn_query_and_group",
           "interpolation"]
