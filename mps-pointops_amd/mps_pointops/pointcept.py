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


def _points(value: Tensor, name: str) -> None:
    if not isinstance(value, Tensor) or value.ndim != 2 or value.shape[1] != 3:
        raise ValueError(f"{name} must be a tensor of shape (N, 3)")
    if value.dtype != torch.float32:
        raise ValueError(f"{name} must be float32")


def _offsets(value: Tensor, count: int | None, device: torch.device, name: str) -> list[int]:
    """Inclusive cumulative counts -> [0, *ends] (pointcept.py:47-58)."""
    if not isinstance(value, Tensor) or value.ndim != 1 or value.dtype not in (torch.int32, torch.int64):
        raise ValueError(f"{name} must be a one-dimensional int32/int64 tensor")
    if value.device != device:
        raise ValueError(f"{name} must be on {device}")
    ends = value.tolist()
    if count is not None and ((ends and ends[-1] != count) or (not ends and count != 0)):
        raise ValueError(f"{name} must end at its point count ({count})")
    if any(end < start for start, end in zip((0, *ends[:-1]), ends)):
        raise ValueError(f"{name} must be nondecreasing and nonnegative")
    return [0, *ends]


def _pairs(xyz: Tensor, offset: Tensor, new_xyz: Tensor | None,
           new_offset: Tensor | None) -> tuple[Tensor, list[int], list[int]]:
    """pointcept.py:61-77."""
    _points(xyz, "xyz")
    if new_xyz is None and new_offset is None:
        new_xyz, new_offset = xyz, offset
    elif new_xyz is None or new_offset is None:
        raise ValueError("new_xyz and new_offset must be provided together")
    _points(new_xyz, "new_xyz")
    if xyz.device != new_xyz.device:
        raise ValueError("xyz and new_xyz must be on the same device")
    ref_ends = _offsets(offset, len(xyz), xyz.device, "offset")
    query_ends = _offsets(new_offset, len(new_xyz), xyz.device, "new_offset")
    if len(ref_ends) != len(query_ends):
        raise ValueError("offset and new_offset must have the same batch count")
    return new_xyz, ref_ends, query_ends


def farthest_point_sampling(xyz: Tensor, offset: Tensor, new_offset: Tensor) -> Tensor:
    """Global int32 FPS indices, starting at each batch's first point
    (pointcept.py:80-104): one ragged launch for every batch."""
    _points(xyz, "xyz")
    source = _offsets(offset, len(xyz), xyz.device, "offset")
    target = _offsets(new_offset, None, xyz.device, "new_offset")
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
    the relative positions first, (M, K, 3+C) (pointcept.py:175-210)."""
    _points(xyz, "xyz")
    if not isinstance(feat, Tensor) or feat.ndim != 2 or len(feat) != len(xyz):
        raise ValueError("feat must have shape (N, C) matching xyz")
    if feat.dtype != torch.float32 or feat.device != xyz.device:
        raise ValueError("feat must be float32 on the xyz device")
    if not isinstance(idx, Tensor) or idx.ndim != 2 or idx.dtype not in (torch.int32, torch.int64):
        raise ValueError("idx must be a two-dimensional int32/int64 tensor")
    if idx.device != xyz.device:
        raise ValueError("idx must be on the xyz device")
    if bool((idx < -1).any()) or bool((idx >= len(xyz)).any()):
        raise ValueError("idx contains an out-of-range point index")
    valid = idx >= 0
    safe = torch.where(valid, idx.long(), len(xyz))
    grouped = torch.cat((feat, feat.new_zeros((1, feat.shape[1]))), dim=0)[safe]
    if not with_xyz:
        return grouped
    if new_xyz is None:
        new_xyz = xyz
    _points(new_xyz, "new_xyz")
    if new_xyz.device != xyz.device or len(new_xyz) != len(idx):
        raise ValueError("new_xyz must have one row per idx row on the xyz device")
    relative = torch.cat((xyz, xyz.new_zeros((1, 3))), dim=0)[safe] - new_xyz.unsqueeze(1)
    relative = torch.where(valid.unsqueeze(-1), relative, 0)
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
    over their k nearest (pointcept.py:228-253): -1 neighbours weigh 0, an
    empty reference batch gives 0, weights are constants for autograd."""
    if not isinstance(feat, Tensor) or feat.ndim != 2 or len(feat) != len(xyz):
        raise ValueError("feat must have shape (N, C) matching xyz")
    if feat.dtype != torch.float32 or feat.device != xyz.device:
        raise ValueError("feat must be float32 on the xyz device")
    idx, dist = knn_query(k, xyz, offset, new_xyz, new_offset)
    valid = idx >= 0
    reciprocal = torch.where(valid, 1.0 / (dist + 1e-8), 0.0)
    weight = reciprocal / reciprocal.sum(dim=1, keepdim=True).clamp_min(1e-20)
    padded = torch.cat((feat, feat.new_zeros((1, feat.shape[1]))), dim=0)
    safe = torch.where(valid, idx.long(), len(feat))
    return (padded[safe] * weight.unsqueeze(-1)).sum(dim=1)


__all__ = ["farthest_point_sampling", "knn_query", "grouping", "knn_query_and_group",
           "interpolation"]
