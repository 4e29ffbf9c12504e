"""Flat point-cloud operators in the ``torch_cluster`` convention, on ROCm.

Signatures, defaults, exception types and messages are those of
/root/reference/mps_pointops/flat.py (with _flat_fps_mps.py and
_flat_search_mps.py); the code is this package's own.  ``x`` holds the
reference points and ``y`` the queries as flat ``(N, D)`` rows, clouds are
contiguous runs described by a sorted batch vector (or, for ``fps``, an
offset array ``ptr``), and every result uses global row indices.  FPS and
radius take 3-D coordinates; kNN takes any positive dimension.

All clouds of a call go to one ragged launch (``pointops_fps_flat``,
``pointops_knn_flat``, ``pointops_radius_flat_*``).  A batch vector is
validated with one device-to-host read (first id, sortedness and last id
together); its offsets are a bincount prefix sum on the device.
"""

from __future__ import annotations

import math
import struct
from dataclasses import dataclass
from typing import Sequence

import torch
from torch import Tensor

from . import _native
from ._ball_query import _checked_radius_and_k

_KNN_MAX_K = 256          # widest neighbour list of the native kNN (ops.py:30)
_MAX_CLOUD = (1 << 32) - 1  # longest cloud a ragged FPS launch indexes
_FLOWS = ("source_to_target", "target_to_source")


# ----------------------------------------------------------- validation


def _rows(value, name: str, *, coordinates: bool) -> None:
    """A floating-point (N, 3) coordinate table or (N, D >= 1) feature table."""
    if not isinstance(value, Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if coordinates and (value.ndim != 2 or value.shape[1] != 3):
        raise ValueError(f"{name} must have shape (N, 3), got {tuple(value.shape)}")
    if not coordinates and (value.ndim != 2 or value.shape[1] < 1):
        raise ValueError(f"{name} must have shape (N, D) with D >= 1, got {tuple(value.shape)}")
    if not value.is_floating_point():
        raise TypeError(f"{name} must have a floating-point dtype")


def _count_arg(value, name: str) -> int:
    """A non-negative Python int (bool excluded)."""
    if isinstance(value, bool) or not isinstance(value, int) or value < 0:
        raise ValueError(f"{name} must be a non-negative integer")
    return value


def _optional_batch_size(value) -> int | None:
    return None if value is None else _count_arg(value, "batch_size")


def _clouds_in(batch, rows: int, device: torch.device, name: str) -> int:
    """Number of clouds a sorted batch vector names (its last id + 1; 0 for
    no vector or no rows).  One device-to-host read covers the checks."""
    if batch is None:
        return 0
    if not isinstance(batch, Tensor):
        raise TypeError(f"{name} must be a torch.Tensor or None")
    if batch.ndim != 1 or batch.numel() != rows:
        raise ValueError(f"{name} must have shape ({rows},)")
    if batch.device != device:
        raise ValueError(f"{name} must be on {device}")
    if batch.dtype not in (torch.int32, torch.int64):
        raise TypeError(f"{name} must have an integer dtype (int32 or int64)")
    if rows == 0:
        return 0
    ids = batch.long()
    first, descending, last = torch.stack(
        (ids[0], (ids[1:] < ids[:-1]).any().long(), ids[-1])).tolist()
    if first < 0 or descending:
        raise ValueError(f"{name} must be sorted with non-negative batch IDs")
    return last + 1


def _offsets(batch: Tensor | None, rows: int, device: torch.device, clouds: int) -> Tensor:
    """(clouds + 1,) int64 row offsets of a sorted batch vector; without a
    vector all rows form one cloud (even when there are none)."""
    if batch is None:
        return torch.tensor([0, rows], dtype=torch.long, device=device)
    offsets = torch.zeros(clouds + 1, dtype=torch.long, device=device)
    if clouds:
        offsets[1:] = torch.bincount(batch.long(), minlength=clouds).cumsum(0)
    return offsets


@dataclass(frozen=True)
class _SearchLayout:
    """Offsets of the reference and query clouds of one search call."""

    x_offsets: Tensor
    y_offsets: Tensor

    @property
    def clouds(self) -> int:
        return len(self.x_offsets) - 1

    @classmethod
    def of(cls, x: Tensor, y: Tensor, batch_x, batch_y, batch_size) -> "_SearchLayout":
        requested = _optional_batch_size(batch_size)
        in_x = _clouds_in(batch_x, len(x), x.device, "batch_x")
        in_y = _clouds_in(batch_y, len(y), y.device, "batch_y")
        clouds = max(1, in_x, in_y, requested or 0)
        if clouds > 1 and (batch_x is None or batch_y is None):
            raise ValueError("batch_x and batch_y are both required for multiple batches")
        if requested is not None and requested < max(in_x, in_y):
            raise ValueError("batch_size is smaller than the largest batch ID")
        return cls(_offsets(batch_x, len(x), x.device, clouds),
                   _offsets(batch_y, len(y), y.device, clouds))


def _fps_offsets(x: Tensor, batch, batch_size, ptr) -> Tensor:
    """Cloud offsets for fps: an explicit ``ptr`` wins over ``batch``."""
    if ptr is None:
        requested = _optional_batch_size(batch_size)
        named = _clouds_in(batch, len(x), x.device, "batch")
        if requested is not None and requested < named:
            raise ValueError("batch_size is smaller than the largest batch ID")
        clouds = max(named, requested or 0)
        if batch is None:
            clouds = max(1, clouds)
        return _offsets(batch, len(x), x.device, clouds)
    if isinstance(ptr, Tensor):
        if ptr.device != x.device or ptr.dtype not in (torch.int32, torch.int64):
            raise ValueError("ptr must be an integer tensor on the same device as x")
        offsets = ptr.long()
    elif isinstance(ptr, (list, tuple)):
        offsets = torch.tensor(ptr, dtype=torch.long, device=x.device)
    else:
        raise TypeError("ptr must be a tensor, a sequence of integers, or None")
    if offsets.ndim != 1 or len(offsets) == 0:
        raise ValueError("ptr must be a non-empty one-dimensional offset array")
    head, tail, descending = torch.stack(
        (offsets[0], offsets[-1], (offsets[1:] < offsets[:-1]).any().long())).tolist()
    if head != 0 or tail != len(x):
        raise ValueError("ptr must start at 0 and end at len(x)")
    if descending:
        raise ValueError("ptr must be non-decreasing")
    return offsets.contiguous()


def _ratio_tensor(value, dtype: torch.dtype) -> Tensor:
    """The sampling ratio as the CPU tensor torch_cluster computes with: a
    Python number becomes a 0-d tensor of the points' dtype, a tensor ratio
    keeps its own dtype and shape (0-d and [1] promote differently)."""
    if value is None:
        value = 0.5
    if isinstance(value, Tensor):
        if value.numel() != 1 or value.ndim > 1:
            raise ValueError("ratio tensor must be scalar or a length-one vector")
        ratio = value.detach().to("cpu")
    elif isinstance(value, bool) or not isinstance(value, (int, float)):
        raise TypeError("ratio must be a number or scalar tensor")
    else:
        ratio = torch.tensor(float(value), dtype=dtype)
    number = float(ratio)
    if not (math.isfinite(number) and number >= 0):
        raise ValueError("ratio must be finite and non-negative")
    return ratio


def _samples_per_cloud(lengths: list[int], ratio: Tensor) -> list[int]:
    """torch_cluster's GPU rule: ceil(length.to(ratio.dtype) * ratio)."""
    return torch.ceil(torch.tensor(lengths, dtype=ratio.dtype) * ratio).long().tolist()


def _radius_sq_torch_cluster(r: float) -> float:
    """The torch_cluster threshold: r * r in double, then rounded to float32
    (inf when that overflows)."""
    try:
        return struct.unpack("f", struct.pack("f", r * r))[0]
    except OverflowError:
        return math.inf


# ---------------------------------------------------------------- fps


def fps(
    x: Tensor,
    batch: Tensor | None = None,
    ratio: float | Tensor | None = None,
    random_start: bool = True,
    batch_size: int | None = None,
    ptr: Tensor | Sequence[int] | None = None,
) -> Tensor:
    """Global indices of farthest point samples, ``ceil(len * ratio)`` per
    cloud (the torch_cluster count rule), flat.py:161-217.  ``ratio=None``
    means 0.5; ``ptr`` takes precedence over ``batch``; without
    ``random_start`` each cloud starts at its first point.  int64 on
    ``x.device``."""
    _rows(x, "x", coordinates=True)
    _native.require_device(x.device)
    if x.dtype != torch.float32:
        raise TypeError("x must be float32 on ROCm")
    ratio_t = _ratio_tensor(ratio, x.dtype)
    offsets = _fps_offsets(x, batch, batch_size, ptr)
    bounds = offsets.tolist()
    lengths = [b - a for a, b in zip(bounds, bounds[1:])]
    counts = _samples_per_cloud(lengths, ratio_t)
    out_bounds = [0]
    for count in counts:
        out_bounds.append(out_bounds[-1] + count)
    total = out_bounds[-1]
    if total == 0:
        return torch.empty(0, dtype=torch.long, device=x.device)
    if random_start:
        sizes = torch.tensor(lengths, dtype=torch.long, device=x.device)
        draw = (torch.rand(len(lengths), device=x.device) * sizes).long()
        starts = torch.minimum(draw, (sizes - 1).clamp_min(0))
    else:
        starts = torch.zeros(len(lengths), dtype=torch.long, device=x.device)
    longest = max(lengths)
    if longest > _MAX_CLOUD or any(c > 0 and n == 0 for c, n in zip(counts, lengths)):
        raise ValueError("invalid ptr, out_ptr, or starts for the input point clouds")
    points = x.contiguous()
    out = torch.empty(total, dtype=torch.long, device=x.device)
    out_ptr = torch.tensor(out_bounds, dtype=torch.long, device=x.device)
    scratch_bytes = _native.size_query("pointops_fps_flat_scratch_bytes", len(points), longest)
    scratch = torch.empty(scratch_bytes, dtype=torch.uint8, device=x.device) if scratch_bytes else None
    _native.call("pointops_fps_flat", points.data_ptr(), offsets.data_ptr(), out_ptr.data_ptr(),
                 starts.contiguous().data_ptr(), out.data_ptr(), _native.ptr(scratch),
                 len(lengths), len(points), longest, _native.stream(x.device))
    return out


# ------------------------------------------------------ kNN and radius


def _search_pair(x, y, *, coordinates: bool) -> None:
    _rows(x, "x", coordinates=coordinates)
    _rows(y, "y", coordinates=coordinates)
    if x.shape[1] != y.shape[1]:
        raise ValueError(f"x and y feature dimensions differ: {x.shape[1]} and {y.shape[1]}")
    if x.device != y.device:
        raise ValueError(f"x and y must be on the same device, got {x.device} and {y.device}")
    if x.dtype != y.dtype:
        raise TypeError(f"x and y must have the same dtype, got {x.dtype} and {y.dtype}")


def _edge_index(table: Tensor) -> Tensor:
    """[2, E] (query row, reference row) pairs of a -1 padded (Q, K) table,
    row-major."""
    queries, slots = torch.nonzero(table >= 0, as_tuple=True)
    return torch.stack((queries, table[queries, slots]))


def knn_indices(x: Tensor, y: Tensor, ptr_x: Tensor, ptr_y: Tensor, k: int) -> Tensor:
    """(Q, k) global x rows nearest to each y row, ordered by (squared
    distance, index), -1 where a cloud has fewer than k rows."""
    table = torch.empty((len(y), k), dtype=torch.int64, device=x.device)
    if len(y) and k:
        _native.call("pointops_knn_flat", y.data_ptr(), x.data_ptr(), ptr_y.contiguous().data_ptr(),
                     ptr_x.contiguous().data_ptr(), table.data_ptr(), len(y), len(ptr_x) - 1,
                     x.shape[1], k, _native.stream(x.device))
    return table


def radius_indices(x: Tensor, y: Tensor, ptr_x: Tensor, ptr_y: Tensor, r: float,
                   max_num_neighbors: int, ignore_same_index: bool = False) -> Tensor:
    """(Q, max_num_neighbors) first x rows in index order with squared
    distance below fl32(r * r in double), -1 padded; with
    ``ignore_same_index`` a row equal to the query's own row number is
    skipped before the cap (_flat_search_mps.py:111-147)."""
    if x.dtype not in (torch.float32, torch.float16) or y.dtype != x.dtype:
        raise TypeError("flat radius requires matching float32 or float16 x and y")
    radius_f32, _ = _checked_radius_and_k(r, max_num_neighbors)
    table = torch.empty((len(y), max_num_neighbors), dtype=torch.int64, device=x.device)
    if len(y) == 0 or max_num_neighbors == 0:
        return table
    if radius_f32 == 0.0:
        return table.fill_(-1)
    entry = "pointops_radius_flat_f32" if x.dtype == torch.float32 else "pointops_radius_flat_f16"
    _native.call(entry, y.data_ptr(), x.data_ptr(), ptr_y.contiguous().data_ptr(),
                 ptr_x.contiguous().data_ptr(), table.data_ptr(), len(y), len(ptr_x) - 1,
                 max_num_neighbors, _radius_sq_torch_cluster(float(r)), int(ignore_same_index),
                 _native.stream(x.device))
    return table


def knn(
    x: Tensor,
    y: Tensor,
    k: int,
    batch_x: Tensor | None = None,
    batch_y: Tensor | None = None,
    cosine: bool = False,
    num_workers: int = 1,
    batch_size: int | None = None,
) -> Tensor:
    """``[2, E]`` (query, reference) edges to the ``k`` nearest references of
    each query within its cloud (flat.py:291-329).  ``min(k, len(x))`` must
    be at most 256; ``cosine=True`` is not implemented; ``num_workers`` has
    no effect."""
    _search_pair(x, y, coordinates=False)
    k = _count_arg(k, "k")
    if cosine:
        raise NotImplementedError("cosine kNN is not supported")
    _count_arg(num_workers, "num_workers")
    _native.require_device(x.device)
    if x.dtype != torch.float32:
        raise TypeError("x and y must be float32 for kNN on ROCm")
    if k == 0 or len(x) == 0 or len(y) == 0:
        return torch.empty((2, 0), dtype=torch.long, device=x.device)
    layout = _SearchLayout.of(x, y, batch_x, batch_y, batch_size)
    width = min(k, len(x))
    if width > _KNN_MAX_K:
        raise ValueError(f"effective k must be at most {_KNN_MAX_K} on ROCm, got {width}")
    table = knn_indices(x.contiguous(), y.contiguous(), layout.x_offsets, layout.y_offsets, width)
    return _edge_index(table)


def radius(
    x: Tensor,
    y: Tensor,
    r: float,
    batch_x: Tensor | None = None,
    batch_y: Tensor | None = None,
    max_num_neighbors: int = 32,
    num_workers: int = 1,
    batch_size: int | None = None,
    ignore_same_index: bool = False,
) -> Tensor:
    """``[2, E]`` (query, reference) edges to the first references of each
    query's cloud, in index order, with squared distance below ``r**2``
    (flat.py:332-373); at most ``max_num_neighbors`` per query.
    ``ignore_same_index=True`` is not implemented, as in the reference."""
    _search_pair(x, y, coordinates=True)
    limit = _count_arg(max_num_neighbors, "max_num_neighbors")
    _count_arg(num_workers, "num_workers")
    if ignore_same_index:
        raise NotImplementedError("ignore_same_index=True is not supported")
    if isinstance(r, bool) or not isinstance(r, (int, float)) or not math.isfinite(float(r)) \
            or float(r) < 0:
        raise ValueError("r must be a finite non-negative number")
    _native.require_device(x.device)
    if x.dtype not in (torch.float16, torch.float32):
        raise TypeError("x and y must be float16 or float32 for radius on ROCm")
    if limit == 0 or len(x) == 0 or len(y) == 0:
        return torch.empty((2, 0), dtype=torch.long, device=x.device)
    layout = _SearchLayout.of(x, y, batch_x, batch_y, batch_size)
    table = radius_indices(x.contiguous(), y.contiguous(), layout.x_offsets, layout.y_offsets,
                           float(r), min(limit, len(x)))
    return _edge_index(table)


# --------------------------------------------------------------- graphs


def _check_flow(flow: str) -> None:
    if flow not in _FLOWS:
        raise ValueError("flow must be 'source_to_target' or 'target_to_source'")


def _as_graph(edges: Tensor, loop: bool, flow: str) -> Tensor:
    """torch_cluster 1.6.3 orientation of self-search edges: (source,
    target) rows, reference first for ``source_to_target``; without ``loop``
    the edges from a point to itself are dropped."""
    if not loop:
        edges = edges[:, edges[0] != edges[1]]
    return edges.flip(0) if flow == "source_to_target" else edges


def knn_graph(
    x: Tensor,
    k: int,
    batch: Tensor | None = None,
    loop: bool = False,
    flow: str = "source_to_target",
    cosine: bool = False,
    num_workers: int = 1,
    batch_size: int | None = None,
) -> Tensor:
    """kNN graph of ``x`` (flat.py:386-404): ``k + 1`` neighbours are searched
    when self loops are removed."""
    k = _count_arg(k, "k")
    _check_flow(flow)
    edges = knn(x, x, k if loop else k + 1, batch, batch, cosine=cosine,
                num_workers=num_workers, batch_size=batch_size)
    return _as_graph(edges, loop, flow)


def radius_graph(
    x: Tensor,
    r: float,
    batch: Tensor | None = None,
    loop: bool = False,
    max_num_neighbors: int = 32,
    flow: str = "source_to_target",
    num_workers: int = 1,
    batch_size: int | None = None,
) -> Tensor:
    """Radius graph of ``x`` (flat.py:407-425): ``max_num_neighbors + 1``
    candidates when self loops are removed."""
    limit = _count_arg(max_num_neighbors, "max_num_neighbors")
    _check_flow(flow)
    edges = radius(x, x, r, batch, batch, limit if loop else limit + 1,
                   num_workers=num_workers, batch_size=batch_size)
    return _as_graph(edges, loop, flow)


__all__ = ["fps", "knn", "radius", "knn_graph", "radius_graph"]
