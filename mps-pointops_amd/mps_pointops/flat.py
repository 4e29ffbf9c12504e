"""Flat point-cloud operators with the ``torch_cluster`` index convention, on
ROCm (signatures and validation of /root/reference/mps_pointops/flat.py and
its native helpers _flat_fps_mps.py / _flat_search_mps.py).

``x`` holds reference points, ``y`` query points, batch vectors are sorted,
and results use global indices into the flat tensors.  FPS and radius use 3-D
coordinates; kNN accepts feature vectors of any positive dimension.
"""

from __future__ import annotations

import math
import struct
from typing import Sequence

import torch
from torch import Tensor

from . import _native
from ._ball_query import _checked_radius_and_k

_KNN_MAX_K = 256
_UINT_MAX = (1 << 32) - 1


def _points(value: Tensor, name: str) -> None:
    if not isinstance(value, Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if value.ndim != 2 or value.shape[1] != 3:
        raise ValueError(f"{name} must have shape (N, 3), got {tuple(value.shape)}")
    if not value.is_floating_point():
        raise TypeError(f"{name} must have a floating-point dtype")


def _features(value: Tensor, name: str) -> None:
    if not isinstance(value, Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if value.ndim != 2 or value.shape[1] < 1:
        raise ValueError(f"{name} must have shape (N, D) with D >= 1, got {tuple(value.shape)}")
    if not value.is_floating_point():
        raise TypeError(f"{name} must have a floating-point dtype")


def _batch_size(value: int | None) -> int | None:
    if value is None:
        return None
    if isinstance(value, bool) or not isinstance(value, int) or value < 0:
        raise ValueError("batch_size must be a non-negative integer")
    return value


def _check_batch(batch: Tensor | None, count: int, device: torch.device, name: str) -> int:
    """flat.py:49-64 (host syncs for sortedness and the largest id)."""
    if batch is None:
        return 0
    if not isinstance(batch, Tensor):
        raise TypeError(f"{name} must be a torch.Tensor or None")
    if batch.ndim != 1 or batch.numel() != count:
        raise ValueError(f"{name} must have shape ({count},)")
    if batch.device != device:
        raise ValueError(f"{name} must be on {device}")
    if batch.dtype not in (torch.int32, torch.int64):
        raise TypeError(f"{name} must have an integer dtype (int32 or int64)")
    if not count:
        return 0
    if bool((batch[0] < 0).item()) or bool((batch[1:] < batch[:-1]).any().item()):
        raise ValueError(f"{name} must be sorted with non-negative batch IDs")
    return int(batch[-1].item()) + 1


def _ptr_from_batch(batch: Tensor | None, count: int, device: torch.device, size: int) -> Tensor:
    if batch is None:
        return torch.tensor([0, count], dtype=torch.long, device=device)
    if size == 0:
        return torch.zeros(1, dtype=torch.long, device=device)
    boundaries = torch.arange(size + 1, dtype=torch.long, device=device)
    return torch.searchsorted(batch.contiguous().long(), boundaries).long()


def _pair_ptrs(x, y, batch_x, batch_y, batch_size):
    explicit_size = _batch_size(batch_size)
    size_x = _check_batch(batch_x, len(x), x.device, "batch_x")
    size_y = _check_batch(batch_y, len(y), y.device, "batch_y")
    size = max(1, size_x, size_y, explicit_size or 0)
    if size > 1 and (batch_x is None or batch_y is None):
        raise ValueError("batch_x and batch_y are both required for multiple batches")
    if explicit_size is not None and explicit_size < max(size_x, size_y):
        raise ValueError("batch_size is smaller than the largest batch ID")
    return (
        _ptr_from_batch(batch_x, len(x), x.device, size),
        _ptr_from_batch(batch_y, len(y), y.device, size),
    )


def _fps_ptr(x, batch, batch_size, ptr) -> Tensor:
    """flat.py:100-122."""
    if ptr is not None:
        if isinstance(ptr, Tensor):
            if ptr.device != x.device or ptr.dtype not in (torch.int32, torch.int64):
                raise ValueError("ptr must be an integer tensor on the same device as x")
            result = ptr.long()
        elif isinstance(ptr, (list, tuple)):
            result = torch.tensor(ptr, dtype=torch.long, device=x.device)
        else:
            raise TypeError("ptr must be a tensor, a sequence of integers, or None")
        if result.ndim != 1 or len(result) == 0:
            raise ValueError("ptr must be a non-empty one-dimensional offset array")
        if int(result[0].item()) != 0 or int(result[-1].item()) != len(x):
            raise ValueError("ptr must start at 0 and end at len(x)")
        if bool((result[1:] < result[:-1]).any().item()):
            raise ValueError("ptr must be non-decreasing")
        return result.contiguous()
    explicit_size = _batch_size(batch_size)
    inferred_size = _check_batch(batch, len(x), x.device, "batch")
    if explicit_size is not None and explicit_size < inferred_size:
        raise ValueError("batch_size is smaller than the largest batch ID")
    size = (max(1, inferred_size, explicit_size or 0) if batch is None
            else max(inferred_size, explicit_size or 0))
    return _ptr_from_batch(batch, len(x), x.device, size)


def _ratio(value, dtype: torch.dtype) -> Tensor:
    """The ratio as the CPU scalar tensor torch_cluster would use (flat.py:125-147)."""
    if value is None:
        value = 0.5
    if isinstance(value, Tensor):
        if value.numel() != 1 or value.ndim > 1:
            raise ValueError("ratio tensor must be scalar or a length-one vector")
        result = value.detach().to("cpu")
    elif isinstance(value, bool) or not isinstance(value, (int, float)):
        raise TypeError("ratio must be a number or scalar tensor")
    else:
        result = torch.tensor(float(value), dtype=dtype)
    if not math.isfinite(float(result)) or float(result) < 0:
        raise ValueError("ratio must be finite and non-negative")
    return result


def _sample_counts(lengths: list[int], ratio: Tensor) -> list[int]:
    """torch_cluster's GPU count rule: ceil(deg.to(ratio.dtype) * ratio)
    (flat.py:150-158 with mps=True)."""
    sizes = torch.tensor(lengths, dtype=ratio.dtype)
    return torch.ceil(sizes * ratio).to(torch.long).tolist()


def fps(
    x: Tensor,
    batch: Tensor | None = None,
    ratio: float | Tensor | None = None,
    random_start: bool = True,
    batch_size: int | None = None,
    ptr: Tensor | Sequence[int] | None = None,
) -> Tensor:
    """Sample global point indices with the torch_cluster count rule
    (flat.py:161-217).  ``ratio=None`` means 0.5; ``ptr`` takes precedence over
    ``batch``; ``random_start=False`` starts from the first point of each
    non-empty cloud.  Returns int64 indices on ``x.device``.
    """
    _points(x, "x")
    _native.require_device(x.device)
    if x.dtype != torch.float32:
        raise TypeError("x must be float32 on ROCm")
    sample_ratio = _ratio(ratio, x.dtype)
    offsets = _fps_ptr(x, batch, batch_size, ptr)
    offset_values = offsets.cpu().tolist()
    lengths = [hi - lo for lo, hi in zip(offset_values, offset_values[1:])]
    counts = _sample_counts(lengths, sample_ratio)
    output_offsets = [0]
    for count in counts:
        output_offsets.append(output_offsets[-1] + count)
    if output_offsets[-1] == 0:
        return torch.empty(0, dtype=torch.long, device=x.device)
    if random_start:
        length_tensor = torch.tensor(lengths, dtype=torch.long, device=x.device)
        starts = (torch.rand(len(lengths), device=x.device) * length_tensor).long()
        starts = torch.minimum(starts, (length_tensor - 1).clamp_min(0))
    else:
        starts = torch.zeros(len(lengths), dtype=torch.long, device=x.device)
    if any(c > 0 and n == 0 for c, n in zip(counts, lengths)):
        raise ValueError("invalid ptr, out_ptr, or starts for the input point clouds")
    max_len = max(lengths) if lengths else 0
    if max_len > _UINT_MAX:
        raise ValueError("invalid ptr, out_ptr, or starts for the input point clouds")
    out = torch.empty(output_offsets[-1], dtype=torch.long, device=x.device)
    x = x.contiguous()
    out_ptr = torch.tensor(output_offsets, dtype=torch.long, device=x.device)
    size = _native.size_query("pointops_fps_flat_scratch_bytes", len(x), max_len)
    scratch = torch.empty(size, dtype=torch.uint8, device=x.device) if size else None
    _native.call("pointops_fps_flat", x.data_ptr(), offsets.data_ptr(), out_ptr.data_ptr(),
                 starts.contiguous().data_ptr(), out.data_ptr(), _native.ptr(scratch),
                 len(lengths), len(x), max_len, _native.stream(x.device))
    return out


def _search_inputs(x: Tensor, y: Tensor, *, feature_space: bool = False) -> None:
    validate = _features if feature_space else _points
    validate(x, "x")
    validate(y, "y")
    if x.shape[1] != y.shape[1]:
        raise ValueError(f"x and y feature dimensions differ: {x.shape[1]} and {y.shape[1]}")
    if x.device != y.device:
        raise ValueError(f"x and y must be on the same device, got {x.device} and {y.device}")
    if x.dtype != y.dtype:
        raise TypeError(f"x and y must have the same dtype, got {x.dtype} and {y.dtype}")


def _nonnegative_int(value: int, name: str) -> int:
    if isinstance(value, bool) or not isinstance(value, int) or value < 0:
        raise ValueError(f"{name} must be a non-negative integer")
    return value


def _edges(indices: Tensor) -> Tensor:
    """Drop -1 padding: [2, E] (query, reference) edges (flat.py:247-253)."""
    if indices.numel() == 0:
        return torch.empty((2, 0), dtype=torch.long, device=indices.device)
    valid = indices >= 0
    queries = torch.arange(indices.shape[0], device=indices.device, dtype=torch.long)
    queries = queries[:, None].expand_as(indices)[valid]
    return torch.stack((queries, indices[valid]), dim=0)


def _torch_cluster_radius_sq(r: float) -> float:
    """fl32(r * r) with r * r in double (_flat_search_mps.py:66-76)."""
    try:
        return struct.unpack("f", struct.pack("f", r * r))[0]
    except OverflowError:
        return math.inf


def knn_indices(x: Tensor, y: Tensor, ptr_x: Tensor, ptr_y: Tensor, k: int) -> Tensor:
    """(Q, k) global x indices by (squared distance, index), -1 padded."""
    out = torch.empty((len(y), k), dtype=torch.int64, device=x.device)
    if len(y) == 0 or k == 0:
        return out
    _native.call("pointops_knn_flat", y.data_ptr(), x.data_ptr(), ptr_y.contiguous().data_ptr(),
                 ptr_x.contiguous().data_ptr(), out.data_ptr(), len(y), len(ptr_x) - 1,
                 x.shape[1], k, _native.stream(x.device))
    return out


def radius_indices(x: Tensor, y: Tensor, ptr_x: Tensor, ptr_y: Tensor, r: float,
                   max_num_neighbors: int, ignore_same_index: bool = False) -> Tensor:
    """First valid global x indices per query, -1 padded
    (_flat_search_mps.py:111-147)."""
    if x.dtype not in (torch.float32, torch.float16) or y.dtype != x.dtype:
        raise TypeError("flat radius requires matching float32 or float16 x and y")
    radius_f32, _ = _checked_radius_and_k(r, max_num_neighbors)
    radius_sq = _torch_cluster_radius_sq(float(r))
    out = torch.empty((len(y), max_num_neighbors), dtype=torch.int64, device=x.device)
    if len(y) == 0 or max_num_neighbors == 0:
        return out
    if radius_f32 == 0.0:
        out.fill_(-1)
        return out
    name = "pointops_radius_flat_f32" if x.dtype == torch.float32 else "pointops_radius_flat_f16"
    _native.call(name, y.data_ptr(), x.data_ptr(), ptr_y.contiguous().data_ptr(),
                 ptr_x.contiguous().data_ptr(), out.data_ptr(), len(y), len(ptr_x) - 1,
                 max_num_neighbors, radius_sq, int(ignore_same_index), _native.stream(x.device))
    return out


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
    """Global ``[query, reference]`` edges for the nearest points
    (flat.py:291-329).  The effective ``min(k, len(x))`` must be at most 256;
    ``cosine=True`` is not implemented; ``num_workers`` has no effect.
    """
    _search_inputs(x, y, feature_space=True)
    k = _nonnegative_int(k, "k")
    if cosine:
        raise NotImplementedError("cosine kNN is not supported")
    _nonnegative_int(num_workers, "num_workers")
    _native.require_device(x.device)
    if x.dtype != torch.float32:
        raise TypeError("x and y must be float32 for kNN on ROCm")
    if k == 0 or len(x) == 0 or len(y) == 0:
        return torch.empty((2, 0), dtype=torch.long, device=x.device)
    ptr_x, ptr_y = _pair_ptrs(x, y, batch_x, batch_y, batch_size)
    width = min(k, len(x))
    if width > _KNN_MAX_K:
        raise ValueError(f"effective k must be at most {_KNN_MAX_K} on ROCm, got {width}")
    return _edges(knn_indices(x.contiguous(), y.contiguous(), ptr_x, ptr_y, width))


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
    """Global ``[query, reference]`` edges with squared distance ``< r^2``
    (flat.py:332-373): neighbours in reference input order, at most
    ``max_num_neighbors`` per query.  ``ignore_same_index=True`` is not
    implemented (as in the reference's public API).
    """
    _search_inputs(x, y)
    limit = _nonnegative_int(max_num_neighbors, "max_num_neighbors")
    _nonnegative_int(num_workers, "num_workers")
    if ignore_same_index:
        raise NotImplementedError("ignore_same_index=True is not supported")
    if isinstance(r, bool) or not isinstance(r, (int, float)):
        raise ValueError("r must be a finite non-negative number")
    r = float(r)
    if not math.isfinite(r) or r < 0:
        raise ValueError("r must be a finite non-negative number")
    _native.require_device(x.device)
    if x.dtype not in (torch.float16, torch.float32):
        raise TypeError("x and y must be float16 or float32 for radius on ROCm")
    if limit == 0 or len(x) == 0 or len(y) == 0:
        return torch.empty((2, 0), dtype=torch.long, device=x.device)
    ptr_x, ptr_y = _pair_ptrs(x, y, batch_x, batch_y, batch_size)
    width = min(limit, len(x))
    return _edges(radius_indices(x.contiguous(), y.contiguous(), ptr_x, ptr_y, r, width))


def _graph_edges(edges: Tensor, loop: bool, flow: str) -> Tensor:
    if flow not in ("source_to_target", "target_to_source"):
        raise ValueError("flow must be 'source_to_target' or 'target_to_source'")
    if flow == "source_to_target":
        edges = edges.flip(0)
    if not loop:
        edges = edges[:, edges[0] != edges[1]]
    return edges


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
    """kNN graph with torch_cluster 1.6.3 edge orientation (flat.py:386-404)."""
    k = _nonnegative_int(k, "k")
    if flow not in ("source_to_target", "target_to_source"):
        raise ValueError("flow must be 'source_to_target' or 'target_to_source'")
    edges = knn(x, x, k if loop else k + 1, batch, batch,
                cosine=cosine, num_workers=num_workers, batch_size=batch_size)
    return _graph_edges(edges, loop, flow)


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
    """Radius graph with torch_cluster 1.6.3 edge orientation (flat.py:407-425)."""
    limit = _nonnegative_int(max_num_neighbors, "max_num_neighbors")
    if flow not in ("source_to_target", "target_to_source"):
        raise ValueError("flow must be 'source_to_target' or 'target_to_source'")
    edges = radius(x, x, r, batch, batch, limit if loop else limit + 1,
                   num_workers=num_workers, batch_size=batch_size)
    return _graph_edges(edges, loop, flow)


__all__ = ["fps", "knn", "radius", "knn_graph", "radius_graph"]
