"""PyTorch3D-style ``ball_query`` call surface on the native ball query
(pytorch3d.py:67-125 of the reference).

Import explicitly: ``from mps_pointops.pytorch3d import ball_query``.  It
neither imports nor replaces PyTorch3D.  Results are this package's ball
query (first ``K`` points in index order strictly inside the radius, squared
distances, ``-1`` / ``0`` padding, ragged lengths) with the neighbours'
coordinates gathered when ``return_nn`` (zeros in padded slots).  Inputs are
float32 ROCm (``device='cuda'``) tensors of shape ``(B, Q, 3)`` and
``(B, P, 3)``; the reference's CPU fallback has no counterpart here.
"""

from __future__ import annotations

from typing import NamedTuple

import torch

from ._ball_query import _checked_radius_and_k
from ._ball_query import ball_query as _ball_query


class KNN(NamedTuple):
    """PyTorch3D-style ``(dists, idx, knn)`` result (pytorch3d.py:19-24)."""

    dists: torch.Tensor
    idx: torch.Tensor
    knn: torch.Tensor | None


def _gather_neighbors(points: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
    """(B, Q, K, 3) coordinates of the neighbours, zeros where the index is
    -1; differentiable in ``points`` (pytorch3d.py:27-39)."""
    batch, queries, k = indices.shape
    if indices.numel() == 0:
        return points[:, :0, :].reshape(batch, queries, k, 3)
    if points.shape[1] == 0:
        return points.new_zeros((batch, queries, k, 3)) + points.sum() * 0.0
    valid = indices >= 0
    gathered = points.gather(1, indices.clamp_min(0).reshape(batch, -1, 1).expand(-1, -1, 3))
    gathered = gathered.reshape(batch, queries, k, 3)
    return torch.where(valid.unsqueeze(-1), gathered, torch.zeros_like(gathered))


def ball_query(
    p1: torch.Tensor,
    p2: torch.Tensor,
    lengths1: torch.Tensor | None = None,
    lengths2: torch.Tensor | None = None,
    K: int = 500,
    radius: float = 0.2,
    return_nn: bool = True,
    skip_points_outside_cube: bool = False,
) -> KNN:
    """First ``K`` points of ``p2`` within ``radius`` of each ``p1`` point
    (pytorch3d.py:67-125): ``dists`` squared, ``idx`` with ``-1`` padding,
    ``knn`` gathered coordinates (zero padded) when ``return_nn``.
    ``skip_points_outside_cube`` is accepted as a hint and changes nothing.
    Argument errors follow the reference's order and messages."""
    if not isinstance(p1, torch.Tensor) or not isinstance(p2, torch.Tensor):
        raise TypeError("p1 and p2 must be torch.Tensor values")
    if p1.ndim != 3 or p2.ndim != 3 or p1.shape[-1] != 3 or p2.shape[-1] != 3:
        raise ValueError("p1 and p2 must have shapes (B, Q, 3) and (B, P, 3)")
    if p1.shape[0] != p2.shape[0]:
        raise ValueError("p1 and p2 must have the same batch dimension")
    if p1.device != p2.device:
        raise ValueError("p1 and p2 must be on the same device")
    if p1.dtype != torch.float32 or p2.dtype != torch.float32:
        raise TypeError("PyTorch3D-style Ball Query currently requires float32 coordinates")
    if not isinstance(return_nn, bool) or not isinstance(skip_points_outside_cube, bool):
        raise TypeError("return_nn and skip_points_outside_cube must be bool")
    _checked_radius_and_k(radius, K)
    result = _ball_query(p1, p2, radius=radius, k=K, query_lengths=lengths1,
                         point_lengths=lengths2)
    dists, idx = result.distances, result.indices
    knn = _gather_neighbors(p2, idx) if return_nn else None
    return KNN(dists=dists, idx=idx, knn=knn)
