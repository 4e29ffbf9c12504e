"""PyTorch3D-style ``ball_query`` call surface on the native ball query.

Import explicitly: ``from mps_pointops.pytorch3d import ball_query``.  It
neither imports nor replaces PyTorch3D.  The call signature, argument checks
and messages are those of /root/reference/mps_pointops/pytorch3d.py:67-125;
results are this package's ball query (the first ``K`` points in index order
strictly inside the radius, squared distances, ``-1`` / ``0`` padding,
ragged lengths) plus, with ``return_nn``, the neighbours' coordinates (zeros
in padded slots).  Inputs are float32 ROCm (``device='cuda'``) tensors of
shape ``(B, Q, 3)`` and ``(B, P, 3)``; the reference's CPU fallback has no
counterpart here.
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


def _neighbour_coordinates(points: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
    """(B, Q, K, 3) coordinates of the selected points, zeros for index -1,
    differentiable in ``points``: the cloud gets one extra all-zero row and
    every -1 reads that row, so padding needs no separate mask and its
    gradient (into the extra row) is dropped."""
    batch, queries, k = indices.shape
    count = points.shape[1]
    padded = torch.cat((points, points.new_zeros((batch, 1, 3))), dim=1)
    rows = torch.where(indices >= 0, indices, count).reshape(batch, queries * k, 1)
    return padded.gather(1, rows.expand(-1, -1, 3)).reshape(batch, queries, k, 3)


def _check_clouds(p1, p2) -> None:
    """The reference's argument checks, in its order."""
    if not isinstance(p1, torch.Tensor) or not isinstance(p2, torch.Tensor):
        raise TypeError("p1 and p2 must be torch.Tensor values")
    shapes_ok = p1.ndim == 3 and p2.ndim == 3 and p1.shape[-1] == 3 and p2.shape[-1] == 3
    checks = (
        (shapes_ok, ValueError, "p1 and p2 must have shapes (B, Q, 3) and (B, P, 3)"),
        (lambda: p1.shape[0] == p2.shape[0], ValueError,
         "p1 and p2 must have the same batch dimension"),
        (lambda: p1.device == p2.device, ValueError, "p1 and p2 must be on the same device"),
        (lambda: p1.dtype == torch.float32 and p2.dtype == torch.float32, TypeError,
         "PyTorch3D-style Ball Query currently requires float32 coordinates"),
    )
    for ok, error, message in checks:
        if not (ok() if callable(ok) else ok):
            raise error(message)


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
    ``knn`` the gathered coordinates (zero padded) when ``return_nn``.
    ``skip_points_outside_cube`` is accepted as a hint and changes nothing.
    Length vectors are checked by the ball query itself (one host read)."""
    _check_clouds(p1, p2)
    if not isinstance(return_nn, bool) or not isinstance(skip_points_outside_cube, bool):
        raise TypeError("return_nn and skip_points_outside_cube must be bool")
    _checked_radius_and_k(radius, K)
    found = _ball_query(p1, p2, radius=radius, k=K, query_lengths=lengths1,
                        point_lengths=lengths2)
    coordinates = _neighbour_coordinates(p2, found.indices) if return_nn else None
    return KNN(dists=found.distances, idx=found.indices, knn=coordinates)
