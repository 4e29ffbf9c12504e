"""Optional stand-ins for ``pointnet2_ops``, ``knn_cuda`` and ``torch_cluster``
(the neighbourhood-search part of /root/reference/mps_pointops/compat.py).

Call ``install()`` before importing code that uses them::

    import mps_pointops.compat
    mps_pointops.compat.install()

    from pointnet2_ops import pointnet2_utils  # served by mps_pointops
    from knn_cuda import KNN
    from torch_cluster import fps, knn, radius

A name that is already importable (for example the real CUDA package) is left
alone unless ``force=True``.  Covered: ``furthest_point_sample``,
``gather_operation``, ``grouping_operation`` and ``ball_query`` from
``pointnet2_utils``, plus its ``QueryAndGroup`` and ``GroupAll`` modules on
the fused grouping kernel (not in the reference's stand-in); ``KNN`` from ``knn_cuda``; ``fps``, ``knn``, ``radius``,
``knn_graph`` and ``radius_graph`` from ``torch_cluster``.  The reference's
graph/cluster extras (graclus, grid, random_walk, nearest) are outside this
package's scope; ``install(pointcept=True)`` adds the Pointcept v1.2.1 PTv1
``pointops`` module (``mps_pointops.pointcept``).
"""

from __future__ import annotations

import importlib.util
import sys
import types
from importlib.machinery import ModuleSpec

import torch
from torch import Tensor

from . import flat, group, ops
from . import pointcept as pointcept_ops


def furthest_point_sample(xyz: Tensor, npoint: int) -> Tensor:
    """Like ``pointnet2_ops.pointnet2_utils.furthest_point_sample``: (B, N, 3)
    float32 -> (B, npoint) int32, start at 0, points with x^2+y^2+z^2 <= 1e-3
    never picked (compat.py:53-59)."""
    return ops.furthest_point_sample(xyz, npoint, skip_near_origin=True).int()


def gather_operation(features: Tensor, idx: Tensor) -> Tensor:
    """(B, C, N), (B, npoint) -> (B, C, npoint) (compat.py:62-65): the
    native gather on the GPU, with its scatter-add gradient."""
    return group.group_points(features, idx)


def grouping_operation(features: Tensor, idx: Tensor) -> Tensor:
    """(B, C, N), (B, npoint, nsample) -> (B, C, npoint, nsample)
    (compat.py:68-73): the same gather over the flattened index."""
    if idx.ndim != 3:
        raise ValueError("indices must have shape (B, npoint, nsample)")
    B, npoint, nsample = idx.shape
    out = group.group_points(features, idx.reshape(B, npoint * nsample))
    return out.reshape(B, features.shape[1], npoint, nsample)


def ball_query(radius: float, nsample: int, xyz: Tensor, new_xyz: Tensor) -> Tensor:
    """(B, N, 3), (B, npoint, 3) -> (B, npoint, nsample) int32 (compat.py:76-85).

    The first ``nsample`` points in input order with squared distance
    ``< radius**2``; empty slots repeat the first neighbour and a query with no
    neighbour gets all zeros, as in pointnet2_ops.
    """
    _, idx = ops.ball_query(new_xyz, xyz, radius, nsample)
    first = idx[..., :1].clamp(min=0)
    return torch.where(idx >= 0, idx, first).int()


class KNN(torch.nn.Module):
    """Like ``knn_cuda.KNN`` (compat.py:91-112).

    With ``transpose_mode=True`` ``ref`` is (B, N, D), ``query`` (B, M, D) and
    the outputs (B, M, k); otherwise (B, D, N), (B, D, M) and (B, k, M).
    ``dist`` is Euclidean.  No gradients flow.
    """

    def __init__(self, k: int, transpose_mode: bool = False):
        super().__init__()
        self.k = k
        self.transpose_mode = transpose_mode

    def forward(self, ref: Tensor, query: Tensor) -> tuple[Tensor, Tensor]:
        if not self.transpose_mode:
            ref, query = ref.transpose(1, 2), query.transpose(1, 2)
        with torch.no_grad():
            dist, idx = ops.knn(query.float(), ref.float(), self.k)
        if not self.transpose_mode:
            dist, idx = dist.transpose(1, 2), idx.transpose(1, 2)
        return dist, idx


def _module(name: str, **attrs) -> types.ModuleType:
    module = types.ModuleType(name)
    module.__dict__.update(attrs)
    module.__spec__ = ModuleSpec(name, loader=None, is_package="__path__" in attrs)
    return module


def install(force: bool = False, *, pointcept: bool = False) -> list[str]:
    """Register the stand-ins in ``sys.modules`` (compat.py:125-172); with
    ``pointcept=True`` also the Pointcept v1.2.1 PTv1 ``pointops`` surface."""
    pointnet2_utils = _module(
        "pointnet2_ops.pointnet2_utils",
        furthest_point_sample=furthest_point_sample,
        gather_operation=gather_operation,
        grouping_operation=grouping_operation,
        ball_query=ball_query,
        QueryAndGroup=group.QueryAndGroup,
        GroupAll=group.GroupAll,
    )
    packages = {
        "pointnet2_ops": {
            "pointnet2_ops": _module("pointnet2_ops", pointnet2_utils=pointnet2_utils, __path__=[]),
            "pointnet2_ops.pointnet2_utils": pointnet2_utils,
        },
        "knn_cuda": {"knn_cuda": _module("knn_cuda", KNN=KNN)},
        "torch_cluster": {
            "torch_cluster": _module(
                "torch_cluster",
                fps=flat.fps,
                knn=flat.knn,
                radius=flat.radius,
                knn_graph=flat.knn_graph,
                radius_graph=flat.radius_graph,
            )
        },
    }
    if pointcept:
        packages["pointops"] = {
            "pointops": _module(
                "pointops",
                farthest_point_sampling=pointcept_ops.farthest_point_sampling,
                knn_query=pointcept_ops.knn_query,
                grouping=pointcept_ops.grouping,
                knn_query_and_group=pointcept_ops.knn_query_and_group,
                interpolation=pointcept_ops.interpolation,
            ),
        }
    installed = []
    for top, modules in packages.items():
        if not force and (top in sys.modules or importlib.util.find_spec(top) is not None):
            continue
        sys.modules.update(modules)
        installed.extend(modules)
    return installed
