"""Stand-ins for ``pointnet2_ops``, ``knn_cuda`` and ``torch_cluster`` on the
native ROCm kernels (the neighbourhood-search surface of
/root/reference/mps_pointops/compat.py).

Call ``install()`` before importing code that uses them::

    import mps_pointops.compat
    mps_pointops.compat.install()

    from pointnet2_ops import pointnet2_utils  # served by mps_pointops
    from knn_cuda import KNN
    from torch_cluster import fps, knn, radius

A top-level name that is already importable (for example the real CUDA
package) is left alone unless ``force=True``.  Served: ``pointnet2_utils``'s
``furthest_point_sample``, ``gather_operation``, ``grouping_operation`` and
``ball_query`` (plus ``QueryAndGroup`` / ``GroupAll`` on the fused grouping
kernel, which the reference's stand-in lacks); ``knn_cuda.KNN``;
``torch_cluster``'s ``fps``, ``knn``, ``radius``, ``knn_graph`` and
``radius_graph``.  The reference's graph/cluster extras (graclus, grid,
random_walk, nearest) are outside this package.  ``install(pointcept=True)``
adds the Pointcept v1.2.1 PTv1 ``pointops`` module
(``mps_pointops.pointcept``).
"""

from __future__ import annotations

import importlib.util
import sys
import types
from importlib.machinery import ModuleSpec

import torch
from torch import Tensor

from . import _native, flat, group, ops
from . import pointcept as pointcept_ops


def furthest_point_sample(xyz: Tensor, npoint: int) -> Tensor:
    """pointnet2_ops' FPS: (B, N, 3) float32 -> (B, npoint) int32, starting
    at index 0, never picking points with x^2+y^2+z^2 <= 1e-3
    (compat.py:53-59)."""
    return ops.furthest_point_sample(xyz, npoint, skip_near_origin=True).int()


def gather_operation(features: Tensor, idx: Tensor) -> Tensor:
    """(B, C, N), (B, npoint) -> (B, C, npoint) (compat.py:62-65): the
    native gather, with its deterministic scatter-add gradient."""
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
    """pointnet2_ops' ball query (compat.py:76-85): (B, N, 3), (B, npoint, 3)
    -> (B, npoint, nsample) int32 holding the first ``nsample`` points in
    input order with squared distance ``< radius**2``; unused slots repeat
    the query's first neighbour, and a query without neighbours is all 0."""
    fused = _ball_query_pointnet2(new_xyz, xyz, radius, nsample)
    if fused is not None:
        return fused
    _, idx = ops.ball_query(new_xyz, xyz, radius, nsample)
    if idx.shape[-1] == 0:
        return idx.int()
    first = idx.narrow(-1, 0, 1).clamp_min(0)
    return idx.where(idx >= 0, first).int()


def _ball_query_pointnet2(queries: Tensor, points: Tensor, radius: float, k: int) -> Tensor | None:
    """The padded int32 result in one launch (pointops_ball_query_pn2_f32) for
    float32 ROCm clouds the index-order kernel serves (fewer points than the
    grid search takes, at most 65535 clouds); None otherwise.  Arguments are
    checked as ops.ball_query checks them."""
    from . import _ball_query

    if not (isinstance(queries, Tensor) and isinstance(points, Tensor)):
        return None
    if (queries.dim() != 3 or points.dim() != 3 or queries.shape[-1] != 3
            or points.shape[-1] != 3 or queries.shape[0] != points.shape[0]
            or queries.device != points.device or queries.device.type != "cuda"
            or queries.dtype != torch.float32 or points.dtype != torch.float32
            or queries.shape[0] > 65_535 or points.shape[1] >= _ball_query._GRID_MIN_POINTS):
        return None  # the general path raises or serves these
    _, radius_sq = _ball_query._checked_radius_and_k(radius, k)
    _native.require_device(queries.device)
    B, Q, _ = queries.shape
    idx = torch.empty((B, Q, k), dtype=torch.int32, device=queries.device)
    if idx.numel():
        _native.call("pointops_ball_query_pn2_f32", queries.contiguous().data_ptr(),
                     points.contiguous().data_ptr(), idx.data_ptr(), B, Q, points.shape[1], k,
                     radius_sq, _native.stream(queries.device))
    return idx


class KNN(torch.nn.Module):
    """``knn_cuda.KNN(k, transpose_mode)`` (compat.py:91-112): Euclidean
    distances and indices of the ``k`` nearest references, no gradient.
    ``transpose_mode=True`` takes (B, N, D) / (B, M, D) and returns (B, M, k);
    otherwise the layouts are (B, D, N) / (B, D, M) -> (B, k, M)."""

    def __init__(self, k: int, transpose_mode: bool = False):
        super().__init__()
        self.k = k
        self.transpose_mode = transpose_mode

    def _rows(self, t: Tensor) -> Tensor:
        """The point-major (B, count, D) view of an input or (B, count, k)
        result in this module's layout."""
        return t if self.transpose_mode else t.transpose(1, 2)

    @torch.no_grad()
    def forward(self, ref: Tensor, query: Tensor) -> tuple[Tensor, Tensor]:
        dist, idx = ops.knn(self._rows(query).float(), self._rows(ref).float(), self.k)
        return self._rows(dist), self._rows(idx)


def _stand_in(name: str, package: bool = False, **attrs) -> types.ModuleType:
    """A module object for sys.modules with a spec, so importlib treats it
    like an imported module (a package when ``package``)."""
    module = types.ModuleType(name)
    module.__spec__ = ModuleSpec(name, loader=None, is_package=package)
    if package:
        module.__path__ = []
    module.__dict__.update(attrs)
    return module


def _stand_ins(pointcept: bool) -> dict[str, list[types.ModuleType]]:
    """Top-level name -> the modules registered for it."""
    utils = _stand_in("pointnet2_ops.pointnet2_utils",
                      furthest_point_sample=furthest_point_sample,
                      gather_operation=gather_operation,
                      grouping_operation=grouping_operation,
                      ball_query=ball_query,
                      QueryAndGroup=group.QueryAndGroup,
                      GroupAll=group.GroupAll)
    table = {
        "pointnet2_ops": [_stand_in("pointnet2_ops", package=True, pointnet2_utils=utils), utils],
        "knn_cuda": [_stand_in("knn_cuda", KNN=KNN)],
        "torch_cluster": [_stand_in("torch_cluster", fps=flat.fps, knn=flat.knn,
                                    radius=flat.radius, knn_graph=flat.knn_graph,
                                    radius_graph=flat.radius_graph)],
    }
    if pointcept:
        table["pointops"] = [_stand_in("pointops", **{
            name: getattr(pointcept_ops, name) for name in pointcept_ops.__all__})]
    return table


def _importable(name: str) -> bool:
    return name in sys.modules or importlib.util.find_spec(name) is not None


def install(force: bool = False, *, pointcept: bool = False) -> list[str]:
    """Register the stand-ins in ``sys.modules`` (compat.py:125-172) and
    return the module names registered; ``pointcept=True`` adds the
    Pointcept v1.2.1 PTv1 ``pointops`` surface."""
    registered: list[str] = []
    for top, modules in _stand_ins(pointcept).items():
        if not force and _importable(top):
            continue
        for module in modules:
            sys.modules[module.__name__] = module
            registered.append(module.__name__)
    return registered
