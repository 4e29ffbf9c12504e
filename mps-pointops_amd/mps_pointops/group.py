"""Point gathers of PointNet++ set abstraction on the native kernels.

``group_points`` is the gather of compat.py:62-73 (``gather_operation`` and
``grouping_operation``: ``torch.gather`` along the point axis) with its
scatter-add gradient; ``query_and_group`` fuses the set-abstraction step
after ball query (tests/test_pointnet2_e2e.py:36-45): grouped xyz less the
query centre, and grouped features, written once into the concatenated
``(B, 3+C, npoint, nsample)`` tensor.  ``QueryAndGroup`` and ``GroupAll``
are the ``pointnet2_ops.pointnet2_utils`` modules of those names built on
it (the reference's stand-in stops at the four functions).

float32 GPU tensors (``device='cuda'``) run ``libpointops_hip.so``; other
devices and dtypes keep the reference's ``torch.gather`` formulation.  Index
gradients are none; feature and xyz gradients are float sums over each
point's entries in increasing entry order (deterministic), like a sequential
scatter-add, for points gathered at most 256 times; a point gathered more
often sums in an unspecified order.
"""

from __future__ import annotations

import torch
from torch import Tensor, nn
from torch.autograd.function import once_differentiable

from . import _native

_MAX_INDEX = (1 << 31) - 1


def _index_arg(idx: Tensor) -> tuple[Tensor, int]:
    """The index tensor as int32 or int64 (contiguous) and its width."""
    if idx.dtype == torch.int32:
        return idx.contiguous(), 32
    if idx.dtype == torch.int64:
        return idx.contiguous(), 64
    if idx.dtype.is_floating_point or idx.dtype in (torch.bool, torch.complex64, torch.complex128):
        raise TypeError("indices must be an integer tensor")
    return idx.long().contiguous(), 64


def _check_range(idx: Tensor, n: int) -> None:
    """torch.gather's index rule (one device-to-host sync)."""
    if idx.numel() and torch.any((idx < 0) | (idx >= n)).item():
        raise IndexError(f"indices must lie in [0, {n})")


def _scatter_back(g: Tensor, batch_stride: int, index: Tensor, bits: int, C: int, N: int,
                  P: int) -> Tensor:
    """(B, C, N) gradient of the gather: the sum over each point's entries in
    increasing p.  `g` points at channel 0 of a (B, *, P) float32 tensor
    whose batches are `batch_stride` elements apart."""
    B = index.shape[0]
    out = torch.empty((B, C, N), dtype=torch.float32, device=g.device)
    if out.numel():
        size = _native.size_query("pointops_group_points_backward_workspace_bytes", B, C, N, P)
        ws = torch.empty(max(size, 1), dtype=torch.uint8, device=g.device)
        _native.call("pointops_group_points_backward", g.data_ptr(), batch_stride,
                     index.data_ptr(), bits, out.data_ptr(), ws.data_ptr(), B, C, N, P,
                     _native.stream(g.device))
    return out


class _GroupPoints(torch.autograd.Function):
    """out[b,c,p] = features[b,c,idx[b,p]] and its scatter-add gradient."""

    @staticmethod
    def forward(ctx, features: Tensor, idx: Tensor) -> Tensor:
        B, C, N = features.shape
        P = idx.shape[1]
        index, bits = _index_arg(idx)
        out = torch.empty((B, C, P), dtype=torch.float32, device=features.device)
        if out.numel():
            _native.call("pointops_group_points", features.contiguous().data_ptr(),
                         index.data_ptr(), bits, out.data_ptr(), B, C, N, P,
                         _native.stream(features.device))
        ctx.save_for_backward(index)
        ctx.bits, ctx.n = bits, N
        return out

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_out: Tensor | None):
        if grad_out is None or not ctx.needs_input_grad[0]:
            return None, None
        (index,) = ctx.saved_tensors
        B, C, P = grad_out.shape
        g = grad_out.contiguous()
        return _scatter_back(g, C * P, index, ctx.bits, C, ctx.n, P), None


def _validate_features(features: Tensor, idx: Tensor) -> None:
    if not isinstance(features, Tensor) or not isinstance(idx, Tensor):
        raise TypeError("features and indices must be tensors")
    if features.ndim != 3:
        raise ValueError("features must have shape (B, C, N)")
    if idx.ndim != 2 or idx.shape[0] != features.shape[0]:
        raise ValueError("indices must have shape (B, P) with the features' batch size")
    if features.device != idx.device:
        raise ValueError("features and indices must be on the same device")
    if features.shape[2] > _MAX_INDEX:
        raise ValueError("at most 2**31-1 points")


def group_points(features: Tensor, idx: Tensor, check: bool = True) -> Tensor:
    """``(B, C, N)`` features gathered at ``(B, P)`` indices -> ``(B, C, P)``."""
    _validate_features(features, idx)
    if features.device.type != "cuda" or features.dtype != torch.float32:
        B, C, _ = features.shape
        return features.gather(2, idx.long().unsqueeze(1).expand(B, C, -1))
    if check:
        _check_range(idx, features.shape[2])
    return _GroupPoints.apply(features, idx)


class _GroupPointsRel(torch.autograd.Function):
    """(B, 3+C, M, S): grouped xyz - centre, then grouped features."""

    @staticmethod
    def forward(ctx, xyz: Tensor, centres: Tensor, features: Tensor | None, idx: Tensor) -> Tensor:
        B, N, _ = xyz.shape
        M, S = idx.shape[1], idx.shape[2]
        C = 0 if features is None else features.shape[1]
        index, bits = _index_arg(idx)
        out = torch.empty((B, 3 + C, M, S), dtype=torch.float32, device=xyz.device)
        feats = None if features is None else features.contiguous()
        if out.numel():
            _native.call("pointops_group_points_rel", xyz.contiguous().data_ptr(),
                         centres.contiguous().data_ptr(),
                         None if feats is None else feats.data_ptr(), index.data_ptr(), bits,
                         out.data_ptr(), B, C, N, M, S, _native.stream(xyz.device))
        ctx.save_for_backward(index)
        ctx.bits, ctx.n, ctx.c = bits, N, C
        return out

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_out: Tensor | None):
        if grad_out is None:
            return None, None, None, None
        (index,) = ctx.saved_tensors
        B, _, M, S = grad_out.shape
        P, N, C = M * S, ctx.n, ctx.c
        g = grad_out.contiguous()
        stride = (3 + C) * P
        g_xyz = g_centres = g_feat = None
        if ctx.needs_input_grad[0]:
            g_xyz = _scatter_back(g, stride, index, ctx.bits, 3, N, P).transpose(1, 2).contiguous()
        if ctx.needs_input_grad[1]:
            g_centres = -g[:, :3].sum(dim=-1).transpose(1, 2).contiguous()
        if C and ctx.needs_input_grad[2]:
            g_feat = _scatter_back(g[:, 3:], stride, index, ctx.bits, C, N, P)
        return g_xyz, g_centres, g_feat, None


def query_and_group(xyz: Tensor, centres: Tensor, features: Tensor | None, idx: Tensor,
                    check: bool = True) -> Tensor:
    """Grouped ``xyz - centre`` and grouped features for ``(B, M, S)`` indices:
    ``(B, N, 3)``, ``(B, M, 3)``, ``(B, C, N)`` or None -> ``(B, 3+C, M, S)``.

    The same values as ``cat([grouping_operation(xyz^T, idx) - centres^T[..., None],
    grouping_operation(features, idx)], 1)`` (tests/test_pointnet2_e2e.py:41-44).
    """
    if xyz.ndim != 3 or xyz.shape[-1] != 3 or centres.ndim != 3 or centres.shape[-1] != 3:
        raise ValueError("xyz and centres must have shape (B, N, 3) and (B, M, 3)")
    if idx.ndim != 3 or idx.shape[:2] != centres.shape[:2] or xyz.shape[0] != idx.shape[0]:
        raise ValueError("indices must have shape (B, M, S) matching the centres")
    if features is not None and (features.ndim != 3 or features.shape[0] != xyz.shape[0]
                                 or features.shape[2] != xyz.shape[1]):
        raise ValueError("features must have shape (B, C, N) matching xyz")
    tensors = [xyz, centres] + ([] if features is None else [features])
    if xyz.device.type != "cuda" or any(t.dtype != torch.float32 for t in tensors):
        B, M, S = idx.shape
        flat = idx.long().reshape(B, 1, M * S)
        gx = xyz.transpose(1, 2).gather(2, flat.expand(B, 3, -1)).reshape(B, 3, M, S)
        parts = [gx - centres.transpose(1, 2).unsqueeze(-1)]
        if features is not None:
            C = features.shape[1]
            parts.append(features.gather(2, flat.expand(B, C, -1)).reshape(B, C, M, S))
        return torch.cat(parts, dim=1)
    if any(t.device != xyz.device for t in tensors + [idx]):
        raise ValueError("all inputs must be on the same device")
    if xyz.shape[1] > _MAX_INDEX:
        raise ValueError("at most 2**31-1 points")
    if check:
        _check_range(idx, xyz.shape[1])
    return _GroupPointsRel.apply(xyz, centres, features, idx)


class QueryAndGroup(nn.Module):
    """``pointnet2_ops.pointnet2_utils.QueryAndGroup``: ball query (first
    ``nsample`` in index order, pointnet2_ops padding) then grouping, as
    ``(B, 3+C, npoint, nsample)`` (xyz relative to the centre first when
    ``use_xyz``)."""

    def __init__(self, radius: float, nsample: int, use_xyz: bool = True):
        super().__init__()
        self.radius, self.nsample, self.use_xyz = radius, nsample, use_xyz

    def forward(self, xyz: Tensor, new_xyz: Tensor, features: Tensor | None = None) -> Tensor:
        from . import compat

        idx = compat.ball_query(self.radius, self.nsample, xyz, new_xyz)
        if not self.use_xyz:
            if features is None:
                raise ValueError("use_xyz=False needs features")
            B, M, S = idx.shape
            return group_points(features, idx.reshape(B, M * S), check=False).reshape(
                B, features.shape[1], M, S)
        return query_and_group(xyz, new_xyz, features, idx, check=False)


class GroupAll(nn.Module):
    """``pointnet2_ops.pointnet2_utils.GroupAll``: every point in one group,
    ``(B, 3+C, 1, N)`` (absolute xyz first when ``use_xyz``)."""

    def __init__(self, use_xyz: bool = True):
        super().__init__()
        self.use_xyz = use_xyz

    def forward(self, xyz: Tensor, new_xyz: Tensor | None = None,
                features: Tensor | None = None) -> Tensor:
        grouped_xyz = xyz.transpose(1, 2).unsqueeze(2)
        if features is None:
            return grouped_xyz
        grouped = features.unsqueeze(2)
        return torch.cat([grouped_xyz, grouped], dim=1) if self.use_xyz else grouped
