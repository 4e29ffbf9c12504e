"""PointNet++ three-neighbour search and weighted feature propagation on ROCm
(signatures, validation and autograd of /root/reference/mps_pointops/pointnet2.py).
"""

from __future__ import annotations

import torch
from torch import Tensor
from torch.autograd.function import once_differentiable

from . import _native

_MAX_INDEX = (1 << 31) - 1
# The deterministic CSR backward covers up to this many known / unknown points.
_CSR_MAX_KNOWN = 4096
_CSR_MAX_UNKNOWN = 4096


def _validate_three_nn(unknown: Tensor, known: Tensor) -> tuple[int, int, int]:
    """pointnet2.py:30-51."""
    if not isinstance(unknown, Tensor) or not isinstance(known, Tensor):
        raise TypeError("unknown and known must be tensors")
    if unknown.ndim != 3 or unknown.shape[-1] != 3:
        raise ValueError("unknown must have shape (B, N, 3)")
    if known.ndim != 3 or known.shape[-1] != 3:
        raise ValueError("known must have shape (B, M, 3)")
    if unknown.shape[0] != known.shape[0]:
        raise ValueError("unknown and known must have the same batch size")
    if unknown.device != known.device:
        raise ValueError("unknown and known must be on the same device")
    if unknown.dtype != torch.float32 or known.dtype != torch.float32:
        raise TypeError("unknown and known must be float32")
    batch, queries, _ = unknown.shape
    points = known.shape[1]
    if batch and queries and points < 3:
        raise ValueError("three_nn needs at least 3 known points for nonempty queries")
    if points > _MAX_INDEX:
        raise ValueError("three_nn supports at most 2**31-1 known points")
    if batch * queries > (1 << 32) - 1:
        raise ValueError("three_nn query count exceeds the native index range")
    return batch, queries, points


def three_nn(unknown: Tensor, known: Tensor) -> tuple[Tensor, Tensor]:
    """Return the three nearest known points for every unknown point.

    ``unknown`` is ``(B, N, 3)`` and ``known`` is ``(B, M, 3)`` float32, with
    ``M >= 3`` whenever ``B*N > 0``.  Returns Euclidean distances ``(B, N, 3)``
    in float32 and known indices ``(B, N, 3)`` in int32.  Equal squared
    distances prefer the smaller known index.  As in PointNet++, selection and
    distances carry no coordinate gradient (pointnet2.py:75-100).
    """
    batch, queries, points = _validate_three_nn(unknown, known)
    _native.require_device(unknown.device)
    distances = torch.empty((batch, queries, 3), dtype=torch.float32, device=unknown.device)
    indices = torch.empty((batch, queries, 3), dtype=torch.int32, device=unknown.device)
    if batch * queries:
        _native.call("pointops_three_nn", unknown.contiguous().data_ptr(),
                     known.contiguous().data_ptr(), distances.data_ptr(), indices.data_ptr(),
                     batch, queries, points, _native.stream(unknown.device))
    return distances, indices


def _validate_interpolate(features: Tensor, indices: Tensor, weights: Tensor):
    """pointnet2.py:103-132 (one device-to-host sync for the index bounds)."""
    if not all(isinstance(t, Tensor) for t in (features, indices, weights)):
        raise TypeError("features, indices, and weights must be tensors")
    if features.ndim != 3:
        raise ValueError("features must have shape (B, C, M)")
    if indices.ndim != 3 or indices.shape[-1] != 3:
        raise ValueError("indices must have shape (B, N, 3)")
    if weights.shape != indices.shape:
        raise ValueError("weights must have the same (B, N, 3) shape as indices")
    if features.shape[0] != indices.shape[0]:
        raise ValueError("features and indices must have the same batch size")
    if features.device != indices.device or features.device != weights.device:
        raise ValueError("features, indices, and weights must be on the same device")
    if features.dtype != torch.float32 or weights.dtype != torch.float32:
        raise TypeError("features and weights must be float32")
    if indices.dtype not in (torch.int32, torch.int64):
        raise TypeError("indices must be int32 or int64")
    batch, channels, points = features.shape
    queries = indices.shape[1]
    if batch and queries and points == 0:
        raise ValueError("nonempty interpolation requires at least one source point")
    if points > _MAX_INDEX:
        raise ValueError("three_interpolate supports at most 2**31-1 source points")
    if batch * channels * queries > (1 << 32) - 1:
        raise ValueError("three_interpolate output exceeds the native index range")
    if indices.numel() and torch.any((indices < 0) | (indices >= points)).item():
        raise IndexError(f"indices must lie in [0, {points})")
    return batch, channels, points, queries


def _csr_eligible(points: int, queries: int, batch: int) -> bool:
    """Shapes the CSR backward serves (pointops_three_interpolate_backward_csr)."""
    return (0 < points <= _CSR_MAX_KNOWN and 0 < queries <= _CSR_MAX_UNKNOWN
            and queries % 4 == 0 and batch <= 65535)


class _ThreeInterpolate(torch.autograd.Function):
    """Native forward and backward; zero weight gradient
    (pointnet2.py:150-188)."""

    @staticmethod
    def forward(ctx, features: Tensor, indices: Tensor, weights: Tensor) -> Tensor:
        batch, channels, points = features.shape
        queries = indices.shape[1]
        output = torch.empty((batch, channels, queries), dtype=torch.float32,
                             device=features.device)
        stream = _native.stream(features.device)
        if output.numel():
            _native.call("pointops_three_interpolate", features.contiguous().data_ptr(),
                         indices.data_ptr(), weights.data_ptr(), output.data_ptr(),
                         batch, channels, points, queries, stream)
        ctx.save_for_backward(indices, weights)
        ctx.points = points
        ctx.channels = channels
        # The backward's CSR of the entries depends only on the indices and
        # weights: built here, behind the forward on the same stream, so the
        # backward only gathers.
        ctx.csr = None
        if ctx.needs_input_grad[0] and batch * channels and _csr_eligible(points, queries, batch):
            size = _native.size_query("pointops_three_interpolate_backward_workspace_bytes",
                                      batch, points, queries)
            ctx.csr = torch.empty(size, dtype=torch.uint8, device=features.device)
            _native.call("pointops_three_interpolate_csr_build", indices.data_ptr(),
                         weights.data_ptr(), ctx.csr.data_ptr(), batch, points, queries, stream)
        return output

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_output: Tensor | None):
        if grad_output is None:
            return None, None, None
        indices, weights = ctx.saved_tensors
        batch, queries, _ = indices.shape
        grad_features = None
        if ctx.needs_input_grad[0]:
            shape = (batch, ctx.channels, ctx.points)
            stream = _native.stream(indices.device)
            if _csr_eligible(ctx.points, queries, batch):
                # Deterministic gather over the CSR the forward built; writes
                # every element, so no zero fill.
                grad_features = torch.empty(shape, device=indices.device, dtype=torch.float32)
                if batch * ctx.channels:
                    _native.call("pointops_three_interpolate_backward_from_csr",
                                 grad_output.contiguous().data_ptr(), ctx.csr.data_ptr(),
                                 grad_features.data_ptr(), batch, ctx.channels, ctx.points,
                                 queries, stream)
            else:
                grad_features = torch.zeros(shape, device=indices.device, dtype=torch.float32)
                if batch * ctx.channels * queries:
                    _native.call("pointops_three_interpolate_backward",
                                 grad_output.contiguous().data_ptr(), indices.data_ptr(),
                                 weights.data_ptr(), grad_features.data_ptr(), batch,
                                 ctx.channels, ctx.points, queries, stream)
        grad_weights = torch.zeros_like(weights) if ctx.needs_input_grad[2] else None
        return grad_features, None, grad_weights


def three_interpolate(features: Tensor, indices: Tensor, weights: Tensor) -> Tensor:
    """Interpolate ``(B,C,M)`` features at ``(B,N,3)`` source indices.

    ``out[b,c,n] = (features[b,c,i0]*w0 + features[b,c,i1]*w1) + features[b,c,i2]*w2``.
    Backward accumulates ``grad_out * w`` at the selected source positions
    in (n, t) order, deterministic, for up to 4096 sources and 4096 queries
    (a multiple of 4)
    (beyond that by hardware float atomics, whose order sets the last bits); the weight
    gradient is an explicit zero tensor, as in the original PointNet++ wrapper
    (pointnet2.py:191-211).
    """
    _validate_interpolate(features, indices, weights)
    _native.require_device(features.device)
    index32 = indices.contiguous() if indices.dtype == torch.int32 else indices.to(torch.int32)
    return _ThreeInterpolate.apply(features, index32, weights.contiguous())


__all__ = ["three_nn", "three_interpolate"]
