"""PyTorch-CPU port of the reference's CPU algorithms, used ONLY as the CPU
baseline that bench.py times beside the GPU (cpu_baseline.kind = "port").

TEST INFRASTRUCTURE ONLY: the shipped package never imports this module.
Each function restates /root/reference/mps_pointops/reference.py:
furthest_point_sample (:27-58), knn (:61-80, cdist + topk, the reference's
own CPU kNN) and ball_query (:83-121, chunks of at most 2**24 pairs); and
the squared-L2 Chamfer loss of /root/reference/mps_pointops/chamfer.py on
CPU tensors: first nearest neighbour by tiles of coordinate differences
(_nearest_indices, :162-230), the selected squared distance with autograd
(_selected_squared_distance, :297-308), mean over points and batch.
"""

from __future__ import annotations

import torch
from torch import Tensor

PAIRS_PER_CHUNK = 1 << 24


def _sqdist(a: Tensor, b: Tensor) -> Tensor:
    d = a - b
    return (d[..., 0] * d[..., 0] + d[..., 1] * d[..., 1]) + d[..., 2] * d[..., 2]


def furthest_point_sample(xyz: Tensor, npoint: int, start_idx: int = 0) -> Tensor:
    B, N, _ = xyz.shape
    idx = torch.empty(B, npoint, dtype=torch.long)
    min_d2 = torch.full((B, N), float("inf"), dtype=xyz.dtype)
    farthest = torch.full((B,), start_idx, dtype=torch.long)
    batch = torch.arange(B)
    for i in range(npoint):
        idx[:, i] = farthest
        centroid = xyz[batch, farthest].unsqueeze(1)
        min_d2 = torch.minimum(min_d2, _sqdist(xyz, centroid))
        farthest = min_d2.argmax(-1)
    return idx


def knn(query: Tensor, ref: Tensor, k: int) -> tuple[Tensor, Tensor]:
    return torch.cdist(query, ref).topk(k, dim=-1, largest=False, sorted=True)


def ball_query(query: Tensor, ref: Tensor, radius: float, K: int) -> tuple[Tensor, Tensor]:
    B, M, _ = query.shape
    N = ref.shape[1]
    r32 = torch.tensor(radius, dtype=torch.float32)
    r2 = (r32 * r32).item()
    kk = min(K, N)
    idx = torch.full((B, M, K), -1, dtype=torch.long)
    dist2 = torch.zeros(B, M, K, dtype=query.dtype)
    if kk == 0 or M == 0:
        return dist2, idx
    order = torch.arange(N)
    step = max(1, PAIRS_PER_CHUNK // max(1, B * N))
    for lo in range(0, M, step):
        d2 = _sqdist(query[:, lo:lo + step, None, :], ref[:, None, :, :])
        cand = torch.where(d2 < r2, order, N)
        first = cand.topk(kk, dim=-1, largest=False, sorted=True).values
        valid = first < N
        idx[:, lo:lo + step, :kk] = torch.where(valid, first, -1)
        dist2[:, lo:lo + step, :kk] = torch.where(valid, d2.gather(-1, first.clamp(max=N - 1)), 0.0)
    return dist2, idx


def nearest_indices(query: Tensor, ref: Tensor, tile: int = 1 << 22) -> Tensor:
    """First minimum of the coordinate-difference squared distance (B, M)."""
    B, M, _ = query.shape
    N = ref.shape[1]
    q_step = max(1, min(M, tile // max(1, B * N)))
    out = torch.empty(B, M, dtype=torch.long)
    for q0 in range(0, M, q_step):
        d2 = _sqdist(query[:, q0:q0 + q_step, None, :], ref[:, None, :, :])
        out[:, q0:q0 + q_step] = d2.argmin(-1)  # first minimum
    return out


def chamfer_l2(x: Tensor, y: Tensor) -> Tensor:
    """Mean/mean squared-L2 Chamfer loss of equal-length clouds, both
    directions, differentiable in x and y."""
    def directed(a: Tensor, b: Tensor) -> Tensor:
        with torch.no_grad():
            ia = nearest_indices(a, b)
        near = b.gather(1, ia[..., None].expand(-1, -1, 3))
        return _sqdist(a, near).mean(dim=1)
    return (directed(x, y) + directed(y, x)).mean()
