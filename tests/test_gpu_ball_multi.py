"""GPU parity of the multi-radius ball query (pointops_ball_query_multi_f32):
every radius's output equals the single-radius query's bit for bit, and the
single-radius query is pinned to the oracle (reference.py:83-121 semantics)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import bench
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def host(t) -> np.ndarray:
    return t.detach().cpu().numpy() if isinstance(t, torch.Tensor) else np.asarray(t)


def same_bits(a, b):
    a = np.ascontiguousarray(np.asarray(a, np.float32))
    b = np.ascontiguousarray(np.asarray(b, np.float32))
    np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))


def _check(query, ref, radii, ks, against_oracle=False):
    import mps_pointops as mp

    qg, rg = query.cuda(), ref.cuda()
    print(f"ball_query_multi B={query.shape[0]} Q={query.shape[1]} P={ref.shape[1]} "
          f"radii={radii} ks={ks}", flush=True)
    outs = mp.ball_query_multi(qg, rg, radii, ks)
    assert len(outs) == len(radii)
    for (d, i), r, k in zip(outs, radii, ks):
        want_d, want_i = mp.ball_query(qg, rg, r, k)
        np.testing.assert_array_equal(host(i), host(want_i))
        same_bits(host(d), host(want_d))
        if against_oracle:
            od, oi = O.ball_query(query, ref, r, k)
            np.testing.assert_array_equal(host(i), oi)
            same_bits(host(d), od)


def test_config2_three_radii(cuda_device):
    """The benchmark's three radii around FPS-like centres of config 2."""
    x = bench.make_c2(B=4)
    g = torch.Generator().manual_seed(5)
    centres = x[:, torch.randperm(4096, generator=g)[:1024]].contiguous()
    _check(centres, x, [0.1, 0.2, 0.4], [16, 32, 128], against_oracle=True)


@pytest.mark.parametrize("radii,ks", [
    ([0.05, 0.1, 0.2, 0.3, 0.5], [8, 16, 32, 64, 100]),   # two scans (4 + 1 radii)
    ([0.3, 0.3, 0.1], [5, 40, 1]),                         # equal radii, different K
    ([0.2, 0.0, 0.4], [8, 8, 8]),                          # radius 0 matches nothing
    ([0.2, 0.4], [0, 12]),                                 # K = 0 writes nothing
    ([10.0, 0.1, 0.2, 0.3, 0.4, 0.5, 0.6, 0.7], [3] * 8),  # eight radii; everything in range
    ([0.15], [300]),                                       # K above the points in reach
])
def test_radius_sets(cuda_device, radii, ks):
    g = torch.Generator().manual_seed(len(radii) * 100 + sum(ks))
    ref = torch.rand(3, 2500, 3, generator=g)
    query = torch.rand(3, 333, 3, generator=g)
    _check(query, ref, radii, ks)


def test_ragged_and_tiny_sizes(cuda_device):
    g = torch.Generator().manual_seed(11)
    for B, Q, P in ((1, 1, 1), (2, 3, 5), (5, 67, 130), (1, 9, 4097)):
        ref = torch.rand(B, P, 3, generator=g)
        query = torch.rand(B, Q, 3, generator=g)
        _check(query, ref, [0.2, 0.5, 0.9], [2, 7, 64])


def test_non_finite_points_and_queries(cuda_device):
    g = torch.Generator().manual_seed(12)
    ref = torch.rand(2, 3000, 3, generator=g)
    ref[0, 5] = float("nan")
    ref[0, 9, 1] = float("inf")
    ref[1, :2990] = float("nan")
    query = torch.rand(2, 200, 3, generator=g)
    query[0, 3] = float("nan")
    query[1, 7, 2] = -float("inf")
    _check(query, ref, [0.1, 0.3, 1.0], [4, 16, 32], against_oracle=True)


def test_duplicates_and_empty_cloud_rows(cuda_device):
    """Many points at one position (every hit at the same distance) and
    queries far from everything."""
    ref = torch.full((1, 1000, 3), 0.5)
    query = torch.cat([torch.full((1, 10, 3), 0.5), torch.full((1, 10, 3), 9.0)], 1)
    _check(query, ref, [0.01, 0.5, 20.0], [3, 64, 200], against_oracle=True)
