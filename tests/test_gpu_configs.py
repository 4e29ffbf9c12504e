"""GPU parity at the full sizes of the large configurations (3, 4 and 5).

The oracle (multi-threaded C) runs the same inputs on the host; where its
cost would be quadratic in the full size (config 4's 131072 x 1M kNN) a fixed
subset of rows is compared, every row of which is computed by the GPU in the
same full-size launch.  Indices are bit-exact, distances bit-identical,
Chamfer loss within 1e-5 relative and gradients within 1e-4 relative.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import bench
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def host(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy()


def same_bits(a, b):
    a = np.ascontiguousarray(np.asarray(a, np.float32))
    b = np.ascontiguousarray(np.asarray(b, np.float32))
    np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.fixture(scope="module")
def c3():
    return bench.make_c3()


def test_c3_large_fps_full(cuda_device, c3):
    """1,048,576-point slab -> 16384 samples, persistent all-CU kernel."""
    import mps_pointops as mp

    got = mp.furthest_point_sample(c3.cuda(), 16384)
    want = O.fps(c3, 16384)
    np.testing.assert_array_equal(host(got), want)


def test_c3_ball_query_from_samples_full(cuda_device, c3):
    import mps_pointops as mp

    samples = c3.gather(1, torch.from_numpy(O.fps(c3, 16384))[..., None].expand(-1, -1, 3))
    want_d, want_i = O.ball_query(samples, c3, 0.5, 32)
    d, i = mp.ball_query(samples.contiguous().cuda(), c3.cuda(), 0.5, 32)
    np.testing.assert_array_equal(host(i), want_i)
    same_bits(host(d), want_d)


def test_c4_knn_at_scale_rows(cuda_device):
    """131072 queries x 1,048,576 references, K=16, in one launch; every
    32nd query row is checked against the oracle."""
    import mps_pointops as mp

    ref, query, _ = bench.make_c4()
    d, i = mp.knn(query.cuda(), ref.cuda(), 16)
    rows = torch.arange(0, query.shape[1], 32)
    want_d, want_i = O.knn3(query[:, rows].contiguous(), ref, 16)
    np.testing.assert_array_equal(host(i)[:, rows.numpy()], want_i)
    same_bits(host(d)[:, rows.numpy()], want_d)


def test_c4_clustered_knn_rows(cuda_device):
    """Config 4's sizes on clustered references queried uniformly (almost
    every query goes to the pruned linear pass): every 64th row against the
    oracle, and every row against the brute-force kernel of the same
    launch sizes."""
    import mps_pointops as mp
    from mps_pointops import _native

    ref, query = bench.make_c4_clustered()
    qd, rd = query.cuda(), ref.cuda()
    d, i = mp.knn(qd, rd, 16)
    rows = torch.arange(0, query.shape[1], 64)
    want_d, want_i = O.knn3(query[:, rows].contiguous(), ref, 16)
    np.testing.assert_array_equal(host(i)[:, rows.numpy()], want_i)
    same_bits(host(d)[:, rows.numpy()], want_d)
    bd, bi = torch.empty_like(d), torch.empty_like(i)
    _native.call("pointops_knn3", qd.data_ptr(), rd.data_ptr(), bd.data_ptr(), bi.data_ptr(),
                 1, query.shape[1], ref.shape[1], 16, _native.stream(qd.device))
    assert torch.equal(i, bi)
    same_bits(host(d), host(bd))


def test_c4_dgcnn_feature_knn_full(cuda_device):
    """DGCNN feature-space kNN: (8, 2048, 64), query is ref (self included)."""
    import mps_pointops as mp

    _, _, feat = bench.make_c4()
    d, i = mp.knn(feat.cuda(), feat.cuda(), 20)
    want_d, want_i = O.knn_feat(feat, feat, 20)
    np.testing.assert_array_equal(host(i), want_i)
    same_bits(host(d), want_d)


def test_dgcnn_feature_knn_d128(cuda_device):
    """DGCNN's deeper layer width: (2, 2048, 128), K = 20, query is ref."""
    import mps_pointops as mp

    feat = torch.randn(2, 2048, 128, generator=torch.Generator().manual_seed(44))
    d, i = mp.knn(feat.cuda(), feat.cuda(), 20)
    want_d, want_i = O.knn_feat(feat, feat, 20)
    np.testing.assert_array_equal(host(i), want_i)
    same_bits(host(d), want_d)


def test_c5_chamfer_forward_backward_full(cuda_device):
    """B=32, P1=P2=8192, mean/mean: loss and both gradients against the
    closed form on the oracle's nearest pairs."""
    import mps_pointops as mp

    y1, y2 = bench.make_c5()
    a = y1.cuda().requires_grad_()
    b = y2.cuda().requires_grad_()
    loss, _ = mp.chamfer_distance(a, b)
    loss.backward()
    d12, i12 = O.chamfer_nearest(y1, y2)
    d21, i21 = O.chamfer_nearest(y2, y1)
    want_loss = (d12.astype(np.float64).mean(1) + d21.astype(np.float64).mean(1)).mean()
    np.testing.assert_allclose(loss.item(), want_loss, rtol=1e-5)
    B, P, _ = y1.shape
    g = 1.0 / (B * P)
    ga = np.zeros((B, P, 3))
    gb = np.zeros((B, P, 3))
    y1n, y2n = y1.numpy().astype(np.float64), y2.numpy().astype(np.float64)
    for bb in range(B):
        diff = y1n[bb] - y2n[bb, i12[bb]]
        ga[bb] += 2 * g * diff
        np.add.at(gb[bb], i12[bb], -2 * g * diff)
        diff = y2n[bb] - y1n[bb, i21[bb]]
        gb[bb] += 2 * g * diff
        np.add.at(ga[bb], i21[bb], -2 * g * diff)
    np.testing.assert_allclose(host(a.grad), ga, rtol=1e-4, atol=1e-9)
    np.testing.assert_allclose(host(b.grad), gb, rtol=1e-4, atol=1e-9)
