"""Host-side checks that need no GPU: the C ABI library, argument validation,
error behaviour of the public API, torch_cluster count rules, compat install,
and the CPU-baseline port."""

from __future__ import annotations

import ctypes
import math
import re
import sys

import numpy as np
import pytest
import torch

from conftest import ROOT
from oracle import oracle as O

HEADER = ROOT / "include" / "pointops_hip.h"


def declared_symbols() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(pointops_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    from mps_pointops import _native

    lib = _native.library()
    names = declared_symbols()
    assert len(names) >= 20
    for name in names:
        assert hasattr(lib, name), name
    assert lib.pointops_abi_version() == 1


def test_header_and_binding_agree():
    from mps_pointops import _native

    bound = set(_native._SIGNATURES) | set(_native._SIZE_QUERIES) | {
        "pointops_abi_version", "pointops_device_supported"}
    assert bound == set(declared_symbols())


def test_capi_rejects_bad_arguments_before_any_launch():
    """Argument errors return hipErrorInvalidValue (1) without touching a
    device; empty work returns hipSuccess (0)."""
    from mps_pointops import _native

    lib = _native.library()
    assert lib.pointops_knn3(None, None, None, None, 1, 1, 300, 257, None) == 1  # K > 256
    assert lib.pointops_knn3(None, None, None, None, 1, 1, 10, 11, None) == 1   # K > N
    assert lib.pointops_knn3(None, None, None, None, 0, 5, 10, 3, None) == 0    # B == 0
    assert lib.pointops_knn_feat(None, None, None, None, 1, 1, 10, 0, 3, None) == 1  # D == 0
    assert lib.pointops_fps_dense(None, None, None, 1, 10, 4, 10, 0, None) == 1  # start >= N
    assert lib.pointops_fps_dense(None, None, None, 2, 0, 0, 0, 0, None) == 0    # npoint == 0
    assert lib.pointops_fps_large(None, None, None, 1 << 32, 4, 0, 0, None) == 1
    assert lib.pointops_three_nn(None, None, None, None, 1, 5, 2, None) == 1     # M < 3
    assert lib.pointops_ball_query_f32(None, None, None, None, None, None, 1, 1, 1, -1,
                                       ctypes.c_float(1.0), None) == 1
    assert lib.pointops_chamfer_nearest_f32(None, None, None, None, None, None, 1, 1, 1, 3, 3,
                                            None) == 1  # norm 3
    assert lib.pointops_three_interpolate(None, None, None, None, 1, 2, 0, 4, None) == 1  # M == 0


def test_ball_query_multi_rejects_bad_arguments():
    """The multi-radius entry checks every radius before any launch: at most
    8 radii, K in [0, 2^31), an output pair for each radius with K >= 1;
    empty work succeeds."""
    from mps_pointops import _native

    lib = _native.library()
    r2 = (ctypes.c_float * 9)(*([0.01] * 9))
    ks = (ctypes.c_int64 * 9)(*([4] * 9))
    ptrs = (ctypes.c_void_p * 9)(*([8] * 9))
    nul = (ctypes.c_void_p * 9)()
    f = lib.pointops_ball_query_multi_f32
    assert f(None, None, 9, r2, ks, ptrs, ptrs, 1, 1, 1, None) == 1            # > 8 radii
    assert f(None, None, 2, None, ks, ptrs, ptrs, 1, 1, 1, None) == 1          # no radii array
    assert f(None, None, 2, r2, ks, nul, ptrs, 1, 1, 1, None) == 1             # no idx output
    bad = (ctypes.c_int64 * 2)(4, -1)
    assert f(None, None, 2, r2, bad, ptrs, ptrs, 1, 1, 1, None) == 1           # K < 0
    big = (ctypes.c_int64 * 1)(1 << 31)
    assert f(None, None, 1, r2, big, ptrs, ptrs, 1, 1, 1, None) == 1           # K >= 2^31
    assert f(None, None, 2, r2, ks, ptrs, ptrs, 0, 5, 5, None) == 0            # B == 0
    assert f(None, None, 2, r2, ks, ptrs, ptrs, 3, 0, 5, None) == 0            # Q == 0
    assert f(None, None, 2, r2, ks, ptrs, ptrs, 65536, 1, 5, None) == 1        # B > 65535
    zero = (ctypes.c_int64 * 2)(0, 0)
    assert f(None, None, 2, r2, zero, nul, nul, 2, 3, 5, None) == 1            # no coordinates


def test_ball_query_multi_python_validation():
    import mps_pointops as mp

    q, r = torch.zeros(1, 4, 3), torch.zeros(1, 8, 3)
    with pytest.raises(ValueError, match="same length"):
        mp.ball_query_multi(q, r, [0.1, 0.2], [4])
    with pytest.raises(ValueError, match="at most 8"):
        mp.ball_query_multi(q, r, [0.1] * 9, [4] * 9)
    with pytest.raises(ValueError, match="radius"):
        mp.ball_query_multi(q, r, [-1.0], [4])
    with pytest.raises(ValueError, match="shapes"):
        mp.ball_query_multi(q[..., :2], r, [0.1], [4])
    with pytest.raises(TypeError, match="float32"):
        mp.ball_query_multi(q.double(), r.double(), [0.1], [4])
    with pytest.raises(ValueError, match="ROCm"):
        mp.ball_query_multi(q, r, [0.1], [4])  # CPU tensors are not computed


def test_scratch_size_queries():
    from mps_pointops import _native

    assert _native.size_query("pointops_fps_dense_scratch_bytes", 32, 4096) == 0
    assert _native.size_query("pointops_fps_dense_scratch_bytes", 2, 100_000) == 2 * 100_000 * 4
    assert _native.size_query("pointops_fps_flat_scratch_bytes", 50_000, 9000) == 50_000 * 4
    assert _native.size_query("pointops_fps_large_workspace_bytes", 1 << 20, 16384) > 0
    # Above 2^21 points the running distances live in the workspace too.
    small = _native.size_query("pointops_fps_large_workspace_bytes", 1 << 21, 16)
    assert _native.size_query("pointops_fps_large_workspace_bytes", 3 << 20, 16) == small + (3 << 22)


# ------------------------------------------------------------ public API

def test_cpu_tensors_are_rejected_not_computed():
    """No CPU fallback: host tensors raise instead of silently running."""
    import mps_pointops as mp

    x = torch.rand(1, 10, 3)
    with pytest.raises(ValueError, match="cuda"):
        mp.furthest_point_sample(x, 4)
    with pytest.raises(ValueError, match="cuda"):
        mp.knn(x, x, 3)
    with pytest.raises(ValueError, match="cuda"):
        mp.ball_query(x, x, 0.5, 3)
    with pytest.raises(ValueError, match="cuda"):
        mp.three_nn(x, x)
    with pytest.raises(ValueError, match="cuda"):
        mp.chamfer_distance(x, x)
    with pytest.raises(ValueError, match="cuda"):
        mp.flat.fps(x[0])


def test_fps_validation_order():
    """ops.py:84-100: shape/strategy/npoint/start checks before dispatch."""
    import mps_pointops as mp

    with pytest.raises(ValueError):
        mp.furthest_point_sample(torch.randn(10, 3), 4)
    with pytest.raises(ValueError, match="strategy"):
        mp.furthest_point_sample(torch.randn(1, 8, 3), 2, strategy="unknown")
    with pytest.raises(ValueError):
        mp.furthest_point_sample(torch.randn(1, 0, 3), 4)
    with pytest.raises(IndexError):
        mp.furthest_point_sample(torch.randn(1, 10, 3), 4, start_idx=10)
    with pytest.raises(ValueError, match="npoint"):
        mp.furthest_point_sample(torch.randn(1, 10, 3), -1)


def test_knn_validation_order():
    import mps_pointops as mp

    ref = torch.randn(1, 300, 3)
    with pytest.raises(ValueError):
        mp.knn(ref, ref, 301)
    with pytest.raises(ValueError, match="batch"):
        mp.knn(ref, torch.randn(2, 300, 3), 4)
    with pytest.raises(ValueError, match="ref must have shape"):
        mp.knn(torch.zeros(1, 5, 64), torch.zeros(1, 5, 128), 2)
    with pytest.raises(ValueError, match="D >= 1"):
        mp.knn(torch.zeros(1, 5, 0), torch.zeros(1, 5, 0), 0)


@pytest.mark.parametrize("radius", [-0.1, float("inf"), float("nan"), 1e-40, 1e39, True])
def test_ball_query_rejects_bad_radius(radius):
    """tests/test_ball_query_api.py:37-42: the same radius rules everywhere."""
    import mps_pointops as mp

    xyz = torch.rand(1, 20, 3)
    with pytest.raises(ValueError):
        mp.ball_query(xyz[:, :4], xyz, radius, 4)


@pytest.mark.parametrize("K", [-1, 1.5, True])
def test_ball_query_rejects_bad_k(K):
    import mps_pointops as mp

    xyz = torch.rand(1, 20, 3)
    with pytest.raises(ValueError):
        mp.ball_query(xyz[:, :4], xyz, 0.5, K)


def test_checked_radius_and_k_rules():
    """_ball_query_mps.py:87-119 and tests/test_ball_query_mps.py:596-618."""
    from mps_pointops._ball_query_mps import _checked_radius_and_k

    assert _checked_radius_and_k(0.1, 1)[1] == O.ball_radius_sq(0.1)
    assert _checked_radius_and_k(1e20, 1)[1] == math.inf
    assert _checked_radius_and_k(0.0, 0) == (0.0, 0.0)
    minimum = 2.0 ** -112
    assert _checked_radius_and_k(minimum, 1)[0] == minimum
    below = float(np.nextafter(np.float32(minimum), np.float32(0)))
    with pytest.raises(ValueError, match="2\\*\\*-112"):
        _checked_radius_and_k(below, 1)
    with pytest.raises(ValueError, match="float32"):
        _checked_radius_and_k(1e-100, 1)
    with pytest.raises(ValueError, match="normal float32"):
        _checked_radius_and_k(1e-40, 1)
    with pytest.raises(ValueError, match="radius"):
        _checked_radius_and_k(10 ** 1000, 1)
    with pytest.raises(ValueError, match="radius"):
        _checked_radius_and_k(torch.tensor(1.0), 1)
    with pytest.raises(ValueError, match="k"):
        _checked_radius_and_k(1.0, 1 << 63)
    # torch_cluster's threshold differs by one ulp at r=0.21 and r=0.1
    # (tests/test_flat.py:207-224).
    from mps_pointops.flat import _radius_sq_torch_cluster

    r21 = np.float32(0.21)
    assert np.float32(r21 * r21) < np.float32(_radius_sq_torch_cluster(0.21))
    r01 = np.float32(0.1)
    assert np.float32(r01 * r01) > np.float32(_radius_sq_torch_cluster(0.1))


def test_pointnet2_validation():
    """tests/test_pointnet2.py:151-165."""
    from mps_pointops import three_interpolate, three_nn

    points = torch.zeros((1, 2, 3))
    with pytest.raises(ValueError, match="at least 3"):
        three_nn(points, points)
    with pytest.raises(TypeError, match="float32"):
        three_nn(points.half(), torch.zeros((1, 3, 3)).half())
    with pytest.raises(ValueError, match="batch"):
        three_nn(points, torch.zeros((2, 3, 3)))
    with pytest.raises(TypeError, match="indices"):
        three_interpolate(torch.zeros((1, 2, 3)), torch.zeros((1, 2, 3)), torch.ones((1, 2, 3)))
    with pytest.raises(ValueError, match="source point"):
        three_interpolate(torch.zeros((1, 2, 0)), torch.zeros((1, 2, 3), dtype=torch.int32),
                          torch.ones((1, 2, 3)))
    with pytest.raises(IndexError):
        three_interpolate(torch.zeros((1, 2, 4)), torch.tensor([[[0, -1, 1]]], dtype=torch.int32),
                          torch.ones((1, 1, 3)))


def test_chamfer_argument_validation():
    """tests/test_chamfer.py:285-304 (argument checks precede device work)."""
    from mps_pointops import chamfer_distance

    x = torch.zeros((1, 2, 3))
    y = torch.ones((1, 2, 3))
    with pytest.raises(ValueError, match="batch_reduction"):
        chamfer_distance(x, y, point_reduction=None)
    with pytest.raises(ValueError, match="1 or 2 norm"):
        chamfer_distance(x, y, norm=3)
    with pytest.raises(ValueError, match="Normals must be None"):
        chamfer_distance(x, y, x_normals=x, point_reduction="max")
    with pytest.raises(ValueError, match="D >= 1"):
        chamfer_distance(torch.empty((1, 2, 0)), torch.empty((1, 2, 0)))


def test_flat_sample_counts_follow_torch_cluster_gpu_rule():
    """tests/test_flat.py:155-204: ceil(deg * ratio) in the ratio's dtype."""
    from mps_pointops.flat import _ratio_tensor, _samples_per_cloud

    for n, ratio, expected in ((25, 0.6, 16), (45, 0.6, 28), (50, 0.3, 16), (90, 0.3, 28),
                               (10, 0.5, 5), (7, 0.5, 4), (9, 1.0, 9)):
        assert _samples_per_cloud([n], _ratio_tensor(ratio, torch.float32)) == [expected]
    # A float64 tensor ratio keeps its dtype on the GPU rule: 15 for 0-D and [1].
    assert _samples_per_cloud([25], _ratio_tensor(torch.tensor(0.6, dtype=torch.float64), torch.float32)) == [15]
    assert _samples_per_cloud([25], _ratio_tensor(torch.tensor([0.6], dtype=torch.float64), torch.float32)) == [15]
    with pytest.raises(ValueError, match="ratio"):
        _ratio_tensor(-0.1, torch.float32)


def test_flat_validation():
    from mps_pointops import flat

    x = torch.tensor([[0., 0, 0], [2., 0, 0], [5., 0, 0], [10., 0, 0], [12., 0, 0]])
    y = torch.tensor([[1., 0, 0], [0., 0, 0]])
    with pytest.raises(NotImplementedError, match="cosine"):
        flat.knn(x, y, 2, cosine=True)
    with pytest.raises(NotImplementedError, match="ignore_same_index"):
        flat.radius(x, y, 1, ignore_same_index=True)
    with pytest.raises(ValueError, match="dimensions differ"):
        flat.knn(torch.zeros(3, 64), torch.zeros(3, 128), 2)


NAMES = ["pointnet2_ops", "pointnet2_ops.pointnet2_utils", "knn_cuda", "torch_cluster"]


@pytest.fixture
def installed():
    from mps_pointops import compat

    saved = {n: sys.modules.pop(n) for n in NAMES if n in sys.modules}
    compat.install(force=True)
    yield compat
    for n in NAMES:
        sys.modules.pop(n, None)
    sys.modules.update(saved)


def test_compat_install_serves_imports(installed):
    """tests/test_compat.py:28-66."""
    compat = installed
    from knn_cuda import KNN
    from pointnet2_ops import pointnet2_utils
    from torch_cluster import fps, knn, knn_graph, radius, radius_graph

    import pointnet2_ops.pointnet2_utils as direct

    assert direct is pointnet2_utils
    assert pointnet2_utils.furthest_point_sample is compat.furthest_point_sample
    assert pointnet2_utils.ball_query is compat.ball_query
    assert KNN is compat.KNN
    assert fps is compat.flat.fps and knn is compat.flat.knn and radius is compat.flat.radius
    assert knn_graph is compat.flat.knn_graph and radius_graph is compat.flat.radius_graph
    marker = object()
    sys.modules["knn_cuda"] = marker
    assert "knn_cuda" not in compat.install()
    assert sys.modules["knn_cuda"] is marker


def test_compat_gather_and_grouping():
    """tests/test_compat.py:121-137 (pure PyTorch gathers, any device)."""
    from mps_pointops import compat

    features = torch.randn(2, 4, 30)
    idx = torch.randint(0, 30, (2, 7), dtype=torch.int32)
    out = compat.gather_operation(features, idx)
    assert out.shape == (2, 4, 7) and torch.equal(out[1, :, 3], features[1, :, idx[1, 3]])
    gidx = torch.randint(0, 30, (2, 7, 5), dtype=torch.int32)
    out = compat.grouping_operation(features, gidx)
    assert out.shape == (2, 4, 7, 5) and torch.equal(out[0, :, 6, 2], features[0, :, gidx[0, 6, 2]])
    f = torch.randn(1, 3, 10, requires_grad=True)
    compat.gather_operation(f, torch.tensor([[2, 2, 5]])).sum().backward()
    assert f.grad[0, 0].tolist() == [0, 0, 2, 0, 0, 1, 0, 0, 0, 0]


def test_bench_rejects_multi_gpu():
    import subprocess

    proc = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                          capture_output=True, text=True, timeout=120)
    assert proc.returncode == 2 and "one" in proc.stdout


# --------------------------------------------------------- CPU baseline

def test_torch_port_matches_oracle():
    """The CPU baseline port restates reference.py: FPS and ball query agree
    with the oracle bit for bit; cdist+topk kNN agrees on distances to
    tolerance (reference.py:61-80 is not exact by design)."""
    from oracle import torch_port

    g = torch.Generator().manual_seed(0)
    x = torch.rand(3, 500, 3, generator=g)
    idx = torch_port.furthest_point_sample(x, 64)
    np.testing.assert_array_equal(idx.numpy(), O.fps(x, 64))
    c = x.gather(1, idx[..., None].expand(-1, -1, 3))
    d, i = torch_port.ball_query(c, x, 0.2, 32)
    od, oi = O.ball_query(c, x, 0.2, 32)
    np.testing.assert_array_equal(i.numpy(), oi)
    np.testing.assert_array_equal(d.numpy(), od)
    d, i = torch_port.knn(c, x, 16)
    od, oi = O.knn3(c, x, 16)
    # cdist may take a matrix-multiply path: self-distances come out ~1e-3
    # instead of 0 (README.md:295-297 documents this inexactness).
    np.testing.assert_allclose(d.numpy(), od, rtol=1e-4, atol=2e-3)


def test_pytorch3d_adapter_argument_errors():
    """tests/test_pytorch3d_adapter.py:121-133: dtype and flag errors come
    before any device work."""
    from mps_pointops.pytorch3d import ball_query

    points = torch.zeros((1, 2, 3))
    with pytest.raises(TypeError, match="float32"):
        ball_query(points.half(), points.half(), K=1, radius=1.0)
    with pytest.raises(TypeError, match="bool"):
        ball_query(points, points, K=1, radius=1.0, skip_points_outside_cube=1)
    with pytest.raises(ValueError, match="shapes"):
        ball_query(points[0], points, K=1, radius=1.0)


def test_pointcept_offsets_and_optional_registration():
    """tests/test_pointcept.py:146-168: offset errors precede device work;
    install() adds ``pointops`` only with pointcept=True."""
    from mps_pointops import compat, pointcept

    xyz = torch.zeros((3, 3))
    with pytest.raises(ValueError, match="end at"):
        pointcept.farthest_point_sampling(xyz, torch.tensor([2]), torch.tensor([1]))
    with pytest.raises(ValueError, match="more FPS"):
        pointcept.farthest_point_sampling(xyz, torch.tensor([3]), torch.tensor([4]))
    names = ("pointnet2_ops", "pointnet2_ops.pointnet2_utils", "knn_cuda", "torch_cluster", "pointops")
    saved = {name: sys.modules.pop(name) for name in names if name in sys.modules}
    try:
        assert "pointops" not in compat.install()
        assert "pointops" in compat.install(force=True, pointcept=True)
        import pointops

        assert pointops.knn_query is pointcept.knn_query
        assert pointops.interpolation is pointcept.interpolation
    finally:
        for name in names:
            sys.modules.pop(name, None)
        sys.modules.update(saved)


def test_chamfer_grid_eligibility():
    """The grid nearest search serves squared-L2 3-D float32 clouds without
    lengths, large enough for its build to pay; everything else keeps the
    linear scan (shape checks only, no device work)."""
    from mps_pointops import chamfer

    def clouds(b, m, n, d=3, dtype=torch.float32):
        return torch.zeros(1, 1, d, dtype=dtype).expand(b, m, d), \
            torch.zeros(1, 1, d, dtype=dtype).expand(b, n, d)

    q, r = clouds(32, 8192, 8192)
    assert chamfer._grid_eligible(q, r, 2, True)
    assert not chamfer._grid_eligible(q, r, 2, False)  # lengths given
    assert not chamfer._grid_eligible(q, r, 1, True)  # L1
    assert not chamfer._grid_eligible(*clouds(32, 8192, 8192, dtype=torch.float64), 2, True)
    assert not chamfer._grid_eligible(*clouds(32, 8192, 8192, d=4), 2, True)
    assert not chamfer._grid_eligible(*clouds(32, 8192, 4096), 2, True)  # too few references
    assert not chamfer._grid_eligible(*clouds(32, 2048, 8192), 2, True)  # too few queries
    assert not chamfer._grid_eligible(*clouds(1, 4096, 8192), 2, True)  # too few pairs
    assert not chamfer._grid_eligible(*clouds(70000, 4096, 8192), 2, True)  # batch limit


def test_flat_layout_offsets_match_searchsorted():
    """Batch vectors -> cloud offsets (one bincount prefix sum) against
    numpy's searchsorted, including empty clouds and a larger batch_size."""
    from mps_pointops import flat

    rng = np.random.default_rng(4)
    for trial in range(20):
        nx, ny = int(rng.integers(1, 300)), int(rng.integers(1, 200))
        bx = np.sort(rng.integers(0, 6, nx))
        by = np.sort(rng.integers(0, 6, ny))
        extra = int(rng.integers(0, 3)) if trial % 2 else None
        size = max(int(bx[-1]), int(by[-1])) + 1 + (extra or 0)
        x, y = torch.rand(nx, 3), torch.rand(ny, 3)
        layout = flat._SearchLayout.of(x, y, torch.from_numpy(bx), torch.from_numpy(by).int(),
                                       None if extra is None else size)
        assert layout.x_offsets.tolist() == np.searchsorted(bx, np.arange(size + 1)).tolist()
        assert layout.y_offsets.tolist() == np.searchsorted(by, np.arange(size + 1)).tolist()
    one = flat._SearchLayout.of(torch.rand(7, 3), torch.rand(2, 3), None, None, None)
    assert one.x_offsets.tolist() == [0, 7] and one.y_offsets.tolist() == [0, 2]


def test_flat_layout_errors_follow_reference_messages():
    """flat.py:49-98: the reference's checks and messages, in its order."""
    from mps_pointops import flat

    x = torch.rand(4, 3)
    with pytest.raises(ValueError, match="batch_size must be a non-negative integer"):
        flat._SearchLayout.of(x, x, None, None, -1)
    with pytest.raises(TypeError, match="batch_x must be a torch.Tensor or None"):
        flat._SearchLayout.of(x, x, [0, 0, 0, 0], None, None)
    with pytest.raises(ValueError, match=r"batch_x must have shape \(4,\)"):
        flat._SearchLayout.of(x, x, torch.zeros(3, dtype=torch.long), None, None)
    with pytest.raises(TypeError, match="integer dtype"):
        flat._SearchLayout.of(x, x, torch.zeros(4), None, None)
    with pytest.raises(ValueError, match="sorted with non-negative batch IDs"):
        flat._SearchLayout.of(x, x, torch.tensor([0, 1, 0, 1]), torch.zeros(4, dtype=torch.long),
                              None)
    with pytest.raises(ValueError, match="sorted with non-negative batch IDs"):
        flat._SearchLayout.of(x, x, torch.tensor([-1, 0, 0, 0]), None, None)
    with pytest.raises(ValueError, match="both required for multiple batches"):
        flat._SearchLayout.of(x, x, torch.tensor([0, 0, 1, 1]), None, None)
    with pytest.raises(ValueError, match="batch_size is smaller than the largest batch ID"):
        b = torch.tensor([0, 0, 2, 2])
        flat._SearchLayout.of(x, x, b, b, 2)


def test_flat_fps_offsets_ptr_and_batch():
    from mps_pointops import flat

    x = torch.rand(10, 3)
    assert flat._fps_offsets(x, None, None, [0, 4, 10]).tolist() == [0, 4, 10]
    assert flat._fps_offsets(x, None, None, torch.tensor([0, 10], dtype=torch.int32)).tolist() \
        == [0, 10]
    assert flat._fps_offsets(x, None, None, None).tolist() == [0, 10]
    b = torch.tensor([0, 0, 0, 1, 1, 3, 3, 3, 3, 3])
    assert flat._fps_offsets(x, b, None, None).tolist() == [0, 3, 5, 5, 10]
    assert flat._fps_offsets(x, b, 6, None).tolist() == [0, 3, 5, 5, 10, 10, 10]
    assert flat._fps_offsets(torch.rand(0, 3), torch.zeros(0, dtype=torch.long), None,
                             None).tolist() == [0]
    with pytest.raises(TypeError, match="ptr must be a tensor, a sequence of integers, or None"):
        flat._fps_offsets(x, None, None, 3)
    with pytest.raises(ValueError, match="non-empty one-dimensional offset array"):
        flat._fps_offsets(x, None, None, [])
    with pytest.raises(ValueError, match="start at 0 and end at len"):
        flat._fps_offsets(x, None, None, [0, 9])
    with pytest.raises(ValueError, match="non-decreasing"):
        flat._fps_offsets(x, None, None, [0, 6, 4, 10])
    with pytest.raises(ValueError, match="integer tensor on the same device"):
        flat._fps_offsets(x, None, None, torch.tensor([0.0, 10.0]))
    with pytest.raises(ValueError, match="batch_size is smaller"):
        flat._fps_offsets(x, b, 2, None)


def test_compat_install_registers_and_respects_existing(monkeypatch):
    import sys as _sys
    import types

    from mps_pointops import compat

    for name in ("pointnet2_ops", "pointnet2_ops.pointnet2_utils", "knn_cuda", "torch_cluster",
                 "pointops"):
        monkeypatch.delitem(_sys.modules, name, raising=False)
    monkeypatch.setitem(_sys.modules, "knn_cuda", types.ModuleType("knn_cuda"))
    names = compat.install()
    assert names == ["pointnet2_ops", "pointnet2_ops.pointnet2_utils", "torch_cluster"]
    from pointnet2_ops import pointnet2_utils
    assert pointnet2_utils.ball_query is compat.ball_query
    assert _sys.modules["pointnet2_ops"].__path__ == []
    from torch_cluster import knn_graph
    assert knn_graph.__module__ == "mps_pointops.flat"
    assert compat.install(force=True, pointcept=True)[-1] == "pointops"
    from pointops import interpolation  # noqa: F401
