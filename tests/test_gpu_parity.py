"""GPU parity: the native kernels against the oracle and the golden vectors.

Integer outputs (indices) must be bit-identical; float outputs computed by
the same operation sequence (squared distances, sqrt, interpolation) are
compared bit for bit as well; atomics-accumulated gradients are compared with
a tolerance (rtol 1e-5 / atol 1e-6, stated per test).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import bench
from conftest import GOLDEN, load_known_answers, load_pointnet2_parity
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def cuda(x, dtype=torch.float32):
    return torch.as_tensor(np.asarray(x), dtype=dtype).cuda()


def host(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy()


def same_bits(a, b):
    a = np.ascontiguousarray(np.asarray(a, np.float32))
    b = np.ascontiguousarray(np.asarray(b, np.float32))
    np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))


# ------------------------------------------------------------ known answers

@pytest.mark.parametrize("case", load_known_answers("fps"), ids=lambda c: c["name"])
def test_fps_known_answers(cuda_device, case):
    import mps_pointops as mp
    from mps_pointops import compat

    xyz = cuda(case["xyz"])
    if case["skip"]:
        got = compat.furthest_point_sample(xyz, case["npoint"])
        assert got.dtype == torch.int32
    else:
        got = mp.furthest_point_sample(xyz, case["npoint"], case["start_idx"])
        assert got.dtype == torch.long
    assert got.cpu().tolist() == case["expect"], case["source"]
    if case["npoint"] > 1:
        large = mp.furthest_point_sample(xyz, case["npoint"], case["start_idx"], case["skip"],
                                         strategy="multigroup")
        assert large.cpu().tolist() == case["expect"]


@pytest.mark.parametrize("case", load_known_answers("fps_flat"), ids=lambda c: c["name"])
def test_fps_flat_known_answers(cuda_device, case):
    from mps_pointops import flat

    x = cuda(case["x"])
    # Both transcribed cases use ratio 0.5 (tests/test_flat.py:20-29).
    got = flat.fps(x, ptr=case["ptr"], ratio=0.5, random_start=False)
    assert got.cpu().tolist() == case["expect"], case["source"]


@pytest.mark.parametrize("case", load_known_answers("knn"), ids=lambda c: c["name"])
def test_knn_known_answers(cuda_device, case):
    import mps_pointops as mp

    d, i = mp.knn(cuda(case["query"]), cuda(case["ref"]), case["k"])
    assert i.cpu().tolist() == case["expect_idx"], case["source"]
    np.testing.assert_allclose(host(d), np.array(case["expect_dist"], np.float32), rtol=1e-6)


def _batch(v):
    return None if v is None else torch.tensor(v, dtype=torch.long).cuda()


@pytest.mark.parametrize("case", load_known_answers("knn_flat"), ids=lambda c: c["name"])
def test_knn_flat_known_answers(cuda_device, case):
    from mps_pointops import flat

    got = flat.knn(cuda(case["x"]), cuda(case["y"]), case["k"], _batch(case["batch_x"]),
                   _batch(case["batch_y"]))
    assert got.cpu().tolist() == case["expect"], case["source"]


@pytest.mark.parametrize("case", load_known_answers("radius_flat"), ids=lambda c: c["name"])
def test_radius_flat_known_answers(cuda_device, case):
    from mps_pointops import flat

    got = flat.radius(cuda(case["x"]), cuda(case["y"]), case["r"], _batch(case["batch_x"]),
                      _batch(case["batch_y"]), max_num_neighbors=case["k"])
    assert got.cpu().tolist() == case["expect"], case["source"]


@pytest.mark.parametrize("case", load_known_answers("ball_query"), ids=lambda c: c["name"])
def test_ball_query_known_answers(cuda_device, case):
    import mps_pointops as mp
    from mps_pointops import compat

    q = cuda(case["query"]).requires_grad_(case.get("expect_grad_p") is not None)
    p = cuda(case["ref"]).requires_grad_(case.get("expect_grad_p") is not None)
    dist, idx = mp.ball_query(q, p, case["radius"], case["k"])
    assert idx.cpu().tolist() == case["expect_idx"], case["source"]
    if case.get("expect_dist") is not None:
        np.testing.assert_allclose(host(dist), np.array(case["expect_dist"], np.float32),
                                   rtol=1e-6, atol=0)
    if case.get("expect_dist_bits") is not None:
        assert host(dist).view(np.uint32).tolist() == case["expect_dist_bits"]
    if case.get("compat") is not None:
        got = compat.ball_query(case["radius"], case["k"], p.detach(), q.detach())
        assert got.dtype == torch.int32 and got.cpu().tolist() == case["compat"]
    if case.get("expect_grad_p") is not None:
        g = case.get("grad_out")
        grad = torch.ones_like(dist) if g is None else cuda(g)
        dist.backward(grad)
        want_p = np.array(case["expect_grad_p"], np.float32).reshape(host(p.grad).shape)
        np.testing.assert_allclose(host(p.grad), want_p, rtol=1e-6, atol=1e-7)
        if case.get("expect_grad_q") is not None:
            np.testing.assert_allclose(host(q.grad), np.array(case["expect_grad_q"], np.float32),
                                       rtol=1e-6, atol=1e-7)
        if case.get("expect_grad_q_row0") is not None:
            np.testing.assert_allclose(host(q.grad)[0, 0], case["expect_grad_q_row0"], rtol=1e-6)
            assert np.all(host(q.grad)[0, 1:] == 0)


@pytest.mark.parametrize("case", load_known_answers("three_nn"), ids=lambda c: c["name"])
def test_three_nn_known_answers(cuda_device, case):
    from mps_pointops import three_nn

    d, i = three_nn(cuda(case["unknown"]), cuda(case["known"]))
    assert i.dtype == torch.int32 and i.cpu().tolist() == case["expect_idx"]
    np.testing.assert_allclose(host(d), np.array(case["expect_dist"], np.float32), rtol=1e-6)


@pytest.mark.parametrize("case", load_known_answers("three_interpolate"), ids=lambda c: c["name"])
def test_three_interpolate_known_answers(cuda_device, case):
    from mps_pointops import three_interpolate

    f = cuda(case["features"]).requires_grad_()
    w = cuda(case["weights"]).requires_grad_()
    out = three_interpolate(f, torch.tensor(case["indices"], dtype=torch.int32).cuda(), w)
    assert out.cpu().tolist() == case["expect"]
    out.backward(cuda(case["grad_out"]))
    assert f.grad.cpu().tolist() == case["expect_grad"]
    assert w.grad is not None and torch.count_nonzero(w.grad).item() == 0


@pytest.mark.parametrize("case", load_known_answers("chamfer_nearest"), ids=lambda c: c["name"])
def test_chamfer_nearest_known_answers(cuda_device, case):
    from mps_pointops import chamfer

    q, r = cuda(case["query"]), cuda(case["ref"])
    B = q.shape[0]
    ql = _batch(case.get("query_lengths") or [q.shape[1]] * B)
    rl = _batch(case.get("ref_lengths") or [r.shape[1]] * B)
    dist, idx = chamfer._nearest_mps(q, r, ql, rl, norm=case["norm"])
    assert idx.cpu().tolist() == case["expect_idx"], case["source"]
    np.testing.assert_array_equal(host(dist), np.array(case["expect_dist"], np.float32))


# ----------------------------------------- reference-recorded selections

def test_segmentation_selections_match_metal_recording(cuda_device):
    """The compat path on the GPU reproduces all 12 index arrays recorded on
    the reference's Metal kernels (docs/parity/pointnet2-segmentation-mps-safe.npz)."""
    from mps_pointops import compat
    from mps_pointops.pointnet2 import three_nn

    z = np.load(GOLDEN / "segmentation_selections.npz")
    xyz = [cuda(z["xyz"])]
    got = []
    for npoint, radius in ((1024, 0.1), (256, 0.2), (64, 0.4), (16, 0.8)):
        x = xyz[-1]
        idx = compat.furthest_point_sample(x, npoint)
        new = compat.gather_operation(x.transpose(1, 2).contiguous(), idx).transpose(1, 2)
        new = new.contiguous()
        got += [idx, compat.ball_query(radius, 32, x, new)]
        xyz.append(new)
    for i in range(4):
        got.append(three_nn(xyz[3 - i], xyz[4 - i])[1])
    names = sorted(k for k in z.files if k.startswith("mps::"))
    for name, arr in zip(names, got):
        np.testing.assert_array_equal(host(arr), z[name], err_msg=name)


def test_pointnet2_parity_fixtures(cuda_device):
    from mps_pointops import three_interpolate, three_nn

    for name, case in load_pointnet2_parity()["cases"].items():
        inp = case["inputs"]
        dist, idx = three_nn(cuda(inp["unknown"]), cuda(inp["known"]))
        want = case["mps_safe"]
        assert idx.cpu().tolist() == want["nearest_indices"], name
        assert idx.cpu().tolist() == case["cuda"]["nearest_indices"], name
        np.testing.assert_allclose(host(dist), np.array(want["distances"], np.float32), rtol=1e-6)
        interp = idx.clone()
        for b, row in inp["override"].items():
            interp[int(b), 0] = torch.tensor(row, dtype=torch.int32)
        f = cuda(inp["features"]).requires_grad_()
        w = cuda(inp["weights"]).requires_grad_()
        out = three_interpolate(f, interp, w)
        np.testing.assert_array_equal(host(out), np.array(want["interpolated"], np.float32))
        out.backward(cuda(inp["gradient"]))
        np.testing.assert_allclose(host(f.grad), np.array(want["feature_gradient"], np.float32),
                                   rtol=1e-6, atol=1e-6)
        assert torch.count_nonzero(w.grad).item() == 0


# ------------------------------------------------------- oracle parity

def rand_cloud(b, n, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(b, n, 3, generator=g) * scale).float()


@pytest.mark.parametrize("n", [1, 2, 31, 32, 33, 63, 64, 65, 255, 256, 257, 1023, 1024, 1025,
                               4095, 4096, 4097, 8192, 8193, 20000])
def test_fps_matches_oracle_edge_sizes(cuda_device, n):
    import mps_pointops as mp

    xyz = rand_cloud(2, n, n)
    npoint = min(n + 3, 300)
    start = n // 3
    want = O.fps(xyz, npoint, start)
    got = mp.furthest_point_sample(xyz.cuda(), npoint, start, strategy="single")
    np.testing.assert_array_equal(host(got), want)


@pytest.mark.parametrize("n", [1, 33, 1025, 4097, 65537, 100_000, 300_000, 1_500_000, 1 << 21])
def test_fps_large_matches_oracle(cuda_device, n):
    import mps_pointops as mp

    xyz = rand_cloud(1, n, 27 + n)
    xyz[0, : n // 7] = xyz[0, n // 7: 2 * (n // 7)]  # duplicates -> ties
    npoint = min(n + 2, 200)
    start = n // 2
    for skip in (False, True):
        want = O.fps(xyz, npoint, start, skip)
        got = mp.furthest_point_sample(xyz.cuda(), npoint, start, skip, strategy="multigroup")
        np.testing.assert_array_equal(host(got), want)


def _fps_large_abi(xyz: torch.Tensor, npoint: int, start: int):
    """pointops_fps_large through the C ABI: (indices, status word)."""
    from mps_pointops import _native

    x = xyz.cuda().contiguous()
    N = x.shape[1]
    out = torch.full((npoint,), -777, dtype=torch.long, device="cuda")
    size = _native.size_query("pointops_fps_large_workspace_bytes", N, npoint)
    ws = torch.zeros(size, dtype=torch.uint8, device="cuda")
    _native.call("pointops_fps_large", x.data_ptr(), out.data_ptr(), ws.data_ptr(), N, npoint,
                 start, 0, _native.stream(x.device))
    torch.cuda.synchronize()
    return host(out), int(ws[:4].view(torch.int32).item())


def test_fps_large_status_word_clear_after_success(cuda_device):
    xyz = rand_cloud(1, 200_000, 5)
    got, status = _fps_large_abi(xyz, 500, 3)
    assert status == 0
    np.testing.assert_array_equal(got, O.fps(xyz, 500, 3)[0])


def test_fps_large_forced_give_up_is_reported(cuda_device, monkeypatch):
    """A poll limit of 0 (set from the host) makes every workgroup give up at
    its first exchange: the status word is raised, the first sample (written
    before any exchange) stays, every other slot is -1, and the public call
    raises.  Every wave exits normally."""
    import mps_pointops as mp

    xyz = rand_cloud(1, 100_000, 6)
    monkeypatch.setenv("POINTOPS_FPS_SPIN_LIMIT", "0")
    got, status = _fps_large_abi(xyz, 300, 11)
    assert status == 1
    assert got[0] == 11 and (got[1:] == -1).all()
    with pytest.raises(RuntimeError, match="incomplete"):
        mp.furthest_point_sample(xyz.cuda(), 300, 11, strategy="multigroup")
    monkeypatch.delenv("POINTOPS_FPS_SPIN_LIMIT")
    got, status = _fps_large_abi(xyz, 300, 11)
    assert status == 0
    np.testing.assert_array_equal(got, O.fps(xyz, 300, 11)[0])


@pytest.mark.parametrize("case", ["random", "ties", "exhausted", "mostly_skipped", "last_start"])
def test_fps_stream_matches_oracle(cuda_device, case):
    """Clouds above 2^21 points (the streaming kernel, running distances in
    the workspace): a random cloud, duplicated points (ties by index), a run
    past the number of distinct points, a cloud whose points are nearly all
    skipped, and a start at the last index of an odd-sized cloud."""
    import mps_pointops as mp

    g = torch.Generator().manual_seed(900 + len(case))
    n = (1 << 21) + 4099
    skip = case == "mostly_skipped"
    start = 12345
    npoint = 300
    if case == "random":
        xyz = torch.randn(1, n, 3, generator=g)
    elif case == "ties":
        xyz = torch.randn(1, n, 3, generator=g)
        xyz[0, : n // 3] = xyz[0, n // 3: 2 * (n // 3)]
    elif case == "exhausted":
        base = torch.randn(250, 3, generator=g)
        xyz = base[torch.randint(0, 250, (n,), generator=g)][None].contiguous()
    elif case == "mostly_skipped":
        xyz = torch.randn(1, n, 3, generator=g) * 1e-3
        xyz[0, ::40_000] = torch.randn(xyz[0, ::40_000].shape[0], 3, generator=g)
        npoint, start = 120, 0
    else:
        n = 3_000_001
        xyz = torch.rand(1, n, 3, generator=g)
        start = n - 1
    print(f"fps stream case={case} n={n} npoint={npoint}", flush=True)
    want = O.fps(xyz, npoint, start, skip)
    got = mp.furthest_point_sample(xyz.cuda(), npoint, start, skip)
    np.testing.assert_array_equal(host(got), want)


def test_fps_stream_status_and_forced_give_up(cuda_device, monkeypatch):
    """The streaming kernel reports success in the status word, and a poll
    limit of 0 (set from the host) makes it give up at its first exchange
    with every later slot -1; every wave exits normally."""
    xyz = rand_cloud(1, (1 << 21) + 1, 8)
    got, status = _fps_large_abi(xyz, 200, 17)
    assert status == 0
    np.testing.assert_array_equal(got, O.fps(xyz, 200, 17)[0])
    monkeypatch.setenv("POINTOPS_FPS_SPIN_LIMIT", "0")
    got, status = _fps_large_abi(xyz, 200, 17)
    assert status == 1
    assert got[0] == 17 and (got[1:] == -1).all()


@pytest.mark.parametrize("n,distinct", [(4096, 300), (1000, 40), (8192, 3000)])
def test_fps_dense_repeated_points(cuda_device, n, distinct):
    """Clouds built from few distinct points (equal distances everywhere, and
    more samples than distinct points): ties must go to the smallest index."""
    import mps_pointops as mp

    g = torch.Generator().manual_seed(n + distinct)
    base = torch.randn(distinct, 3, generator=g)
    xyz = base[torch.randint(0, distinct, (3, n), generator=g)].contiguous()
    npoint = min(n, distinct + 200)
    for start, skip in ((0, False), (n // 3, False), (5, True)):
        want = O.fps(xyz, npoint, start, skip)
        got = mp.furthest_point_sample(xyz.cuda(), npoint, start, skip)
        np.testing.assert_array_equal(host(got), want)


@pytest.mark.parametrize("case", ["long", "exhausted", "mostly_skipped"])
def test_fps_large_long_runs(cuda_device, case):
    """Many exchanges of the persistent kernel: a long run on a random cloud,
    a run past the number of distinct points (every remaining distance ties
    at zero), and a cloud whose points are nearly all skipped."""
    import mps_pointops as mp

    g = torch.Generator().manual_seed({"long": 1, "exhausted": 2, "mostly_skipped": 3}[case])
    skip = case == "mostly_skipped"
    if case == "long":
        xyz = torch.randn(1, 100_000, 3, generator=g)
        npoint, start = 3000, 12345
    elif case == "exhausted":
        base = torch.randn(400, 3, generator=g)
        xyz = base[torch.randint(0, 400, (20_000,), generator=g)][None].contiguous()
        npoint, start = 600, 7
    else:
        xyz = torch.randn(1, 30_000, 3, generator=g) * 1e-3
        xyz[0, ::1000] = torch.randn(30, 3, generator=g)
        npoint, start = 100, 0
    want = O.fps(xyz, npoint, start, skip)
    got = mp.furthest_point_sample(xyz.cuda(), npoint, start, skip, strategy="multigroup")
    np.testing.assert_array_equal(host(got), want)


def test_fps_skip_near_origin_boundary(cuda_device):
    """tests/test_compat.py:96-111: points just inside the 1e-3 radius are
    never picked, the one just outside is."""
    from mps_pointops import compat

    xyz = rand_cloud(1, 2000, 0)
    inside = np.float32(np.sqrt(np.float32(1e-3))) * np.float32(0.999)
    outside = np.float32(np.sqrt(np.float32(1e-3))) * np.float32(1.001)
    g = torch.Generator().manual_seed(1)
    xyz[0, 1:40] = torch.tensor([float(inside), 0.0, 0.0]) * torch.rand(39, 1, generator=g)
    xyz[0, 40] = torch.tensor([float(inside), 0.0, 0.0])
    xyz[0, 41] = torch.tensor([float(outside), 0.0, 0.0])
    got = compat.furthest_point_sample(xyz.cuda(), 2000).cpu()
    want = O.fps(xyz, 2000, 0, True).astype(np.int32)
    np.testing.assert_array_equal(got.numpy(), want)
    picked = set(got[0].tolist())
    assert picked.isdisjoint(range(1, 41)) and 41 in picked


@pytest.mark.parametrize("B,n,npoint,frac,strategy,skip", [
    (2, 1000, 300, 0.05, "single", False),        # one workgroup, leader/follower kernel
    (1, 40, 25, 0.75, "single", False),           # fewer finite points than samples
    (2, 6000, 300, 0.05, "single", True),         # 8192-point tiled kernel
    (2, 9000, 200, 0.05, "single", False),        # running distances in scratch
    (1, 70_000, 200, 0.02, "multigroup", False),  # cooperative lazy kernel
    (1, (1 << 21) + 5, 100, 0.02, "auto", False), # streaming kernel
])
def test_fps_nan_points_never_sampled(cuda_device, B, n, npoint, frac, strategy, skip):
    """A point with a NaN coordinate is never sampled, and the others are
    sampled as if it were absent: in kernels/fps.metal:77-83 its NaN running
    distance never wins `m > best`.  (reference.py:56-57, torch.minimum then
    argmax, would pick the first NaN point instead.)  Expected: the oracle's
    FPS of each cloud without its NaN points, mapped back to the full
    cloud's indices; the start point is finite."""
    import mps_pointops as mp

    print(f"fps nan B={B} n={n} npoint={npoint} strategy={strategy}", flush=True)
    xyz = rand_cloud(B, n, 31 + n)
    g = np.random.default_rng(n)
    start = n // 3
    bad = g.random((B, n)) < frac
    bad[:, start] = False
    axis = g.integers(0, 3, (B, n))
    for b in range(B):
        rows = np.nonzero(bad[b])[0]
        xyz[b, rows, axis[b, rows]] = float("nan")
    got = host(mp.furthest_point_sample(xyz.cuda(), npoint, start, skip, strategy=strategy))
    for b in range(B):
        keep = np.nonzero(~bad[b])[0]
        sub = xyz[b:b + 1, keep].contiguous()
        want = keep[O.fps(sub, npoint, int(np.searchsorted(keep, start)), skip)[0]]
        np.testing.assert_array_equal(got[b], want)
        assert not bad[b, got[b]].any()


def _fps_shape_case(case: str) -> tuple[torch.Tensor, int, int, bool]:
    seeds = {"uniform_exhausted": 1, "blobs_skip": 2, "plane": 3, "duplicates": 4,
             "mixed_scale": 5, "infinite": 6}
    g = torch.Generator().manual_seed(seeds[case])
    if case == "uniform_exhausted":
        return torch.rand(2, 4096, 3, generator=g), 4096, 17, False
    if case == "blobs_skip":
        centres = torch.randn(5, 3, generator=g) * 20
        x = centres[torch.randint(0, 5, (2, 3000), generator=g)] + torch.randn(2, 3000, 3, generator=g)
        x[:, ::10] *= 1e-3  # near the origin: never picked
        return x.contiguous(), 1500, 3, True
    if case == "plane":
        x = torch.rand(3, 2500, 3, generator=g)
        x[..., 2] = 0.0
        return x, 800, 2499, False
    if case == "duplicates":
        base = torch.randn(200, 3, generator=g)
        return base[torch.randint(0, 200, (2, 4096), generator=g)].contiguous(), 600, 0, False
    if case == "mixed_scale":
        x = torch.randn(2, 4000, 3, generator=g) * 1e-3
        x[:, ::7] = torch.randn(2, 572, 3, generator=g) * 1e4
        return x, 1000, 5, False
    if case == "infinite":
        x = torch.randn(1, 3000, 3, generator=g)
        x[0, 10] = torch.tensor([float("inf"), 0.0, 0.0])
        x[0, 2000] = torch.tensor([1.0, float("-inf"), 2.0])
        return x, 500, 0, False
    raise ValueError(case)


@pytest.mark.parametrize("case", ["uniform_exhausted", "blobs_skip", "plane", "duplicates",
                                  "mixed_scale", "infinite"])
def test_fps_cloud_shapes_match_oracle(cuda_device, case):
    """Clouds of 2049..4096 points (eight per thread of the batched kernel):
    exhausted clouds (every remaining distance ties at zero), skipped points,
    a degenerate axis, duplicates, widely mixed scales and infinite
    coordinates."""
    import mps_pointops as mp

    xyz, npoint, start, skip = _fps_shape_case(case)
    want = O.fps(xyz, npoint, start, skip)
    got = mp.furthest_point_sample(xyz.cuda(), npoint, start, skip)
    np.testing.assert_array_equal(host(got), want)


def test_fps_ragged_up_to_4096_matches_oracle(cuda_device):
    """A ragged launch whose longest cloud has 2049..4096 points also holds
    empty, one-point and small clouds."""
    from mps_pointops import flat

    g = torch.Generator().manual_seed(11)
    x = torch.randn(9000, 3, generator=g)
    ptr = [0, 0, 1, 3, 70, 70, 2119, 6215, 9000]
    lengths = np.diff(ptr)
    got = flat.fps(x.cuda(), ptr=ptr, ratio=0.5, random_start=False)
    counts = np.ceil(lengths.astype(np.float32) * np.float32(0.5)).astype(np.int64)
    out_ptr = np.concatenate([[0], np.cumsum(counts)])
    want = O.fps_flat(x, ptr, out_ptr, np.zeros(len(lengths), np.int64))
    np.testing.assert_array_equal(host(got), want)


def test_fps_c1_and_c2_full(cuda_device):
    import mps_pointops as mp

    c1 = bench.make_c1()
    np.testing.assert_array_equal(host(mp.furthest_point_sample(c1.cuda(), 512)), O.fps(c1, 512))
    c2 = bench.make_c2()
    np.testing.assert_array_equal(host(mp.furthest_point_sample(c2.cuda(), 1024)), O.fps(c2, 1024))


@pytest.mark.parametrize("n,k", [(1, 1), (31, 5), (64, 64), (65, 65), (300, 17), (1000, 128),
                                 (700, 256), (5000, 32)])
def test_knn3_matches_oracle(cuda_device, n, k):
    import mps_pointops as mp

    ref = rand_cloud(2, n, n + k)
    ref[:, n // 3:] = torch.round(ref[:, n // 3:] * 2) / 2  # exact ties
    query = torch.cat([ref[:, :5], rand_cloud(2, 9, 1)], 1)
    want_d, want_i = O.knn3(query, ref, k)
    d, i = mp.knn(query.cuda(), ref.cuda(), k)
    np.testing.assert_array_equal(host(i), want_i)
    same_bits(host(d), want_d)


@pytest.mark.parametrize("descending", [False, True])
def test_knn3_spatially_sorted_reference(cuda_device, descending):
    import mps_pointops as mp

    ref = rand_cloud(1, 20000, 0)
    ref = ref[:, ref[0, :, 0].argsort(descending=descending)].contiguous()
    query = rand_cloud(1, 64, 1)
    want_d, want_i = O.knn3(query, ref, 128)
    d, i = mp.knn(query.cuda(), ref.cuda(), 128)
    np.testing.assert_array_equal(host(i), want_i)
    same_bits(host(d), want_d)


def _knn3_grid(query: torch.Tensor, ref: torch.Tensor, k: int):
    """pointops_knn3_grid through the C ABI (any cloud size)."""
    from mps_pointops import _native

    q, r = query.cuda().contiguous(), ref.cuda().contiguous()
    B, M, _ = q.shape
    N = r.shape[1]
    dist = torch.empty(B, M, k, device="cuda")
    idx = torch.empty(B, M, k, dtype=torch.long, device="cuda")
    size = _native.size_query("pointops_knn3_grid_workspace_bytes", B, M, N)
    ws = torch.empty(size, dtype=torch.uint8, device="cuda")
    _native.call("pointops_knn3_grid", q.data_ptr(), r.data_ptr(), dist.data_ptr(), idx.data_ptr(),
                 ws.data_ptr(), B, M, N, k, _native.stream(q.device))
    return host(dist), host(idx)


def _grid_case(name: str):
    g = torch.Generator().manual_seed(sum(map(ord, name)))
    if name == "uniform":
        ref = torch.rand(2, 40_000, 3, generator=g) * 10
        query = torch.rand(2, 3000, 3, generator=g) * 10
    elif name == "slab":
        ref = bench.make_c3(N=60_000)
        query = ref[:, torch.randperm(60_000, generator=g)[:2000]].clone()
    elif name == "ties":  # integer lattice: many equal distances, duplicates
        ref = torch.randint(0, 12, (1, 30_000, 3), generator=g).float()
        query = torch.randint(-1, 13, (1, 1500, 3), generator=g).float() + 0.5 * (
            torch.rand(1, 1500, 1, generator=g) < 0.5).float()
    elif name == "far_queries":  # queries outside the references' box
        ref = torch.rand(1, 20_000, 3, generator=g)
        query = torch.cat([torch.rand(1, 500, 3, generator=g) * 40 - 20,
                           torch.rand(1, 100, 3, generator=g)], 1)
    elif name == "sparse_clusters":  # few references per occupied cell, wide gaps
        centres = torch.rand(1, 40, 3, generator=g) * 100
        ref = (centres.repeat_interleave(50, 1) + torch.randn(1, 2000, 3, generator=g) * 0.1)
        query = torch.rand(1, 700, 3, generator=g) * 100
    elif name == "flat":  # zero extent in z
        ref = torch.cat([torch.rand(1, 10_000, 2, generator=g), torch.zeros(1, 10_000, 1)], 2)
        query = torch.cat([torch.rand(1, 400, 2, generator=g), torch.rand(1, 400, 1, generator=g)], 2)
    elif name == "one_point":  # every reference identical
        ref = torch.full((1, 5000, 3), 0.25)
        query = torch.rand(1, 100, 3, generator=g)
    elif name == "non_finite_refs":
        ref = torch.rand(2, 8000, 3, generator=g)
        ref[0, 7] = float("nan")
        ref[0, 100, 1] = float("inf")
        ref[1, :7990] = float("nan")  # ten finite references: K=16 pads
        query = torch.rand(2, 300, 3, generator=g)
    else:  # non_finite_queries
        ref = torch.rand(1, 8000, 3, generator=g)
        query = torch.rand(1, 300, 3, generator=g)
        query[0, 5] = float("nan")
        query[0, 70, 2] = -float("inf")
    return query.contiguous(), ref.contiguous()


@pytest.mark.parametrize("name", ["uniform", "slab", "ties", "far_queries", "sparse_clusters",
                                  "flat", "one_point", "non_finite_refs", "non_finite_queries"])
@pytest.mark.parametrize("k", [1, 5, 16, 32])
def test_knn3_grid_matches_oracle(cuda_device, name, k):
    """The grid search returns the brute-force answer bit for bit."""
    query, ref = _grid_case(name)
    want_d, want_i = O.knn3(query, ref, k)
    d, i = _knn3_grid(query, ref, k)
    np.testing.assert_array_equal(i, want_i)
    same_bits(d, want_d)


@pytest.mark.parametrize("k", [1, 16, 32])
def test_knn3_grid_listed_far_queries(cuda_device, k):
    """Tight clusters queried both on the clusters and uniformly over their
    box, shuffled, so that the walk lists some quads of a wave for the linear
    pass and finishes the others: every row equals the brute-force answer,
    in two batches with different mixes."""
    g = torch.Generator().manual_seed(40 + k)
    refs, queries = [], []
    for b in range(2):
        centres = torch.rand(10, 3, generator=g) * 100
        ref = centres.repeat_interleave(4000, 0) + torch.randn(40_000, 3, generator=g) * 0.1
        near = ref[torch.randperm(40_000, generator=g)[: 1500 + 1000 * b]]
        far = torch.rand(2500 - 1000 * b, 3, generator=g) * 100
        both = torch.cat([near, far])
        refs.append(ref)
        queries.append(both[torch.randperm(4000, generator=g)])
    query, ref = torch.stack(queries), torch.stack(refs)
    want_d, want_i = O.knn3(query, ref, k)
    d, i = _knn3_grid(query, ref, k)
    np.testing.assert_array_equal(i, want_i)
    same_bits(d, want_d)


def _listed_case(case: str):
    g = torch.Generator().manual_seed(sum(map(ord, case)))
    if case == "clusters":  # 40965 references: the last chunk of 256 holds 5
        centres = torch.rand(30, 3, generator=g) * 100
        ref = centres.repeat_interleave(1366, 0)[:40_965] + torch.randn(40_965, 3, generator=g) * 0.1
        query = torch.rand(5000, 3, generator=g) * 100
        return query[None].contiguous(), ref[None].contiguous()
    if case == "lattice_ties":  # integer points repeated: equal keys across chunks and waves
        centres = torch.randint(0, 60, (20, 1, 3), generator=g)
        offs = torch.stack(torch.meshgrid(*[torch.arange(-1, 2)] * 3, indexing="ij"), -1).reshape(1, 27, 3)
        ref = (centres + offs).reshape(-1, 3).repeat(30, 1).float()
        ref = ref[torch.randperm(ref.shape[0], generator=g)]
        query = torch.randint(-10, 70, (3000, 3), generator=g).float()
        return query[None].contiguous(), ref[None].contiguous()
    # non_finite: cloud 0 holds NaN and inf references (every query listed,
    # chunks with (-inf, +inf) boxes next to pruned ones); cloud 1 non-finite queries.
    refs, queries = [], []
    for b in range(2):
        centres = torch.rand(12, 3, generator=g) * 50
        ref = centres.repeat_interleave(1000, 0) + torch.randn(12_000, 3, generator=g) * 0.2
        query = torch.rand(2500, 3, generator=g) * 50
        if b == 0:
            ref[17] = float("nan")
            ref[5000, 2] = float("inf")
            ref[9000, 0] = -float("inf")
        else:
            query[3] = float("nan")
            query[1000, 1] = float("inf")
        refs.append(ref)
        queries.append(query)
    return torch.stack(queries).contiguous(), torch.stack(refs).contiguous()


@pytest.mark.parametrize("case", ["clusters", "lattice_ties", "non_finite"])
@pytest.mark.parametrize("k", [1, 7, 16, 32])
def test_knn3_grid_listed_pruned(cuda_device, case, k):
    """Queries far from tight clusters go to the pruned linear pass (more than
    one list tile, chunk boxes that skip whole clusters, a last chunk shorter
    than K, equal keys at the K-th place, non-finite chunks and queries): the
    result equals brute force bit for bit."""
    query, ref = _listed_case(case)
    want_d, want_i = O.knn3(query, ref, k)
    d, i = _knn3_grid(query, ref, k)
    np.testing.assert_array_equal(i, want_i)
    same_bits(d, want_d)


def test_knn3_grid_public_path(cuda_device):
    """ops.knn uses the grid search for large clouds; results match the
    brute-force kernel on the same inputs."""
    import mps_pointops as mp
    from mps_pointops import _native

    g = torch.Generator().manual_seed(11)
    ref = torch.rand(1, 70_000, 3, generator=g).cuda()
    query = torch.rand(1, 4000, 3, generator=g).cuda()
    d, i = mp.knn(query, ref, 16)
    bd = torch.empty_like(d)
    bi = torch.empty_like(i)
    _native.call("pointops_knn3", query.data_ptr(), ref.data_ptr(), bd.data_ptr(), bi.data_ptr(),
                 1, 4000, 70_000, 16, _native.stream(query.device))
    np.testing.assert_array_equal(host(i), host(bi))
    same_bits(host(d), host(bd))


def test_knn3_nan_padding_matches_reference_kernel(cuda_device):
    """kernels/knn.metal semantics: NaN distances never insert; unfilled slots
    stay (inf, 2^32-1); inf distances are ordinary candidates."""
    import mps_pointops as mp

    ref = torch.tensor([[[np.nan, 0, 0], [np.inf, 0, 0], [1, 0, 0], [np.nan, 1, 1]]]).float()
    query = torch.tensor([[[0, 0, 0], [np.nan, 0, 0]]]).float()
    want_d, want_i = O.knn3(query, ref, 3)
    d, i = mp.knn(query.cuda(), ref.cuda(), 3)
    assert want_i.tolist() == [[[2, 1, 4294967295], [4294967295] * 3]]
    np.testing.assert_array_equal(host(i), want_i)
    same_bits(host(d), want_d)


@pytest.mark.parametrize("dim,k", [(1, 5), (2, 1), (4, 33), (64, 20), (128, 256), (7, 64)])
def test_knn_feat_matches_oracle(cuda_device, dim, k):
    import mps_pointops as mp

    g = torch.Generator().manual_seed(107 + dim)
    query = torch.randn(2, 9, dim, generator=g)
    ref = torch.randn(2, 300, dim, generator=g)
    ref[:, 20] = ref[:, 3]
    query[:, 0] = ref[:, 3]
    q_view = torch.cat((query, query), dim=1)[:, ::2]
    want_d, want_i = O.knn_feat(q_view, ref, k)
    d, i = mp.knn(q_view.cuda(), ref.cuda(), k)
    np.testing.assert_array_equal(host(i), want_i)
    same_bits(host(d), want_d)


@pytest.mark.parametrize("dim", [64, 128])
@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (63, 15, 8), (65, 17, 9), (130, 100, 16),
                                   (70, 1000, 17), (64, 2049, 32), (3, 40, 33)])
def test_knn_feat_lane_path(cuda_device, m, n, k, dim):
    """D=64 and D=128 with K<=32 run one lane per query with LDS reference
    tiles: ragged tiles and wave ranges, duplicate references (ties),
    non-finite queries and references, and K=33 (wave-per-query path)
    against the oracle."""
    import mps_pointops as mp

    if k > n:
        k = n
    g = torch.Generator().manual_seed(1000 * m + n + k + dim)
    ref = torch.randn(2, n, dim, generator=g)
    query = torch.randn(2, m, dim, generator=g)
    if n > 4:
        ref[:, n - 1] = ref[:, 1]
        ref[:, n // 2] = ref[:, 1]
        ref[0, 2, 7] = float("nan")
        ref[1, 3, 0] = float("inf")
    query[:, 0] = ref[:, min(1, n - 1)]
    if m > 2:
        query[0, 2, 5] = float("inf")
        query[1, 1, dim - 1] = float("nan")
    want_d, want_i = O.knn_feat(query, ref, k)
    d, i = mp.knn(query.cuda(), ref.cuda(), k)
    np.testing.assert_array_equal(host(i), want_i)
    same_bits(host(d), want_d)


@pytest.mark.parametrize("radius,k", [(0.1, 16), (0.2, 32), (0.4, 128), (0.7, 1), (2.0, 65)])
def test_ball_query_matches_oracle(cuda_device, radius, k):
    import mps_pointops as mp

    p = bench.make_c2(seed=11, B=3, N=1500)
    q = p[:, ::5].contiguous()
    want_d, want_i = O.ball_query(q, p, radius, k)
    d, i = mp.ball_query(q.cuda(), p.cuda(), radius, k)
    np.testing.assert_array_equal(host(i), want_i)
    same_bits(host(d), want_d)


def test_ball_query_lengths_poisoned_outputs(cuda_device):
    """tests/test_ball_query_mps.py:127-213: every slot is written (outputs
    poisoned first), lengths respected, NaN/inf points never match."""
    from mps_pointops import _ball_query_mps as bq
    from mps_pointops import _native

    batch, nq, npts = 2, 9, 65
    q = torch.zeros(batch, nq, 3)
    p = torch.zeros(batch, npts, 3)
    for j in range(npts):
        p[:, j, 0] = 2.0 if j % 5 == 1 else (0.25 if j % 3 == 0 else 0.5)
    p[:, 31, 0] = float("nan")
    p[:, 32, 0] = float("inf")
    q[:, 2, 0] = 0.5
    q[:, 4, 0] = 20.0
    ql, pl = [9, 7], [65, 49]
    for dtype in (torch.float32, torch.float16):
        for k in (1, 31, 32, 33, 65):
            want_d, want_i = O.ball_query(q.to(dtype).float(), p.to(dtype).float(), 1.0, k, ql, pl)
            idx = torch.full((batch, nq, k), -777, dtype=torch.int64).cuda()
            dist = torch.full((batch, nq, k), float("nan")).cuda()
            qc, pc = q.to(dtype).cuda(), p.to(dtype).cuda()
            qlc, plc = torch.tensor(ql).cuda(), torch.tensor(pl).cuda()
            _, r2 = bq._checked_radius_and_k(1.0, k)
            name = "pointops_ball_query_f32" if dtype == torch.float32 else "pointops_ball_query_f16"
            _native.call(name, qc.data_ptr(), pc.data_ptr(), qlc.data_ptr(), plc.data_ptr(),
                         idx.data_ptr(), dist.data_ptr(), batch, nq, npts, k, r2,
                         _native.stream(qc.device))
            torch.cuda.synchronize()
            np.testing.assert_array_equal(host(idx), want_i)
            same_bits(host(dist), want_d)
            res = bq.ball_query(qc, pc, radius=1.0, k=k, query_lengths=qlc, point_lengths=plc)
            np.testing.assert_array_equal(host(res.indices), want_i)


def test_ball_query_c1_c2_c3_full(cuda_device):
    import mps_pointops as mp

    c1 = bench.make_c1()
    centres = c1.gather(1, torch.from_numpy(O.fps(c1, 512))[..., None].expand(-1, -1, 3))
    want_d, want_i = O.ball_query(centres, c1, 0.2, 32)
    d, i = mp.ball_query(centres.cuda(), c1.cuda(), 0.2, 32)
    np.testing.assert_array_equal(host(i), want_i)
    same_bits(host(d), want_d)
    c2 = bench.make_c2()
    centres = c2.gather(1, torch.from_numpy(O.fps(c2, 1024))[..., None].expand(-1, -1, 3))
    for radius, k in bench.C2_RADII:
        want_d, want_i = O.ball_query(centres, c2, radius, k)
        d, i = mp.ball_query(centres.cuda(), c2.cuda(), radius, k)
        np.testing.assert_array_equal(host(i), want_i)
        same_bits(host(d), want_d)


def test_knn_c1_c2_full(cuda_device):
    import mps_pointops as mp

    for make, npoint in ((bench.make_c1, 512), (bench.make_c2, 1024)):
        x = make()
        centres = x.gather(1, torch.from_numpy(O.fps(x, npoint))[..., None].expand(-1, -1, 3))
        want_d, want_i = O.knn3(centres, x, 16)
        d, i = mp.knn(centres.cuda(), x.cuda(), 16)
        np.testing.assert_array_equal(host(i), want_i)
        same_bits(host(d), want_d)


def test_three_nn_and_interpolate_c2(cuda_device):
    from mps_pointops import three_interpolate, three_nn

    x = bench.make_c2()
    centres = x.gather(1, torch.from_numpy(O.fps(x, 1024))[..., None].expand(-1, -1, 3))
    want_d, want_i = O.three_nn(x, centres)
    d, i = three_nn(x.cuda(), centres.cuda())
    np.testing.assert_array_equal(host(i), want_i)
    same_bits(host(d), want_d)
    inv = 1.0 / (d + 1e-8)
    w = (inv / inv.sum(-1, keepdim=True)).contiguous()
    g = torch.Generator().manual_seed(9)
    feats = torch.randn(32, 128, 1024, generator=g)
    out = three_interpolate(feats.cuda(), i, w)
    same_bits(host(out), O.three_interpolate(feats, host(i), host(w)))
    fc = feats.cuda().requires_grad_()
    upstream = torch.randn(32, 128, 4096, generator=g)
    three_interpolate(fc, i, w).backward(upstream.cuda())
    want_g = O.three_interpolate_backward(upstream, host(i), host(w), 1024)
    np.testing.assert_allclose(host(fc.grad), want_g, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("m,n", [(64, 300), (5, 40), (1024, 4096), (3000, 200)])
def test_three_interpolate_backward_sequential_order(cuda_device, m, n):
    """The gradient equals its documented float32 order bit for bit -- for up
    to 1024 known points the (n, t)-ordered terms summed in pieces of 12 CSR
    positions, for more (3000 here) the scatter loop over (n, t) in order --
    is the same on every call (no float atomics), and lies within 1e-5 of
    the sequential loop."""
    from test_gpu_interp_backward import pieces_f32

    from mps_pointops import three_interpolate

    g = torch.Generator().manual_seed(m * 7 + n)
    B, C = 2, 5
    feats = torch.randn(B, C, m, generator=g)
    idx = torch.randint(0, m, (B, n, 3), generator=g, dtype=torch.int32)
    idx[:, : n // 3, :] = idx[:, :1, :]  # a hot bucket
    w = torch.rand(B, n, 3, generator=g)
    up = torch.randn(B, C, n, generator=g)
    grads = []
    for _ in range(2):
        fc = feats.cuda().requires_grad_()
        three_interpolate(fc, idx.cuda(), w.cuda()).backward(up.cuda())
        grads.append(host(fc.grad))
    want = np.zeros((B, C, m), np.float32)
    upn, wn, ixn = up.numpy(), w.numpy(), idx.numpy()
    for b in range(B):
        for c in range(C):
            row = want[b, c]
            prod = (upn[b, c][:, None] * wn[b]).astype(np.float32)  # fl32(g * w) per (n, t)
            for j, v in zip(ixn[b].reshape(-1), prod.reshape(-1)):
                row[j] = np.float32(row[j] + v)
    exact = pieces_f32(upn, ixn, wn, m) if m <= 1024 else want
    same_bits(grads[0], exact)
    same_bits(grads[1], grads[0])
    np.testing.assert_allclose(grads[0], want, rtol=1e-5, atol=1e-5)


def test_three_nn_non_finite(cuda_device):
    """NaN distances sort last in index order, +inf ones before them; a NaN
    unknown takes the first three known points (stable argsort)."""
    from mps_pointops import three_nn

    u = rand_cloud(3, 300, 21)
    k = rand_cloud(3, 70, 22)
    k[0, 5] = float("nan")
    k[0, 9, 1] = float("inf")
    k[0, 10, 2] = -float("inf")
    k[1, 2:] = float("nan")  # two finite known points: the third is the first NaN
    k[2, :, 0] = float("inf")  # every distance is +inf or NaN
    k[2, 40] = torch.tensor([1.0, 2.0, 3.0])
    u[0, 3] = float("nan")
    u[1, 7, 0] = -float("inf")
    want_d, want_i = O.three_nn(u, k)
    d, i = three_nn(u.cuda(), k.cuda())
    np.testing.assert_array_equal(host(i), want_i)
    got = host(d)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(want_d))
    fin = ~np.isnan(want_d)
    same_bits(got[fin], want_d[fin])


@pytest.mark.parametrize("m", [3, 4, 50, 1025, 2100])
def test_three_nn_matches_oracle(cuda_device, m):
    from mps_pointops import three_nn

    u = rand_cloud(2, 300, m)
    k = rand_cloud(2, m, m + 1)
    k[:, m // 2:] = k[:, : m - m // 2]
    want_d, want_i = O.three_nn(u, k)
    d, i = three_nn(u.cuda(), k.cuda())
    np.testing.assert_array_equal(host(i), want_i)
    same_bits(host(d), want_d)


def test_three_nn_nonfinite(cuda_device):
    from mps_pointops import three_nn

    u = torch.zeros(1, 2, 3)
    u[0, 1, 0] = float("nan")
    k = torch.tensor([[[np.nan, 0, 0], [np.inf, 0, 0], [1, 0, 0], [np.nan, 0, 0], [2, 0, 0]]]).float()
    want_d, want_i = O.three_nn(u, k)
    d, i = three_nn(u.cuda(), k.cuda())
    np.testing.assert_array_equal(host(i), want_i)


@pytest.mark.parametrize("dim,norm,dtype", [(3, 2, torch.float32), (3, 1, torch.float32),
                                            (5, 2, torch.float32), (64, 1, torch.float32),
                                            (3, 2, torch.float64), (2, 1, torch.float64)])
def test_chamfer_nearest_matches_oracle(cuda_device, dim, norm, dtype):
    from mps_pointops import chamfer

    g = torch.Generator().manual_seed(dim * 10 + norm)
    q = torch.randn(3, 300, dim, generator=g, dtype=torch.float64).to(dtype)
    r = (torch.round(torch.randn(3, 2100, dim, generator=g, dtype=torch.float64) * 2) / 2).to(dtype)
    ql, rl = [300, 40, 299], [2100, 1025, 3]
    want_d, want_i = O.chamfer_nearest(q, r, ql, rl, norm)
    d, i = chamfer._nearest_mps(q.cuda(), r.cuda(), _batch(ql), _batch(rl), norm=norm)
    np.testing.assert_array_equal(host(i), want_i)
    np.testing.assert_array_equal(host(d), want_d)


def test_chamfer_c5_forward_backward_reduced(cuda_device):
    """Config 5 generator at B=4 (the oracle's cost is quadratic): loss and
    both gradients against the closed form on the oracle's pairs."""
    import mps_pointops as mp

    y1, y2 = bench.make_c5(B=4, P=2048)
    a = y1.cuda().requires_grad_()
    b = y2.cuda().requires_grad_()
    loss, _ = mp.chamfer_distance(a, b)
    loss.backward()
    d12, i12 = O.chamfer_nearest(y1, y2)
    d21, i21 = O.chamfer_nearest(y2, y1)
    want_loss = (d12.astype(np.float64).mean(1) + d21.astype(np.float64).mean(1)).mean()
    np.testing.assert_allclose(loss.item(), want_loss, rtol=1e-5)
    B, P = 4, 2048
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


def _nearest_grid_case(case: str) -> tuple[torch.Tensor, torch.Tensor]:
    g = torch.Generator().manual_seed({"c5_xy": 0, "c5_yx": 0, "cube": 1, "duplicates": 2,
                                       "shell_far_queries": 3, "overflow": 4}[case])
    if case in ("c5_xy", "c5_yx"):
        y1, y2 = bench.make_c5()
        return (y1, y2) if case == "c5_xy" else (y2, y1)
    if case == "cube":
        return torch.rand(4, 9000, 3, generator=g), torch.rand(4, 8192, 3, generator=g)
    if case == "duplicates":
        base = torch.randn(500, 3, generator=g)
        pick = torch.randint(0, 500, (3, 12000), generator=g)
        return base[pick[:, :5000]].contiguous(), base[pick[:, 3000:]].contiguous()
    if case == "overflow":  # squared distances of the far half overflow to +inf
        q = torch.rand(2, 5000, 3, generator=g)
        r = torch.rand(2, 9000, 3, generator=g)
        q[:, ::2] *= 3e19
        r[:, 1::3] *= -3e19
        return q, r
    ref = torch.randn(2, 10000, 3, generator=g)
    ref = ref / ref.norm(dim=-1, keepdim=True)  # a shell: the interior is empty
    return torch.rand(2, 6000, 3, generator=g) * 0.2 - 0.1, ref


@pytest.mark.parametrize("case", ["c5_xy", "c5_yx", "cube", "duplicates", "shell_far_queries",
                                  "overflow"])
def test_chamfer_nearest_grid_matches_scan(cuda_device, case):
    """The grid search (and the scan inside it for far queries: every query
    of the shell case is far) returns the linear scan's squared distances
    and indices bit for bit, ties to the smallest index included."""
    from mps_pointops import chamfer

    q, r = (t.cuda().contiguous() for t in _nearest_grid_case(case))
    B, M, N = q.shape[0], q.shape[1], r.shape[1]
    ql = torch.full((B,), M, dtype=torch.int64, device=q.device)
    rl = torch.full((B,), N, dtype=torch.int64, device=q.device)
    assert chamfer._grid_eligible(q, r, 2, True)
    d, i = chamfer._nearest_device(q, r, ql, rl, 2, full=True)
    sd, si = chamfer._nearest_scan(q, r, ql, rl, 2)
    assert torch.equal(i, si)
    assert torch.equal(d.view(torch.int32), sd.view(torch.int32))
    assert int((i < 0).sum()) == 0


def test_chamfer_nearest_grid_matches_oracle(cuda_device):
    """Config 5's clouds at B=2 through the grid path against the oracle."""
    from mps_pointops import chamfer

    y1, y2 = bench.make_c5(B=2)
    for q, r in ((y1, y2), (y2, y1)):
        B, M, N = q.shape[0], q.shape[1], r.shape[1]
        ql = torch.full((B,), M, dtype=torch.int64, device="cuda")
        rl = torch.full((B,), N, dtype=torch.int64, device="cuda")
        qc, rc = q.cuda(), r.cuda()
        assert chamfer._grid_eligible(qc, rc, 2, True) == (B * M * N >= chamfer._GRID_MIN_PAIRS)
        d, i = chamfer._nearest_grid(qc, rc)
        want_d, want_i = O.chamfer_nearest(q, r)
        np.testing.assert_array_equal(host(i), want_i)
        np.testing.assert_array_equal(host(d), want_d)


def test_chamfer_c5_grid_path_equals_scan_path(cuda_device):
    """Full config 5: chamfer_distance without lengths (grid search) and with
    explicit full lengths (linear scan) give bit-identical losses; gradients
    agree to float rounding (the backward accumulates the reference side with
    atomics, so its summation order varies from run to run)."""
    import mps_pointops as mp

    y1, y2 = bench.make_c5()
    out = []
    for lengths in (None, torch.full((y1.shape[0],), y1.shape[1], dtype=torch.int64).cuda()):
        a = y1.cuda().requires_grad_()
        b = y2.cuda().requires_grad_()
        loss, _ = mp.chamfer_distance(a, b, x_lengths=lengths, y_lengths=lengths)
        loss.backward()
        out.append((loss.detach(), a.grad, b.grad))
    assert torch.equal(out[0][0].view(torch.int32), out[1][0].view(torch.int32))
    for got, want in zip(out[0][1:], out[1][1:]):
        torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-9)


@pytest.mark.parametrize("k", [1, 4, 40, 256])
def test_flat_knn_radius_match_oracle(cuda_device, k):
    from mps_pointops import flat

    rng = np.random.default_rng(k)
    x = rng.random((3000, 3), dtype=np.float32)
    y = rng.random((500, 3), dtype=np.float32)
    bx = np.sort(rng.integers(0, 5, 3000))
    by = np.sort(rng.integers(0, 5, 500))
    size = int(max(bx.max(), by.max())) + 1
    px = np.searchsorted(bx, np.arange(size + 1)).astype(np.int64)
    py = np.searchsorted(by, np.arange(size + 1)).astype(np.int64)
    xc, yc = torch.from_numpy(x).cuda(), torch.from_numpy(y).cuda()
    bxc, byc = torch.from_numpy(bx).cuda(), torch.from_numpy(by).cuda()
    got = flat.knn(xc, yc, k, bxc, byc)
    want = O.knn_flat(x, y, px, py, min(k, len(x)))
    q, s = np.nonzero(want >= 0)
    assert got.cpu().tolist() == [q.tolist(), want[q, s].tolist()]
    got = flat.radius(xc, yc, 0.07, bxc, byc, max_num_neighbors=k)
    want = O.radius_flat(x, y, px, py, 0.07, min(k, len(x)))
    q, s = np.nonzero(want >= 0)
    assert got.cpu().tolist() == [q.tolist(), want[q, s].tolist()]
    feats = rng.standard_normal((3000, 16)).astype(np.float32)
    qf = rng.standard_normal((500, 16)).astype(np.float32)
    got = flat.knn(torch.from_numpy(feats).cuda(), torch.from_numpy(qf).cuda(), min(k, 64), bxc, byc)
    want = O.knn_flat(feats, qf, px, py, min(k, 64))
    q, s = np.nonzero(want >= 0)
    assert got.cpu().tolist() == [q.tolist(), want[q, s].tolist()]


def test_flat_fps_ragged_matches_oracle(cuda_device):
    from mps_pointops import flat

    g = torch.Generator().manual_seed(7)
    x = torch.rand(20000, 3, generator=g)
    ptr = [0, 2, 82, 82, 87, 9087, 20000]
    lengths = np.diff(ptr)
    got = flat.fps(x.cuda(), ptr=ptr, ratio=0.25, random_start=False)
    counts = np.ceil(lengths.astype(np.float32) * np.float32(0.25)).astype(np.int64)
    out_ptr = np.concatenate([[0], np.cumsum(counts)])
    want = O.fps_flat(x, ptr, out_ptr, np.zeros(len(lengths), np.int64))
    np.testing.assert_array_equal(host(got), want)


def test_repeated_dispatch_is_stable(cuda_device):
    import mps_pointops as mp

    x = bench.make_c2(B=4).cuda()
    first = mp.furthest_point_sample(x, 256)
    c = x.gather(1, first[..., None].expand(-1, -1, 3)).contiguous()
    bq = mp.ball_query(c, x, 0.2, 32)[1]
    kn = mp.knn(c, x, 16)[1]
    for _ in range(20):
        assert torch.equal(mp.furthest_point_sample(x, 256), first)
        assert torch.equal(mp.ball_query(c, x, 0.2, 32)[1], bq)
        assert torch.equal(mp.knn(c, x, 16)[1], kn)


# ------------------------------------------------------- PointNet++ grouping


def group_backward_pieces(go: np.ndarray, idx: np.ndarray, N: int, piece: int = 32) -> np.ndarray:
    """float32 grouping gradient in the CSR kernel's order: per batch the
    entries sorted by (point, p) -- the CSR -- are cut into pieces at every
    `piece`-th position; each piece is summed from +0 in p order and a
    point's pieces are added in order.  (Lists longer than 256 entries are
    in an unspecified order on the device: callers keep them shorter.)"""
    B, C, P = go.shape
    out = np.zeros((B, C, N), np.float32)
    for b in range(B):
        keys = np.clip(idx[b].reshape(-1).astype(np.int64), 0, N - 1)
        order = np.argsort(keys, kind="stable")
        starts = np.searchsorted(keys[order], np.arange(N + 1))
        vals = go[b][:, order].astype(np.float32)
        for n in range(N):
            q, e = int(starts[n]), int(starts[n + 1])
            total = None
            while q < e:
                cut = min(e, (q // piece + 1) * piece)
                part = np.zeros(C, np.float32)
                for k in range(q, cut):
                    part = (part + vals[:, k]).astype(np.float32)
                total = part if total is None else (total + part).astype(np.float32)
                q = cut
            if total is not None:
                out[b, :, n] = total
    return out


@pytest.mark.parametrize("bits", [32, 64])
@pytest.mark.parametrize("B,C,N,P", [(3, 67, 500, 1000), (2, 16, 4096, 32 * 33), (1, 1, 7, 1)])
def test_group_points_matches_oracle(cuda_device, bits, B, C, N, P):
    """Forward bit for bit; backward (points gathered many times) bit for bit
    against the kernel's documented order (pieces of 32 list positions) and
    within 1e-5 of the sequential scatter-add in p order."""
    from mps_pointops import group

    g = torch.Generator().manual_seed(B * 1000 + C + P)
    f = torch.randn(B, C, N, generator=g)
    idx = torch.randint(0, min(N, 37), (B, P), generator=g, dtype=torch.int64)
    idx = idx.to(torch.int32 if bits == 32 else torch.int64)
    fc = f.cuda().requires_grad_()
    out = group.group_points(fc, idx.cuda())
    np.testing.assert_array_equal(host(out), O.group_points(f.numpy(), idx.numpy()))
    go = torch.randn(B, C, P, generator=g)
    out.backward(go.cuda())
    got = host(fc.grad)
    same_bits(got, group_backward_pieces(go.numpy(), idx.numpy(), N))
    np.testing.assert_allclose(got, O.group_points_backward(go.numpy(), idx.numpy(), N),
                               rtol=1e-5, atol=1e-5)


def test_group_points_backward_c2_set_abstraction(cuda_device):
    """Config 2's set-abstraction gradient (C = 64 + 3 channels, the
    pointnet2-form r = 0.2, K = 32 ball query of the FPS centres: lists up to
    ~200 entries, most points in none): the documented order bit for bit,
    the sequential oracle within 1e-5 of the sum of absolute terms, the
    same bits twice."""
    from mps_pointops import compat

    x = bench.make_c2(B=4)
    xc = x.cuda()
    sampled = compat.furthest_point_sample(xc, 1024)
    centres = compat.gather_operation(xc.transpose(1, 2).contiguous(), sampled)
    idx = compat.ball_query(0.2, 32, xc, centres.transpose(1, 2).contiguous())
    B, M, S = idx.shape
    g = torch.Generator().manual_seed(77)
    f = torch.randn(B, 67, 4096, generator=g).cuda().requires_grad_()
    go = torch.randn(B, 67, M * S, generator=g)
    runs = []
    for _ in range(2):
        f.grad = None
        compat.grouping_operation(f, idx).backward(go.cuda().reshape(B, 67, M, S))
        runs.append(host(f.grad))
    flat = host(idx).reshape(B, M * S)
    lens = np.stack([np.bincount(flat[b], minlength=4096) for b in range(B)])
    assert 50 < lens.max() <= 256
    same_bits(runs[0], group_backward_pieces(go.numpy(), flat, 4096))
    same_bits(runs[1], runs[0])
    want = O.group_points_backward(go.numpy(), flat, 4096)
    scale = O.group_points_backward(np.abs(go.numpy()), flat, 4096)
    assert (np.abs(runs[0] - want) <= 1e-5 * scale + 1e-30).all()


@pytest.mark.parametrize("bits", [32, 64])
@pytest.mark.parametrize("B,C,N,M,S", [(2, 5, 100, 30, 10),    # 8 rows per workgroup, one group
                                       (2, 67, 2049, 70, 9),   # 4 rows, a partial last group
                                       (1, 9, 8193, 50, 7),    # 1 row per workgroup
                                       (1, 3, 20_000, 40, 8),  # rows too long for LDS
                                       (3, 0, 4096, 64, 32)])  # relative xyz only
def test_group_points_and_rel_lds_and_fallback(cuda_device, bits, B, C, N, M, S):
    """Both grouping kernels (LDS-staged rows for clouds whose rows fit, the
    L2 gather otherwise) against the oracle, bit for bit, with out-of-order
    and repeated indices."""
    from mps_pointops import group

    g = torch.Generator().manual_seed(B * 7 + C * 11 + N + M * S + bits)
    x = torch.randn(B, N, 3, generator=g)
    centres = torch.randn(B, M, 3, generator=g)
    f = torch.randn(B, C, N, generator=g)
    idx = torch.randint(0, N, (B, M, S), generator=g, dtype=torch.int64)
    idx[:, :, 1] = idx[:, :, 0]
    idx = idx.to(torch.int32 if bits == 32 else torch.int64)
    xc, cc, fc, ic = x.cuda(), centres.cuda(), f.cuda(), idx.cuda()
    print(f"group lds B={B} C={C} N={N} M={M} S={S} bits={bits}", flush=True)
    rel = group.query_and_group(xc, cc, fc if C else None, ic)
    want = O.group_points_rel(x.numpy(), centres.numpy(), f.numpy() if C else None, idx.numpy())
    np.testing.assert_array_equal(host(rel), want)
    if C:
        flat = ic.reshape(B, M * S)
        out = group.group_points(fc, flat)
        np.testing.assert_array_equal(host(out), O.group_points(f.numpy(), flat.cpu().numpy()))


@pytest.mark.parametrize("case", ["c2", "sparse", "radius_zero", "non_finite", "k_large", "ragged"])
def test_compat_ball_query_single_launch(cuda_device, case):
    """compat.ball_query's one-launch int32 path (pointnet2 padding in the
    kernel) equals the composition it replaces -- the index-order ball
    query, -1 replaced by the first neighbour (0 without one), int32 -- and
    the oracle's first-K answer."""
    from mps_pointops import compat, ops

    g = torch.Generator().manual_seed(len(case) * 13)
    radius, k = 0.2, 32
    if case == "c2":
        x = bench.make_c2(B=3)
        c = x[:, torch.randperm(4096, generator=g)[:500]].clone()
    elif case == "sparse":  # many queries with few or no neighbours
        x = torch.rand(2, 3000, 3, generator=g) * 10
        c = torch.rand(2, 700, 3, generator=g) * 12 - 1
        radius = 0.4
    elif case == "radius_zero":
        x = torch.rand(2, 500, 3, generator=g)
        c = x[:, :64].clone()
        radius = 0.0
    elif case == "non_finite":
        x = torch.rand(2, 2000, 3, generator=g)
        x[0, 5] = float("nan")
        x[1, 17, 2] = float("inf")
        c = torch.rand(2, 300, 3, generator=g)
        c[0, 3] = float("nan")
    elif case == "k_large":
        x = torch.rand(1, 5000, 3, generator=g)
        c = torch.rand(1, 200, 3, generator=g)
        radius, k = 0.3, 130
    else:
        x = torch.rand(3, 1037, 3, generator=g)
        c = torch.rand(3, 77, 3, generator=g)
        k = 5
    xc, cc = x.cuda().contiguous(), c.cuda().contiguous()
    got = compat.ball_query(radius, k, xc, cc)
    assert got.dtype == torch.int32 and got.shape == (x.shape[0], c.shape[1], k)
    _, idx = ops.ball_query(cc, xc, radius, k)
    first = idx.narrow(-1, 0, 1).clamp_min(0)
    want = idx.where(idx >= 0, first).int()
    np.testing.assert_array_equal(host(got), host(want))
    _, oi = O.ball_query(c, x, radius, k)
    of = np.where(oi[..., :1] >= 0, oi[..., :1], 0)
    np.testing.assert_array_equal(host(got), np.where(oi >= 0, oi, of).astype(np.int32))


def test_compat_gather_grouping_known_answers(cuda_device):
    """tests/test_compat.py:121-137 on the GPU path."""
    from mps_pointops import compat

    features = torch.randn(2, 4, 30).cuda()
    idx = torch.randint(0, 30, (2, 7), dtype=torch.int32).cuda()
    out = compat.gather_operation(features, idx)
    assert out.shape == (2, 4, 7)
    assert torch.equal(out[1, :, 3], features[1, :, idx[1, 3]])
    gidx = torch.randint(0, 30, (2, 7, 5), dtype=torch.int32).cuda()
    out = compat.grouping_operation(features, gidx)
    assert out.shape == (2, 4, 7, 5)
    assert torch.equal(out[0, :, 6, 2], features[0, :, gidx[0, 6, 2]])
    leaf = torch.randn(1, 3, 10).cuda().requires_grad_()
    compat.gather_operation(leaf, torch.tensor([[2, 2, 5]]).cuda()).sum().backward()
    assert leaf.grad[0, 0].tolist() == [0, 0, 2, 0, 0, 1, 0, 0, 0, 0]
    with pytest.raises(IndexError):
        compat.gather_operation(features, torch.tensor([[0, 30]] * 2).cuda())


def test_query_and_group_matches_oracle_and_composition(cuda_device):
    """The fused grouping equals the oracle bit for bit and the reference
    layer's composition (tests/test_pointnet2_e2e.py:38-44: gather, ball
    query, two groupings, subtraction, concatenation); gradients match the
    composition's autograd on the CPU."""
    from mps_pointops import compat, group

    x = bench.make_c2(B=4, N=1024)
    feats = torch.randn(4, 19, 1024, generator=torch.Generator().manual_seed(9))
    xc, fc = x.cuda(), feats.cuda()
    sampled = compat.furthest_point_sample(xc, 128)
    new_xyz = compat.gather_operation(xc.transpose(1, 2).contiguous(), sampled).transpose(1, 2).contiguous()
    idx = compat.ball_query(0.2, 24, xc, new_xyz)
    fused = group.QueryAndGroup(0.2, 24)(xc, new_xyz, fc)
    want = O.group_points_rel(x.numpy(), host(new_xyz), feats.numpy(), host(idx))
    np.testing.assert_array_equal(host(fused), want)
    gx = compat.grouping_operation(xc.transpose(1, 2).contiguous(), idx) - new_xyz.transpose(1, 2).unsqueeze(-1)
    composed = torch.cat((gx, compat.grouping_operation(fc, idx)), dim=1)
    assert torch.equal(fused, composed)
    # Centres are cloud points: wherever a centre is grouped with its own
    # point the relative channels are exactly 0.
    own = host(idx) == host(sampled)[:, :, None]
    assert own.any()
    assert (host(fused)[:, :3][np.broadcast_to(own[:, None], (4, 3) + own.shape[1:])] == 0).all()
    assert group.QueryAndGroup(0.2, 24, use_xyz=False)(xc, new_xyz, fc).shape == (4, 19, 128, 24)
    # Gradients to xyz, centres and features.
    a = xc.clone().requires_grad_()
    c = new_xyz.clone().requires_grad_()
    f = fc.clone().requires_grad_()
    go = torch.randn(fused.shape, generator=torch.Generator().manual_seed(10))
    group.query_and_group(a, c, f, idx).backward(go.cuda())
    ac, cc, fcp = (t.detach().cpu().requires_grad_() for t in (xc, new_xyz, fc))
    il = host(idx).astype(np.int64)
    B, M, S = il.shape
    flat = torch.from_numpy(il).reshape(B, 1, M * S)
    rel = ac.transpose(1, 2).gather(2, flat.expand(B, 3, -1)).reshape(B, 3, M, S) - cc.transpose(1, 2).unsqueeze(-1)
    ref_out = torch.cat((rel, fcp.gather(2, flat.expand(B, 19, -1)).reshape(B, 19, M, S)), 1)
    ref_out.backward(go)
    for got, ref in ((a, ac), (c, cc), (f, fcp)):
        np.testing.assert_allclose(host(got.grad), ref.grad.numpy(), rtol=1e-5, atol=1e-5)


# ------------------------------------------------ PyTorch3D-style ball query
# Known answers of tests/test_pytorch3d_adapter.py, on the ROCm device.


def test_pytorch3d_defaults_and_zero_padded_neighbors(cuda_device):
    from mps_pointops.pytorch3d import KNN, ball_query

    queries = torch.zeros((1, 1, 3), device="cuda")
    points = torch.tensor([[[0.125, 0.0, 0.0], [2.0, 0.0, 0.0]]], device="cuda")
    result = ball_query(queries, points)
    assert isinstance(result, KNN)
    assert result._fields == ("dists", "idx", "knn")
    assert result.dists.shape == result.idx.shape == (1, 1, 500)
    assert result.knn.shape == (1, 1, 500, 3)
    assert result.dists.dtype == torch.float32 and result.idx.dtype == torch.int64
    assert result.idx[0, 0, 0].item() == 0 and torch.all(result.idx[0, 0, 1:] == -1)
    assert result.dists[0, 0, 0].item() == 0.015625 and torch.all(result.dists[0, 0, 1:] == 0)
    assert torch.equal(result.knn[0, 0, 0], points[0, 0])
    assert torch.all(result.knn[0, 0, 1:] == 0)


def test_pytorch3d_ragged_lengths_and_cube_hint(cuda_device):
    from mps_pointops.pytorch3d import ball_query

    queries = torch.tensor([[[0.0, 0, 0], [0.0, 0, 0]], [[3.0, 0, 0], [0.0, 0, 0]]], device="cuda")
    points = torch.tensor([[[0.5, 0, 0], [0.25, 0, 0], [0.125, 0, 0], [2.0, 0, 0]],
                           [[0.125, 0, 0], [0.25, 0, 0], [2.0, 0, 0], [3.0, 0, 0]]], device="cuda")
    l1 = torch.tensor([1, 2], device="cuda")
    l2 = torch.tensor([2, 1], device="cuda")
    default = ball_query(queries, points, l1, l2, 3, 1.0, True, False)
    cube = ball_query(queries, points, l1, l2, 3, 1.0, True, True)
    no_nn = ball_query(queries, points, l1, l2, 3, 1.0, False, True)
    assert default.idx.cpu().tolist() == [[[0, 1, -1], [-1, -1, -1]], [[-1, -1, -1], [0, -1, -1]]]
    assert default.dists.cpu().tolist() == [[[0.25, 0.0625, 0], [0, 0, 0]], [[0, 0, 0], [0.015625, 0, 0]]]
    assert torch.equal(cube.idx, default.idx) and torch.equal(cube.dists, default.dists)
    assert no_nn.knn is None
    assert default.knn[0, 0, 0, 0].item() == 0.5 and default.knn[0, 0, 1, 0].item() == 0.25
    assert torch.all(default.knn[default.idx == -1] == 0)


@pytest.mark.parametrize("B,Q,P,k", [(1, 2, 0, 3), (1, 2, 2, 0), (1, 0, 2, 3), (0, 2, 2, 3)])
def test_pytorch3d_empty_dimensions(cuda_device, B, Q, P, k):
    from mps_pointops.pytorch3d import ball_query

    result = ball_query(torch.zeros((B, Q, 3), device="cuda"), torch.zeros((B, P, 3), device="cuda"),
                        K=k, radius=1.0)
    assert result.dists.shape == result.idx.shape == (B, Q, k)
    assert result.knn.shape == (B, Q, k, 3)
    assert torch.all(result.idx == -1) and torch.all(result.dists == 0) and torch.all(result.knn == 0)


def test_pytorch3d_gradients(cuda_device):
    from mps_pointops.pytorch3d import ball_query

    q = torch.zeros((1, 1, 3), device="cuda", requires_grad=True)
    p = torch.tensor([[[0.25, 0.0, 0.0]]], device="cuda", requires_grad=True)
    r = ball_query(q, p, K=2, radius=1.0)
    (r.dists.sum() + r.knn.sum()).backward()
    assert q.grad.cpu().tolist() == [[[-0.5, 0.0, 0.0]]]
    assert p.grad.cpu().tolist() == [[[1.5, 1.0, 1.0]]]
    for P, k in ((0, 2), (2, 0)):
        pts = torch.zeros((1, P, 3), device="cuda", requires_grad=True)
        ball_query(torch.zeros((1, 1, 3), device="cuda"), pts, K=k, radius=1.0).knn.sum().backward()
        assert pts.grad is not None and torch.all(pts.grad == 0)


def test_pytorch3d_rejects_invalid_lengths(cuda_device):
    from mps_pointops.pytorch3d import ball_query

    points = torch.zeros((1, 2, 3), device="cuda")
    with pytest.raises(ValueError, match="lengths1|query_lengths"):
        ball_query(points, points, lengths1=torch.tensor([3], device="cuda"), K=1, radius=1.0)


# ------------------------------------------------------- Pointcept shim
# Known answers of tests/test_pointcept.py, on the ROCm device.


def test_pointcept_fps_offsets_and_int32(cuda_device):
    from mps_pointops import pointcept

    xyz = torch.tensor([[0., 0, 0], [1., 0, 0], [4., 0, 0], [9., 0, 0], [10., 0, 0], [11., 0, 0],
                        [15., 0, 0]], device="cuda")
    out = pointcept.farthest_point_sampling(xyz, torch.tensor([4, 7], dtype=torch.int32, device="cuda"),
                                            torch.tensor([2, 4], dtype=torch.int32, device="cuda"))
    assert out.dtype == torch.int32 and out.cpu().tolist() == [0, 3, 4, 6]


def test_pointcept_knn_padding_ties_ceiling_nonfinite(cuda_device):
    from mps_pointops import pointcept

    xyz = torch.tensor([[0., 0, 0], [2., 0, 0], [10., 0, 0], [12., 0, 0], [14., 0, 0]],
                       device="cuda", requires_grad=True)
    query = torch.tensor([[0.5, 0, 0], [11., 0, 0]], device="cuda", requires_grad=True)
    idx, dist = pointcept.knn_query(4, xyz, torch.tensor([2, 5], device="cuda"), query,
                                    torch.tensor([1, 2], dtype=torch.int32, device="cuda"))
    assert idx.dtype == torch.int32 and idx.cpu().tolist() == [[0, 1, -1, -1], [2, 3, 4, -1]]
    assert dist.cpu().tolist() == [[0.5, 1.5, 1e5, 1e5], [1., 1., 3., 1e5]]
    assert not dist.requires_grad
    x = torch.arange(16, dtype=torch.float32, device="cuda") * 0.25
    line = torch.stack((x, torch.zeros_like(x), torch.zeros_like(x)), dim=1)
    idx, dist = pointcept.knn_query(8, line, torch.tensor([16], dtype=torch.int32, device="cuda"))
    assert idx[2].cpu().tolist() == [2, 1, 3, 0, 4, 5, 6, 7]
    assert dist[2].cpu().tolist() == [0., 0.25, 0.25, 0.5, 0.5, 0.75, 1., 1.25]
    far = torch.tensor([[99_999., 0, 0], [100_000., 0, 0], [100_001., 0, 0]], device="cuda")
    one = torch.tensor([1], dtype=torch.int32, device="cuda")
    idx, dist = pointcept.knn_query(3, far, torch.tensor([3], dtype=torch.int32, device="cuda"),
                                    torch.zeros((1, 3), device="cuda"), one)
    assert idx.cpu().tolist() == [[0, -1, -1]]
    assert dist.cpu().tolist() == [[99_999., 100_000., 100_000.]]
    q0 = torch.zeros((1, 3), device="cuda")
    nb = torch.tensor([0, 1], dtype=torch.int32, device="cuda")
    for bad in (float("nan"), float("inf")):
        pts = torch.tensor([[0., 0, 0], [bad, 0, 0]], device="cuda")
        idx, dist = pointcept.knn_query(1, pts, torch.tensor([1, 2], dtype=torch.int32, device="cuda"), q0, nb)
        assert idx.cpu().tolist() == [[-1]] and dist.cpu().tolist() == [[100_000.]]
        pts = torch.tensor([[0., 0, 0], [bad, 0, 0], [1., 0, 0]], device="cuda")
        idx, dist = pointcept.knn_query(2, pts, torch.tensor([1, 3], dtype=torch.int32, device="cuda"), q0, nb)
        assert idx.cpu().tolist() == [[2, -1]] and dist.cpu().tolist() == [[1., 100_000.]]


def test_pointcept_grouping_query_and_group_interpolation(cuda_device):
    from mps_pointops import pointcept

    xyz = torch.tensor([[0., 0, 0], [1., 0, 0], [2., 0, 0]], device="cuda", requires_grad=True)
    feat = torch.tensor([[1., 2.], [3., 4.], [5., 6.]], device="cuda", requires_grad=True)
    query = torch.tensor([[1., 0, 0]], device="cuda", requires_grad=True)
    idx = torch.tensor([[2, -1, 2]], dtype=torch.int32, device="cuda")
    result = pointcept.grouping(idx, feat, xyz, query, with_xyz=True)
    assert result.shape == (1, 3, 5)
    assert result[0, 1].cpu().tolist() == [0.] * 5 and result[0, 0].cpu().tolist() == [1., 0, 0, 5, 6]
    result.sum().backward()
    assert feat.grad.cpu().tolist() == [[0., 0], [0, 0], [2, 2]]
    assert xyz.grad.cpu().tolist() == [[0., 0, 0], [0, 0, 0], [2, 2, 2]]
    assert query.grad.cpu().tolist() == [[-2., -2, -2]]

    xyz = torch.tensor([[0., 0, 0], [2., 0, 0]], device="cuda", requires_grad=True)
    feat = torch.tensor([[2.], [10.]], device="cuda", requires_grad=True)
    query = torch.tensor([[0.5, 0, 0]], device="cuda", requires_grad=True)
    off = torch.tensor([2], dtype=torch.int32, device="cuda")
    noff = torch.tensor([1], dtype=torch.int32, device="cuda")
    grouped, idx = pointcept.knn_query_and_group(feat, xyz, off, query, noff, nsample=3, with_xyz=True)
    assert idx.cpu().tolist() == [[0, 1, -1]]
    reused, same = pointcept.knn_query_and_group(feat, xyz, idx=idx, new_xyz=query)
    assert same is idx and torch.equal(reused, grouped[..., 3:])
    out = pointcept.interpolation(xyz, query, feat, off, noff, k=3)
    torch.testing.assert_close(out.cpu(), torch.tensor([[4.]]), atol=1e-5, rtol=1e-5)
    out.sum().backward()
    torch.testing.assert_close(feat.grad.cpu(), torch.tensor([[0.75], [0.25]]), atol=1e-5, rtol=1e-5)
    assert xyz.grad is None and query.grad is None
    # An empty reference batch interpolates to 0.
    feat = torch.tensor([[3.]], device="cuda", requires_grad=True)
    out = pointcept.interpolation(torch.tensor([[10., 0, 0]], device="cuda"),
                                  torch.tensor([[0., 0, 0], [10., 0, 0]], device="cuda"), feat,
                                  torch.tensor([0, 1], dtype=torch.int32, device="cuda"),
                                  torch.tensor([1, 2], dtype=torch.int32, device="cuda"))
    assert out.cpu().tolist() == [[0.], [3.]]
    out.sum().backward()
    assert feat.grad.cpu().tolist() == [[1.]]


def test_pointcept_knn_matches_oracle_ragged(cuda_device):
    """Random ragged batches against the oracle's flat kNN (global indices,
    (squared distance, index) order), with the 1e5 padding of short batches."""
    from mps_pointops import pointcept

    g = torch.Generator().manual_seed(21)
    counts, qcounts = [300, 0, 7, 1000], [50, 20, 30, 40]
    xyz = torch.rand(sum(counts), 3, generator=g)
    q = torch.rand(sum(qcounts), 3, generator=g)
    ends = torch.tensor(counts).cumsum(0)
    qends = torch.tensor(qcounts).cumsum(0)
    idx, dist = pointcept.knn_query(16, xyz.cuda(), ends.cuda(), q.cuda(), qends.cuda())
    ptr_x = np.concatenate([[0], ends.numpy()])
    ptr_y = np.concatenate([[0], qends.numpy()])
    want = O.knn_flat(xyz.numpy(), q.numpy(), ptr_x, ptr_y, 16)
    np.testing.assert_array_equal(host(idx), want)
    d = host(dist)
    assert (d[want < 0] == 1e5).all()
    sel = want >= 0
    qq = np.repeat(q.numpy()[:, None, :], 16, 1)[sel]
    delta = (qq - xyz.numpy()[want[sel]]).astype(np.float32)
    squared = (delta[:, 0] * delta[:, 0] + delta[:, 1] * delta[:, 1]) + delta[:, 2] * delta[:, 2]
    same_bits(d[sel], np.sqrt(squared))


def test_group_points_backward_heavily_repeated_point(cuda_device):
    """A point gathered far more than 256 times (all-zero indices, as the
    pointnet2 padding of queries without neighbours produces) sums in an
    unspecified order; with quarter-integer gradients every order is exact,
    so the result still equals the sequential oracle bit for bit (a dropped
    or repeated term would not)."""
    from mps_pointops import group

    g = torch.Generator().manual_seed(31)
    f = torch.randn(2, 70, 100, generator=g).cuda().requires_grad_()
    idx = torch.zeros(2, 40_000, dtype=torch.int32)
    idx[:, ::7] = torch.randint(0, 100, (2, len(range(0, 40_000, 7))), generator=g, dtype=torch.int32)
    go = torch.randint(-8, 9, (2, 70, 40_000), generator=g).float() / 4
    group.group_points(f, idx.cuda()).backward(go.cuda())
    same_bits(host(f.grad), O.group_points_backward(go.numpy(), idx.numpy(), 100))


@pytest.mark.parametrize("B,C,N,P,repeat", [(2, 70, 100, 30_000, True),   # CSR, one huge list
                                             (3, 5, 4096, 32_768, False),  # CSR at its limits
                                             (2, 7, 5000, 3000, False)])   # inverse-index path
def test_group_points_backward_paths(cuda_device, B, C, N, P, repeat):
    """Both backward designs (the per-batch CSR for P <= 32768 and N <= 4096,
    the inverse index with the transposed gradient otherwise) equal the
    sequential oracle bit for bit; a point listed more than 256 times sums in
    the scatter's order, exact here with quarter-integer gradients."""
    from mps_pointops import group

    g = torch.Generator().manual_seed(B + C + N + P)
    f = torch.randn(B, C, N, generator=g).cuda().requires_grad_()
    idx = torch.randint(0, N, (B, P), generator=g, dtype=torch.int32)
    if repeat:
        idx[:, ::7] = 0
        idx[:, 1::7] = 0
        idx[:, 2::3] = 0
    go = torch.randint(-8, 9, (B, C, P), generator=g).float() / 4
    print(f"group backward B={B} C={C} N={N} P={P}", flush=True)
    group.group_points(f, idx.cuda()).backward(go.cuda())
    same_bits(host(f.grad), O.group_points_backward(go.numpy(), idx.numpy(), N))


def _grid_sweep_case(seed: int):
    """Random shapes and distributions for the grid search: uniform boxes,
    Gaussian blobs, sphere surfaces, points on a line (degenerate extents)
    and heavily duplicated points."""
    g = torch.Generator().manual_seed(1000 + seed)
    B = int(torch.randint(1, 4, (1,), generator=g))
    N = int(torch.randint(2000, 40_000, (1,), generator=g))
    M = int(torch.randint(50, 2500, (1,), generator=g))
    kind = seed % 5
    if kind == 0:
        ref = torch.rand(B, N, 3, generator=g) * float(torch.rand(1, generator=g) * 100 + 0.01)
    elif kind == 1:
        cen = torch.randn(B, 8, 3, generator=g) * 5
        ref = cen[:, torch.randint(0, 8, (N,), generator=g)] + torch.randn(B, N, 3, generator=g) * 0.3
    elif kind == 2:
        d = torch.randn(B, N, 3, generator=g)
        ref = d / d.norm(dim=-1, keepdim=True)
    elif kind == 3:
        t = torch.rand(B, N, 1, generator=g)
        ref = t * torch.tensor([1.0, 2.0, -0.5]) + 3.0
    else:
        base = torch.rand(B, N // 50 + 1, 3, generator=g)
        ref = base[:, torch.randint(0, base.shape[1], (N,), generator=g)]
    pick = torch.randint(0, N, (M,), generator=g)
    query = ref[:, pick] + torch.randn(B, M, 3, generator=g) * 0.05
    return query.contiguous(), ref.contiguous()


@pytest.mark.parametrize("seed", range(10))
@pytest.mark.parametrize("k", [3, 12, 32])
def test_knn3_grid_random_sweep(cuda_device, seed, k):
    query, ref = _grid_sweep_case(seed)
    want_d, want_i = O.knn3(query, ref, k)
    d, i = _knn3_grid(query, ref, k)
    np.testing.assert_array_equal(i, want_i)
    same_bits(d, want_d)


# ------------------------------------------------------- grid ball query


def _ball_grid(query: torch.Tensor, ref: torch.Tensor, radius: float, k: int):
    """pointops_ball_query_grid_f32 through the C ABI (any cloud size)."""
    from mps_pointops import _native

    q, r = query.cuda().contiguous(), ref.cuda().contiguous()
    B, Q, _ = q.shape
    P = r.shape[1]
    dist = torch.empty(B, Q, k, device="cuda")
    idx = torch.empty(B, Q, k, dtype=torch.long, device="cuda")
    size = _native.size_query("pointops_ball_query_grid_workspace_bytes", B, Q, P)
    ws = torch.empty(size, dtype=torch.uint8, device="cuda")
    _native.call("pointops_ball_query_grid_f32", q.data_ptr(), r.data_ptr(), idx.data_ptr(),
                 dist.data_ptr(), ws.data_ptr(), B, Q, P, k, O.ball_radius_sq(radius),
                 _native.stream(q.device))
    return host(dist), host(idx)


@pytest.mark.parametrize("name,radius", [("uniform", 0.4), ("slab", 0.5), ("ties", 1.0),
                                         ("far_queries", 0.3), ("sparse_clusters", 2.0),
                                         ("flat", 0.05), ("one_point", 0.5),
                                         ("non_finite_refs", 0.2), ("non_finite_queries", 0.2),
                                         ("uniform", 0.0), ("uniform", 1e30)])
@pytest.mark.parametrize("k", [1, 16, 32, 64])
def test_ball_query_grid_matches_oracle(cuda_device, name, radius, k):
    """The grid ball query returns the index-order first-K answer bit for bit
    (also radius 0: no hit, and a radius whose square overflows: every finite
    point)."""
    query, ref = _grid_case(name)
    want_d, want_i = O.ball_query(query, ref, radius, k)
    d, i = _ball_grid(query, ref, radius, k)
    np.testing.assert_array_equal(i, want_i)
    same_bits(d, want_d)


@pytest.mark.parametrize("seed", range(6))
def test_ball_query_grid_random_sweep(cuda_device, seed):
    query, ref = _grid_sweep_case(seed)
    span = float((ref.amax(1) - ref.amin(1)).max())
    for frac, k in ((0.01, 8), (0.05, 32), (0.2, 64)):
        want_d, want_i = O.ball_query(query, ref, span * frac, k)
        d, i = _ball_grid(query, ref, span * frac, k)
        np.testing.assert_array_equal(i, want_i)
        same_bits(d, want_d)


def test_ball_query_grid_public_path(cuda_device):
    """ops.ball_query uses the grid search for large clouds without lengths;
    results equal the index-order kernel's, and gradients still flow."""
    import mps_pointops as mp
    from mps_pointops import _native

    g = torch.Generator().manual_seed(12)
    ref = bench.make_c3(N=80_000)
    query = ref[:, torch.randperm(80_000, generator=g)[:3000]].clone()
    q, r = query.cuda().requires_grad_(), ref.cuda()
    d, i = mp.ball_query(q, r, 0.5, 32)
    bd = torch.empty_like(d)
    bi = torch.empty_like(i)
    _native.call("pointops_ball_query_f32", q.data_ptr(), r.data_ptr(), None, None, bi.data_ptr(),
                 bd.data_ptr(), 1, 3000, 80_000, 32, O.ball_radius_sq(0.5), _native.stream(q.device))
    np.testing.assert_array_equal(host(i), host(bi))
    same_bits(host(d), host(bd))
    d.sum().backward()
    assert q.grad is not None and torch.isfinite(q.grad).all()


def _expected_choice(ref: np.ndarray, radius_sq: float, k: int) -> int:
    """The documented grid/index-order rule restated on the host: lambda =
    P (4/3) pi r^3 / V, V the smallest per-cloud box volume (float32, each
    side at least 2r), grid while lambda < sqrt(P K / 6.4)."""
    if not 0.0 < radius_sq < math.inf:
        return 0
    r = math.sqrt(radius_sq)
    side = np.float32(2.0 * r)
    volumes = []
    for cloud in ref:
        finite = cloud[np.isfinite(cloud).all(axis=1)]
        ext = (finite.max(0) - finite.min(0)) if len(finite) else np.full(3, -np.inf, np.float32)
        ext = np.maximum(ext.astype(np.float32), side)
        volumes.append(np.float32(np.float32(ext[0] * ext[1]) * ext[2]))
    v = float(min(volumes))
    if not 0.0 < v < math.inf:
        return 0
    n = ref.shape[1]
    return int(n * (4.0 / 3.0) * math.pi * r ** 3 / v < math.sqrt(n * k / 6.4))


def _ball_auto(query: torch.Tensor, ref: torch.Tensor, radius: float, k: int):
    """pointops_ball_query_auto_f32 through the C ABI into outputs filled
    with garbage (every slot must be written); returns the device's choice."""
    from mps_pointops import _native

    q, r = query.cuda().contiguous(), ref.cuda().contiguous()
    B, Q, _ = q.shape
    P = r.shape[1]
    dist = torch.full((B, Q, k), float("nan"), device="cuda")
    idx = torch.full((B, Q, k), 7, dtype=torch.long, device="cuda")
    size = _native.size_query("pointops_ball_query_auto_workspace_bytes", B, Q, P)
    ws = torch.full((size,), 0xAB, dtype=torch.uint8, device="cuda")
    _native.call("pointops_ball_query_auto_f32", q.data_ptr(), r.data_ptr(), idx.data_ptr(),
                 dist.data_ptr(), ws.data_ptr(), B, Q, P, k, O.ball_radius_sq(radius),
                 _native.stream(q.device))
    choice = int(ws[:4].view(torch.int32).item())
    return host(dist), host(idx), choice


@pytest.mark.parametrize("name,radius,k", [
    ("uniform", 0.4, 16), ("uniform", 3.0, 64), ("uniform", 0.0, 8), ("uniform", 1e30, 4),
    ("slab", 0.5, 32), ("one_point", 0.5, 16), ("non_finite_refs", 0.2, 16),
    ("far_queries", 0.3, 1), ("sparse_clusters", 2.0, 64), ("ties", 1.0, 32)])
def test_ball_query_auto_choice_and_results(cuda_device, name, radius, k):
    """The device-side choice follows the documented rule, and whichever
    search it takes, the result is the index-order answer bit for bit with
    every output slot written."""
    query, ref = _grid_case(name)
    want_d, want_i = O.ball_query(query, ref, radius, k)
    d, i, choice = _ball_auto(query, ref, radius, k)
    assert choice == _expected_choice(ref.numpy(), O.ball_radius_sq(radius), k)
    np.testing.assert_array_equal(i, want_i)
    same_bits(d, want_d)


def test_ball_query_auto_takes_both_paths(cuda_device):
    """The cases above cover both choices (sparse balls: grid, dense or
    degenerate ones: index order)."""
    query, ref = _grid_case("uniform")
    assert _ball_auto(query, ref, 0.4, 16)[2] == 1
    assert _ball_auto(query, ref, 3.0, 64)[2] == 0


def test_ball_query_public_path_in_a_graph(cuda_device):
    """ops.ball_query on a grid-eligible shape synchronises nothing, so it
    can be captured; every replay (new point data copied into the captured
    input between replays, which flips the device-side choice, and eager
    work in between) equals the eager call on the same data."""
    import mps_pointops as mp

    g = torch.Generator().manual_seed(21)
    sparse = torch.rand(1, 40_000, 3, generator=g) * 10
    dense = torch.rand(1, 40_000, 3, generator=g) * 0.5
    queries = (torch.rand(1, 3000, 3, generator=g) * 10).cuda()
    points = sparse.cuda()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        mp.ball_query(queries, points, 0.4, 16)  # warm-up off the capture
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        d, i = mp.ball_query(queries, points, 0.4, 16)
    for cloud in (sparse, dense, sparse, dense):
        points.copy_(cloud.cuda())
        graph.replay()
        torch.cuda.synchronize()
        want_d, want_i = mp.ball_query(queries, points, 0.4, 16)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(host(i), host(want_i))
        same_bits(host(d), host(want_d))
    oracle_d, oracle_i = O.ball_query(queries.cpu(), dense, 0.4, 16)
    np.testing.assert_array_equal(host(i), oracle_i)
    same_bits(host(d), oracle_d)


