"""Pin the CPU oracle before trusting it (CPU only).

Each oracle function is checked against (a) known answers transcribed from the
reference's tests, (b) index arrays the reference recorded on its Metal
kernels, and (c) independent numpy formulations (lexsort, stable argsort,
brute-force first-K, from-scratch max-min).  Mutant formulations show that the
checks discriminate the plausible mistakes (non-strict radius, wrong tie
order, FMA accumulation).
"""

from __future__ import annotations

import struct

import numpy as np
import pytest

from conftest import GOLDEN, load_known_answers, load_pointnet2_parity
from oracle import oracle as O


def sq32(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """((dx*dx + dy*dy) + dz*dz) in float32, one rounding per op."""
    d = (a - b).astype(np.float32)
    s = d[..., 0] * d[..., 0]
    s = s + d[..., 1] * d[..., 1]
    return s + d[..., 2] * d[..., 2]


# ----------------------------------------------------------- known answers

@pytest.mark.parametrize("case", load_known_answers("fps"), ids=lambda c: c["name"])
def test_fps_known_answers(case):
    got = O.fps(np.array(case["xyz"], np.float32), case["npoint"], case["start_idx"], case["skip"])
    assert got.tolist() == case["expect"], case["source"]


@pytest.mark.parametrize("case", load_known_answers("fps_flat"), ids=lambda c: c["name"])
def test_fps_flat_known_answers(case):
    got = O.fps_flat(np.array(case["x"], np.float32), case["ptr"], case["out_ptr"], case["starts"])
    assert got.tolist() == case["expect"], case["source"]


@pytest.mark.parametrize("case", load_known_answers("knn"), ids=lambda c: c["name"])
def test_knn_known_answers(case):
    dist, idx = O.knn(np.array(case["query"], np.float32), np.array(case["ref"], np.float32),
                      case["k"])
    assert idx.tolist() == case["expect_idx"], case["source"]
    np.testing.assert_allclose(dist, np.array(case["expect_dist"], np.float32), rtol=1e-6)


def _ptr(batch, n):
    if batch is None:
        return np.array([0, n], np.int64)
    b = np.asarray(batch, np.int64)
    size = int(b.max()) + 1 if len(b) else 0
    return np.searchsorted(b, np.arange(size + 1)).astype(np.int64)


def _edges(indices: np.ndarray) -> list:
    q, slot = np.nonzero(indices >= 0)
    return [q.tolist(), indices[q, slot].tolist()]


def _pair_ptrs(case, nx, ny):
    bx, by = case["batch_x"], case["batch_y"]
    if bx is None and by is None:
        return _ptr(None, nx), _ptr(None, ny)
    size = max(max(bx) + 1, max(by) + 1)
    return (np.searchsorted(np.asarray(bx), np.arange(size + 1)).astype(np.int64),
            np.searchsorted(np.asarray(by), np.arange(size + 1)).astype(np.int64))


@pytest.mark.parametrize("case", load_known_answers("knn_flat"), ids=lambda c: c["name"])
def test_knn_flat_known_answers(case):
    x, y = np.array(case["x"], np.float32), np.array(case["y"], np.float32)
    px, py = _pair_ptrs(case, len(x), len(y))
    width = min(case["k"], len(x))
    assert _edges(O.knn_flat(x, y, px, py, width)) == case["expect"], case["source"]


@pytest.mark.parametrize("case", load_known_answers("radius_flat"), ids=lambda c: c["name"])
def test_radius_flat_known_answers(case):
    x, y = np.array(case["x"], np.float32), np.array(case["y"], np.float32)
    px, py = _pair_ptrs(case, len(x), len(y))
    width = min(case["k"], len(x))
    assert _edges(O.radius_flat(x, y, px, py, case["r"], width)) == case["expect"], case["source"]


@pytest.mark.parametrize("case", load_known_answers("ball_query"), ids=lambda c: c["name"])
def test_ball_query_known_answers(case):
    dist, idx = O.ball_query(np.array(case["query"], np.float32), np.array(case["ref"], np.float32),
                             case["radius"], case["k"])
    assert idx.tolist() == case["expect_idx"], case["source"]
    if case.get("expect_dist") is not None:
        np.testing.assert_allclose(dist, np.array(case["expect_dist"], np.float32), rtol=1e-6,
                                   atol=0)
    if case.get("expect_dist_bits") is not None:
        assert dist.view(np.uint32).tolist() == case["expect_dist_bits"]
    if case.get("compat") is not None:
        first = np.clip(idx[..., :1], 0, None)
        assert np.where(idx >= 0, idx, first).tolist() == case["compat"]


@pytest.mark.parametrize("case", load_known_answers("three_nn"), ids=lambda c: c["name"])
def test_three_nn_known_answers(case):
    dist, idx = O.three_nn(np.array(case["unknown"], np.float32), np.array(case["known"], np.float32))
    assert idx.tolist() == case["expect_idx"]
    np.testing.assert_allclose(dist, np.array(case["expect_dist"], np.float32), rtol=1e-6)


@pytest.mark.parametrize("case", load_known_answers("three_interpolate"), ids=lambda c: c["name"])
def test_three_interpolate_known_answers(case):
    f = np.array(case["features"], np.float32)
    out = O.three_interpolate(f, case["indices"], np.array(case["weights"], np.float32))
    assert out.tolist() == case["expect"]
    grad = O.three_interpolate_backward(np.array(case["grad_out"], np.float32), case["indices"],
                                        np.array(case["weights"], np.float32), f.shape[-1])
    assert grad.tolist() == case["expect_grad"]


@pytest.mark.parametrize("case", load_known_answers("chamfer_nearest"), ids=lambda c: c["name"])
def test_chamfer_nearest_known_answers(case):
    dist, idx = O.chamfer_nearest(np.array(case["query"], np.float32),
                                  np.array(case["ref"], np.float32),
                                  case.get("query_lengths"), case.get("ref_lengths"), case["norm"])
    assert idx.tolist() == case["expect_idx"], case["source"]
    np.testing.assert_array_equal(dist, np.array(case["expect_dist"], np.float32))


# --------------------------------------------- reference-recorded selections

def test_segmentation_selections_match_metal_recording():
    """docs/parity/pointnet2-segmentation-mps-safe.npz: 4 FPS (skip near
    origin), 4 first-hit-padded ball queries and 4 three_nn on a 1152-point
    cloud, recorded on the reference's Metal kernels.  Every index must match."""
    z = np.load(GOLDEN / "segmentation_selections.npz")
    xyz = [z["xyz"]]
    got = []
    for npoint, radius in ((1024, 0.1), (256, 0.2), (64, 0.4), (16, 0.8)):
        x = xyz[-1]
        idx = O.fps(x, npoint, 0, True)
        new = np.take_along_axis(x, np.repeat(idx[..., None], 3, -1), 1)
        _, bi = O.ball_query(new, x, radius, 32)
        got += [idx, np.where(bi >= 0, bi, np.clip(bi[..., :1], 0, None))]
        xyz.append(new)
    for i in range(4):
        got.append(O.three_nn(xyz[3 - i], xyz[4 - i])[1])
    names = sorted(k for k in z.files if k.startswith("mps::"))
    assert len(names) == 12
    for name, arr in zip(names, got):
        np.testing.assert_array_equal(arr, z[name], err_msg=name)


def test_pointnet2_parity_fixtures():
    """docs/parity/pointnet2-{mps-safe,cuda}.json (tools/pointnet2parity.py)."""
    data = load_pointnet2_parity()
    for name, case in data["cases"].items():
        inp = case["inputs"]
        unknown = np.array(inp["unknown"], np.float32)
        known = np.array(inp["known"], np.float32)
        dist, idx = O.three_nn(unknown, known)
        for backend in ("mps_safe", "cuda"):
            want = case[backend]
            assert idx.tolist() == want["nearest_indices"], (name, backend)
            np.testing.assert_allclose(dist, np.array(want["distances"], np.float32),
                                       rtol=1e-6, err_msg=f"{name} {backend}")
        interp_idx = idx.astype(np.int64)
        for b, row in inp["override"].items():
            interp_idx[int(b), 0] = row
        assert interp_idx.tolist() == case["mps_safe"]["interpolate_indices"]
        feats = np.array(inp["features"], np.float32)
        w = np.array(inp["weights"], np.float32)
        out = O.three_interpolate(feats, interp_idx, w)
        np.testing.assert_allclose(out, np.array(case["mps_safe"]["interpolated"], np.float32),
                                   rtol=0, atol=0)
        grad = O.three_interpolate_backward(np.array(inp["gradient"], np.float32), interp_idx, w,
                                            feats.shape[-1])
        np.testing.assert_allclose(grad, np.array(case["mps_safe"]["feature_gradient"]),
                                   rtol=1e-6, atol=1e-6)


# ------------------------------------------- independent numpy formulations

def np_fps_maxmin(xyz: np.ndarray, npoint: int, start: int) -> list:
    """From-scratch max-min: step i takes the first point maximising the
    minimum distance to ALL previously selected points (no running state)."""
    out = [start]
    for _ in range(1, npoint):
        sel = xyz[out]
        d = sq32(xyz[:, None, :], sel[None, :, :])  # (N, i)
        m = d.min(axis=1)
        out.append(int(np.argmax(m)))
    return out


@pytest.mark.parametrize("n,npoint,start", [(1, 3, 0), (33, 33, 5), (200, 64, 0), (257, 300, 17)])
def test_fps_matches_from_scratch_maxmin(n, npoint, start):
    rng = np.random.default_rng(n)
    xyz = rng.standard_normal((2, n, 3)).astype(np.float32)
    xyz[1, : n // 2] = xyz[1, n // 2: n // 2 * 2]  # duplicates -> ties
    got = O.fps(xyz, npoint, start)
    for b in range(2):
        assert got[b].tolist() == np_fps_maxmin(xyz[b], npoint, start)


def np_knn(query, ref, k):
    d = sq32(ref[:, None, :, :], query[:, :, None, :])  # (B, M, N)
    order = np.lexsort((np.broadcast_to(np.arange(d.shape[-1]), d.shape), d), axis=-1)[..., :k]
    return np.sqrt(np.take_along_axis(d, order, -1)), order


@pytest.mark.parametrize("n,k", [(1, 1), (31, 5), (64, 64), (300, 17), (700, 256)])
def test_knn3_matches_lexsort(n, k):
    rng = np.random.default_rng(7 + n)
    ref = rng.standard_normal((2, n, 3)).astype(np.float32)
    ref[:, n // 3:] = np.round(ref[:, n // 3:] * 2) / 2  # many exact ties
    query = np.concatenate([ref[:, :5], rng.standard_normal((2, 9, 3)).astype(np.float32)], 1)
    want_d, want_i = np_knn(query, ref, k)
    dist, idx = O.knn3(query, ref, k)
    np.testing.assert_array_equal(idx, want_i)
    np.testing.assert_array_equal(dist, want_d)


def np_feature_knn(q, x, k):
    """Scalar float32 loop of tests/test_feature_knn.py:16-35 (numpy)."""
    rows = []
    for row in q:
        ranked = []
        for j, point in enumerate(x):
            delta = np.float32(point[0] - row[0])
            score = np.float32(delta * delta)
            for t in range(1, len(row)):
                delta = np.float32(point[t] - row[t])
                score = np.float32(score + np.float32(delta * delta))
            ranked.append((float(score), j))
        ranked.sort()
        rows.append([j for _, j in ranked[:k]])
    return np.array(rows)


@pytest.mark.parametrize("dim,k", [(1, 5), (2, 1), (4, 33), (64, 20)])
def test_knn_feat_matches_scalar_loop(dim, k):
    rng = np.random.default_rng(dim)
    ref = rng.standard_normal((1, 97, dim)).astype(np.float32)
    ref[:, 20] = ref[:, 3]
    query = rng.standard_normal((1, 9, dim)).astype(np.float32)
    query[:, 0] = ref[:, 3]
    _, idx = O.knn_feat(query, ref, k)
    np.testing.assert_array_equal(idx[0], np_feature_knn(query[0], ref[0], k))


def np_ball_query(q, p, radius, k):
    r2 = np.float32(O.ball_radius_sq(radius))
    d = sq32(q[:, :, None, :], p[:, None, :, :])
    idx = np.full(q.shape[:2] + (k,), -1, np.int64)
    dist = np.zeros(q.shape[:2] + (k,), np.float32)
    for b in range(q.shape[0]):
        for i in range(q.shape[1]):
            hits = np.nonzero(d[b, i] < r2)[0][:k]
            idx[b, i, : len(hits)] = hits
            dist[b, i, : len(hits)] = d[b, i, hits]
    return dist, idx


@pytest.mark.parametrize("radius,k", [(0.1, 16), (0.3, 32), (0.7, 128), (2.0, 5)])
def test_ball_query_matches_bruteforce(radius, k):
    rng = np.random.default_rng(int(radius * 100) + k)
    p = (rng.random((2, 400, 3), dtype=np.float32) * 2 - 1)
    q = p[:, ::7].copy()
    want_d, want_i = np_ball_query(q, p, radius, k)
    dist, idx = O.ball_query(q, p, radius, k)
    np.testing.assert_array_equal(idx, want_i)
    np.testing.assert_array_equal(dist, want_d)


def test_ball_query_lengths_and_padding():
    """tests/test_ball_query_mps.py:127-213 pattern: binary-fraction coordinates,
    a NaN and an inf point, short query/point lengths, K crossing blocks."""
    batch, nq, npts = 2, 9, 65
    q = np.zeros((batch, nq, 3), np.float32)
    p = np.zeros((batch, npts, 3), np.float32)
    for j in range(npts):
        p[:, j, 0] = 2.0 if j % 5 == 1 else (0.25 if j % 3 == 0 else 0.5)
    p[:, 31, 0] = np.nan
    p[:, 32, 0] = np.inf
    q[:, 2, 0] = 0.5
    q[:, 4, 0] = 20.0
    qlen, plen = [9, 7], [65, 49]
    for k in (1, 31, 32, 33, 65):
        dist, idx = O.ball_query(q, p, 1.0, k, qlen, plen)
        for b in range(batch):
            for i in range(nq):
                hits = []
                if i < qlen[b]:
                    for j in range(plen[b]):
                        dd = sum((float(a) - float(c)) ** 2 for a, c in zip(q[b, i], p[b, j]))
                        if dd < 1.0:
                            hits.append(j)
                hits = hits[:k]
                assert idx[b, i].tolist() == hits + [-1] * (k - len(hits))


def test_ball_query_membership_outside_boundary_band():
    """tests/test_ball_query_mps.py:288-331: decisions more than 4 float32 ulps
    of r^2 away from the boundary agree with binary64 arithmetic."""
    for radius in (0.1, 0.3, 1.0, 3.0):
        r32 = np.float32(radius)
        r2 = np.float32(np.float64(r32) * np.float64(r32))
        band = 4.0 * float(np.nextafter(r2, np.float32(np.inf)) - r2)
        lower = upper = r32
        vecs = [[0.0, 0.0, 0.0], [0.5 * float(r32), 0.0, 0.0]]
        for _ in range(12):
            lower = np.nextafter(lower, np.float32(0))
            upper = np.nextafter(upper, np.float32(np.inf))
            vecs += [[float(lower), 0, 0], [float(upper), 0, 0]]
        vecs += [[0.6 * float(r32), 0.8 * float(r32), 0], [1.5 * float(r32), 0, 0]]
        pts = np.array([vecs], np.float32)
        _, idx = O.ball_query(np.zeros((1, 1, 3), np.float32), pts, radius, len(vecs))
        got = set(j for j in idx.ravel().tolist() if j >= 0)
        amb = inside = outside = 0
        for j, v in enumerate(pts[0].tolist()):
            dd = sum(float(c) ** 2 for c in v)
            if abs(dd - float(r2)) <= band:
                amb += 1
                continue
            assert (j in got) == (dd < float(r2))
            inside += dd < float(r2)
            outside += dd >= float(r2)
        assert amb and inside and outside


@pytest.mark.parametrize("m", [3, 4, 50, 513])
def test_three_nn_matches_stable_argsort(m):
    rng = np.random.default_rng(59 + m)
    u = rng.standard_normal((2, 37, 3)).astype(np.float32)
    k = rng.standard_normal((2, m, 3)).astype(np.float32)
    k[:, m // 2:] = k[:, : m - m // 2][:, : m - m // 2]  # duplicate known points
    d2 = sq32(u[:, :, None, :], k[:, None, :, :])
    want_i = np.argsort(d2, axis=-1, kind="stable")[..., :3]
    want_d = np.sqrt(np.take_along_axis(d2, want_i, -1))
    dist, idx = O.three_nn(u, k)
    np.testing.assert_array_equal(idx, want_i)
    np.testing.assert_array_equal(dist, want_d)


def test_three_nn_nonfinite_order_matches_stable_argsort():
    """NaN sorts after every number (torch/numpy argsort), inf before NaN."""
    u = np.zeros((1, 1, 3), np.float32)
    k = np.array([[[np.nan, 0, 0], [np.inf, 0, 0], [1, 0, 0], [np.nan, 0, 0], [2, 0, 0]]],
                 np.float32)
    _, idx = O.three_nn(u, k)
    d2 = sq32(u[:, :, None, :], k[:, None, :, :])
    assert idx.tolist() == np.argsort(d2, axis=-1, kind="stable")[..., :3].tolist() == [[[2, 4, 1]]]


def test_three_interpolate_matches_gather():
    rng = np.random.default_rng(77)
    f = rng.standard_normal((2, 5, 12)).astype(np.float32)
    ix = rng.integers(0, 12, size=(2, 7, 3))
    w = rng.standard_normal((2, 7, 3)).astype(np.float32)
    sel = np.take_along_axis(f[:, :, None, :], ix[:, None, :, :].repeat(5, 1), -1)  # (B,C,N,3)
    prod = sel * w[:, None]
    want = (prod[..., 0] + prod[..., 1]) + prod[..., 2]
    np.testing.assert_array_equal(O.three_interpolate(f, ix, w), want)
    g = rng.standard_normal((2, 5, 7)).astype(np.float32)
    want_g = np.zeros((2, 5, 12))
    for b in range(2):
        for n in range(7):
            for t in range(3):
                want_g[b, :, ix[b, n, t]] += (g[b, :, n] * w[b, n, t]).astype(np.float64)
    np.testing.assert_allclose(O.three_interpolate_backward(g, ix, w, 12), want_g, rtol=1e-12)


@pytest.mark.parametrize("dim,norm", [(3, 2), (3, 1), (5, 2), (64, 1)])
def test_chamfer_nearest_matches_argmin(dim, norm):
    rng = np.random.default_rng(dim * 10 + norm)
    q = rng.standard_normal((3, 13, dim)).astype(np.float32)
    r = np.round(rng.standard_normal((3, 67, dim)).astype(np.float32) * 2) / 2
    ql, rl = [13, 4, 9], [67, 39, 3]
    dist, idx = O.chamfer_nearest(q, r, ql, rl, norm)
    for b in range(3):
        for i in range(13):
            if i >= ql[b]:
                assert idx[b, i] == -1 and dist[b, i] == 0
                continue
            delta = (q[b, i][None] - r[b, : rl[b]]).astype(np.float32)
            terms = np.abs(delta) if norm == 1 else delta * delta
            acc = terms[:, 0].copy()
            for t in range(1, dim):
                acc = acc + terms[:, t]
            assert idx[b, i] == int(np.argmin(acc))
            assert dist[b, i] == acc.min()


def test_chamfer_nearest_float64():
    rng = np.random.default_rng(3)
    q = rng.standard_normal((2, 11, 3))
    r = rng.standard_normal((2, 29, 3))
    dist, idx = O.chamfer_nearest(q, r)
    assert dist.dtype == np.float64
    d = ((q[:, :, None, 0] - r[:, None, :, 0]) ** 2 + (q[:, :, None, 1] - r[:, None, :, 1]) ** 2) \
        + (q[:, :, None, 2] - r[:, None, :, 2]) ** 2
    np.testing.assert_array_equal(idx, d.argmin(-1))


@pytest.mark.parametrize("k", [1, 4, 40])
def test_knn_flat_and_radius_flat_match_segment_bruteforce(k):
    rng = np.random.default_rng(k)
    x = rng.random((120, 3), dtype=np.float32)
    y = rng.random((50, 3), dtype=np.float32)
    bx = np.sort(rng.integers(0, 4, 120))
    by = np.sort(rng.integers(0, 4, 50))
    size = max(bx.max(), by.max()) + 1
    px = np.searchsorted(bx, np.arange(size + 1)).astype(np.int64)
    py = np.searchsorted(by, np.arange(size + 1)).astype(np.int64)
    kn = O.knn_flat(x, y, px, py, k)
    rad = O.radius_flat(x, y, px, py, 0.3, k)
    r2 = np.float32(0.3 * 0.3)
    for q in range(50):
        b = by[q]
        lo, hi = px[b], px[b + 1]
        d = sq32(x[lo:hi], y[q][None])
        order = np.lexsort((np.arange(hi - lo), d))[:k]
        want = list(order + lo) + [-1] * (k - len(order))
        assert kn[q].tolist() == want
        hits = list(np.nonzero(d < r2)[0][:k] + lo)
        assert rad[q].tolist() == hits + [-1] * (k - len(hits))


def test_radius_flat_ignore_same_index():
    x = np.array([[0, 0, 0], [0.1, 0, 0], [0.2, 0, 0]], np.float32)
    ptr = np.array([0, 3], np.int64)
    out = O.radius_flat(x, x, ptr, ptr, 0.5, 2, ignore_same_index=True)
    assert out.tolist() == [[1, 2], [0, 2], [0, 1]]


# ----------------------------------------------------- discriminating power

def test_mutants_fail_the_goldens():
    """Plausible oracle mistakes, planted in numpy copies, are caught."""
    # Non-strict radius (<=) admits the exact-boundary point of
    # tests/test_ball_query_mps.py:230-245.
    pts = np.array([[[np.nextafter(np.float32(1), np.float32(0)), 0, 0], [1, 0, 0]]], np.float32)
    d = sq32(np.zeros((1, 1, 1, 3), np.float32), pts[:, None])
    r2 = np.float32(O.ball_radius_sq(1.0))
    assert (d <= r2).sum() == 2 and (d < r2).sum() == 1
    _, idx = O.ball_query(np.zeros((1, 1, 3), np.float32), pts, 1.0, 2)
    assert idx.tolist() == [[[0, -1]]]
    # Largest-index tie order breaks the README/test_knn tie answers.
    case = [c for c in load_known_answers("knn") if c["name"] == "readme_square"][0]
    q, r = np.array(case["query"], np.float32), np.array(case["ref"], np.float32)
    dd = sq32(r[:, None, :, :], q[:, :, None, :])
    wrong = np.lexsort((-np.arange(4)[None, None].repeat(2, 1), dd), axis=-1)[..., :2]
    assert wrong.tolist() != case["expect_idx"]
    # r^2 squared in double then rounded differs from fl32(fl32(r)^2) at r=0.1:
    # the 0x3C23D70A point is excluded by the torch_cluster threshold.
    p01 = np.array([[[0.09999999403953552, 3.112176273134537e-05, 0.0]]], np.float32)
    dist = sq32(np.zeros(3, np.float32), p01[0, 0])
    assert struct.unpack("<I", struct.pack("<f", float(dist)))[0] == 0x3C23D70A
    assert dist < np.float32(O.ball_radius_sq(0.1))
    assert not dist < np.float32(O.torch_cluster_radius_sq(0.1))
    # FMA accumulation changes d^2 bits on inputs where rounding differs.
    rng = np.random.default_rng(0)
    a = rng.standard_normal((20000, 3)).astype(np.float32)
    unfused = sq32(a, np.zeros(3, np.float32))
    fused = (a[:, 0].astype(np.float64) ** 2).astype(np.float32)
    fused = (a[:, 1].astype(np.float64) * a[:, 1] + fused).astype(np.float32)
    fused = (a[:, 2].astype(np.float64) * a[:, 2] + fused).astype(np.float32)
    assert (unfused != fused).any()


# ------------------------------------------------------- PointNet++ grouping


def test_group_points_backward_known_answer():
    """tests/test_compat.py:134-137: the gradient of a gather with index
    [[2, 2, 5]] under sum() is 2 at point 2 and 1 at point 5, per channel."""
    grad = O.group_points_backward(np.ones((1, 3, 3), np.float32), [[2, 2, 5]], 10)
    assert grad[0, 0].tolist() == [0, 0, 2, 0, 0, 1, 0, 0, 0, 0]
    assert (grad[0] == grad[0, 0]).all()


def test_group_points_matches_indexing():
    """tests/test_compat.py:121-131 element identities over whole arrays, for
    the flat (gather) and the (npoint, nsample) (grouping) index."""
    rng = np.random.default_rng(3)
    f = rng.standard_normal((2, 4, 30)).astype(np.float32)
    idx = rng.integers(0, 30, size=(2, 7))
    out = O.group_points(f, idx)
    assert out.shape == (2, 4, 7)
    np.testing.assert_array_equal(out[1, :, 3], f[1, :, idx[1, 3]])
    np.testing.assert_array_equal(out, np.stack([f[b][:, idx[b]] for b in range(2)]))
    gidx = rng.integers(0, 30, size=(2, 7, 5))
    grouped = O.group_points(f, gidx.reshape(2, 35)).reshape(2, 4, 7, 5)
    np.testing.assert_array_equal(grouped[0, :, 6, 2], f[0, :, gidx[0, 6, 2]])


def test_group_points_backward_matches_add_at():
    """np.add.at adds in index order, in float32: the sequential
    scatter-add the oracle restates, bit for bit."""
    rng = np.random.default_rng(4)
    g = rng.standard_normal((2, 3, 40)).astype(np.float32)
    idx = rng.integers(0, 9, size=(2, 40))  # heavy repetition
    want = np.zeros((2, 3, 9), np.float32)
    for b in range(2):
        for c in range(3):
            np.add.at(want[b, c], idx[b], g[b, c])
    np.testing.assert_array_equal(O.group_points_backward(g, idx, 9), want)
    # Conservation: every gradient element lands somewhere exactly once.
    np.testing.assert_allclose(O.group_points_backward(g, idx, 9).sum(-1, dtype=np.float64),
                               g.astype(np.float64).sum(-1), rtol=1e-5)


def test_group_points_rel_matches_composition_and_self_zero():
    """Channels 0-2 are grouped xyz minus the centre (one float32
    subtraction), then the grouped features; a centre grouped with its own
    point is exactly 0 in the relative channels."""
    rng = np.random.default_rng(5)
    xyz = rng.standard_normal((2, 50, 3)).astype(np.float32)
    sel = rng.integers(0, 50, size=(2, 6))
    centres = np.stack([xyz[b, sel[b]] for b in range(2)])
    feats = rng.standard_normal((2, 4, 50)).astype(np.float32)
    idx = rng.integers(0, 50, size=(2, 6, 5))
    idx[:, :, 0] = sel
    out = O.group_points_rel(xyz, centres, feats, idx)
    assert out.shape == (2, 7, 6, 5)
    gx = np.stack([xyz[b, idx[b]] for b in range(2)])  # (B,M,S,3)
    want_rel = (gx - centres[:, :, None, :]).transpose(0, 3, 1, 2)
    np.testing.assert_array_equal(out[:, :3], want_rel)
    np.testing.assert_array_equal(out[:, 3:], np.stack([feats[b][:, idx[b]] for b in range(2)]))
    assert (out[:, :3, :, 0] == 0).all()
    assert O.group_points_rel(xyz, centres, None, idx).shape == (2, 3, 6, 5)
