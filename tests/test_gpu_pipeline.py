"""fps_ball_knn (one call, queries overlapped with FPS) against the separate
calls it replaces, bit for bit, and the samples against the oracle; calls
that overlap on two streams; the give-up path forced from the host."""

import os

import pytest
import torch

import bench

pytestmark = pytest.mark.gpu


def _separate(mp, xyz, npoint, radii, ks, knn_k, start, skip):
    samples = mp.furthest_point_sample(xyz, npoint, start, skip)
    centres = xyz.gather(1, samples[..., None].expand(-1, -1, 3)).contiguous()
    balls = [mp.ball_query(centres, xyz, r, k) for r, k in zip(radii, ks)]
    knn = mp.knn(centres, xyz, knn_k) if knn_k else None
    return samples, centres, balls, knn


def _cloud(B, N, seed):
    if (B, N, seed) == (32, 4096, 2):
        return bench.make_c2().to("cuda")  # the benchmarked config-2 input
    g = torch.Generator().manual_seed(seed)
    return torch.rand(B, N, 3, generator=g).to("cuda")


def _assert_same(out, ref, knn_k):
    samples, centres, balls, knn = out
    assert torch.equal(samples, ref[0])
    assert torch.equal(centres, ref[1])
    for (d, i), (rd, ri) in zip(balls, ref[2]):
        assert torch.equal(i, ri) and torch.equal(d, rd)
    if knn_k:
        assert torch.equal(knn[1], ref[3][1]) and torch.equal(knn[0], ref[3][0])


C2 = (bench.C2_NPOINT, tuple(r for r, _ in bench.C2_RADII), tuple(k for _, k in bench.C2_RADII),
      bench.C2_KNN_K)


@pytest.mark.parametrize("B,N,seed,npoint,chunk,radii,ks,knn_k,start,skip", [
    (32, 4096, 2, *C2[:1], 256, *C2[1:], 0, False),   # config 2, the benchmarked call
    (32, 4096, 2, *C2[:1], 128, *C2[1:], 0, False),
    (3, 500, 7, 77, 16, (0.3,), (8,), 5, 7, False),       # npoint not a multiple of chunk
    (2, 1000, 8, 1000, 4096, (0.2, 0.5), (4, 64), 32, 0, True),   # one chunk, every point
    (5, 8192, 9, 300, 64, (0.05,), (32,), 0, 3, False),   # no kNN, the largest cloud
    (4, 2048, 10, 1, 1, (), (), 1, 0, False),              # one sample, no ball query
    # Six radii (two multi-radius scans), K above 128, a zero and a huge radius.
    (3, 3000, 12, 200, 64, (0.1, 0.0, 0.3, 0.05, 2.0, 0.2), (16, 8, 200, 1, 3, 65), 8, 0, False),
])
def test_fps_ball_knn_matches_separate_calls(B, N, seed, npoint, chunk, radii, ks, knn_k, start,
                                             skip):
    import mps_pointops as mp

    print(f"case B={B} N={N} npoint={npoint} chunk={chunk}", flush=True)
    xyz = _cloud(B, N, seed)
    if skip:
        xyz[:, ::7] *= 1e-3  # points near the origin that FPS must never pick
    # Two calls in a row, the second queued behind the first.
    outs = [mp.fps_ball_knn(xyz, npoint, radii, ks, knn_k, start, skip, chunk=chunk, check=True)
            for _ in range(2)]
    ref = _separate(mp, xyz, npoint, radii, ks, knn_k, start, skip)
    torch.cuda.synchronize()
    for out in outs:
        _assert_same(out, ref, knn_k)


def test_fps_ball_knn_samples_match_oracle():
    import mps_pointops as mp
    from oracle import oracle

    xyz = _cloud(2, 1500, 5)
    samples, *_ = mp.fps_ball_knn(xyz, 200, (0.2,), (16,), 8, chunk=32, check=True)
    want = oracle.fps(xyz.cpu().numpy(), 200, 0, False)
    assert (samples.cpu().numpy() == want).all()


def test_fps_ball_knn_back_to_back_on_shared_stream():
    """Many calls queued without synchronising: every call's chunks wait for
    that call's own samples (tags grow per call)."""
    import mps_pointops as mp

    xyzs = [_cloud(8, 4096, s) for s in range(6)]
    outs = [mp.fps_ball_knn(x, 512, (0.2,), (32,), 16, chunk=64) for x in xyzs]
    for x, (samples, centres, balls, knn) in zip(xyzs, outs):
        ref = _separate(mp, x, 512, (0.2,), (32,), 16, 0, False)
        assert torch.equal(samples, ref[0]) and torch.equal(balls[0][1], ref[2][0][1])
        assert torch.equal(knn[1], ref[3][1])


def test_fps_ball_knn_overlapping_calls_on_two_streams():
    """Same-shape calls issued from two default-priority streams without any
    synchronisation between them: each call's gates wait for that call's own
    samples, so every output equals the separate calls bit for bit."""
    import mps_pointops as mp

    npoint, radii, ks, knn_k = C2
    xyzs = [bench.make_c2(seed=s).to("cuda") for s in (2, 3)]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    torch.cuda.synchronize()
    outs = [[], []]
    for _ in range(3):  # calls interleaved over the two streams
        for k, (stream, xyz) in enumerate(zip(streams, xyzs)):
            with torch.cuda.stream(stream):
                outs[k].append(mp.fps_ball_knn(xyz, npoint, radii, ks, knn_k, chunk=256))
    torch.cuda.synchronize()
    for xyz, calls in zip(xyzs, outs):
        ref = _separate(mp, xyz, npoint, radii, ks, knn_k, 0, False)
        torch.cuda.synchronize()
        for out in calls:
            _assert_same(out, ref, knn_k)


def test_fps_ball_knn_give_up_is_flagged(monkeypatch):
    """The gates' poll budget forced to 0 from the host: every gate gives up
    without reading a progress word, and every kernel still ends.  The call
    reports it (status word, check=True raises), its centres are NaN and its
    queries are those of NaN centres; the samples stay exact.  The next call
    with the default budget is exact again."""
    import mps_pointops as mp

    npoint, radii, ks, knn_k = 256, (0.2, 0.4), (16, 32), 16
    xyz = _cloud(4, 2048, 11)
    ref = _separate(mp, xyz, npoint, radii, ks, knn_k, 0, False)
    monkeypatch.setenv("POINTOPS_PIPELINE_SPIN_LIMIT", "0")
    with pytest.raises(RuntimeError, match="gave up"):
        mp.fps_ball_knn(xyz, npoint, radii, ks, knn_k, chunk=64, check=True)
    samples, centres, balls, knn = mp.fps_ball_knn(xyz, npoint, radii, ks, knn_k, chunk=64)
    torch.cuda.synchronize()
    assert torch.equal(samples, ref[0])
    assert torch.isnan(centres).all()
    nan_ref = [mp.ball_query(centres, xyz, r, k) for r, k in zip(radii, ks)]
    for (d, i), (rd, ri) in zip(balls, nan_ref):
        assert torch.equal(i, ri) and torch.equal(d, rd)
        assert (i == -1).all() and (d == 0).all()
    kd, ki = mp.knn(centres, xyz, knn_k)
    assert torch.equal(knn[1], ki) and torch.equal(knn[0], kd)
    assert (knn[1] == 0xFFFFFFFF).all() and torch.isinf(knn[0]).all()
    monkeypatch.delenv("POINTOPS_PIPELINE_SPIN_LIMIT")
    _assert_same(mp.fps_ball_knn(xyz, npoint, radii, ks, knn_k, chunk=64, check=True), ref, knn_k)
