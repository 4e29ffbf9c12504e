"""fps_ball_knn (one call, queries overlapped with FPS) against the separate
calls it replaces, bit for bit, and the samples against the oracle."""

import pytest
import torch

pytestmark = pytest.mark.gpu


def _separate(mp, xyz, npoint, radii, ks, knn_k, start, skip):
    samples = mp.furthest_point_sample(xyz, npoint, start, skip)
    centres = xyz.gather(1, samples[..., None].expand(-1, -1, 3)).contiguous()
    balls = [mp.ball_query(centres, xyz, r, k) for r, k in zip(radii, ks)]
    knn = mp.knn(centres, xyz, knn_k) if knn_k else None
    return samples, centres, balls, knn


def _cloud(B, N, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.rand(B, N, 3, generator=g).to("cuda")


@pytest.mark.parametrize("B,N,npoint,chunk,radii,ks,knn_k,start,skip", [
    (32, 4096, 1024, 128, (0.1, 0.2, 0.4), (16, 32, 128), 16, 0, False),   # config 2
    (3, 500, 77, 16, (0.3,), (8,), 5, 7, False),       # npoint not a multiple of chunk
    (2, 1000, 1000, 4096, (0.2, 0.5), (4, 64), 32, 0, True),   # one chunk, every point
    (5, 8192, 300, 64, (0.05,), (32,), 0, 3, False),   # no kNN, the largest cloud
    (4, 2048, 1, 1, (), (), 1, 0, False),              # one sample, no ball query
])
def test_fps_ball_knn_matches_separate_calls(B, N, npoint, chunk, radii, ks, knn_k, start, skip):
    import mps_pointops as mp

    print(f"case B={B} N={N} npoint={npoint} chunk={chunk}", flush=True)
    xyz = _cloud(B, N, B * 1000 + N)
    if skip:
        xyz[:, ::7] *= 1e-3  # points near the origin that FPS must never pick
    # Two calls in a row (the second reuses the workspace and its progress words).
    for _ in range(2):
        samples, centres, balls, knn = mp.fps_ball_knn(
            xyz, npoint, radii, ks, knn_k, start, skip, chunk=chunk, check=True)
    ref = _separate(mp, xyz, npoint, radii, ks, knn_k, start, skip)
    torch.cuda.synchronize()
    assert torch.equal(samples, ref[0])
    assert torch.equal(centres, ref[1])
    for (d, i), (rd, ri) in zip(balls, ref[2]):
        assert torch.equal(i, ri) and torch.equal(d, rd)
    if knn_k:
        assert torch.equal(knn[1], ref[3][1]) and torch.equal(knn[0], ref[3][0])


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
