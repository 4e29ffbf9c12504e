"""Backward of the dense ball query (pointops_ball_query_backward_*) against
the gradients _ball_query_mps.py:168-203 defines: d(d2)/dq = 2 (q - p) and
d(d2)/dp = -2 (q - p) per valid slot, padded slots masked.

* the config-2 set-abstraction queries at the three radii, indices from the
  oracle: float64 closed form, error within 1e-4 of the sum of absolute
  contributions, NaN gradients planted in every padded slot;
* the kernel's fixed summation order (for a query, four partial sums over
  the slots k = l mod 4 in order, added in order; for a point, rows in order
  within 8 row segments, then the segments in order)
  emulated in float32 numpy: the same bits;
* two runs give the same bits; float16 inputs; clouds spanning several
  512-point tiles; empty shapes; one-sided gradients."""

import numpy as np
import pytest
import torch

import bench
from oracle import oracle

pytestmark = pytest.mark.gpu

SEGMENTS = 8


def _contributions(q, p, idx, g):
    """Per-slot contributions in float32, as the kernels form them:
    fl(2 g) * fl(q - p), zero (and masked) at padded slots."""
    B, Q, K = idx.shape
    valid = idx >= 0
    safe = np.where(valid, idx, 0)
    gathered = np.stack([p[b][safe[b]] for b in range(B)])  # (B, Q, K, 3)
    delta = (q[:, :, None, :] - gathered).astype(np.float32)
    g2 = (np.float32(2) * np.where(valid, g, 0).astype(np.float32))[..., None]
    return np.where(valid[..., None], (g2 * delta).astype(np.float32), np.float32(0)), valid


def _emulate(q, p, idx, g):
    """The kernels' float32 sums in their order."""
    c, valid = _contributions(q, p, idx, g)
    B, Q, K = idx.shape
    P = p.shape[1]
    parts = []
    for lane in range(4):
        acc = np.zeros((B, Q, 3), np.float32)
        for k in range(lane, K, 4):
            acc = np.where(valid[:, :, k, None], (acc + c[:, :, k]).astype(np.float32), acc)
        parts.append(acc)
    gq = parts[0]
    for part in parts[1:]:
        gq = (gq + part).astype(np.float32)
    gp = np.zeros((B, P, 3), np.float32)
    for b in range(B):
        parts = []
        for w in range(SEGMENTS):
            acc = np.zeros((P, 3), np.float32)
            for r in range(Q * w // SEGMENTS, Q * (w + 1) // SEGMENTS):
                m = valid[b, r]
                acc[idx[b, r][m]] = (acc[idx[b, r][m]] + c[b, r][m]).astype(np.float32)
            parts.append(acc)
        total = parts[0]
        for part in parts[1:]:
            total = (total + part).astype(np.float32)
        gp[b] = -total
    return gq, gp


def _closed_form(q, p, idx, g):
    """float64 gradients and the sums of absolute contributions (the error scale)."""
    B, Q, K = idx.shape
    valid = idx >= 0
    safe = np.where(valid, idx, 0)
    gathered = np.stack([p[b][safe[b]] for b in range(B)]).astype(np.float64)
    c = np.where(valid[..., None],
                 2.0 * np.where(valid, g, 0)[..., None].astype(np.float64)
                 * (q[:, :, None, :].astype(np.float64) - gathered), 0.0)
    gq = c.sum(axis=2)
    gq_abs = np.abs(c).sum(axis=2)
    gp = np.zeros(p.shape, np.float64)
    gp_abs = np.zeros(p.shape, np.float64)
    for b in range(B):
        m = valid[b]
        np.add.at(gp[b], idx[b][m], -c[b][m])
        np.add.at(gp_abs[b], idx[b][m], np.abs(c[b][m]))
    return gq, gq_abs, gp, gp_abs


def _run(mp, q, p, radius, k, g, need=(True, True)):
    ql = q.clone().requires_grad_(need[0])
    pl = p.clone().requires_grad_(need[1])
    d, i = mp.ball_query(ql, pl, radius, k)
    d.backward(g)
    return i, ql.grad, pl.grad


@pytest.mark.parametrize("radius,k", bench.C2_RADII)
def test_c2_radii_closed_form(radius, k):
    import mps_pointops as mp

    print(f"case c2 r={radius} K={k}", flush=True)
    xyz = bench.make_c2()
    samples = oracle.fps(xyz.numpy(), bench.C2_NPOINT, 0, False)
    centres = np.stack([xyz.numpy()[b][samples[b]] for b in range(xyz.shape[0])])
    _, want_idx = oracle.ball_query(centres, xyz.numpy(), radius, k)
    rng = np.random.default_rng(int(radius * 10) + k)
    g = rng.standard_normal(want_idx.shape).astype(np.float32)
    g[want_idx < 0] = np.nan  # padded slots must not reach the sums
    idx, gq, gp = _run(mp, torch.from_numpy(centres).cuda(), xyz.cuda(), radius, k,
                       torch.from_numpy(g).cuda())
    assert np.array_equal(idx.cpu().numpy(), want_idx)
    cq, cq_abs, cp, cp_abs = _closed_form(centres, xyz.numpy(), want_idx, g)
    gq, gp = gq.cpu().numpy().astype(np.float64), gp.cpu().numpy().astype(np.float64)
    assert np.isfinite(gq).all() and np.isfinite(gp).all()
    assert (np.abs(gq - cq) <= 1e-4 * cq_abs + 1e-30).all()
    assert (np.abs(gp - cp) <= 1e-4 * cp_abs + 1e-30).all()


@pytest.mark.parametrize("B,Q,P,K,radius,seed", [
    (2, 300, 5000, 32, 0.3, 1),   # ten 512-point tiles, rows skipped per tile
    (3, 77, 1000, 16, 0.5, 2),    # one partial tile
    (1, 9, 2048, 128, 2.0, 3),    # every row full, K > 64
    (2, 64, 1, 4, 1.0, 4),        # a one-point cloud
    (1, 5, 300, 8, 0.5, 5),       # fewer rows than segments: empty segments
    (1, 2100, 600, 128, 0.5, 6),  # many rows per segment, K > 64
    (1, 40, 9000, 16, 0.3, 7),    # more than 16 tiles: rows missing a tile skipped
])
def test_fixed_order_bits_and_repeatability(B, Q, P, K, radius, seed):
    import mps_pointops as mp

    print(f"case B={B} Q={Q} P={P} K={K}", flush=True)
    gen = torch.Generator().manual_seed(seed)
    p = torch.rand(B, P, 3, generator=gen)
    q = torch.rand(B, Q, 3, generator=gen)
    g = torch.randn(B, Q, K, generator=gen)
    runs = [_run(mp, q.cuda(), p.cuda(), radius, K, g.cuda()) for _ in range(2)]
    idx = runs[0][0].cpu().numpy()
    wq, wp = _emulate(q.numpy(), p.numpy(), idx, g.numpy())
    for _, gq, gp in runs:
        assert np.array_equal(gq.cpu().numpy().view(np.uint32), wq.view(np.uint32))
        assert np.array_equal(gp.cpu().numpy().view(np.uint32), wp.view(np.uint32))


def test_float16_inputs():
    import mps_pointops as mp

    gen = torch.Generator().manual_seed(7)
    p = (torch.rand(2, 700, 3, generator=gen)).half()
    q = (torch.rand(2, 50, 3, generator=gen)).half()
    g = torch.randn(2, 50, 24, generator=gen)
    idx, gq, gp = _run(mp, q.cuda(), p.cuda(), 0.3, 24, g.cuda())
    assert gq.dtype == torch.float16 and gp.dtype == torch.float16
    wq, wp = _emulate(q.float().numpy(), p.float().numpy(), idx.cpu().numpy(), g.numpy())
    assert np.array_equal(gq.cpu().numpy(), wq.astype(np.float16))
    assert np.array_equal(gp.cpu().numpy(), wp.astype(np.float16))


def test_one_sided_and_empty():
    import mps_pointops as mp

    gen = torch.Generator().manual_seed(8)
    p = torch.rand(2, 300, 3, generator=gen)
    q = torch.rand(2, 40, 3, generator=gen)
    g = torch.randn(2, 40, 8, generator=gen)
    idx, gq, gp = _run(mp, q.cuda(), p.cuda(), 0.4, 8, g.cuda(), need=(True, False))
    wq, wp = _emulate(q.numpy(), p.numpy(), idx.cpu().numpy(), g.numpy())
    assert gp is None and np.array_equal(gq.cpu().numpy(), wq)
    idx, gq, gp = _run(mp, q.cuda(), p.cuda(), 0.4, 8, g.cuda(), need=(False, True))
    assert gq is None and np.array_equal(gp.cpu().numpy(), wp)
    # No neighbour anywhere (r = 0), K = 0 and no queries: zero gradients.
    for qq, k, r in ((q, 8, 0.0), (q, 0, 0.4), (q[:, :0], 8, 0.4)):
        _, gq, gp = _run(mp, qq.cuda(), p.cuda(), r, k,
                         torch.ones(2, qq.shape[1], k).cuda())
        assert (gq == 0).all() and (gp == 0).all() and gp.shape == p.shape
