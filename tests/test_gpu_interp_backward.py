"""GPU parity of the CSR three_interpolate backward
(pointops_three_interpolate_backward_csr): bit for bit, on every call, equal
to its documented float32 order -- for up to 1024 known points, a known
point's terms fl32(grad_out * w) in (n, t) order summed in pieces cut at
every 12th position of the batch's CSR (emulated in numpy here); for more,
the float32 scatter loop over (n, t) in order (numpy's unbuffered add.at,
which applies the updates in index order) -- and within 1e-5 of the
oracle's three_interpolate_backward (the same loop accumulated in double,
kernels/pointnet2.metal:85-103)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def host(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy()


def sequential_f32(up: np.ndarray, idx: np.ndarray, w: np.ndarray, m: int) -> np.ndarray:
    """float32 grad[b, c, idx[b, n, t]] += fl32(up[b, c, n] * w[b, n, t]) in (n, t) order."""
    B, C, _ = up.shape
    out = np.zeros((B, C, m), np.float32)
    for b in range(B):
        flat = idx[b].reshape(-1)
        for c in range(C):
            prod = (up[b, c][:, None] * w[b]).astype(np.float32).reshape(-1)
            np.add.at(out[b, c], flat, prod)
    return out


def pieces_f32(up: np.ndarray, idx: np.ndarray, w: np.ndarray, m: int, piece: int = 12) -> np.ndarray:
    """The CSR gather's order for M <= 1024 known points: per batch the
    entries e = 3n + t sorted by (known index, e) are cut into pieces at
    every `piece`-th position; each piece sums fl32(up[c, n] * w[e]) from +0
    in order and a known point's pieces are added in order."""
    B, C, _ = up.shape
    out = np.zeros((B, C, m), np.float32)
    for b in range(B):
        keys = idx[b].reshape(-1).astype(np.int64)
        valid = np.nonzero((keys >= 0) & (keys < m))[0]
        order = valid[np.argsort(keys[valid], kind="stable")]
        sk = keys[order]
        starts = np.searchsorted(sk, np.arange(m + 1))
        terms = (up[b][:, order // 3] * w[b].reshape(-1)[order]).astype(np.float32)  # (C, E)
        for k in range(m):
            q, e = int(starts[k]), int(starts[k + 1])
            total = None
            while q < e:
                cut = min(e, (q // piece + 1) * piece)
                part = np.zeros(C, np.float32)
                for i in range(q, cut):
                    part = (part + terms[:, i]).astype(np.float32)
                total = part if total is None else (total + part).astype(np.float32)
                q = cut
            if total is not None:
                out[b, :, k] = total
    return out


def expected_bits(up, idx, w, m):
    """Known points <= 1024: the piece order; more: the sequential loop."""
    return pieces_f32(up, idx, w, m) if m <= 1024 else sequential_f32(up, idx, w, m)


def backward_csr(grad_out: torch.Tensor, idx: torch.Tensor, w: torch.Tensor, m: int,
                 fill: float = float("nan")) -> np.ndarray:
    """The CSR entry point through the C ABI into an output pre-filled with
    `fill` (every element must be overwritten)."""
    from mps_pointops import _native

    g, i, ww = (t.cuda().contiguous() for t in (grad_out, idx, w))
    B, C, N = g.shape
    out = torch.full((B, C, m), fill, device="cuda")
    size = _native.size_query("pointops_three_interpolate_backward_workspace_bytes", B, m, N)
    ws = torch.empty(size, dtype=torch.uint8, device="cuda")
    print(f"three_interpolate_backward_csr B={B} C={C} M={m} N={N}", flush=True)
    _native.call("pointops_three_interpolate_backward_csr", g.data_ptr(), i.data_ptr(),
                 ww.data_ptr(), out.data_ptr(), ws.data_ptr(), B, C, m, N,
                 _native.stream(g.device))
    return host(out)


@pytest.mark.parametrize("m,n,c", [(1024, 4096, 128), (64, 300, 5), (5, 40, 13), (4096, 4096, 3),
                                   (3000, 200, 9), (1, 12, 2), (700, 4000, 17)])
def test_csr_backward_matches_sequential_loop(cuda_device, m, n, c):
    g = torch.Generator().manual_seed(m * 31 + n + c)
    B = 2
    idx = torch.randint(0, m, (B, n, 3), generator=g, dtype=torch.int32)
    idx[:, : n // 3, :] = idx[:, :1, :]  # a hot bucket, repeated within one n
    w = torch.rand(B, n, 3, generator=g)
    up = torch.randn(B, c, n, generator=g)
    want = expected_bits(up.numpy(), idx.numpy(), w.numpy(), m)
    first = backward_csr(up, idx, w, m)
    np.testing.assert_array_equal(first.view(np.uint32), want.view(np.uint32))
    # float32 against double accumulation; the hot bucket sums up to 4096 terms.
    oracle = O.three_interpolate_backward(up.numpy(), idx.numpy(), w.numpy(), m)
    np.testing.assert_allclose(first, oracle, rtol=1e-5, atol=1e-4)
    again = backward_csr(up, idx, w, m, fill=7.0)
    np.testing.assert_array_equal(again.view(np.uint32), first.view(np.uint32))


def test_csr_backward_unselected_points_are_zero(cuda_device):
    """Known points no entry selects get exactly +0 (the output is not
    zero-filled by the caller here)."""
    B, C, M, N = 1, 4, 100, 52
    idx = torch.zeros(B, N, 3, dtype=torch.int32)
    idx[..., 1:] = 7  # slot 0 selects point 0, slots 1 and 2 point 7
    w = torch.ones(B, N, 3)
    up = torch.ones(B, C, N)
    out = backward_csr(up, idx, w, M)
    assert np.all(out[..., 0] == N) and np.all(out[..., 7] == 2 * N)
    rest = np.delete(out, [0, 7], axis=-1)
    assert np.all(rest.view(np.uint32) == 0)


def test_csr_backward_rejects_out_of_range(cuda_device):
    from mps_pointops import _native

    lib = _native.library()
    g = torch.zeros(1, 1, 4, device="cuda")
    i = torch.zeros(1, 4, 3, dtype=torch.int32, device="cuda")
    w = torch.zeros(1, 4, 3, device="cuda")
    o = torch.zeros(1, 1, 4, device="cuda")
    ws = torch.empty(1 << 20, dtype=torch.uint8, device="cuda")
    a = (g.data_ptr(), i.data_ptr(), w.data_ptr(), o.data_ptr())
    assert lib.pointops_three_interpolate_backward_csr(*a, ws.data_ptr(), 1, 1, 4097, 4, None) != 0
    assert lib.pointops_three_interpolate_backward_csr(*a, ws.data_ptr(), 1, 1, 4, 4100, None) != 0
    assert lib.pointops_three_interpolate_backward_csr(*a, None, 1, 1, 4, 4, None) != 0
    assert lib.pointops_three_interpolate_backward_csr(*a, ws.data_ptr(), 1, 1, 4, 3, None) != 0


def test_public_backward_uses_csr_path(cuda_device, monkeypatch):
    """three_interpolate's autograd forward builds the CSR for config 2's
    shape and its backward gathers over it, giving the sequential-loop
    gradient."""
    from mps_pointops import _native, three_interpolate

    calls = []
    real = _native.call
    monkeypatch.setattr(_native, "call", lambda name, *a: (calls.append(name), real(name, *a))[1])
    g = torch.Generator().manual_seed(3)
    B, C, M, N = 2, 16, 1024, 4096
    idx = torch.randint(0, M, (B, N, 3), generator=g, dtype=torch.int32)
    w = torch.rand(B, N, 3, generator=g)
    up = torch.randn(B, C, N, generator=g)
    f = torch.randn(B, C, M, generator=g).cuda().requires_grad_()
    out = three_interpolate(f, idx.cuda(), w.cuda())
    # The CSR is built right after the forward; the backward only gathers.
    assert calls == ["pointops_three_interpolate", "pointops_three_interpolate_csr_build"]
    out.backward(up.cuda(), retain_graph=True)
    assert calls[2:] == ["pointops_three_interpolate_backward_from_csr"]
    want = pieces_f32(up.numpy(), idx.numpy(), w.numpy(), M)
    np.testing.assert_array_equal(host(f.grad).view(np.uint32), want.view(np.uint32))
    # A second backward over the same graph reuses the CSR: the same bits again.
    f.grad = None
    out.backward(up.cuda())
    np.testing.assert_array_equal(host(f.grad).view(np.uint32), want.view(np.uint32))
    # Without a feature gradient no CSR is built.
    calls.clear()
    three_interpolate(f.detach(), idx.cuda(), w.cuda())
    assert calls == ["pointops_three_interpolate"]
