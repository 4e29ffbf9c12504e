"""pointops_fps_large_noalloc (the entry point that allocates nothing)
against pointops_fps_large, through the C ABI: bit-identical indices on two
calls in a row, the second with a smaller cloud (the array keeps the first
call's records and must be cleared), and the size limit rejected before any
launch."""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _cloud(n: int, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    xyz = torch.randn(1, n, 3, generator=g)
    xyz[0, : n // 9] = xyz[0, n // 9: 2 * (n // 9)]  # duplicates: index ties
    return xyz.cuda().contiguous()


def _with_workspace(xyz: torch.Tensor, npoint: int, start: int, skip: int) -> np.ndarray:
    from mps_pointops import _native

    N = xyz.shape[1]
    out = torch.full((npoint,), -777, dtype=torch.long, device="cuda")
    size = _native.size_query("pointops_fps_large_workspace_bytes", N, npoint)
    ws = torch.zeros(size, dtype=torch.uint8, device="cuda")
    _native.call("pointops_fps_large", xyz.data_ptr(), out.data_ptr(), ws.data_ptr(), N, npoint,
                 start, skip, _native.stream(xyz.device))
    torch.cuda.synchronize()
    assert int(ws[:4].view(torch.int32).item()) == 0
    return out.cpu().numpy()


def _no_alloc(xyz: torch.Tensor, npoint: int, start: int, skip: int) -> np.ndarray:
    from mps_pointops import _native

    out = torch.full((npoint,), -777, dtype=torch.long, device="cuda")
    _native.call("pointops_fps_large_noalloc", xyz.data_ptr(), out.data_ptr(), xyz.shape[1],
                 npoint, start, skip, _native.stream(xyz.device))
    torch.cuda.synchronize()
    return out.cpu().numpy()


def test_no_alloc_matches_workspace_entry_on_consecutive_calls(cuda_device):
    for n, npoint, start, skip in ((300_000, 2000, 17, 0), (70_000, 700, 5, 1)):
        xyz = _cloud(n, n)
        want = _with_workspace(xyz, npoint, start, skip)
        got = _no_alloc(xyz, npoint, start, skip)
        assert (got >= 0).all()
        np.testing.assert_array_equal(got, want)


def test_no_alloc_repeat_after_larger_call(cuda_device):
    """A small call right after a large one on the same array, twice."""
    big, small = _cloud(1 << 21, 1), _cloud(5000, 2)
    want_small = _with_workspace(small, 900, 0, 0)
    for _ in range(2):
        _no_alloc(big, 3000, 1, 0)
        np.testing.assert_array_equal(_no_alloc(small, 900, 0, 0), want_small)


def test_no_alloc_rejects_sizes_beyond_the_limit(cuda_device):
    from mps_pointops import _native

    lib = _native.library()
    stream = _native.stream(torch.device("cuda", 0))
    out = torch.empty(4, dtype=torch.long, device="cuda")
    # hipErrorInvalidValue (1) before any launch: N above 2^21, start outside.
    assert lib.pointops_fps_large_noalloc(None, out.data_ptr(), (1 << 21) + 1, 4, 0, 0,
                                          stream) == 1
    assert lib.pointops_fps_large_noalloc(None, out.data_ptr(), 100, 4, 100, 0, stream) == 1
    assert lib.pointops_fps_large_noalloc(None, None, 100, 0, 0, 0, stream) == 0  # nothing to do
