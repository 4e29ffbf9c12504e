"""GPU parity of the Morton-window 3-D kNN (pointops_knn3_windowed) against
the oracle.

The starting limit only decides which references are buffered; indices must
equal the brute-force answer of kernels/knn.metal:32-140 bit for bit, and the
distances (sqrt of the same fl32 squared distance) bit for bit as well.
Cases cover the shapes the entry point accepts (N <= 8192, M <= 16384,
K <= 32), the template boundaries of K (8, 16, 32), ties and duplicates,
points outside the references' box, degenerate extents and non-finite
coordinates.
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


def knn3_windowed(query: torch.Tensor, ref: torch.Tensor, k: int):
    """pointops_knn3_windowed through the C ABI."""
    from mps_pointops import _native

    q, r = query.cuda().contiguous(), ref.cuda().contiguous()
    B, M, _ = q.shape
    N = r.shape[1]
    dist = torch.empty(B, M, k, device="cuda")
    idx = torch.empty(B, M, k, dtype=torch.long, device="cuda")
    size = _native.size_query("pointops_knn3_windowed_workspace_bytes", B, M, N)
    ws = torch.empty(size, dtype=torch.uint8, device="cuda")
    print(f"knn3_windowed B={B} M={M} N={N} K={k}", flush=True)
    _native.call("pointops_knn3_windowed", q.data_ptr(), r.data_ptr(), dist.data_ptr(),
                 idx.data_ptr(), ws.data_ptr(), B, M, N, k, _native.stream(q.device))
    return host(dist), host(idx)


def _case(name: str):
    g = torch.Generator().manual_seed(sum(map(ord, name)))
    if name == "uniform":
        ref = torch.rand(3, 8192, 3, generator=g) * 10
        query = torch.rand(3, 5000, 3, generator=g) * 10
    elif name == "config2":  # the BASELINE config 2 clouds, queries = FPS-like subset
        ref = bench.make_c2(B=2)
        query = ref[:, torch.randperm(4096, generator=g)[:1024]].clone()
    elif name == "ties":  # integer lattice: many equal distances, duplicates
        ref = torch.randint(0, 12, (1, 6000, 3), generator=g).float()
        query = torch.randint(-1, 13, (1, 1500, 3), generator=g).float() + 0.5 * (
            torch.rand(1, 1500, 1, generator=g) < 0.5).float()
    elif name == "far_queries":  # queries outside the references' box
        ref = torch.rand(1, 5000, 3, generator=g)
        query = torch.cat([torch.rand(1, 500, 3, generator=g) * 40 - 20,
                           torch.rand(1, 100, 3, generator=g)], 1)
    elif name == "sparse_clusters":  # tight clusters with wide gaps
        centres = torch.rand(1, 40, 3, generator=g) * 100
        ref = centres.repeat_interleave(50, 1) + torch.randn(1, 2000, 3, generator=g) * 0.1
        query = torch.rand(1, 700, 3, generator=g) * 100
    elif name == "flat":  # zero extent in z
        ref = torch.cat([torch.rand(1, 6000, 2, generator=g), torch.zeros(1, 6000, 1)], 2)
        query = torch.cat([torch.rand(1, 400, 2, generator=g), torch.rand(1, 400, 1, generator=g)], 2)
    elif name == "one_point":  # every reference identical
        ref = torch.full((1, 5000, 3), 0.25)
        query = torch.rand(1, 100, 3, generator=g)
    elif name == "non_finite_refs":
        ref = torch.rand(2, 8000, 3, generator=g)
        ref[0, 7] = float("nan")
        ref[0, 100, 1] = float("inf")
        ref[0, 200] = -float("inf")
        ref[1, :7990] = float("nan")  # ten finite references: K=16 pads
        query = torch.rand(2, 300, 3, generator=g)
    elif name == "non_finite_queries":
        ref = torch.rand(1, 8000, 3, generator=g)
        query = torch.rand(1, 300, 3, generator=g)
        query[0, 5] = float("nan")
        query[0, 70, 2] = -float("inf")
        query[0, 71] = float("inf")
    elif name == "max_size":
        ref = torch.randn(1, 8192, 3, generator=g)
        query = torch.randn(1, 16384, 3, generator=g)
    else:  # "ragged": N and M not multiples of 16 or 64
        ref = torch.rand(2, 1037, 3, generator=g)
        query = torch.rand(2, 77, 3, generator=g)
    return query.contiguous(), ref.contiguous()


CASES = ["uniform", "config2", "ties", "far_queries", "sparse_clusters", "flat", "one_point",
         "non_finite_refs", "non_finite_queries", "max_size", "ragged"]


@pytest.mark.parametrize("name", CASES)
@pytest.mark.parametrize("k", [1, 8, 9, 16, 17, 32])
def test_knn3_windowed_matches_oracle(cuda_device, name, k):
    query, ref = _case(name)
    want_d, want_i = O.knn3(query, ref, k)
    d, i = knn3_windowed(query, ref, k)
    np.testing.assert_array_equal(i, want_i)
    same_bits(d, want_d)


@pytest.mark.parametrize("n,k", [(1, 1), (2, 2), (15, 15), (16, 16), (17, 16), (31, 32), (32, 32),
                                 (33, 32)])
def test_knn3_windowed_tiny_clouds(cuda_device, n, k):
    """K up to N (every reference a neighbour); window narrower than 8 groups."""
    k = min(k, n)
    g = torch.Generator().manual_seed(n * 100 + k)
    ref = torch.rand(2, n, 3, generator=g)
    query = torch.rand(2, 65, 3, generator=g)
    want_d, want_i = O.knn3(query, ref, k)
    d, i = knn3_windowed(query, ref, k)
    np.testing.assert_array_equal(i, want_i)
    same_bits(d, want_d)


def _sweep_case(seed: int):
    """Random sizes and distributions: uniform boxes, Gaussian blobs, sphere
    surfaces, points on a line and heavily duplicated points."""
    g = torch.Generator().manual_seed(2000 + seed)
    B = int(torch.randint(1, 4, (1,), generator=g))
    N = int(torch.randint(32, 8193, (1,), generator=g))
    M = int(torch.randint(1, 3000, (1,), generator=g))
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
def test_knn3_windowed_random_sweep(cuda_device, seed, k):
    query, ref = _sweep_case(seed)
    want_d, want_i = O.knn3(query, ref, k)
    d, i = knn3_windowed(query, ref, k)
    np.testing.assert_array_equal(i, want_i)
    same_bits(d, want_d)


def test_knn3_windowed_config2_full_equals_lane_kernel(cuda_device):
    """Config 2 at full size (B=32, FPS centres as queries, K=16): the
    windowed search equals the plain kernel, twice in a row on one workspace
    (nothing carried over between calls)."""
    import mps_pointops as mp
    from mps_pointops import _native

    x = bench.make_c2().cuda()
    centres = x.gather(1, mp.furthest_point_sample(x, 1024)[..., None].expand(-1, -1, 3))
    centres = centres.contiguous()
    B, M, N, K = 32, 1024, 4096, 16
    bd = torch.empty(B, M, K, device="cuda")
    bi = torch.empty(B, M, K, dtype=torch.long, device="cuda")
    _native.call("pointops_knn3", centres.data_ptr(), x.data_ptr(), bd.data_ptr(), bi.data_ptr(),
                 B, M, N, K, _native.stream(x.device))
    for _ in range(2):
        d, i = knn3_windowed(centres, x, K)
        np.testing.assert_array_equal(i, host(bi))
        same_bits(d, host(bd))


def test_knn3_windowed_rejects_out_of_range(cuda_device):
    """Sizes beyond the windowed search's limits are refused (hipErrorInvalidValue)."""
    from mps_pointops import _native

    lib = _native.library()
    q = torch.zeros(1, 4, 3, device="cuda")
    r = torch.zeros(1, 8193, 3, device="cuda")
    d = torch.empty(1, 4, 1, device="cuda")
    i = torch.empty(1, 4, 1, dtype=torch.long, device="cuda")
    ws = torch.empty(1 << 20, dtype=torch.uint8, device="cuda")
    args = (q.data_ptr(), r.data_ptr(), d.data_ptr(), i.data_ptr(), ws.data_ptr())
    assert lib.pointops_knn3_windowed(*args, 1, 4, 8193, 1, None) != 0  # N > 8192
    assert lib.pointops_knn3_windowed(*args, 1, 4, 8, 33, None) != 0    # K > 32
    assert lib.pointops_knn3_windowed(*args, 1, 4, 8, 9, None) != 0     # K > N
    assert lib.pointops_knn3_windowed(q.data_ptr(), r.data_ptr(), d.data_ptr(), i.data_ptr(), None,
                                   1, 4, 8, 1, None) != 0            # no workspace


def test_public_knn_takes_windowed_path(cuda_device, monkeypatch):
    """ops.knn sends config-2-sized clouds to the windowed entry point and
    smaller ones (config 1) to the plain kernel; both equal the plain kernel."""
    import mps_pointops as mp
    from mps_pointops import _native

    calls = []
    real_call = _native.call

    def spy(name, *args):
        calls.append(name)
        return real_call(name, *args)

    monkeypatch.setattr(_native, "call", spy)
    g = torch.Generator().manual_seed(5)
    for n, want in ((4096, "pointops_knn3_windowed"), (1024, "pointops_knn3")):
        ref = torch.rand(4, n, 3, generator=g).cuda()
        query = torch.rand(4, 300, 3, generator=g).cuda()
        calls.clear()
        d, i = mp.knn(query, ref, 16)
        assert calls == [want]
        bd = torch.empty_like(d)
        bi = torch.empty_like(i)
        real_call("pointops_knn3", query.data_ptr(), ref.data_ptr(), bd.data_ptr(), bi.data_ptr(),
                  4, 300, n, 16, _native.stream(query.device))
        np.testing.assert_array_equal(host(i), host(bi))
        same_bits(host(d), host(bd))
