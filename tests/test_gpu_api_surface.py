"""GPU tests of the public option surface: every chamfer_distance option, the
flat graph wrappers, the float16 flat radius and the knn_cuda stand-in.

The expected values are the reference's own test literals (file:line cited
per test, /root/reference/tests/...) and, for random inputs, the CPU oracle:
indices bit-exact, Chamfer losses within 1e-5 relative and gradients within
1e-4 relative (the tolerances of the contract), closed-form literals exactly.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def dev(values, dtype=torch.float32, grad=False):
    t = torch.tensor(values, dtype=dtype, device="cuda")
    return t.requires_grad_(grad)


def host(t):
    return t.detach().cpu()


def exact(actual, expected):
    torch.testing.assert_close(host(actual), torch.as_tensor(expected, dtype=actual.dtype),
                               rtol=0, atol=0)


# ------------------------------------------------------------------ Chamfer


def test_chamfer_bidirectional_tie_gradient(cuda_device):
    """tests/test_chamfer.py:8-20: y picks x[0] on the tie."""
    from mps_pointops import chamfer_distance

    x = dev([[[0.0, 0.0, 0.0], [2.0, 0.0, 0.0]]], grad=True)
    y = dev([[[1.0, 0.0, 0.0]]], grad=True)
    loss, normals = chamfer_distance(x, y, batch_reduction="sum")
    assert normals is None and loss.item() == 2.0
    loss.backward()
    exact(x.grad, [[[-3.0, 0.0, 0.0], [1.0, 0.0, 0.0]]])
    exact(y.grad, [[[2.0, 0.0, 0.0]]])


def test_chamfer_lengths_hide_nonfinite_padding(cuda_device):
    """tests/test_chamfer.py:23-36."""
    from mps_pointops import chamfer_distance

    x = dev([[[0.0, 0.0, 0.0], [math.nan, 0.0, 0.0]]], grad=True)
    y = dev([[[1.0, 0.0, 0.0], [math.inf, 0.0, 0.0]]], grad=True)
    lengths = torch.tensor([1], device="cuda")
    loss, _ = chamfer_distance(x, y, lengths, lengths)
    assert loss.item() == 2.0
    loss.backward()
    exact(x.grad[0, 0], [-4.0, 0.0, 0.0])
    exact(y.grad[0, 0], [4.0, 0.0, 0.0])
    exact(x.grad[0, 1], [0.0, 0.0, 0.0])
    exact(y.grad[0, 1], [0.0, 0.0, 0.0])


def test_chamfer_reductions_weights_single_direction(cuda_device):
    """tests/test_chamfer.py:39-53."""
    from mps_pointops import chamfer_distance

    x = torch.zeros((2, 1, 3), device="cuda")
    y = dev([[[1.0, 0.0, 0.0]], [[2.0, 0.0, 0.0]]])
    weights = dev([0.1, 0.2])
    mean, _ = chamfer_distance(x, y, weights=weights)
    torch.testing.assert_close(host(mean), torch.tensor(6.0))
    summed, _ = chamfer_distance(x, y, weights=weights, point_reduction="sum",
                                 batch_reduction="sum")
    torch.testing.assert_close(host(summed), torch.tensor(1.8))
    per_batch, _ = chamfer_distance(x, y, point_reduction="max", batch_reduction=None)
    torch.testing.assert_close(host(per_batch), torch.tensor([1.0, 4.0]))
    one_way, _ = chamfer_distance(x, y, single_directional=True, batch_reduction=None)
    torch.testing.assert_close(host(one_way), torch.tensor([1.0, 4.0]))
    zero_weight, _ = chamfer_distance(x, y, weights=torch.zeros(2, device="cuda"))
    assert zero_weight.item() == 0.0


def test_chamfer_weighted_backward_closed_form(cuda_device):
    """tests/test_chamfer.py:56-67."""
    from mps_pointops import chamfer_distance

    x = torch.zeros((2, 1, 3), device="cuda", requires_grad=True)
    y = dev([[[1.0, 0.0, 0.0]], [[2.0, 0.0, 0.0]]], grad=True)
    loss, _ = chamfer_distance(x, y, weights=dev([1.0, 3.0]))
    loss.backward()
    exact(loss, 6.5)
    exact(x.grad[:, 0, 0], [-1.0, -6.0])
    exact(y.grad[:, 0, 0], [1.0, 6.0])


@pytest.mark.parametrize("norm", [1, 2])
def test_chamfer_all_zero_weights_zero_gradient(cuda_device, norm):
    """tests/test_chamfer.py:70-85."""
    from mps_pointops import chamfer_distance

    x = torch.zeros((1, 1, 3), device="cuda", requires_grad=True)
    y = dev([[[2.0, 0.0, 0.0]]], grad=True)
    weights = torch.zeros(1, device="cuda", requires_grad=True)
    loss, _ = chamfer_distance(x, y, weights=weights, norm=norm)
    loss.backward()
    assert loss.item() == 0.0
    exact(x.grad, torch.zeros((1, 1, 3)))
    exact(y.grad, torch.zeros((1, 1, 3)))
    exact(weights.grad, torch.zeros(1))


@pytest.mark.parametrize("norm", [1, 2])
@pytest.mark.parametrize("point_reduction", ["mean", "sum", "max", None])
@pytest.mark.parametrize("single_directional", [False, True])
def test_chamfer_all_zero_weights_return_structure(cuda_device, norm, point_reduction,
                                                   single_directional):
    """tests/test_chamfer.py:88-127: (B, B) zeros, connected to x, weights and
    (bidirectional only) y."""
    from mps_pointops import chamfer_distance

    x = dev([[[0.0, 0.0, 0.0], [2.0, 0.0, 0.0]], [[3.0, 0.0, 0.0], [4.0, 0.0, 0.0]]], grad=True)
    y = dev([[[1.0, 0.0, 0.0], [2.0, 0.0, 0.0]], [[3.0, 0.0, 0.0], [5.0, 0.0, 0.0]]], grad=True)
    weights = torch.zeros(2, device="cuda", requires_grad=True)
    loss, normals = chamfer_distance(x, y, weights=weights, point_reduction=point_reduction,
                                     batch_reduction=None, single_directional=single_directional,
                                     norm=norm)
    parts = loss if isinstance(loss, tuple) else (loss,)
    assert len(parts) == (1 if single_directional or point_reduction is not None else 2)
    for part in parts:
        assert part.shape == (2, 2)
        exact(part, torch.zeros(2, 2))
    if point_reduction == "max" and not single_directional:
        assert normals is None
    elif isinstance(loss, tuple):
        assert isinstance(normals, tuple) and len(normals) == 2
        assert all(part.shape == (2, 2) for part in normals)
    else:
        assert isinstance(normals, torch.Tensor) and normals.shape == (2, 2)
    grads = torch.autograd.grad(sum(part.sum() for part in parts), (x, y, weights),
                                allow_unused=True)
    assert grads[0] is not None and grads[2] is not None
    assert (grads[1] is None) == single_directional
    for grad in grads:
        if grad is not None:
            exact(grad, torch.zeros_like(host(grad)))


@pytest.mark.parametrize("point_reduction,loss_value,x_grad,y_grad",
                         [("sum", 6.0, [-4.0, 4.0], 0.0), ("max", 4.0, [0.0, 4.0], -4.0)])
def test_chamfer_point_reduction_backward_scaling(cuda_device, point_reduction, loss_value,
                                                  x_grad, y_grad):
    """tests/test_chamfer.py:130-152."""
    from mps_pointops import chamfer_distance

    x = dev([[[0.0, 0.0, 0.0], [3.0, 0.0, 0.0]]], grad=True)
    y = dev([[[1.0, 0.0, 0.0]]], grad=True)
    loss, _ = chamfer_distance(x, y, point_reduction=point_reduction)
    loss.backward()
    assert loss.item() == loss_value
    exact(x.grad[0, :, 0], x_grad)
    assert y.grad[0, 0, 0].item() == y_grad


def test_chamfer_unreduced_distances_zero_padding(cuda_device):
    """tests/test_chamfer.py:155-162."""
    from mps_pointops import chamfer_distance

    x = dev([[[0.0, 0.0, 0.0], [8.0, 0.0, 0.0]]])
    y = dev([[[1.0, 0.0, 0.0], [9.0, 0.0, 0.0]]])
    lengths = torch.tensor([1], device="cuda")
    pair, normals = chamfer_distance(x, y, lengths, lengths, point_reduction=None,
                                     batch_reduction=None)
    assert normals is None and isinstance(pair, tuple)
    exact(pair[0], [[1.0, 0.0]])
    exact(pair[1], [[1.0, 0.0]])


def test_chamfer_lowest_index_tie_in_loss_gradient(cuda_device):
    """tests/test_chamfer.py:165-175: references 1 and 4 tie at distance 1;
    the gradient goes to reference 1."""
    from mps_pointops import chamfer_distance

    x = dev([[[0.0, 0.0, 0.0]]], grad=True)
    y = dev([[[8.0, 0.0, 0.0], [1.0, 0.0, 0.0], [9.0, 0.0, 0.0], [10.0, 0.0, 0.0],
              [-1.0, 0.0, 0.0]]], grad=True)
    loss, _ = chamfer_distance(x, y, single_directional=True)
    assert loss.item() == 1.0
    loss.backward()
    assert y.grad[0, 1, 0].item() == 2.0
    assert y.grad[0, 4, 0].item() == 0.0


def test_chamfer_overflow_keeps_first_index(cuda_device):
    """tests/test_chamfer.py:178-197: every squared distance overflows; index 0
    is kept for the backward gather."""
    from mps_pointops import chamfer, chamfer_distance

    x = dev([[[1e20, 0.0, 0.0]]], grad=True)
    y = dev([[[0.0, 0.0, 0.0], [1.0, 0.0, 0.0]]], grad=True)
    distances, indices = chamfer._nearest_mps(x, y, torch.tensor([1], device="cuda"),
                                              torch.tensor([2], device="cuda"))
    assert torch.isinf(distances).all().item()
    exact(indices, [[0]])
    loss, _ = chamfer_distance(x, y, single_directional=True)
    assert torch.isinf(loss).item()
    loss.backward()
    torch.testing.assert_close(host(x.grad), torch.tensor([[[2e20, 0.0, 0.0]]]))
    torch.testing.assert_close(host(y.grad), torch.tensor([[[-2e20, 0.0, 0.0], [0.0, 0.0, 0.0]]]))


@pytest.mark.parametrize("norm,y_values", [
    (2, [[[1.0, 0.1, 0.2], [4.0, 0.8, 0.7]]]),     # tests/test_chamfer.py:200-203
    (1, [[[1.0, 0.11, 0.21], [4.0, 0.8, 0.7]]]),   # tests/test_chamfer.py:206-209
])
def test_chamfer_float64_gradcheck(cuda_device, norm, y_values):
    """The float64 kernels against finite differences, away from ties and
    (L1) cusps."""
    from mps_pointops import chamfer_distance

    x = dev([[[0.1, 0.2, 0.3], [2.1, 0.4, 0.5]]], torch.float64, grad=True)
    y = dev(y_values, torch.float64, grad=True)
    assert torch.autograd.gradcheck(lambda a, b: chamfer_distance(a, b, norm=norm)[0], (x, y))


def test_chamfer_l1_ranks_by_absolute_sum(cuda_device):
    """tests/test_chamfer.py:212-226."""
    from mps_pointops import chamfer_distance

    x = torch.zeros((1, 1, 3), device="cuda", requires_grad=True)
    y = dev([[[3.0, 0.0, 0.0], [2.0, 2.0, 0.0]]], grad=True)
    l1, _ = chamfer_distance(x, y, norm=1, single_directional=True)
    l2, _ = chamfer_distance(x, y, norm=2, single_directional=True)
    assert l1.item() == 3.0 and l2.item() == 8.0
    l1.backward()
    exact(x.grad, [[[-1.0, -1.0, -1.0]]])
    exact(y.grad, [[[1.0, 1.0, 1.0], [0.0, 0.0, 0.0]]])


def test_chamfer_l1_tie_first_reference_and_padding(cuda_device):
    """tests/test_chamfer.py:229-250."""
    from mps_pointops import chamfer, chamfer_distance

    x = dev([[[0.0, 0.0, 0.0], [math.nan, 0.0, 0.0]]], grad=True)
    y = dev([[[1.0, 0.0, 0.0], [-1.0, 0.0, 0.0]]], grad=True)
    lx = torch.tensor([1], device="cuda")
    ly = torch.tensor([2], device="cuda")
    distances, indices = chamfer._nearest_mps(x, y, lx, ly, norm=1)
    exact(distances, [[1.0, 0.0]])
    exact(indices, [[0, -1]])
    loss, _ = chamfer_distance(x, y, lx, ly, norm=1, single_directional=True)
    assert loss.item() == 1.0
    loss.backward()
    exact(x.grad[0, 0], [-1.0, -1.0, -1.0])
    exact(x.grad[0, 1], [0.0, 0.0, 0.0])
    exact(y.grad[0, 0], [1.0, 1.0, 1.0])
    exact(y.grad[0, 1], [0.0, 0.0, 0.0])


def test_chamfer_l1_coincidence_minus_one_subgradient(cuda_device):
    """tests/test_chamfer.py:253-266."""
    from mps_pointops import chamfer_distance

    query = torch.zeros((1, 1, 3), device="cuda", requires_grad=True)
    ref = torch.zeros((1, 1, 3), device="cuda", requires_grad=True)
    loss, _ = chamfer_distance(query, ref, norm=1, single_directional=True,
                               point_reduction="sum", batch_reduction="sum")
    assert loss.item() == 0.0
    loss.backward()
    exact(query.grad, -torch.ones((1, 1, 3)))
    exact(ref.grad, torch.ones((1, 1, 3)))


def test_chamfer_l1_tie_stable_across_lanes_and_dispatches(cuda_device):
    """tests/test_chamfer.py:269-285: equal L1 distances at references 0, 31,
    32 and 64 all resolve to 0, on every one of 32 dispatches."""
    from mps_pointops import chamfer

    query = torch.zeros((2, 17, 3), device="cuda")
    ref = torch.full((2, 65, 3), 100.0, device="cuda")
    ref[:, 0] = dev([1.0, 0.0, 0.0])
    ref[:, 31] = dev([-1.0, 0.0, 0.0])
    ref[:, 32] = dev([0.0, 1.0, 0.0])
    ref[:, 64] = dev([0.0, -1.0, 0.0])
    ql = torch.tensor([17, 17], device="cuda")
    rl = torch.tensor([65, 65], device="cuda")
    outputs = [chamfer._nearest_mps(query, ref, ql, rl, norm=1) for _ in range(32)]
    for distances, indices in outputs:
        exact(distances, torch.ones((2, 17)))
        exact(indices, torch.zeros((2, 17), dtype=torch.long))


def test_chamfer_rejects_invalid_inputs(cuda_device):
    """tests/test_chamfer.py:288-306 on ROCm tensors."""
    from mps_pointops import chamfer_distance

    x = torch.zeros((1, 2, 3), device="cuda")
    y = torch.ones((1, 2, 3), device="cuda")
    with pytest.raises(ValueError, match="batch_reduction"):
        chamfer_distance(x, y, point_reduction=None)
    with pytest.raises(ValueError, match="1 or 2 norm"):
        chamfer_distance(x, y, norm=3)
    assert chamfer_distance(x, y, x_normals=x)[1] is None
    with pytest.raises(ValueError, match="Normals must be None"):
        chamfer_distance(x, y, x_normals=x, point_reduction="max")
    with pytest.raises(ValueError, match="same \\(B, P, 3\\) shape"):
        chamfer_distance(x, y, x_normals=torch.zeros((1, 1, 3), device="cuda"))
    empty_loss, _ = chamfer_distance(x, y, torch.tensor([0], device="cuda"),
                                     torch.tensor([2], device="cuda"))
    assert empty_loss.item() == 0.0
    with pytest.raises(ValueError, match=r"\[0, 2\]"):
        chamfer_distance(x, y, torch.tensor([3], device="cuda"), torch.tensor([2], device="cuda"))
    with pytest.raises(ValueError, match="finite"):
        chamfer_distance(x.clone().fill_(math.nan), y)
    with pytest.raises(ValueError, match="nonnegative"):
        chamfer_distance(x, y, weights=dev([-1.0]))


@pytest.mark.parametrize("abs_cosine", [False, True])
def test_chamfer_normal_loss_and_gradients(cuda_device, abs_cosine):
    """tests/test_chamfer.py:309-327."""
    from mps_pointops import chamfer_distance

    x = dev([[[0., 0., 0.], [2., 0., 0.]]], grad=True)
    y = dev([[[1., 0., 0.]]], grad=True)
    xn = dev([[[1., 0., 0.], [0., 1., 0.]]], grad=True)
    yn = dev([[[-1., 0., 0.]]], grad=True)
    loss, normals = chamfer_distance(x, y, x_normals=xn, y_normals=yn, abs_cosine=abs_cosine)
    assert normals is not None
    exact(normals, 0.5 if abs_cosine else 3.5)
    grads = torch.autograd.grad(loss + normals, (x, y, xn, yn))
    exact(grads[0], [[[-3., 0., 0.], [1., 0., 0.]]])
    exact(grads[1], [[[2., 0., 0.]]])
    assert grads[2].shape == xn.shape and grads[3].shape == yn.shape
    assert torch.isfinite(grads[2]).all() and torch.isfinite(grads[3]).all()


def test_chamfer_zero_normals_padding_and_one_sided(cuda_device):
    """tests/test_chamfer.py:330-351."""
    from mps_pointops import chamfer_distance

    x = dev([[[0., 0., 0.], [99., 0., 0.]]], grad=True)
    y = dev([[[1., 0., 0.], [88., 0., 0.]]], grad=True)
    xn = dev([[[0., 0., 0.], [math.nan, 0., 0.]]], grad=True)
    yn = dev([[[0., 0., 0.], [math.nan, 0., 0.]]], grad=True)
    lengths = torch.tensor([1], device="cuda")
    loss, normals = chamfer_distance(x, y, lengths, lengths, x_normals=xn, y_normals=yn,
                                     point_reduction=None, batch_reduction=None)
    assert isinstance(loss, tuple) and isinstance(normals, tuple)
    for part in normals:
        exact(part, [[1., 0.]])
    gxn, gyn = torch.autograd.grad(sum(part.sum() for part in normals), (xn, yn))
    assert torch.isfinite(gxn).all() and torch.isfinite(gyn).all()
    exact(gxn, torch.zeros((1, 2, 3)))
    exact(gyn, torch.zeros((1, 2, 3)))
    _, only_one = chamfer_distance(x, y, lengths, lengths, x_normals=xn)
    assert only_one is None


@pytest.mark.parametrize("x_empty", [True, False])
def test_chamfer_empty_cloud_zero_loss_and_gradient(cuda_device, x_empty):
    """tests/test_chamfer.py:381-395."""
    from mps_pointops import chamfer_distance

    x = torch.zeros((1, 0 if x_empty else 2, 3), device="cuda", requires_grad=True)
    y = torch.ones((1, 2 if x_empty else 0, 3), device="cuda", requires_grad=True)
    loss, normals = chamfer_distance(x, y)
    assert normals is None and loss.item() == 0.0
    gx, gy = torch.autograd.grad(loss, (x, y))
    assert gx.shape == x.shape and gy.shape == y.shape
    exact(gx, torch.zeros(x.shape))
    exact(gy, torch.zeros(y.shape))


def test_chamfer_empty_cloud_inside_uneven_batch(cuda_device):
    """tests/test_chamfer.py:398-419."""
    from mps_pointops import chamfer_distance

    x = dev([[[0., 0., 0.], [9., 0., 0.]], [[0., 0., 0.], [2., 0., 0.]]], grad=True)
    y = dev([[[1., 0., 0.], [2., 0., 0.]], [[1., 0., 0.], [3., 0., 0.]]], grad=True)
    xn = dev([[[1., 0., 0.], [0., 0., 1.]], [[1., 0., 0.], [0., 1., 0.]]], grad=True)
    yn = dev([[[1., 0., 0.], [0., 1., 0.]], [[1., 0., 0.], [0., 1., 0.]]], grad=True)
    distance, normal = chamfer_distance(x, y, x_lengths=torch.tensor([0, 2], device="cuda"),
                                        y_lengths=torch.tensor([2, 2], device="cuda"),
                                        x_normals=xn, y_normals=yn, batch_reduction=None)
    assert normal is not None
    assert distance[0].item() == 0.0 and normal[0].item() == 1.0
    grads = torch.autograd.grad(distance.sum() + normal.sum(), (x, y, xn, yn))
    for grad in grads:
        assert torch.isfinite(grad).all()
    exact(grads[0][0], torch.zeros((2, 3)))
    exact(grads[2][0], torch.zeros((2, 3)))


def test_chamfer_nearest_writes_every_row_first_tie(cuda_device):
    """tests/test_chamfer.py:443-469: ties at references 0, 31 and 36 choose 0;
    rows beyond the lengths are (0, -1)."""
    from mps_pointops import chamfer

    query = torch.zeros((2, 9, 3))
    ref = torch.full((2, 37, 3), 9.0)
    ref[:, 0] = torch.tensor([1.0, 0.0, 0.0])
    ref[:, 31] = torch.tensor([-1.0, 0.0, 0.0])
    ref[:, 36] = torch.tensor([0.0, 1.0, 0.0])
    query[0, 8] = torch.tensor([math.nan, 0.0, 0.0])
    query[1, 7:] = torch.tensor([math.nan, 0.0, 0.0])
    distance, index = chamfer._nearest_mps(query.cuda(), ref.cuda(),
                                           torch.tensor([8, 7], device="cuda"),
                                           torch.tensor([37, 32], device="cuda"))
    want_d = torch.ones((2, 9))
    want_d[0, 8] = 0.0
    want_d[1, 7:] = 0.0
    want_i = torch.zeros((2, 9), dtype=torch.long)
    want_i[0, 8] = -1
    want_i[1, 7:] = -1
    exact(distance, want_d)
    exact(index, want_i)


def _chamfer_expected(x, y, lx, ly, weights, norm, point_reduction, batch_reduction,
                      single_directional):
    """Loss and coordinate gradients in float64 numpy from the oracle's nearest
    indices: PyTorch3D's definitions (chamfer.py:342-488), written from the
    closed form of each term."""
    B = x.shape[0]
    w = np.ones(B) if weights is None else weights.astype(np.float64)
    gx = np.zeros(x.shape)
    gy = np.zeros(y.shape)
    terms = []
    pairs = [(x, y, lx, ly, gx, gy)]
    if not single_directional:
        pairs.append((y, x, ly, lx, gy, gx))
    for q, r, lq, lr, gq, gr in pairs:
        d, i = O.chamfer_nearest(q, r, lq, lr, norm)
        per_cloud = np.zeros(B)
        for b in range(B):
            n = int(lq[b])
            if n == 0 or lr[b] == 0:
                continue
            vals = d[b, :n].astype(np.float64) * w[b]
            scale = w[b] / max(n, 1) if point_reduction == "mean" else w[b]
            per_cloud[b] = vals.sum() / max(n, 1) if point_reduction == "mean" else vals.sum()
            delta = q[b, :n].astype(np.float64) - r[b, i[b, :n]].astype(np.float64)
            local = 2.0 * delta if norm == 2 else np.where(delta > 0, 1.0, -1.0)
            gq[b, :n] += scale * local
            np.add.at(gr[b], i[b, :n], -scale * local)
        terms.append(per_cloud)
    loss = sum(terms)
    if batch_reduction is not None:
        denominator = 1.0
        if batch_reduction == "mean":
            denominator = max(B, 1) if weights is None else (w.sum() if w.sum() > 0 else 1.0)
        loss = loss.sum() / denominator
        gx /= denominator
        gy /= denominator
    return loss, gx, gy


@pytest.mark.parametrize("norm", [1, 2])
@pytest.mark.parametrize("point_reduction,batch_reduction", [("mean", "mean"), ("sum", "sum"),
                                                             ("mean", "sum"), ("sum", None)])
@pytest.mark.parametrize("weighted,single", [(False, False), (True, False), (True, True)])
def test_chamfer_random_uneven_matches_closed_form(cuda_device, norm, point_reduction,
                                                   batch_reduction, weighted, single):
    """Random ragged clouds: the public loss and both gradients against the
    float64 closed form over the oracle's nearest indices (loss rtol 1e-5,
    gradients rtol 1e-4 / atol 1e-6)."""
    from mps_pointops import chamfer_distance

    rng = np.random.default_rng(100 * norm + 10 * weighted + single)
    B, P1, P2 = 5, 300, 257
    x = rng.standard_normal((B, P1, 3)).astype(np.float32)
    y = rng.standard_normal((B, P2, 3)).astype(np.float32)
    lx = np.array([300, 1, 150, 0, 299], np.int64)
    ly = np.array([257, 200, 2, 100, 0], np.int64)
    w = rng.random(B).astype(np.float32) if weighted else None
    xd = torch.from_numpy(x).cuda().requires_grad_()
    yd = torch.from_numpy(y).cuda().requires_grad_()
    loss, _ = chamfer_distance(xd, yd, torch.from_numpy(lx).cuda(), torch.from_numpy(ly).cuda(),
                               weights=None if w is None else torch.from_numpy(w).cuda(),
                               norm=norm, point_reduction=point_reduction,
                               batch_reduction=batch_reduction, single_directional=single)
    want, gx, gy = _chamfer_expected(x, y, lx, ly, w, norm, point_reduction, batch_reduction,
                                     single)
    np.testing.assert_allclose(host(loss).numpy(), want, rtol=1e-5, atol=1e-6)
    loss.sum().backward()
    np.testing.assert_allclose(host(xd.grad).numpy(), gx, rtol=1e-4, atol=1e-6)
    np.testing.assert_allclose(host(yd.grad).numpy(), gy, rtol=1e-4, atol=1e-6)


def test_chamfer_nearest_small_oracle_strided(cuda_device):
    """tests/test_chamfer.py:472-503: uneven lengths, strided views."""
    from mps_pointops import chamfer

    g = torch.Generator().manual_seed(137)
    query = torch.randn((3, 13, 3), generator=g)
    ref = torch.randn((3, 67, 3), generator=g)
    ql = torch.tensor([13, 4, 9])
    rl = torch.tensor([67, 39, 3])
    query = query.repeat_interleave(2, dim=1)[:, ::2, :]
    ref = ref.repeat_interleave(2, dim=1)[:, ::2, :]
    distance, index = chamfer._nearest_mps(query.cuda(), ref.cuda(), ql.cuda(), rl.cuda())
    want_d, want_i = O.chamfer_nearest(query.contiguous(), ref.contiguous(), ql, rl)
    np.testing.assert_array_equal(host(index).numpy(), want_i)
    np.testing.assert_array_equal(host(distance).numpy().view(np.uint32), want_d.view(np.uint32))


# ------------------------------------------------------- flat graph wrappers


def test_flat_graph_orientation_and_self_loops(cuda_device):
    """tests/test_flat_graph.py:7-22."""
    from mps_pointops import flat

    x = dev([[0.0, 0.0, 0.0], [1.0, 0.0, 0.0], [2.0, 0.0, 0.0]])
    forward = torch.tensor([[1, 0, 1], [0, 1, 2]])
    reverse = forward.flip(0)
    assert torch.equal(host(flat.knn_graph(x, 1)), forward)
    assert torch.equal(host(flat.knn_graph(x, 1, flow="target_to_source")), reverse)
    assert torch.equal(host(flat.radius_graph(x, 1.1, max_num_neighbors=1)), forward)
    assert torch.equal(host(flat.radius_graph(x, 1.1, max_num_neighbors=1,
                                              flow="target_to_source")), reverse)
    assert flat.knn_graph(x, 1, loop=True).shape == (2, len(x))
    assert flat.radius_graph(x, 0.5, loop=True).shape == (2, len(x))


def test_flat_knn_features_and_graph(cuda_device):
    """tests/test_feature_knn.py:139-152: 64-dimensional features."""
    from mps_pointops import flat

    x = torch.zeros((5, 64), device="cuda")
    x[:, 0] = dev([0.0, 1.0, 4.0, 10.0, 11.0])
    y = x[[0, 3]] + 0.1
    bx = torch.tensor([0, 0, 0, 1, 1], device="cuda")
    by = torch.tensor([0, 1], device="cuda")
    assert flat.knn(x, y, 2, bx, by).cpu().tolist() == [[0, 0, 1, 1], [0, 1, 3, 4]]
    graph = flat.knn_graph(x, 1, bx, loop=False)
    assert graph.shape == (2, 5)
    assert all(a != b for a, b in zip(*graph.cpu().tolist()))


@pytest.mark.parametrize("loop", [False, True])
@pytest.mark.parametrize("flow", ["source_to_target", "target_to_source"])
def test_flat_graphs_match_oracle_ragged(cuda_device, loop, flow):
    """knn_graph / radius_graph over three ragged clouds against the oracle's
    flat searches (k + 1 requested and self edges dropped without loop;
    torch_cluster's (source, target) orientation)."""
    from mps_pointops import flat

    rng = np.random.default_rng(7 + loop)
    x = rng.random((900, 3), dtype=np.float32)
    x[100:140] = x[0]  # exact duplicates: ties resolved by index
    batch = np.sort(rng.integers(0, 3, 900))
    ptr = np.searchsorted(batch, np.arange(4)).astype(np.int64)
    xc, bc = torch.from_numpy(x).cuda(), torch.from_numpy(batch).cuda()

    def expect(table):
        q, s = np.nonzero(table >= 0)
        src, dst = table[q, s], q
        if not loop:
            keep = src != dst
            src, dst = src[keep], dst[keep]
        edges = np.stack([src, dst]) if flow == "source_to_target" else np.stack([dst, src])
        return edges.tolist()

    k = 6
    got = flat.knn_graph(xc, k, bc, loop=loop, flow=flow)
    assert got.cpu().tolist() == expect(O.knn_flat(x, x, ptr, ptr, k if loop else k + 1))
    got = flat.radius_graph(xc, 0.08, bc, loop=loop, max_num_neighbors=k, flow=flow)
    assert got.cpu().tolist() == expect(O.radius_flat(x, x, ptr, ptr, 0.08,
                                                      k if loop else k + 1))


# --------------------------------------------------------- float16 radius


@pytest.mark.parametrize("r,k", [(0.05, 8), (0.21, 32), (0.1, 300)])
def test_flat_radius_float16_matches_oracle(cuda_device, r, k):
    """Half coordinates widen exactly to float32, so the float16 search equals
    the float32 oracle on the widened values (threshold fl32(r*r in double),
    tests/test_flat.py:207-224)."""
    from mps_pointops import flat

    rng = np.random.default_rng(int(r * 1000) + k)
    x = rng.random((2000, 3)).astype(np.float16)
    y = rng.random((400, 3)).astype(np.float16)
    y[:50] = x[:50]  # queries on top of references
    bx = np.sort(rng.integers(0, 4, 2000))
    by = np.sort(rng.integers(0, 4, 400))
    size = int(max(bx.max(), by.max())) + 1
    px = np.searchsorted(bx, np.arange(size + 1)).astype(np.int64)
    py = np.searchsorted(by, np.arange(size + 1)).astype(np.int64)
    got = flat.radius(torch.from_numpy(x).cuda(), torch.from_numpy(y).cuda(), r,
                      torch.from_numpy(bx).cuda(), torch.from_numpy(by).cuda(),
                      max_num_neighbors=k)
    want = O.radius_flat(x.astype(np.float32), y.astype(np.float32), px, py, r,
                         min(k, len(x)))
    q, s = np.nonzero(want >= 0)
    assert len(q) > 0
    assert got.cpu().tolist() == [q.tolist(), want[q, s].tolist()]


def test_radius_graph_float16(cuda_device):
    """radius_graph on half coordinates equals the float32 graph of the
    widened coordinates."""
    from mps_pointops import flat

    rng = np.random.default_rng(3)
    x = rng.random((600, 3)).astype(np.float16)
    half = flat.radius_graph(torch.from_numpy(x).cuda(), 0.1, max_num_neighbors=16)
    full = flat.radius_graph(torch.from_numpy(x.astype(np.float32)).cuda(), 0.1,
                             max_num_neighbors=16)
    assert half.shape[1] > 0
    assert torch.equal(half.cpu(), full.cpu())


# ------------------------------------------------------------ knn_cuda.KNN


@pytest.mark.parametrize("transpose_mode", [True, False])
def test_compat_knn_module_layouts(cuda_device, transpose_mode):
    """tests/test_compat.py:150-160, against the exact oracle."""
    from mps_pointops import compat

    g0, g1 = torch.Generator().manual_seed(0), torch.Generator().manual_seed(1)
    ref = torch.randn(2, 3000, 3, generator=g0)
    query = torch.randn(2, 100, 3, generator=g1)
    want_d, want_i = O.knn3(query, ref, 16)
    module = compat.KNN(16, transpose_mode=transpose_mode)
    if transpose_mode:
        d, i = module(ref.cuda(), query.cuda())
    else:
        d, i = module(ref.transpose(1, 2).cuda(), query.transpose(1, 2).cuda())
        assert d.shape == (2, 16, 100) and i.shape == (2, 16, 100)
        d, i = d.transpose(1, 2), i.transpose(1, 2)
    np.testing.assert_array_equal(host(i).numpy(), want_i)
    np.testing.assert_array_equal(host(d).numpy().view(np.uint32), want_d.view(np.uint32))
    assert not d.requires_grad


def test_compat_knn_module_feature_dims(cuda_device):
    """knn_cuda layouts with D = 5 (the feature kernel)."""
    from mps_pointops import compat

    rng = np.random.default_rng(11)
    ref = rng.standard_normal((3, 5, 700)).astype(np.float32)   # (B, D, N)
    query = rng.standard_normal((3, 5, 90)).astype(np.float32)  # (B, D, M)
    d, i = compat.KNN(7)(torch.from_numpy(ref).cuda(), torch.from_numpy(query).cuda())
    want_d, want_i = O.knn_feat(query.transpose(0, 2, 1), ref.transpose(0, 2, 1), 7)
    np.testing.assert_array_equal(host(i).numpy(), want_i.transpose(0, 2, 1))
    np.testing.assert_array_equal(host(d).numpy().view(np.uint32),
                                  want_d.transpose(0, 2, 1).view(np.uint32))
