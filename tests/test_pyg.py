"""pyg-lib operator registration (the reference's tests/test_pyg28.py).

pyg-lib is not installed here, so its ``pyg::fps/knn/radius`` schemas are
stood in for by the same signatures (pyg.py:75-135 of the reference) under a
scratch namespace, and a stand-in ``pyg_lib`` module; registration and the
known answers then run exactly as they would against pyg-lib's own schemas.
"""

from __future__ import annotations

import sys
import types

import pytest
import torch

from mps_pointops import pyg

_NS = "pyg_rocm_standin"
_SCHEMAS = {
    "fps": "fps(Tensor src, Tensor ptr, float ratio=0.5, bool random_start=True) -> Tensor",
    "knn": "knn(Tensor x, Tensor y, Tensor? ptr_x=None, Tensor? ptr_y=None, int k=1, "
           "bool cosine=False, int num_workers=1) -> Tensor",
    "radius": "radius(Tensor x, Tensor y, Tensor? ptr_x=None, Tensor? ptr_y=None, float r=1.0, "
              "int max_num_neighbors=32, int num_workers=1, bool ignore_same_index=False) -> Tensor",
}
_DEFS: list[torch.library.Library] = []


def _define_standin_schemas() -> None:
    if not _DEFS:
        library = torch.library.Library(_NS, "DEF")
        for schema in _SCHEMAS.values():
            library.define(schema)
        _DEFS.append(library)


def _fake_pyg_lib(names=("fps", "knn", "radius")) -> types.ModuleType:
    module = types.ModuleType("pyg_lib")
    module.ops = types.SimpleNamespace(**{name: object() for name in names})
    return module


@pytest.fixture
def standin(monkeypatch):
    _define_standin_schemas()
    monkeypatch.setitem(sys.modules, "pyg_lib", _fake_pyg_lib())
    monkeypatch.setattr(pyg, "_NAMESPACE", _NS)
    monkeypatch.setattr(pyg, "_LIBRARY", None)
    yield getattr(torch.ops, _NS)


def test_register_requires_pyg_lib(monkeypatch):
    monkeypatch.setitem(sys.modules, "pyg_lib", None)
    monkeypatch.setattr(pyg, "_LIBRARY", None)
    with pytest.raises(ImportError, match="pyg-lib>=0.6"):
        pyg.register_rocm()


def test_register_rejects_missing_operator(monkeypatch):
    _define_standin_schemas()
    monkeypatch.setitem(sys.modules, "pyg_lib", _fake_pyg_lib(("fps", "knn")))
    monkeypatch.setattr(pyg, "_NAMESPACE", _NS)
    monkeypatch.setattr(pyg, "_LIBRARY", None)
    with pytest.raises(RuntimeError, match="does not provide pyg::radius"):
        pyg.register_rocm()


def test_register_adds_cuda_kernels_once(standin):
    """test_pyg28.py:27-31: every operator gets a kernel on the ROCm key, a
    second call registers nothing; register_mps is the same call."""
    assert pyg.register_mps is pyg.register_rocm
    assert sorted(pyg.register_rocm()) == ["fps", "knn", "radius"]
    assert all(torch._C._dispatch_has_kernel_for_dispatch_key(f"{_NS}::{name}", "CUDA")
               for name in _SCHEMAS)
    assert pyg.register_rocm() == []


@pytest.mark.gpu
def test_registered_operators_known_answers(cuda_device, standin):
    """test_pyg28.py:27-50 and 53-58: fps, knn and radius on two clouds, and
    ignore_same_index applied before the neighbour limit."""
    ops = standin
    pyg.register_rocm()
    x = torch.tensor([[0.0, 0, 0], [1.0, 0, 0], [10.0, 0, 0], [11.0, 0, 0]], device="cuda")
    y = torch.tensor([[0.1, 0, 0], [10.1, 0, 0]], device="cuda")
    ptr_x = torch.tensor([0, 2, 4], dtype=torch.long, device="cuda")
    ptr_y = torch.tensor([0, 1, 2], dtype=torch.long, device="cuda")
    assert ops.fps(x, ptr_x, 0.5, False).cpu().tolist() == [0, 2]
    expected = [[0, 0, 1, 1], [0, 1, 2, 3]]
    assert ops.knn(x, y, ptr_x, ptr_y, 2).cpu().tolist() == expected
    assert ops.radius(x, y, ptr_x, ptr_y, 1.0).cpu().tolist() == expected
    x3 = torch.tensor([[0.0, 0, 0], [0.1, 0, 0], [0.2, 0, 0]], device="cuda")
    y3 = torch.tensor([[0.0, 0, 0]], device="cuda")
    assert ops.radius(x3, y3, None, None, 1.0, 1, 1, True).cpu().tolist() == [[0], [1]]


@pytest.mark.gpu
def test_registered_operators_defaults_and_batches(cuda_device, standin):
    """test_pyg28.py:70-106: schema defaults, feature-space kNN, the k limit,
    and a query batch without a reference batch (every reference serves
    every query)."""
    ops = standin
    pyg.register_rocm()
    x = torch.tensor([[0.0, 0, 0], [2.0, 0, 0]], device="cuda")
    y = torch.tensor([[0.1, 0, 0]], device="cuda")
    assert ops.knn(x, y).cpu().tolist() == [[0], [0]]
    assert ops.radius(x, y).cpu().tolist() == [[0], [0]]

    f = torch.zeros((4, 64), device="cuda")
    f[:, 0] = torch.tensor([0.0, 1.0, 10.0, 11.0], device="cuda")
    q = f[[0, 2]] + 0.1
    pf = torch.tensor([0, 2, 4], device="cuda")
    pq = torch.tensor([0, 1, 2], device="cuda")
    assert ops.knn(f, q, pf, pq, 2).cpu().tolist() == [[0, 0, 1, 1], [0, 1, 2, 3]]

    for dims in (3, 64):
        big = torch.arange(257, dtype=torch.float32, device="cuda")[:, None].expand(-1, dims)
        big = big.contiguous()
        with pytest.raises(ValueError, match="effective k must be at most 256 on ROCm"):
            ops.knn(big, big[:1], None, None, 257)
        assert ops.knn(big[:256], big[:1], None, None, 300).shape == (2, 256)

    x2 = torch.tensor([[0.0, 0, 0], [10.0, 0, 0]], device="cuda")
    y2 = x2.clone()
    ptr_y = torch.tensor([0, 1, 2], dtype=torch.long, device="cuda")
    assert ops.knn(x2, y2, None, ptr_y, 1).cpu().tolist() == [[0, 1], [0, 1]]
    assert ops.radius(x2, y2, None, ptr_y, 1.0, 2).cpu().tolist() == [[0, 1], [0, 1]]
