"""ROCm kernels for pyg-lib's point-cloud operators (pyg.py of the reference).

``register_rocm()`` adds implementations of ``pyg::fps``, ``pyg::knn`` and
``pyg::radius`` on the CUDA dispatch key (the key ROCm tensors carry) to
pyg-lib's existing operator schemas, for builds of pyg-lib without kernels
of their own there; kernels pyg-lib already has are left in place
(pyg.py:144-181).  Like the reference it needs pyg-lib >= 0.6 and raises
ImportError without it.  ``register_mps`` is the reference's name for the
same call.  Not covered: ``pyg::grid_cluster`` (the graph/cluster extras are
outside this package), and the reference's PyG 2.8 CSR bridge for MPS
(pyg.py:23-56), which ROCm does not need.
"""

from __future__ import annotations

import torch
from torch import Tensor

from . import flat

_NAMESPACE = "pyg"
_LIBRARY: torch.library.Library | None = None


def _check_ptr(ptr: Tensor, count: int, device: torch.device, name: str) -> Tensor:
    if not isinstance(ptr, Tensor) or ptr.ndim != 1 or ptr.dtype not in (torch.int32, torch.int64):
        raise ValueError(f"{name} must be a one-dimensional integer tensor")
    if ptr.device != device:
        raise ValueError(f"{name} must be on {device}")
    values = ptr.long()
    if len(values) == 0 or int(values[0]) != 0 or int(values[-1]) != count:
        raise ValueError(f"{name} must start at 0 and end at {count}")
    if bool((values[1:] < values[:-1]).any()):
        raise ValueError(f"{name} must be non-decreasing")
    return values.contiguous()


def _ptrs(x: Tensor, y: Tensor, ptr_x: Tensor | None, ptr_y: Tensor | None, *,
          feature_space: bool = False) -> tuple[Tensor, Tensor]:
    """pyg.py:59-72: an unbatched x is the whole reference set for every
    query (ptr_y is then ignored); ptr_x needs ptr_y."""
    flat._search_pair(x, y, coordinates=not feature_space)
    if ptr_x is None:
        return (torch.tensor([0, len(x)], dtype=torch.long, device=x.device),
                torch.tensor([0, len(y)], dtype=torch.long, device=y.device))
    if ptr_y is None:
        raise ValueError("ptr_y is required when ptr_x is given")
    ptr_x = _check_ptr(ptr_x, len(x), x.device, "ptr_x")
    ptr_y = _check_ptr(ptr_y, len(y), y.device, "ptr_y")
    if len(ptr_x) != len(ptr_y):
        raise ValueError("ptr_x and ptr_y must describe the same number of clouds")
    return ptr_x, ptr_y


def _knn_rocm(x: Tensor, y: Tensor, ptr_x: Tensor | None = None, ptr_y: Tensor | None = None,
              k: int = 1, cosine: bool = False, num_workers: int = 1) -> Tensor:
    """pyg-lib's query-major ``[query, reference]`` edges (pyg.py:75-101)."""
    ptr_x, ptr_y = _ptrs(x, y, ptr_x, ptr_y, feature_space=True)
    k = flat._count_arg(k, "k")
    flat._count_arg(num_workers, "num_workers")
    if cosine:
        raise NotImplementedError("cosine kNN is not supported for ROCm point clouds")
    if x.dtype != torch.float32:
        raise TypeError("x and y must be float32 for kNN on ROCm")
    if k == 0 or len(x) == 0 or len(y) == 0:
        return torch.empty((2, 0), dtype=torch.long, device=x.device)
    width = min(k, len(x))
    if width > flat._KNN_MAX_K:
        raise ValueError(f"effective k must be at most {flat._KNN_MAX_K} on ROCm, got {width}")
    return flat._edge_index(flat.knn_indices(x.contiguous(), y.contiguous(), ptr_x, ptr_y, width))


def _radius_rocm(x: Tensor, y: Tensor, ptr_x: Tensor | None = None, ptr_y: Tensor | None = None,
                 r: float = 1.0, max_num_neighbors: int = 32, num_workers: int = 1,
                 ignore_same_index: bool = False) -> Tensor:
    """The first neighbours in x order, optionally without equal indices
    (pyg.py:104-130)."""
    ptr_x, ptr_y = _ptrs(x, y, ptr_x, ptr_y)
    limit = flat._count_arg(max_num_neighbors, "max_num_neighbors")
    flat._count_arg(num_workers, "num_workers")
    if x.dtype not in (torch.float16, torch.float32):
        raise TypeError("x and y must be float16 or float32 for radius on ROCm")
    if limit == 0 or len(x) == 0 or len(y) == 0:
        return torch.empty((2, 0), dtype=torch.long, device=x.device)
    width = min(limit, len(x))
    indices = flat.radius_indices(x.contiguous(), y.contiguous(), ptr_x, ptr_y, r, width,
                                  ignore_same_index=ignore_same_index)
    return flat._edge_index(indices)


def _fps_rocm(src: Tensor, ptr: Tensor, ratio: float = 0.5, random_start: bool = True) -> Tensor:
    """FPS on pyg-lib's pointer-shaped call (pyg.py:133-135)."""
    return flat.fps(src, ratio=ratio, random_start=random_start, ptr=ptr)


_IMPLEMENTATIONS = {"fps": _fps_rocm, "knn": _knn_rocm, "radius": _radius_rocm}


def register_rocm() -> list[str]:
    """Register ROCm kernels for pyg-lib's point search operators; returns
    the operator names this call registered (none on a repeated call)."""
    global _LIBRARY
    if _LIBRARY is not None:
        return []
    try:
        import pyg_lib
    except ImportError as exc:
        raise ImportError(
            "PyG integration requires pyg-lib>=0.6 with a wheel matching "
            "your PyTorch version"
        ) from exc
    namespace = getattr(torch.ops, _NAMESPACE)
    for name in _IMPLEMENTATIONS:
        if not hasattr(pyg_lib.ops, name) or not hasattr(namespace, name):
            raise RuntimeError(f"pyg-lib does not provide pyg::{name}; pyg-lib>=0.6 is required")
    library = torch.library.Library(_NAMESPACE, "IMPL", "CUDA")
    registered = []
    for name, implementation in _IMPLEMENTATIONS.items():
        if not torch._C._dispatch_has_kernel_for_dispatch_key(f"{_NAMESPACE}::{name}", "CUDA"):
            library.impl(name, implementation)
            registered.append(name)
    _LIBRARY = library  # registrations live as long as the Library object
    return registered


register_mps = register_rocm  # the reference's name (pyg.py:144)

__all__ = ["register_rocm", "register_mps"]
