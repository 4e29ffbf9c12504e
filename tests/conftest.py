"""Shared pytest setup: import paths, the ``gpu`` marker, golden loaders."""

from __future__ import annotations

import json
import math
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG_ROOT = ROOT / "mps-pointops_amd"
for path in (str(ROOT), str(PKG_ROOT)):
    if path not in sys.path:
        sys.path.insert(0, path)

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (ROCm device visible to torch)")


def _decode(value):
    """JSON fixtures spell non-finite floats as strings."""
    if isinstance(value, list):
        return [_decode(v) for v in value]
    if value == "nan":
        return math.nan
    if value == "inf":
        return math.inf
    if value == "-inf":
        return -math.inf
    return value


def load_known_answers(op: str | None = None) -> list[dict]:
    cases = json.loads((GOLDEN / "known_answers.json").read_text())["cases"]
    out = []
    for case in cases:
        if op is None or case["op"] == op:
            out.append({k: _decode(v) for k, v in case.items()})
    return out


def load_pointnet2_parity() -> dict:
    return json.loads((GOLDEN / "pointnet2_parity.json").read_text())


@pytest.fixture(scope="session")
def cuda_device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    return torch.device("cuda", 0)
