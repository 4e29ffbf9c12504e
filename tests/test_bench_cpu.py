"""bench.py's contract pieces that need no GPU: the refusal of more than one
GPU and the CPU baseline's fields."""

from __future__ import annotations

import json
import subprocess
import sys
from pathlib import Path

import bench

ROOT = Path(__file__).resolve().parents[1]


def test_more_than_one_gpu_exits_with_a_message():
    proc = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                          capture_output=True, text=True, timeout=300)
    assert proc.returncode == 2
    line = json.loads(proc.stdout.strip().splitlines()[-1])
    assert "one MI355X" in line["error"] and line["n_gpus"] == 2


def test_cpu_baseline_fields():
    """One cloud of config 2 through the CPU port: points/s, the cores used,
    the kind of baseline and what was sampled."""
    xyz = bench.make_c2(B=1)
    out = bench.cpu_baseline(xyz, 1, warmup=1, repeats=3)
    assert out["value"] > 0 and out["unit"] == "points/s"
    assert out["kind"] == "port" and out["cores"] >= 1
    assert out["sample"].startswith("1 of 32 clouds of config 2")
    assert "median of 3 passes after 1 warmups" in out["sample"]
