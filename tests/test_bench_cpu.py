"""bench.py's command-line contract, on the CPU: it runs on one GPU only, says
so for any other --gpus as a one-line JSON error, and reads the committed
HBM-traffic table that its roofline line cites."""

from __future__ import annotations

import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.parametrize("gpus", ["2", "8"])
def test_more_than_one_gpu_is_refused_with_a_json_line(gpus):
    proc = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", gpus],
                          capture_output=True, text=True, timeout=120, cwd=ROOT)
    assert proc.returncode == 2
    lines = [ln for ln in proc.stdout.splitlines() if ln.strip()]
    assert len(lines) == 1
    msg = json.loads(lines[0])
    assert "one GPU" in msg["error"]


def test_no_gpu_is_reported_as_a_json_error():
    env = dict(os.environ, HIP_VISIBLE_DEVICES="", CUDA_VISIBLE_DEVICES="")
    proc = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--steps", "1", "--warmup", "0"],
                          capture_output=True, text=True, timeout=300, cwd=ROOT, env=env)
    assert proc.returncode != 0
    msg = json.loads([ln for ln in proc.stdout.splitlines() if ln.strip()][-1])
    assert "error" in msg


def test_traffic_table_covers_the_headline_kernel():
    sys.path.insert(0, ROOT)
    import bench

    traffic = bench._traffic("rmsnorm_residual")
    assert traffic is not None
    alg = 8192 * 4096 * 8 + 4096 * 2
    assert 0.98 * alg <= traffic <= 1.05 * alg
