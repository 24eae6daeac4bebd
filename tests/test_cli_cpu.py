"""The developer CLI (python -m custom_cuda_kernals_amd.cli) on the CPU:
the registry is consistent with the repository (tests, sources, bench.py
ops, C entry points declared in the header, Python API names), and the
commands that need no GPU render (help, list, info, doctor, visualize from
a stored bench line)."""

from __future__ import annotations

import json
import os
import re

import pytest
from typer.testing import CliRunner

from custom_cuda_kernals_amd import kernels
from custom_cuda_kernals_amd.cli import app as cli_app
from custom_cuda_kernals_amd.cli import runners
from custom_cuda_kernals_amd.cli.registry import REGISTRY, list_ops
from tests import _cck

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
runner = CliRunner()


def _bench_op_patterns() -> list[re.Pattern]:
    text = open(os.path.join(ROOT, "bench.py")).read()
    names = re.findall(r'Op\(\s*f?"([A-Za-z0-9_{}]+)"', text)
    return [re.compile("^" + re.sub(r"\{[a-z_]+\}", r"\\d+", n) + "$") for n in names]


@pytest.mark.parametrize("op_id", sorted(REGISTRY))
def test_registry_matches_repository(op_id):
    s = REGISTRY[op_id]
    for f in s.test_files + s.sources:
        assert os.path.exists(os.path.join(ROOT, f)), f
    declared = _cck.declared_functions()
    for fn in s.c_entry_points:
        assert fn in declared, fn
    for fn in s.python_api:
        assert hasattr(kernels, fn), fn
    pats = _bench_op_patterns()
    for b in s.bench_ops:
        assert any(p.match(b) for p in pats), b


def test_help_and_list():
    r = runner.invoke(cli_app.app, [])
    assert r.exit_code == 0 and "doctor" in r.output and "profile OP" in r.output
    r = runner.invoke(cli_app.app, ["list"])
    assert r.exit_code == 0
    for s in list_ops():
        assert s.id in r.output


def test_info_and_unknown_op():
    r = runner.invoke(cli_app.app, ["info", "fp8_quant"])
    assert r.exit_code == 0 and "launch_fp8_quant_tensor_noalloc_fwd" in r.output
    r = runner.invoke(cli_app.app, ["info", "rmsnorm"])
    assert r.exit_code == 1


def test_doctor_reports_every_check():
    from custom_cuda_kernals_amd.cli.env_checks import run_checks

    checks = run_checks()
    names = [c.name for c in checks]
    assert any("hipcc" in n for n in names) and any("gfx950" in n for n in names)
    lib = [c for c in checks if c.name == "libcustom_kernels_amd.so"][0]
    assert lib.status == "ok", lib.detail  # the in-tree build holds a gfx950 code object
    r = runner.invoke(cli_app.app, ["doctor"])
    assert "PyTorch" in r.output


def test_benchmark_shows_a_stored_result_without_a_gpu(tmp_path, monkeypatch):
    """Without --rerun, `benchmark` renders the stored bench line (no GPU needed);
    --full adds the recorded detail columns."""
    monkeypatch.setattr(runners, "RESULTS", tmp_path)
    line = {"ops": {"rope_inplace": {"workload": "rope_inplace_bf16_8x4096", "us": 102.1, "GB_per_s": 6593.0,
                                     "frac_of_8TBps": 0.8242, "algorithmic_bytes": 673185792, "shape": [8, 4096],
                                     "steps": 100, "buffer_sets": 4,
                                     "per_call": {"median_us": 110.2, "iqr_us": 0.5, "calls": 30}}}}
    (tmp_path / "bench_rope.json").write_text(json.dumps(line))
    r = runner.invoke(cli_app.app, ["benchmark", "rope"])
    assert r.exit_code == 0, r.output
    assert "102.10" in r.output and "stored result" in r.output
    r = runner.invoke(cli_app.app, ["benchmark", "rope", "--full"])
    assert r.exit_code == 0 and "673185792" in r.output


def test_visualize_from_a_stored_bench_line(tmp_path, monkeypatch):
    monkeypatch.setattr(runners, "RESULTS", tmp_path)
    monkeypatch.setattr(cli_app, "RESULTS", tmp_path)
    line = {"ops": {"swiglu": {"workload": "swiglu_bf16_8192x14336", "us": 107.5, "GB_per_s": 6554.0,
                               "frac_of_8TBps": 0.8193}}}
    (tmp_path / "bench_swiglu.json").write_text(json.dumps(line))
    r = runner.invoke(cli_app.app, ["visualize", "swiglu"])
    assert r.exit_code == 0, r.output
    png = tmp_path / "swiglu_bandwidth.png"
    assert png.exists() and png.read_bytes()[:4] == b"\x89PNG"
