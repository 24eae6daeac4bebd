"""The developer CLI's GPU commands: `compare` times the kernel against the
reference's eager formula, `benchmark` runs bench.py for an op, `profile`
captures a rocprofv3 kernel trace of one."""

from __future__ import annotations

import pytest
from typer.testing import CliRunner

from custom_cuda_kernals_amd.cli import app as cli_app
from custom_cuda_kernals_amd.cli import runners
from custom_cuda_kernals_amd.cli.registry import REGISTRY

pytestmark = pytest.mark.gpu
runner = CliRunner()


@pytest.mark.parametrize("op_id", ["rmsnorm_residual", "swiglu", "fp8_quant"])
def test_compare_times_kernel_and_eager(op_id):
    """`compare` times both sides; the speed-up is reported, not asserted (a
    timing inside the correctness suite would flake on a loaded box)."""
    r = runners.time_pair(REGISTRY[op_id].build_target("cuda"), iters=5, warmup=2)
    print(f"\n{op_id}: {r}")
    assert r["kernel_us"] > 0 and r["eager_us"] > 0 and r["speedup"] > 0


def test_benchmark_and_profile_commands(tmp_path, monkeypatch):
    monkeypatch.setattr(runners, "RESULTS", tmp_path)
    r = runner.invoke(cli_app.app, ["benchmark", "moe_router", "--steps", "5", "--rerun"])
    assert r.exit_code == 0, r.output
    assert (tmp_path / "bench_moe_router.json").exists()
    r = runner.invoke(cli_app.app, ["profile", "moe_router", "--warmup", "2", "--iters", "3", "-o",
                                    str(tmp_path / "prof"), "--timeout", "100"])
    assert r.exit_code == 0, r.output
    assert "moe_router" in r.output
    assert list((tmp_path / "prof").rglob("*.pftrace")), "no Perfetto trace written"
