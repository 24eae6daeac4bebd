"""Process and measurement plumbing for the `verify`, `benchmark`,
`compare`, `visualize` and `profile` commands (the reference keeps the
same split, custom_cuda/cli/runners.py:60-157): pytest and bench.py run as
subprocesses, profiles come from rocprofv3's kernel trace (in place of
torch.profiler), and `compare` times the library's kernel against the
reference's eager formula with HIP events."""

from __future__ import annotations

import csv
import dataclasses
import json
import os
import re
import shutil
import subprocess
import sys
import time
from pathlib import Path

REPO_ROOT = Path(__file__).resolve().parent.parent.parent
RESULTS = REPO_ROOT / "cli_results"

__all__ = ["REPO_ROOT", "RESULTS", "PytestSummary", "run_pytest", "run_bench", "load_bench", "time_pair",
           "ProfileResult", "run_profile"]


@dataclasses.dataclass(frozen=True)
class PytestSummary:
    passed: int
    failed: int
    skipped: int
    errors: int
    duration_s: float
    returncode: int
    stdout: str

    @property
    def ok(self) -> bool:
        return self.returncode == 0


_TOKEN = re.compile(r"(\d+) (passed|failed|skipped|deselected|error|errors)")
_DURATION = re.compile(r"in ([\d.]+)s")


def run_pytest(files: list[str], marker: str, timeout: int) -> PytestSummary:
    existing = [f for f in files if (REPO_ROOT / f).exists()]
    cmd = [sys.executable, "-m", "pytest", *existing, "-q", "-m", marker, "-p", "no:cacheprovider"]
    t0 = time.monotonic()
    proc = subprocess.run(cmd, cwd=REPO_ROOT, capture_output=True, text=True, timeout=timeout)
    tail = "\n".join(proc.stdout.strip().splitlines()[-5:])
    counts = {"passed": 0, "failed": 0, "skipped": 0, "errors": 0}
    for n, label in _TOKEN.findall(tail):
        key = {"error": "errors", "deselected": "skipped"}.get(label, label)
        counts[key] += int(n)
    m = _DURATION.search(tail)
    return PytestSummary(counts["passed"], counts["failed"], counts["skipped"], counts["errors"],
                         float(m.group(1)) if m else time.monotonic() - t0, proc.returncode, proc.stdout)


def _bench_path(op_id: str) -> Path:
    return RESULTS / f"bench_{op_id}.json"


def run_bench(op_id: str, bench_ops: tuple[str, ...], steps: int, timeout: int) -> dict:
    """bench.py over the op's benchmark entries; the JSON line is kept under cli_results/."""
    cmd = [sys.executable, "bench.py", "--ops", ",".join(bench_ops), "--steps", str(steps),
           "--no-cpu-baseline", "--no-ceilings"]
    proc = subprocess.run(cmd, cwd=REPO_ROOT, capture_output=True, text=True, timeout=timeout)
    lines = [ln for ln in proc.stdout.splitlines() if ln.startswith("{")]
    if proc.returncode != 0 or not lines:
        raise RuntimeError(f"bench.py failed (exit {proc.returncode}):\n{proc.stderr[-3000:]}")
    line = json.loads(lines[-1])
    RESULTS.mkdir(exist_ok=True)
    _bench_path(op_id).write_text(json.dumps(line))
    return line


def load_bench(op_id: str) -> dict | None:
    p = _bench_path(op_id)
    return json.loads(p.read_text()) if p.exists() else None


def time_pair(target, iters: int = 20, warmup: int = 5) -> dict:
    """Median HIP-event time of the kernel call and of the eager formula on
    the same device tensors (each call timed on its own)."""
    import torch

    def med(fn):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        ts = []
        for _ in range(iters):
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record()
            fn()
            e.record()
            torch.cuda.synchronize()
            ts.append(s.elapsed_time(e) * 1000.0)
        ts.sort()
        return ts[len(ts) // 2]

    k_us, e_us = med(target.kernel), med(target.eager)
    return {"kernel_us": k_us, "eager_us": e_us, "speedup": e_us / k_us,
            "kernel_GB_per_s": target.nbytes / k_us / 1e3}


@dataclasses.dataclass(frozen=True)
class ProfileResult:
    out_dir: Path
    top: list[dict]
    trace: Path | None  # Perfetto trace (ui.perfetto.dev), when rocprofv3 wrote one


def run_profile(op_id: str, iters: int, out_dir: Path, timeout: int, warmup: int = 2) -> ProfileResult:
    """rocprofv3 kernel trace of `warmup` + `iters` calls of the op's
    representative target (the program itself follows `--`, with no launcher
    in between): per-kernel statistics as CSV and the timeline as a Perfetto
    trace, where the reference writes a torch.profiler Chrome trace."""
    rocprof = shutil.which("rocprofv3") or "/opt/rocm/bin/rocprofv3"
    if not os.path.exists(rocprof):
        raise RuntimeError("rocprofv3 not found (ROCm's profiler is needed for `profile`)")
    out_dir.mkdir(parents=True, exist_ok=True)
    cmd = [rocprof, "--kernel-trace", "--stats", "--output-format", "csv", "pftrace", "-d", str(out_dir), "-o", "run",
           "--", sys.executable, "-m", "custom_cuda_kernals_amd.cli.profile_target", op_id, str(iters), str(warmup)]
    proc = subprocess.run(cmd, cwd=REPO_ROOT, capture_output=True, text=True, timeout=timeout)
    stats = sorted(out_dir.rglob("*kernel_stats.csv"))
    if not stats:
        raise RuntimeError(f"rocprofv3 produced no kernel statistics (exit {proc.returncode}):\n"
                           f"{proc.stderr[-3000:]}")
    rows = list(csv.DictReader(open(stats[-1])))
    top = sorted(rows, key=lambda r: -float(r.get("TotalDurationNs", 0)))[:15]
    traces = sorted(out_dir.rglob("*.pftrace"))
    return ProfileResult(out_dir, top, traces[-1] if traces else None)
