"""The validating binding (csrc/native.cpp) built with AddressSanitizer and
UndefinedBehaviorSanitizer (CCK_SANITIZE=1's build), running the binding's
CPU tests: every validation branch with attribute-only fakes (the Python
attribute path) and with real CPU tensors (the at::Tensor path), the empty
and rejected launches, and the header checks. The build goes into a copy of
the package in a temporary directory, so the in-tree binding is untouched;
the tests run in a child process that preloads the sanitizer runtimes.
Any report fails the run (halt_on_error)."""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

from custom_cuda_kernals_amd import build

ROOT = Path(__file__).resolve().parent.parent


def _runtime(name: str) -> str:
    return subprocess.run(["gcc", f"-print-file-name={name}"], capture_output=True, text=True,
                          check=True).stdout.strip()


def test_binding_tests_pass_under_asan_and_ubsan(tmp_path):
    for d in ("custom_cuda_kernals_amd", "include", "oracle", "tests"):
        shutil.copytree(ROOT / d, tmp_path / d,
                        ignore=shutil.ignore_patterns("__pycache__", "_build", "_native*.so", "*.tmp"))
    pkg = tmp_path / "custom_cuda_kernals_amd"
    out = pkg / build.native_ext_path().name
    subprocess.run([*build.native_compile_args(sanitize=True), "-o", str(out)], check=True, capture_output=True,
                   text=True)
    env = dict(os.environ,
               LD_PRELOAD=f"{_runtime('libasan.so')} {_runtime('libstdc++.so.6')}",
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    r = subprocess.run([sys.executable, "-m", "pytest", "tests/test_abi_cpu.py", "-q", "-s", "-p", "no:cacheprovider",
                        "-m", "not gpu"], cwd=tmp_path, env=env, capture_output=True, text=True, timeout=900)
    assert r.returncode == 0, r.stdout[-4000:] + r.stderr[-4000:]
    assert " passed" in r.stdout and "AddressSanitizer" not in r.stderr and "runtime error" not in r.stderr
