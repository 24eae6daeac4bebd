"""Environment inspection behind the `doctor` command: the ROCm toolchain,
PyTorch's HIP build, the GPU and its architecture, OCP FP8 support and the
in-tree native library (the reference checks nvcc, CUDA_PATH, the CUDA GPU
and its PyO3 extension instead: custom_cuda/cli/env_checks.py:27-157)."""

from __future__ import annotations

import dataclasses
import os
import re
import shutil
import subprocess
import sys
from pathlib import Path

__all__ = ["Check", "run_checks", "TARGET_ARCH"]

TARGET_ARCH = "gfx950"
PKG = Path(__file__).resolve().parent.parent
LIB = PKG / "libcustom_kernels_amd.so"


@dataclasses.dataclass(frozen=True)
class Check:
    name: str
    status: str  # "ok" | "fail" | "warn"
    detail: str


def _check_python() -> Check:
    v = sys.version_info
    return Check("Python interpreter", "ok", f"{v.major}.{v.minor}.{v.micro} ({sys.executable})")


def _rocm_path() -> str | None:
    for p in (os.environ.get("ROCM_PATH"), "/opt/rocm"):
        if p and os.path.isdir(p):
            return p
    return None


def _check_rocm() -> Check:
    path = _rocm_path()
    if path is None:
        return Check("ROCm install", "fail", "ROCM_PATH unset and /opt/rocm missing")
    version = "unknown"
    vfile = os.path.join(path, ".info", "version")
    if os.path.exists(vfile):
        version = open(vfile).read().strip()
    return Check("ROCm install", "ok", f"{version} ({path})")


def _check_hipcc() -> Check:
    hipcc = os.environ.get("HIPCC") or shutil.which("hipcc")
    path = _rocm_path()
    if hipcc is None and path and os.path.exists(os.path.join(path, "bin", "hipcc")):
        hipcc = os.path.join(path, "bin", "hipcc")
    if hipcc is None:
        return Check("hipcc (HIP compiler)", "fail",
                     "not found: `python -m custom_cuda_kernals_amd.build` cannot compile csrc/*.hip")
    try:
        out = subprocess.run([hipcc, "--version"], capture_output=True, text=True, timeout=30, check=False)
        m = re.search(r"HIP version: (\S+)", out.stdout)
        return Check("hipcc (HIP compiler)", "ok", f"HIP {m.group(1) if m else 'unknown'} ({hipcc})")
    except (OSError, subprocess.SubprocessError) as e:
        return Check("hipcc (HIP compiler)", "warn", f"found at {hipcc} but failed to run: {e}")


def _check_torch() -> Check:
    try:
        import torch
    except ImportError as e:
        return Check("PyTorch", "fail", f"not importable: {e}")
    hip = getattr(torch.version, "hip", None)
    if not hip:
        return Check("PyTorch", "fail", f"{torch.__version__} is not a ROCm build (torch.version.hip is empty)")
    return Check("PyTorch", "ok", f"{torch.__version__} (HIP {hip})")


def _device_props():
    try:
        import torch
    except ImportError:
        return None
    if not torch.cuda.is_available():
        return None
    return torch.cuda.get_device_properties(0)


def _check_gpu() -> Check:
    props = _device_props()
    if props is None:
        return Check("GPU", "fail", "no HIP device visible to PyTorch")
    return Check("GPU", "ok", f"{props.name}, {props.multi_processor_count} CUs, "
                              f"{props.total_memory / 2**30:.0f} GiB")


def _check_arch() -> Check:
    props = _device_props()
    if props is None:
        return Check(f"GPU architecture ({TARGET_ARCH})", "warn", "no GPU: cannot verify")
    arch = getattr(props, "gcnArchName", "").split(":")[0]
    if arch != TARGET_ARCH:
        return Check(f"GPU architecture ({TARGET_ARCH})", "fail",
                     f"GPU is {arch or 'unknown'}; the kernels are built for {TARGET_ARCH} only")
    return Check(f"GPU architecture ({TARGET_ARCH})", "ok", f"{arch} matches the build target")


def _check_fp8() -> Check:
    try:
        import torch
    except ImportError:
        return Check("OCP FP8 (e4m3fn / e5m2)", "fail", "torch not importable")
    if not hasattr(torch, "float8_e4m3fn") or not hasattr(torch, "float8_e5m2"):
        return Check("OCP FP8 (e4m3fn / e5m2)", "fail", "torch lacks float8_e4m3fn / float8_e5m2")
    props = _device_props()
    if props is None:
        return Check("OCP FP8 (e4m3fn / e5m2)", "warn", "torch dtypes present; no GPU to check the conversion")
    arch = getattr(props, "gcnArchName", "").split(":")[0]
    if arch != TARGET_ARCH:
        return Check("OCP FP8 (e4m3fn / e5m2)", "warn",
                     f"{arch}: v_cvt_pk_fp8_f32 there may use the fnuz encodings, not OCP")
    return Check("OCP FP8 (e4m3fn / e5m2)", "ok", "gfx950 v_cvt_pk_fp8_f32 / v_cvt_pk_bf8_f32 produce OCP codes")


def _check_library() -> Check:
    if not LIB.exists():
        return Check("libcustom_kernels_amd.so", "fail", "not built: run `python -m custom_cuda_kernals_amd.build`")
    data = LIB.read_bytes()
    if f"amdgcn-amd-amdhsa--{TARGET_ARCH}".encode() not in data:
        return Check("libcustom_kernels_amd.so", "warn", f"built, but holds no {TARGET_ARCH} code object")
    return Check("libcustom_kernels_amd.so", "ok", f"{LIB} ({len(data) / 2**20:.1f} MiB, {TARGET_ARCH} code object)")


def _check_native() -> Check:
    try:
        import torch  # noqa: F401  (the binding links against torch's HIP runtime)

        from custom_cuda_kernals_amd import _native
    except ImportError as e:
        return Check("custom_cuda_kernals_amd._native", "fail",
                     f"not importable: run `python -m custom_cuda_kernals_amd.build`: {e}")
    required = ["rmsnorm_residual_fwd", "swiglu_fwd", "rope_fwd", "fp8_quant_block_fwd", "fp8_quant_tensor_fwd"]
    missing = [f for f in required if not hasattr(_native, f)]
    if missing:
        return Check("custom_cuda_kernals_amd._native", "warn", f"imported, but missing {missing}: rebuild")
    return Check("custom_cuda_kernals_amd._native", "ok", f"loaded from {_native.__file__}")


def run_checks() -> list[Check]:
    return [_check_python(), _check_rocm(), _check_hipcc(), _check_torch(), _check_gpu(), _check_arch(),
            _check_fp8(), _check_library(), _check_native()]
