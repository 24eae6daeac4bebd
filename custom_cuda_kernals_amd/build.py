"""Build recipe for the in-tree native artefacts (gfx950 only).

* ``libcustom_kernels_amd.so`` - the HIP kernels behind the C ABI declared in
  ``include/custom_kernels_amd.h`` (hipcc, ``--offload-arch=gfx950``).
* ``_native.<abi>.so`` - the pybind11 validating binding (g++), linked to the
  library above through the C ABI only, found at run time via ``$ORIGIN``.

Both land next to this file so they travel with the source tree. Run as
``python -m custom_cuda_kernals_amd.build``.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
import sysconfig
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libcustom_kernels_amd.so"
HIP_SOURCES = ["fp8_quant.hip", "rmsnorm_residual.hip", "swiglu.hip", "rope.hip", "token_permute.hip", "moe_router.hip",
               "selftest.hip", "calibrate.hip"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Products and sums are rounded separately unless a kernel writes an fma.
    "-ffp-contract=off",
    # Keep hand-written fp32 code scalar (no v_pk_{add,mul,fma}_f32).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Kernel arguments arrive preloaded in SGPRs (a gfx950 dispatch feature)
    # instead of through a scalar load at wave start: measured on MI355X at
    # the config-1 input, the three-launch per-tensor FP8 9.9 vs 10.7 us, the
    # MoE router 4.82 vs 5.0 us, block FP8 6.29 vs 6.35 us; the large-row ops
    # unchanged.
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-Wall",
    "-Wno-unused-function",
    f"-I{ROOT / 'include'}",
]


def native_ext_path() -> Path:
    suffix = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    return PKG / f"_native{suffix}"


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        line for line in proc.stdout.splitlines()
        if "packed-fp32-ops' is not a recognized feature" not in line
    )
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


def build_library() -> Path:
    BUILD.mkdir(exist_ok=True)
    objs = [BUILD / (src.replace(".hip", ".o")) for src in HIP_SOURCES]
    cmds = [
        [HIPCC, *HIP_FLAGS, "-c", str(CSRC / src), "-o", str(obj)]
        for src, obj in zip(HIP_SOURCES, objs)
    ]
    with cf.ThreadPoolExecutor(max_workers=min(len(cmds), os.cpu_count() or 4)) as ex:
        list(ex.map(_run, cmds))
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)])
    os.replace(tmp, LIB)
    return LIB


def _torch_paths() -> tuple[Path, bool]:
    """torch's install directory and whether it was built with the C++11 ABI."""
    import torch

    return Path(torch.__file__).resolve().parent, bool(torch._C._GLIBCXX_USE_CXX11_ABI)


def native_compile_args(sanitize: bool = False) -> list[str]:
    """g++ arguments of the binding: torch's headers (for at::Tensor and c10's
    HIP stream registry; torch's bundled pybind11 comes with them), linked to
    torch's Python, core and HIP libraries and to the kernel library (C ABI
    only). `sanitize` adds AddressSanitizer and UndefinedBehaviorSanitizer
    (host code only; nothing of it is GPU code)."""
    tdir, cxx11 = _torch_paths()
    args = [
        "g++", "-std=c++17", "-shared", "-fPIC", "-Wall",
        "-D__HIP_PLATFORM_AMD__", f"-D_GLIBCXX_USE_CXX11_ABI={int(cxx11)}",
        f"-I{tdir / 'include'}", f"-I{tdir / 'include' / 'torch' / 'csrc' / 'api' / 'include'}",
        "-I/opt/rocm/include",
        f"-I{sysconfig.get_paths()['include']}",
    ]
    args += ["-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
             "-fno-sanitize-recover=undefined"] if sanitize else ["-O2"]
    args += [
        str(CSRC / "native.cpp"),
        f"-L{tdir / 'lib'}", "-ltorch_python", "-ltorch", "-lc10", "-lc10_hip",
        f"-Wl,-rpath,{tdir / 'lib'}",
        f"-L{PKG}", "-lcustom_kernels_amd",
        "-Wl,-rpath,$ORIGIN",
    ]
    return args


def sanitize_requested() -> bool:
    """CCK_SANITIZE=1 builds the binding with AddressSanitizer and
    UndefinedBehaviorSanitizer. Python is not instrumented, so a process that
    imports such a build must preload the runtimes: LD_PRELOAD="$(gcc
    -print-file-name=libasan.so) $(gcc -print-file-name=libstdc++.so.6)" and
    ASAN_OPTIONS=detect_leaks=0 (libstdc++ after libasan, so that the
    sanitizer finds the real exception-throwing routine)."""
    return os.environ.get("CCK_SANITIZE", "") == "1"


def build_native(sanitize: bool | None = None) -> Path:
    out = native_ext_path()
    tmp = out.with_suffix(".tmp")
    _run([*native_compile_args(sanitize_requested() if sanitize is None else sanitize), "-o", str(tmp)])
    os.replace(tmp, out)
    return out


def build_all() -> None:
    build_library()
    build_native()


def is_built() -> bool:
    return LIB.exists() and native_ext_path().exists()


if __name__ == "__main__":
    build_all()
    print(f"built {LIB.name} and {native_ext_path().name}")
