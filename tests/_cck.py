"""ctypes view of the C ABI in include/custom_kernels_amd.h, for tests that
exercise the boundary directly. torch is imported first so that the library
binds to torch's HIP runtime."""

from __future__ import annotations

import ctypes
import os
import re

import torch  # noqa: F401  (load order, see module docstring)

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "custom_kernels_amd.h")
LIB_PATH = os.path.join(ROOT, "custom_cuda_kernals_amd", "libcustom_kernels_amd.so")

_CTYPES = {
    "const void*": ctypes.c_void_p,
    "void*": ctypes.c_void_p,
    "uint8_t*": ctypes.c_void_p,
    "float*": ctypes.c_void_p,
    "const float*": ctypes.c_void_p,
    "const int64_t*": ctypes.c_void_p,
    "int64_t*": ctypes.c_void_p,
    "int32_t*": ctypes.c_void_p,
    "unsigned long long*": ctypes.c_void_p,
    "int64_t": ctypes.c_int64,
    "uint64_t": ctypes.c_uint64,
    "int32_t": ctypes.c_int32,
    "float": ctypes.c_float,
}


def declared_functions() -> dict[str, list[str]]:
    """{name: [param C types]} for every function declared in the header."""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"int32_t\s+(\w+)\s*\(([^)]*)\);", text):
        params = []
        for p in m.group(2).split(","):
            p = " ".join(p.split())
            name_split = re.match(r"(.*?)(\w+)$", p)
            params.append(name_split.group(1).replace(" *", "*").strip())
        out[m.group(1)] = params
    return out


def load():
    lib = ctypes.CDLL(LIB_PATH)
    for name, params in declared_functions().items():
        fn = getattr(lib, name)
        fn.restype = ctypes.c_int32
        fn.argtypes = [_CTYPES[p] for p in params]
    return lib
