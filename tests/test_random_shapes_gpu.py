"""Seeded random shapes for every op, against the same oracles and bars as the
per-op tests (whose checking helpers are reused here).

The fixed case tables pin the reference's shapes; these cases probe the
launchers' shape selection instead: row lengths on and around every
register-resident bucket boundary (BUCKET_VECS vectors, +-1, +-8 elements),
lengths that are not a multiple of the 16-byte vector, single rows and
columns, and mixed dtypes / FP8 formats. Sizes stay small enough for the CPU
oracle to finish in a second or two per case.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import inputs
from tests.test_fp8_quant_gpu import _check as check_fp8
from tests.test_fused_fp8_gpu import _check_rms, _check_swiglu
from tests.test_moe_router_gpu import _check as check_router
from tests.test_rmsnorm_residual_gpu import _run as run_rmsnorm
from tests.test_rope_gpu import _run as run_rope
from tests.test_swiglu_gpu import _run as run_swiglu
from tests.test_token_permute_gpu import _check_combine

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.float16, torch.bfloat16]
# Row capacities (in 16-byte vectors) of the register-resident shapes of the
# row kernels (threads x vectors per thread).
BUCKET_VECS = [64, 128, 192, 256, 320, 384, 448, 512, 768, 896, 1024, 1152, 1536, 2048, 3072, 4096, 8192, 16384]
N_CASES = 16
MAX_ELEMS = 1 << 21


def _cols(rng: np.random.Generator, vec: int) -> int:
    kind = rng.integers(4)
    if kind == 0:
        return int(rng.integers(1, 20001))
    if kind == 1:
        return int(vec * rng.integers(1, 2501))
    if kind == 2:  # around a row-shape bucket boundary
        base = vec * int(rng.choice(BUCKET_VECS))
        return max(1, base + int(rng.choice([-8, -1, 0, 1, 8])))
    return int(rng.integers(1, 65))


def _rows(rng: np.random.Generator, cols: int) -> int:
    cap = max(1, min(300, MAX_ELEMS // max(1, cols)))
    return int(rng.integers(1, cap + 1))


def _cases(name: str, seed: int):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(N_CASES):
        dtype = DTYPES[int(rng.integers(3))]
        vec = 4 if dtype == torch.float32 else 8
        cols = _cols(rng, vec)
        rows = _rows(rng, cols)
        fmt = ["e4m3", "e5m2"][int(rng.integers(2))]
        out.append(pytest.param(rows, cols, dtype, fmt, int(rng.integers(1 << 30)),
                                id=f"{name}{i}-{rows}x{cols}-{str(dtype).split('.')[-1]}-{fmt}"))
    return out


@pytest.mark.parametrize("rows,cols,dtype,fmt,seed", _cases("rms", 1))
def test_rmsnorm_random(rows, cols, dtype, fmt, seed):
    x, r, w = inputs.rmsnorm_inputs(rows, cols, dtype, seed=seed)
    run_rmsnorm(x, r, w, 1e-6)


@pytest.mark.parametrize("static", [None, 0.05])
@pytest.mark.parametrize("rows,cols,dtype,fmt,seed", _cases("rmsfp8", 2))
def test_rmsnorm_fp8_random(rows, cols, dtype, fmt, seed, static):
    x, r, w = inputs.rmsnorm_inputs(rows, cols, dtype, seed=seed)
    _check_rms(x, r, w, 1e-5, fmt, static)


@pytest.mark.parametrize("rows,cols,dtype,fmt,seed", _cases("swiglu", 3))
def test_swiglu_random(rows, cols, dtype, fmt, seed):
    g, u = inputs.swiglu_inputs(rows, cols, dtype, seed=seed)
    run_swiglu(g, u)


@pytest.mark.parametrize("static", [None, 0.05])
@pytest.mark.parametrize("rows,cols,dtype,fmt,seed", _cases("swifp8", 4))
def test_swiglu_fp8_random(rows, cols, dtype, fmt, seed, static):
    g, u = inputs.swiglu_inputs(rows, cols, dtype, seed=seed)
    _check_swiglu(g, u, fmt, static)


@pytest.mark.parametrize("gran", ["token", "block", "tensor", "static"])
@pytest.mark.parametrize("rows,cols,dtype,fmt,seed", _cases("fp8", 5))
def test_fp8_quant_random(rows, cols, dtype, fmt, seed, gran):
    x = inputs.randn((rows, cols), dtype, seed=seed)
    if gran == "static":
        check_fp8(x, fmt, "tensor", scale=0.05)
    else:
        check_fp8(x, fmt, gran)


def _rope_cases(seed: int):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(N_CASES):
        dtype = DTYPES[int(rng.integers(3))]
        d = 2 * int(rng.choice([1, 2, 3, 4, 5, 7, 8, 16, 24, 32, 48, 64, 128, 256]))
        hq = int(rng.integers(1, 41))
        hkv = int(rng.integers(1, hq + 1))
        b = int(rng.integers(1, 4))
        s = max(1, min(int(rng.integers(1, 300)), MAX_ELEMS // (b * (hq + hkv) * d)))
        inplace = bool(rng.integers(2))
        out.append(pytest.param((b, s, hq, hkv, d), dtype, inplace, int(rng.integers(1 << 30)),
                                id=f"rope{i}-{b}x{s}x{hq}x{hkv}x{d}-{str(dtype).split('.')[-1]}-{'ip' if inplace else 'oop'}"))
    return out


@pytest.mark.parametrize("case,dtype,inplace,seed", _rope_cases(6))
def test_rope_random(case, dtype, inplace, seed):
    run_rope(case, dtype, 10000.0, inplace, seed=seed)


@pytest.mark.parametrize("rows,cols,dtype,fmt,seed", _cases("combine", 7))
def test_gather_combine_random(rows, cols, dtype, fmt, seed):
    from custom_cuda_kernals_amd.kernels import token_gather
    from oracle import moe
    from tests._parity import bits_equal

    n_dst = int(np.random.default_rng(seed).integers(1, 2 * rows + 2))
    src, idx = inputs.gather_inputs(rows, n_dst, cols, dtype, seed=seed)
    out = token_gather(src.cuda(), idx.cuda()).cpu()
    assert bits_equal(out, moe.token_gather(src, idx)).all()
    k = int(np.random.default_rng(seed + 1).integers(1, 9))
    eo, ui, w = inputs.combine_inputs(rows, k, cols, dtype, seed=seed)
    _check_combine(eo, ui, w)


def _router_cases(seed: int):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(N_CASES):
        dtype = DTYPES[int(rng.integers(3))]
        e = int(rng.integers(1, 257))
        k = int(rng.integers(1, e + 1)) if rng.integers(2) else int(rng.integers(1, min(e, 8) + 1))
        t = int(rng.integers(1, 600))
        out.append(pytest.param(t, e, k, bool(rng.integers(2)), dtype, int(rng.integers(1 << 30)),
                                id=f"router{i}-{t}x{e}-k{k}-{str(dtype).split('.')[-1]}"))
    return out


@pytest.mark.parametrize("t,e,k,renorm,dtype,seed", _router_cases(8))
def test_router_random(t, e, k, renorm, dtype, seed):
    check_router(inputs.router_inputs(t, e, dtype, seed=seed), k, renorm)
