"""SwiGLU kernel vs the CPU oracle (torch-CPU restatement of
baselines/swiglu.py:107-112): bit-exact in every dtype. fp32 follows
torch-CPU's float32 sigmoid as its vectorised loop evaluates it (SLEEF's
expf, oracle/sigmoid.py), so the comparison is bit for bit there too; every
element is also within one storage-type ulp relative (bf16 2^-7, fp16
2^-10, fp32 1e-5) of the oracle. Shapes: the reference's case table
(baselines/swiglu.py:70-88), the vector-tail sizes n = 1..129 its kernel
tests sweep (tests/test_swiglu_kernel.py:74-93), BASELINE config 3 at full size,
and every one of the 65536 bf16 gate values, alone and shuffled among
neighbours from other ranges. (The LDS SiLU table of the FP8 variants is
checked against this kernel's arithmetic SiLU in test_gpu_selftest.py.)
"""

from __future__ import annotations

import pytest
import torch

from custom_cuda_kernals_amd.kernels import swiglu
from oracle import eager, inputs
from tests._parity import assert_ulp_close, assert_within_rel, bits_equal

pytestmark = pytest.mark.gpu

CASES = [(4, 128, 3072), (2, 2048, 11008), (1, 4096, 11008), (3, 17, 11008), (2, 64, 100), (8, 1, 11008),
         (1, 8192, 4096), (0, 128, 11008), (1, 1, 128)]
DTYPES = [torch.float32, torch.float16, torch.bfloat16]


def _run(g, u):
    y = swiglu(g.cuda(), u.cuda())
    y_ref = eager.swiglu(g, u)
    assert y.shape == g.shape and y.dtype == g.dtype
    if g.numel() == 0:
        return None
    stats = assert_ulp_close(y, y_ref, "y")
    print(f"\n{tuple(g.shape)} {g.dtype}: {stats}")
    assert stats["bit_exact_fraction"] == 1.0, stats
    return stats


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c)))
def test_matches_oracle(case, dtype):
    b, s, d = case
    g, u = inputs.swiglu_inputs(b * s, d, dtype, seed=b + s + d)
    _run(g.view(b, s, d), u.view(b, s, d))


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
def test_vector_tail_sizes(dtype):
    for n in range(1, 130):
        g, u = inputs.swiglu_inputs(1, n, dtype, seed=n)
        _run(g.view(-1), u.view(-1))


def test_config3_full_size():
    rows, cols = inputs.CONFIG_SHAPES["swiglu"]
    g, u = inputs.swiglu_inputs(rows, cols, torch.bfloat16, seed=0)
    stats = _run(g, u)
    assert stats["violations"] == 0 and stats["bit_exact_fraction"] == 1.0


def test_extreme_gate_values():
    g = torch.tensor([0.0, -0.0, 1e-30, -1e-30, 30.0, -30.0, 88.0, -88.0, 100.0, -100.0, -1000.0, 1000.0,
                      float("inf"), float("-inf")], dtype=torch.float32)
    u = torch.full_like(g, 1.5)
    y = swiglu(g.cuda(), u.cuda()).cpu()
    y_ref = eager.swiglu(g, u)
    assert torch.equal(torch.isnan(y), torch.isnan(y_ref))
    fin = ~torch.isnan(y_ref)
    assert_within_rel(y[fin], y_ref[fin], 1e-5, "extreme")
    assert bits_equal(y, y_ref).all()


def _every_bf16() -> torch.Tensor:
    import numpy as np

    return torch.from_numpy(np.arange(1 << 16, dtype=np.uint16).view(np.int16)).view(torch.bfloat16)


def test_every_bf16_gate_independent_of_neighbours():
    """All 2^16 gate patterns (zeros, subnormals, inf, NaN included) with up = 1,
    so y is the rounded SiLU itself. In 16 shuffled copies (1M elements) most
    16-byte vectors mix fast-range gates with gates that need the exact path;
    the plain copy keeps neighbouring patterns together. Each element's result
    must not depend on its neighbours (bitwise equal in both), and stays within
    the ulp bound of the oracle."""
    g = _every_bf16()
    gen = torch.Generator().manual_seed(7)
    perm = torch.randperm(16 << 16, generator=gen)
    g_big = g.repeat(16)[perm]
    y_big = swiglu(g_big.cuda(), torch.ones_like(g_big).cuda()).cpu()
    y_small = swiglu(g.cuda(), torch.ones_like(g).cuda()).cpu()
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(perm.numel())
    y_back = y_big[inv].view(16, -1)
    for c in range(16):
        assert bits_equal(y_back[c], y_small).all(), f"copy {c}: results depend on neighbouring gates"
    y_ref = eager.swiglu(g, torch.ones_like(g))
    nan = torch.isnan(y_ref)
    assert torch.equal(torch.isnan(y_small), nan)
    stats = assert_ulp_close(y_small[~nan], y_ref[~nan], "every bf16 gate")
    print(f"\nevery bf16 gate vs oracle: {stats}")


@pytest.mark.parametrize("n", [(1 << 20) + 8 * 13, (1 << 20) + 8 * 2047 + 5, 77 * 14336])
def test_long_stream_ragged_lengths(n):
    """Long streams (>= 1M elements) whose length is not a multiple of the
    8192-element workgroup tile, plus a scalar tail: equal to the oracle like
    every other size."""
    g, u = inputs.swiglu_inputs(1, n, torch.bfloat16, seed=n % 1000)
    stats = _run(g.view(-1), u.view(-1))
    assert stats["bit_exact_fraction"] == 1.0


def test_every_f16_gate_and_strided_f32_gates():
    """All 2^16 fp16 gate patterns and every 4096th fp32 pattern (1 M values
    spanning every exponent, incl. subnormals, inf and NaN), with up = 1 so
    y is the rounded SiLU itself: within the ulp bound of the oracle, NaN
    exactly where the oracle has NaN. fp16 covers the fast-path edge at
    |g| = 87 that bf16 gates (edge 20) do not reach."""
    import numpy as np

    g16 = torch.from_numpy(np.arange(1 << 16, dtype=np.uint16).view(np.int16)).view(torch.float16)
    g32 = torch.from_numpy((np.arange(1 << 20, dtype=np.uint64) * 4096 + 7).astype(np.uint32).view(np.int32)).view(
        torch.float32)
    for g in (g16, g32):
        y = swiglu(g.cuda(), torch.ones_like(g).cuda()).cpu()
        y_ref = eager.swiglu(g, torch.ones_like(g))
        nan = torch.isnan(y_ref)
        assert torch.equal(torch.isnan(y), nan)
        stats = assert_ulp_close(y[~nan], y_ref[~nan], f"every {g.dtype} gate")
        print(f"\n{g.dtype} gates vs oracle: {stats}")
        assert stats["bit_exact_fraction"] == 1.0, stats


def test_fp32_config3_shape_bit_exact():
    """fp32 at config 3's shape [8192, 14336]: every element bit for bit."""
    rows, cols = inputs.CONFIG_SHAPES["swiglu"]
    g, u = inputs.swiglu_inputs(rows, cols, torch.float32, seed=3)
    stats = _run(g, u)
    assert stats["violations"] == 0
