"""Device-side checks of the two arithmetic shortcuts of the FP8 fast path,
run through the C ABI diagnostics (csrc/selftest.hip):

* gfx950's v_cvt_pk_fp8_f32 / v_cvt_pk_bf8_f32 against the exact encoder
  (itself pinned to torch's cast and to the oracle in test_oracle_fp8.py) for
  all 2^32 fp32 bit patterns;
* the three-op division against IEEE division for every finite bf16 / fp16 x
  and random fp32 x over a large set of scales (random mantissas, every
  dynamic scale a bf16 amax can produce, and edge scales);
* the dynamic scale clamp(amax / FP8_MAX, 1e-12) computed with the exact
  power-of-two step and the fma-corrected division by 7, against IEEE
  division, for every non-negative fp32 amax (2^31 patterns incl. inf / NaN);
* the bf16 SiLU table of the SwiGLU+FP8 kernels: both fills against the
  arithmetic SiLU entry by entry, and the table lookup against the arithmetic
  path for all 2^16 bf16 gates (the arithmetic path itself is checked against
  the oracle for every bf16 gate in test_swiglu_gpu.py);
* the fp32 SwiGLU's sigmoid as the kernels evaluate it (SLEEF's expf with its
  scaling as one ldexp, and a Newton-refined reciprocal in place of the IEEE
  division below 2^64) against the operation-for-operation form, for all
  2^32 fp32 gates, and the reciprocal against IEEE 1 / d for every float in
  [1, 2^64) (the operation-for-operation form is pinned to torch by
  test_oracle_sigmoid.py and checked on the device against the oracle in
  test_swiglu_gpu.py).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests import _cck

pytestmark = pytest.mark.gpu

FMT_TAG = {"e4m3": 3, "e5m2": 4}
FAST_LIMIT = {"e4m3": 65536.0, "e5m2": 65536.0}  # Fp8<FMT>::kFastLimit


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_hw_fp8_convert_matches_exact_encoder_on_fast_domain(fmt):
    lib = _cck.load()
    counters = torch.zeros(8, dtype=torch.int64, device="cuda")
    counters[4:] = -1
    stream = torch.cuda.current_stream().cuda_stream
    chunk = 1 << 30
    for start in range(0, 1 << 32, chunk):
        assert lib.cck_fp8_cvt_selftest(start, chunk, FMT_TAG[fmt], counters.data_ptr(), stream) == 0
    torch.cuda.synchronize()
    c = counters.cpu().numpy().view(np.uint64)
    print(f"\n[{fmt}] hw-vs-exact mismatches: |v|<={FAST_LIMIT[fmt]}: {c[0]}, above: {c[1]} "
          f"(lowest {hex(int(c[5]))}), inf: {c[2]}, nan: {c[3]} (lowest {hex(int(c[7]))})")
    assert c[0] == 0, f"hardware conversion differs inside the fast domain, first pattern {hex(int(c[4]))}"


def _finite_bf16_values() -> np.ndarray:
    v = (np.arange(1 << 16, dtype=np.uint32) << 16).view(np.float32)
    return v[np.isfinite(v)]


def _finite_f16_values() -> np.ndarray:
    v = np.arange(1 << 16, dtype=np.uint16).view(np.float16).astype(np.float32)
    return v[np.isfinite(v)]


def _random_f32_values(n: int = 1 << 16) -> np.ndarray:
    bits = np.random.default_rng(1).integers(0, 1 << 32, size=n, dtype=np.uint64).astype(np.uint32)
    v = bits.view(np.float32)
    return v[np.isfinite(v)]


def _scales() -> np.ndarray:
    rng = np.random.default_rng(0)
    mant = rng.integers(0, 1 << 23, size=1 << 20, dtype=np.uint32)
    random_scales = ((np.uint32(127) << 23) | mant).view(np.float32)  # [1, 2)
    amax = _finite_bf16_values()
    amax = np.abs(amax[amax > 0])
    dyn = []
    for fmax in (448.0, 57344.0):
        s = amax / np.float32(fmax)
        dyn.append(np.where(s < np.float32(1e-12), np.float32(1e-12), s).astype(np.float32))
    edge = np.array([1e-12, 0.05, 1.0, 3.0, 7.0, 1.1754944e-38, 2.0**-100, 2.0**100, 1e30], dtype=np.float32)
    return np.unique(np.concatenate([random_scales, *dyn, edge]).astype(np.float32))


@pytest.mark.parametrize("xset", ["bf16", "f16", "f32_random"])
def test_fast_division_matches_ieee_division(xset):
    lib = _cck.load()
    xvals = {"bf16": _finite_bf16_values, "f16": _finite_f16_values, "f32_random": _random_f32_values}[xset]()
    xs = torch.from_numpy(xvals).cuda()
    ss = torch.from_numpy(_scales()).cuda()
    counters = torch.zeros(5, dtype=torch.int64, device="cuda")
    counters[3] = -1
    stream = torch.cuda.current_stream().cuda_stream
    assert lib.cck_div_selftest(xs.data_ptr(), xs.numel(), ss.data_ptr(), ss.numel(), counters.data_ptr(), stream) == 0
    torch.cuda.synchronize()
    c = counters.cpu().numpy().view(np.uint64)
    print(f"\npairs checked {c[4]}, fp32 bit mismatches {c[0]}, e4m3 code mismatches {c[1]}, "
          f"e5m2 code mismatches {c[2]}")
    if c[0]:
        i = int(c[3])
        x, s = xs[i % xs.numel()].item(), ss[i // xs.numel()].item()
        print(f"first bitwise mismatch: x={x!r} s={s!r}")
    assert c[4] > 10**9
    assert c[1] == 0 and c[2] == 0


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_dynamic_scale_matches_ieee_division_for_every_amax(fmt):
    lib = _cck.load()
    counters = torch.zeros(2, dtype=torch.int64, device="cuda")
    counters[1] = -1
    stream = torch.cuda.current_stream().cuda_stream
    assert lib.cck_scale_selftest(0, 1 << 31, FMT_TAG[fmt], counters.data_ptr(), stream) == 0
    torch.cuda.synchronize()
    c = counters.cpu().numpy().view(np.uint64)
    assert c[0] == 0, f"{c[0]} scale mismatches, lowest amax bits {hex(int(c[1]))}"


def test_silu_table_equals_arithmetic_silu():
    lib = _cck.load()
    counters = torch.zeros(6, dtype=torch.int64, device="cuda")
    counters[2] = -1
    stream = torch.cuda.current_stream().cuda_stream
    assert lib.cck_silu_table_selftest(counters.data_ptr(), stream) == 0
    torch.cuda.synchronize()
    c = counters.cpu().numpy().view(np.uint64)
    assert c[5] == 2 * 65536
    # Both groupings exercise the table and the fallback: the ascending one
    # has whole vectors in range, the permuted one mixes ranges.
    assert 0 < c[4] < 2 * 65536 // 8
    assert c[0] == 0 and c[1] == 0, f"fill mismatches {c[0]}/{c[1]}, lowest index {int(c[2])}"
    assert c[3] == 0, f"{c[3]} lookups differ from the arithmetic SiLU"


def test_fp32_sigmoid_forms_agree_for_every_gate():
    lib = _cck.load()
    counters = torch.zeros(7, dtype=torch.int64, device="cuda")
    counters[4:] = -1
    stream = torch.cuda.current_stream().cuda_stream
    chunk = 1 << 28
    for start in range(0, 1 << 32, chunk):
        assert lib.cck_sigmoid_selftest(start, chunk, counters.data_ptr(), stream) == 0
    torch.cuda.synchronize()
    c = counters.cpu().numpy().view(np.uint64)
    assert c[3] == 64 << 23, c[3]  # every float in [1, 2^64)
    assert c[0] == 0, f"{c[0]} expf mismatches, lowest pattern {hex(int(c[4]))}"
    assert c[1] == 0, f"{c[1]} sigmoid mismatches, lowest pattern {hex(int(c[5]))}"
    assert c[2] == 0, f"{c[2]} reciprocal mismatches, lowest pattern {hex(int(c[6]))}"

