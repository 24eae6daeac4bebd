"""Pins oracle.fp8 (CPU, no GPU needed).

* encode vs torch's own cast (the reference oracle's dependency) over every
  bf16- and fp16-representable value, a strided and a random fp32 sample and
  the neighbourhoods of every format boundary; all 2^32 patterns when
  CCK_SLOW_TESTS=1;
* the quantisation functions vs the reference's eager formula evaluated with
  torch (baselines/fp8_quant.py:162-189, restated here with torch ops) on
  ragged shapes, including NaN / inf / signed-zero inputs;
* the reference's invariant tests (tests/test_fp8_quant.py:56-94): all-zero
  input gives zero codes and a positive finite scale; the dequantised
  round-trip error is bounded by half a format ulp of the scaled value;
* closed forms: scale = amax / FP8_MAX exactly, clamped at float32(1e-12).
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from oracle import fp8

TORCH_DT = {"e4m3": torch.float8_e4m3fn, "e5m2": torch.float8_e5m2}
FMTS = ["e4m3", "e5m2"]


def _torch_codes(v: np.ndarray, fmt: str) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(v, dtype=np.float32)).to(TORCH_DT[fmt]).view(torch.uint8).numpy()


def _check(v: np.ndarray, fmt: str):
    ours, ref = fp8.encode(v, fmt), _torch_codes(v, fmt)
    bad = np.nonzero(ours != ref)[0]
    assert len(bad) == 0, f"{len(bad)} mismatches, first value {v[bad[0]]!r} (bits {v.view(np.uint32)[bad[0]]:#x})"


@pytest.mark.parametrize("fmt", FMTS)
def test_encode_matches_torch_on_all_bf16_and_f16_values(fmt):
    _check((np.arange(1 << 16, dtype=np.uint32) << 16).view(np.float32), fmt)
    _check(np.arange(1 << 16, dtype=np.uint16).view(np.float16).astype(np.float32), fmt)


@pytest.mark.parametrize("fmt", FMTS)
def test_encode_matches_torch_on_fp32_samples(fmt):
    strided = np.arange(0, 1 << 32, 1021, dtype=np.uint64).astype(np.uint32).view(np.float32)
    rnd = np.random.default_rng(0).integers(0, 1 << 32, 1 << 22, dtype=np.uint64).astype(np.uint32).view(np.float32)
    # +-64 ulps around every value of the format and every midpoint between them
    codes = np.arange(256, dtype=np.uint8)
    vals = fp8.decode(codes, fmt)
    vals = vals[np.isfinite(vals)].astype(np.float64)
    mids = (np.sort(vals)[1:] + np.sort(vals)[:-1]) / 2
    centres = np.concatenate([vals, mids, [464.0, 480.0, 57344.0, 61440.0, 65536.0, 2.0**-9, 2.0**-16]]).astype(np.float32)
    offs = np.arange(-64, 65, dtype=np.int64)
    near = (centres.view(np.uint32).astype(np.int64)[:, None] + offs[None, :]).clip(0, (1 << 32) - 1)
    near = near.astype(np.uint32).view(np.float32).ravel()
    for v in (strided, rnd, near, -near):
        _check(v, fmt)


@pytest.mark.skipif(os.environ.get("CCK_SLOW_TESTS") != "1", reason="all 2^32 patterns: set CCK_SLOW_TESTS=1")
@pytest.mark.parametrize("fmt", FMTS)
def test_encode_matches_torch_exhaustively(fmt):
    step = 1 << 26
    for start in range(0, 1 << 32, step):
        _check(np.arange(start, start + step, dtype=np.uint64).astype(np.uint32).view(np.float32), fmt)


@pytest.mark.parametrize("fmt", FMTS)
def test_decode_matches_torch(fmt):
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(TORCH_DT[fmt]).float().numpy()
    np.testing.assert_array_equal(fp8.decode(codes, fmt), ref)


# --- the reference formula with torch ----------------------------------------

def _torch_eager(x32: torch.Tensor, fmt: str, gran: str):
    fmax = torch.finfo(TORCH_DT[fmt]).max
    if gran == "token":
        scale = torch.clamp(x32.abs().amax(dim=-1) / fmax, min=1e-12)
        return (x32 / scale[:, None]).to(TORCH_DT[fmt]), scale
    if gran == "tensor":
        scale = torch.clamp(x32.abs().max() / fmax, min=1e-12)
        return (x32 / scale).to(TORCH_DT[fmt]), scale.reshape(1)
    m, n = x32.shape
    pm, pn = -(-m // 128) * 128, -(-n // 128) * 128
    padded = torch.nn.functional.pad(x32.abs(), (0, pn - n, 0, pm - m))
    amax = padded.view(pm // 128, 128, pn // 128, 128).amax(dim=(1, 3))
    scale = torch.clamp(amax / fmax, min=1e-12)
    expanded = scale.repeat_interleave(128, 0).repeat_interleave(128, 1)[:m, :n]
    return (x32 / expanded).to(TORCH_DT[fmt]), scale


def _inputs():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(131, 259, generator=g)
    x.view(-1)[torch.randperm(x.numel(), generator=g)[:40]] *= 50
    yield "randn", x
    z = x.clone()
    z[0] = -0.0
    z[1, :5] = 0.0
    z[2, 3] = float("inf")
    z[3, 4] = float("-inf")
    z[4, 9] = float("nan")
    z[5, :] = 1e-40
    yield "specials", z
    yield "zeros", torch.zeros(130, 129)


@pytest.mark.parametrize("gran", ["token", "tensor", "block"])
@pytest.mark.parametrize("fmt", FMTS)
def test_quant_matches_torch_formula(fmt, gran):
    f = {"token": fp8.quant_token, "tensor": fp8.quant_tensor, "block": fp8.quant_block}[gran]
    for name, x in _inputs():
        codes, scale = f(x.numpy(), fmt)
        t_codes, t_scale = _torch_eager(x, fmt, gran)
        np.testing.assert_array_equal(codes, t_codes.view(torch.uint8).numpy(), err_msg=name)
        np.testing.assert_array_equal(scale.view(np.uint32) | 0, t_scale.numpy().view(np.uint32) | 0, err_msg=name) \
            if not np.isnan(scale).any() else np.testing.assert_array_equal(np.isnan(scale), np.isnan(t_scale.numpy()))


@pytest.mark.parametrize("fmt", FMTS)
def test_static_matches_torch_formula(fmt):
    for _, x in _inputs():
        for s in (0.05, 0.003, 1e-5):
            ref = (x / s).to(TORCH_DT[fmt]).view(torch.uint8).numpy()
            np.testing.assert_array_equal(fp8.quant_static(x.numpy(), s, fmt), ref)


@pytest.mark.parametrize("gran", ["token", "tensor", "block"])
def test_zero_input_gives_zero_codes_and_min_scale(gran):
    f = {"token": fp8.quant_token, "tensor": fp8.quant_tensor, "block": fp8.quant_block}[gran]
    codes, scale = f(np.zeros((256, 256), np.float32), "e4m3")
    assert (codes == 0).all()
    assert np.all(scale == np.float32(1e-12)) and np.isfinite(scale).all() and (scale > 0).all()


@pytest.mark.parametrize("fmt", FMTS)
def test_roundtrip_error_bounded_by_half_ulp_of_scaled_value(fmt):
    eps = float(torch.finfo(TORCH_DT[fmt]).eps)
    tiny = float(torch.finfo(TORCH_DT[fmt]).smallest_normal) * eps
    x = np.random.default_rng(5).standard_normal((64, 512)).astype(np.float32)
    codes, scale = fp8.quant_token(x, fmt)
    scaled = x / scale[:, None]
    deq = fp8.decode(codes, fmt)
    assert np.all(np.abs(deq - scaled) <= 0.5 * eps * np.abs(scaled) + tiny)


def test_scale_closed_form():
    amax = np.array([0.0, 1e-20, 4.48e-10, 4.4800004e-10, 1.0, 448.0, 3.0e38, np.inf, np.nan], dtype=np.float32)
    x = np.zeros((len(amax), 2), np.float32)
    x[:, 0] = amax
    _, s = fp8.quant_token(x, "e4m3")
    expect = np.maximum(amax.astype(np.float64) / 448.0, 0).astype(np.float32)
    expect = np.where(expect < np.float32(1e-12), np.float32(1e-12), expect)
    np.testing.assert_array_equal(s[:-1], expect[:-1])
    assert np.isnan(s[-1])


def test_block_scales_keep_a_small_tile_resolved_next_to_an_outlier_tile():
    """The reason for 128x128 scales (the reference checks the same property,
    tests/test_fp8_quant.py:95-123): with one tile ~1e4 times larger than
    another, one tensor-wide scale leaves the small tile only the subnormal
    codes near zero (a fixed step of 2^-9 times the scale), while its own
    tile scale resolves it to e4m3's relative precision. Measured as the mean
    absolute error of the dequantised small tile: about 3x smaller with block
    scales here (asserted with a 2x margin), and within e4m3's relative step."""
    rng = np.random.default_rng(11)
    x = np.zeros((256, 256), dtype=np.float32)
    x[:128, :128] = (rng.standard_normal((128, 128)) * 0.01).astype(np.float32)
    x[128:, 128:] = (rng.standard_normal((128, 128)) * 100.0).astype(np.float32)
    small = x[:128, :128].astype(np.float64)
    codes_t, s_t = fp8.quant_tensor(x, "e4m3")
    codes_b, s_b = fp8.quant_block(x, "e4m3")
    deq_t = fp8.decode(codes_t, "e4m3").astype(np.float64) * s_t[0]
    deq_b = fp8.decode(codes_b, "e4m3").astype(np.float64) * np.repeat(np.repeat(s_b, 128, 0), 128, 1)
    err_t = np.abs(deq_t[:128, :128] - small).mean()
    err_b = np.abs(deq_b[:128, :128] - small).mean()
    assert err_b * 2 < err_t, (err_b, err_t)
    assert err_b < 0.04 * np.abs(small).mean()  # within e4m3's relative step


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_torch_per_token_restatement_equals_exact_encoder(fmt):
    """oracle.eager.fp8_quant_token_torch (torch's own cast, timed by the CPU
    baseline) gives the same codes and scales as oracle.fp8.quant_token, on
    rows with outliers, a zero row and signed zeros."""
    from oracle import eager, inputs

    x = inputs.fp8_token_input(64, 4096, torch.bfloat16, seed=2)
    x[3] = 0.0
    x[5, ::2] = -0.0
    codes_t, scale_t = eager.fp8_quant_token_torch(x, fmt)
    codes, scale = fp8.quant_token(x.float().numpy(), fmt)
    np.testing.assert_array_equal(codes_t.numpy(), codes)
    np.testing.assert_array_equal(scale_t.numpy().view(np.uint32), scale.view(np.uint32))
