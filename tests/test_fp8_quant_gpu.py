"""FP8 quantisation kernels vs the CPU oracle: codes and scales bit-exact.

Case matrix follows the reference's (baselines/fp8_quant.py:84-114: standard
and edge shapes x {f32, f16, bf16} x {e4m3, e5m2}), for the reference's two
granularities and the build's per-token and static modes, plus the
BASELINE config-1 workload at full size and the edge inputs the reference
tests (all-zero input, tests/test_fp8_quant_kernel.py:84-89) and those the
domain adds (signed zeros, NaN / inf rows, static-scale overflow, unaligned
pointers, long rows).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from custom_cuda_kernals_amd.kernels import fp8_quant
from oracle import fp8 as ofp8
from oracle import inputs
from tests._parity import assert_codes_equal, assert_f32_bits_equal

pytestmark = pytest.mark.gpu

SHAPES = [(256, 256), (1024, 1024), (4096, 4096), (257, 513), (64, 64), (1, 256), (256, 1), (2048, 128)]
DTYPES = [torch.float32, torch.float16, torch.bfloat16]
FORMATS = ["e4m3", "e5m2"]


def _oracle(x: torch.Tensor, fmt: str, gran: str, scale=None):
    x32 = x.float().numpy()
    if scale is not None:
        return ofp8.quant_static(x32, scale, fmt), np.array([scale], dtype=np.float32)
    return {"token": ofp8.quant_token, "tensor": ofp8.quant_tensor, "block": ofp8.quant_block}[gran](x32, fmt)


def _check(x_cpu: torch.Tensor, fmt: str, gran: str, scale=None, x_dev=None):
    x_dev = x_cpu.cuda() if x_dev is None else x_dev
    q, s = fp8_quant(x_dev, fmt, gran, scale=scale)
    torch.cuda.synchronize()
    codes, s_ref = _oracle(x_cpu, fmt, gran, scale)
    assert q.dtype == ofp8_dtype(fmt) and tuple(q.shape) == tuple(x_cpu.shape)
    assert_codes_equal(q, codes)
    assert_f32_bits_equal(s, s_ref)


def ofp8_dtype(fmt):
    return torch.float8_e4m3fn if fmt == "e4m3" else torch.float8_e5m2


@pytest.mark.parametrize("gran", ["token", "block", "tensor"])
@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: f"{s[0]}x{s[1]}")
def test_dynamic_matches_oracle(shape, dtype, fmt, gran):
    x = inputs.randn(shape, dtype, seed=7 * shape[0] + shape[1] + DTYPES.index(dtype))
    _check(x, fmt, gran)


@pytest.mark.parametrize("scale", [0.05, 0.003, 1e-5])
@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
def test_static_matches_oracle_including_overflow(dtype, fmt, scale):
    x = inputs.randn((257, 1030), dtype, seed=3) * 4
    _check(x.to(dtype), fmt, "tensor", scale=scale)


@pytest.mark.parametrize("fmt", FORMATS)
def test_config1_per_token_full_size(fmt):
    m, n = inputs.CONFIG_SHAPES["fp8_token"]
    x = inputs.fp8_token_input(m, n, seed=0)
    _check(x, fmt, "token")


@pytest.mark.parametrize("gran", ["token", "block", "tensor"])
def test_all_zero_gives_zero_codes_and_min_scale(gran):
    x = torch.zeros(256, 256, dtype=torch.float32)
    q, s = fp8_quant(x.cuda(), "e4m3", gran)
    assert torch.all(q.float() == 0)
    assert torch.all(s == torch.tensor(1e-12, dtype=torch.float32).cuda())
    _check(x, "e4m3", gran)


@pytest.mark.parametrize("gran", ["token", "block", "tensor"])
@pytest.mark.parametrize("fmt", FORMATS)
def test_signed_zeros_nan_inf(gran, fmt):
    x = inputs.randn((130, 264), torch.bfloat16, seed=5)
    x[0, :] = -0.0
    x[1, 3] = float("nan")
    x[2, 7] = float("inf")
    x[3, 9] = float("-inf")
    x[4, 1] = -float("nan")
    x[5, 5:9] = 0.0
    x[5, 6] = -0.0
    x[6, :] = 1e-40  # bf16 subnormals
    if gran == "tensor":
        x[1, 3] = 1.0  # a NaN would make every code NaN; keep the tensor case finite + inf
    _check(x, fmt, gran)


@pytest.mark.parametrize("fmt", FORMATS)
def test_static_nan_inf_and_huge(fmt):
    x = inputs.randn((64, 256), torch.float32, seed=7)
    x[0, 0] = float("nan")
    x[1, 1] = float("inf")
    x[2, 2] = -3.0e38
    x[3, :] = 1e30
    _check(x, fmt, "tensor", scale=0.05)


@pytest.mark.parametrize("gran", ["token", "block", "tensor"])
@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
def test_unaligned_input_pointer(gran, dtype):
    m, n = 33, 264
    base = inputs.randn((m * n + 1,), dtype, seed=9)
    x_cpu = base[1:].view(m, n).clone()
    x_dev = base.cuda()[1:].view(m, n)
    assert x_dev.data_ptr() % 16 != 0
    _check(x_cpu, "e4m3", gran, x_dev=x_dev)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("cols", [64, 512, 1024, 2048, 4096, 8192, 16384, 32768, 65536])
def test_every_row_shape_bucket(cols, dtype):
    _check(inputs.randn((3, cols), dtype, seed=cols), "e4m3", "token")


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
def test_long_rows_use_looping_path(dtype):
    x = inputs.randn((5, 40000), dtype, seed=11)
    _check(x, "e4m3", "token")


def test_rejects_bad_format_and_granularity():
    x = torch.randn(4, 8, device="cuda")
    with pytest.raises(ValueError):
        fp8_quant(x, "e4m4", "block")
    with pytest.raises(ValueError):
        fp8_quant(x, "e4m3", "row")
    with pytest.raises(ValueError):
        fp8_quant(x, "e4m3", "block", scale=0.1)
