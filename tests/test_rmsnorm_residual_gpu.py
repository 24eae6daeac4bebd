"""Fused residual + RMSNorm kernel vs the CPU oracle (torch-CPU restatement of
baselines/rmsnorm_residual.py:123-136).

* residual_out: bit-exact (one rounding of x + residual);
* y: bit-exact in every dtype. The kernel sums the squares in torch-CPU's
  fp32 order (oracle/rowsum.py states it; tests/test_oracle_rowsum.py pins
  it against torch), so the variance, rsqrt and every rounding point match.
  The one-ulp bound (bf16 2^-7, fp16 2^-10, fp32 1e-5) is also checked.
  Torch may split the sum of a single row of 32768 or more elements across
  threads, in an order that depends on the host's thread count; for those
  rows the oracle runs on one thread, the serial order the kernel follows.
Shapes: the reference's standard + edge cases (baselines/rmsnorm_residual.py:75-91),
row lengths that reach every part of the summation order (8-lane vector
tail, leftover vectors, trailing steps, acc2 / acc3 levels, the 32-step
blocks of rows above 2^24 elements) on the register-resident and the
looping kernels, and the BASELINE config-2 workload at full size.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from custom_cuda_kernals_amd.kernels import rmsnorm_residual
from oracle import eager, inputs
from tests._parity import assert_ulp_close, assert_within_rel, bits_equal

pytestmark = pytest.mark.gpu

CASES = [(4, 128, 768), (2, 2048, 4096), (1, 4096, 4096), (3, 17, 4096), (2, 64, 100), (8, 1, 4096),
         (1, 8192, 2048), (0, 128, 4096), (1, 1, 128)]
DTYPES = [torch.float32, torch.float16, torch.bfloat16]


def _run(x, r, w, eps, x_dev=None, r_dev=None):
    y, ro = rmsnorm_residual(x.cuda() if x_dev is None else x_dev, r.cuda() if r_dev is None else r_dev,
                             w.cuda(), eps)
    y_ref, ro_ref = eager.rmsnorm_residual(x, r, w, eps)
    assert y.shape == x.shape and ro.shape == x.shape and y.dtype == x.dtype and ro.dtype == x.dtype
    if x.numel() == 0:
        return None
    assert bits_equal(ro, ro_ref).all(), "residual_out must be bit-exact"
    stats = assert_ulp_close(y, y_ref, "y")
    print(f"\n{tuple(x.shape)} {x.dtype}: {stats}")
    same = bits_equal(y, y_ref)
    if not same.all():
        first = np.argwhere(~same.reshape(same.shape[0], -1) if same.ndim > 1 else ~same)[0].tolist()
        raise AssertionError(f"y: {int((~same).sum())} of {same.size} elements differ from the eager "
                             f"oracle; first at {first}")
    return stats


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c)))
def test_matches_oracle(case, dtype):
    b, s, h = case
    x, r, w = inputs.rmsnorm_inputs(b * s, h, dtype, seed=b + s + h)
    _run(x.view(b, s, h), r.view(b, s, h), w, 1e-6)


def test_config2_full_size():
    rows, cols = inputs.CONFIG_SHAPES["rmsnorm"]
    x, r, w = inputs.rmsnorm_inputs(rows, cols, torch.bfloat16, seed=0)
    stats = _run(x, r, w, inputs.RMS_EPS)
    assert stats["violations"] == 0 and stats["bit_exact_fraction"] == 1.0


# Row lengths around each part of the summation order: < 8 (scalar slots),
# 8-lane vector tails (cols % 8), leftover vectors (nv % 4), trailing steps,
# exact 16-step blocks, 16 blocks (acc2), 256 blocks (acc3).
ORDER_COLS = [1, 3, 4, 5, 7, 8, 12, 16, 24, 40, 100, 256, 264, 516, 520, 1000, 2056, 4104, 8192, 8200,
              11008, 16392, 20000, 40000, 131072, 139272]


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("cols", ORDER_COLS)
def test_summation_order_lengths(cols, dtype):
    rows = 3 if cols < 100000 else 2
    x, r, w = inputs.rmsnorm_inputs(rows, cols, dtype, seed=cols + 7)
    _run(x * 4, r, w, 1e-5)


def test_summation_order_32_step_blocks():
    """Rows above 2^24 elements switch torch's blocks to 32 steps (the looping
    kernel follows)."""
    cols = (1 << 24) + 8 * 4 * 40 + 8 * 3 + 5
    x, r, w = inputs.rmsnorm_inputs(2, cols, torch.bfloat16, seed=5)
    _run(x, r, w, 1e-5)


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
def test_unaligned_and_long_rows(dtype):
    rows, cols = 6, 40000
    x, r, w = inputs.rmsnorm_inputs(rows, cols, dtype, seed=1)
    _run(x, r, w, 1e-5)
    # unaligned base pointers take the scalar path
    xb = torch.cat([torch.zeros(1, dtype=dtype), x[:3, :1000].reshape(-1)])
    rb = torch.cat([torch.zeros(1, dtype=dtype), r[:3, :1000].reshape(-1)])
    xd, rd = xb.cuda()[1:].view(3, 1000), rb.cuda()[1:].view(3, 1000)
    assert xd.data_ptr() % 16 != 0
    _run(x[:3, :1000].contiguous(), r[:3, :1000].contiguous(), w[:1000].contiguous(), 1e-5, xd, rd)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16], ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("cols", [64, 512, 1024, 2048, 2056, 2560, 3072, 3584, 4096, 5120, 6144, 6152, 8192, 10240,
                                  12288, 16384, 32768])
def test_every_row_shape_bucket(cols, dtype):
    x, r, w = inputs.rmsnorm_inputs(5, cols, dtype, seed=cols)
    _run(x, r, w, 1e-5)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("cols", [32768, 65536, (1 << 20) + 13])
def test_single_long_row_against_one_thread_torch(cols, dtype):
    x, r, w = inputs.rmsnorm_inputs(1, cols, dtype, seed=cols + 3)
    prev = torch.get_num_threads()
    torch.set_num_threads(1)
    try:
        _run(x, r, w, 1e-5)
    finally:
        torch.set_num_threads(prev)


def test_rejections():
    x = torch.randn(2, 4, 8, device="cuda")
    with pytest.raises(ValueError):
        rmsnorm_residual(x, torch.randn(2, 4, 8, device="cuda", dtype=torch.float16), torch.randn(8, device="cuda"))
    with pytest.raises(ValueError):
        rmsnorm_residual(x, torch.randn(2, 4, 16, device="cuda")[..., ::2], torch.randn(8, device="cuda"))
    with pytest.raises(ValueError):
        rmsnorm_residual(x, x, torch.randn(9, device="cuda"))
