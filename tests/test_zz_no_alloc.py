"""launch_fp8_quant_tensor_noalloc_fwd (no caller scratch, library-owned
device array) against the reference-ABI launch_fp8_quant_tensor_fwd and the
oracle (baselines/fp8_quant.py:162-178 with one scale for the tensor), bit
for bit: codes and scale. Two calls in a row, the second on a smaller input,
so the second call starts from the array as the first left it; plus the
scalar (unaligned) path, both formats and every input dtype.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import fp8 as ofp8
from oracle import inputs
from tests._parity import assert_codes_equal, assert_f32_bits_equal

pytestmark = pytest.mark.gpu

DTAG = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}
FTAG = {"e4m3": 3, "e5m2": 4}


def _lib():
    from tests import _cck

    return _cck.load()


def _noalloc(x_dev: torch.Tensor, q: torch.Tensor, fmt: str) -> torch.Tensor:
    scale = torch.full((1,), float("nan"), dtype=torch.float32, device="cuda")
    m, n = x_dev.shape
    rc = _lib().launch_fp8_quant_tensor_noalloc_fwd(x_dev.data_ptr(), q.data_ptr(), scale.data_ptr(), m, n,
                                                     DTAG[x_dev.dtype], FTAG[fmt],
                                                     torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    return scale


def _reference_abi(x_dev: torch.Tensor, fmt: str):
    q = torch.empty(x_dev.shape, dtype=torch.uint8, device="cuda")
    scale = torch.empty(1, dtype=torch.float32, device="cuda")
    amax = torch.zeros(1, dtype=torch.int32, device="cuda")
    m, n = x_dev.shape
    rc = _lib().launch_fp8_quant_tensor_fwd(x_dev.data_ptr(), q.data_ptr(), scale.data_ptr(), amax.data_ptr(), m, n,
                                            DTAG[x_dev.dtype], FTAG[fmt], torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    return q, scale


def _check_pair(x: torch.Tensor, fmt: str, q: torch.Tensor | None = None) -> None:
    x_dev = x.cuda()
    if q is None:
        q = torch.full(x.shape, 0x55, dtype=torch.uint8, device="cuda")
    scale = _noalloc(x_dev, q, fmt)
    q_ref, s_ref = _reference_abi(x_dev, fmt)
    torch.cuda.synchronize()
    assert torch.equal(q.cpu(), q_ref.cpu()), "codes differ from launch_fp8_quant_tensor_fwd"
    assert_f32_bits_equal(scale, s_ref.cpu().numpy())
    codes, s_oracle = ofp8.quant_tensor(x.float().numpy(), fmt)
    assert_codes_equal(q, codes)
    assert_f32_bits_equal(scale, s_oracle)


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16], ids=lambda d: str(d).split(".")[-1])
def test_two_calls_second_smaller(dtype, fmt):
    big = inputs.fp8_token_input(2048, 4096, dtype, seed=3)
    small = inputs.randn((300, 520), dtype, seed=4) * 0.01  # a much smaller amax than the first call's
    _check_pair(big, fmt)
    _check_pair(small, fmt)


def test_config1_shape_then_tiny():
    _check_pair(inputs.fp8_token_input(*inputs.CONFIG_SHAPES["fp8_token"], torch.bfloat16, seed=0), "e4m3")
    _check_pair(inputs.randn((2, 3), torch.bfloat16, seed=5), "e4m3")


@pytest.mark.parametrize("shape", [(1, 7), (33, 1001), (4096, 4100), (8192, 8192)], ids=lambda s: f"{s[0]}x{s[1]}")
def test_shapes_and_partial_grids(shape):
    """Sizes from below one workgroup to a grid-stride partial pass (more
    vectors than 512 workgroups take in one round)."""
    x = inputs.randn(shape, torch.bfloat16, seed=shape[1])
    x.view(-1)[x.numel() // 3] = -700.0
    _check_pair(x, "e4m3")


def test_unaligned_buffers_take_the_scalar_path():
    m, n = 513, 777
    x = inputs.randn((m, n), torch.bfloat16, seed=9)
    xb = torch.cat([torch.zeros(1, dtype=torch.bfloat16), x.reshape(-1)]).cuda()
    x_dev = xb[1:].view(m, n)
    assert x_dev.data_ptr() % 16 != 0
    buf = torch.full((m * n + 8,), 0x55, dtype=torch.uint8, device="cuda")
    q = buf[3:3 + m * n].view(m, n)
    scale = _noalloc(x_dev, q, "e4m3")
    torch.cuda.synchronize()
    codes, s_oracle = ofp8.quant_tensor(x.float().numpy(), "e4m3")
    assert_codes_equal(q, codes)
    assert_f32_bits_equal(scale, s_oracle)
    b = buf.cpu().numpy()
    assert (b[:3] == 0x55).all() and (b[3 + m * n:] == 0x55).all(), "wrote outside the codes buffer"


def test_back_to_back_without_synchronising():
    """Several calls queued on one stream without host synchronisation (each
    call's last partial workgroup must leave the counter at zero for the
    next), each checked afterwards against the oracle."""
    xs = [inputs.randn((64 * (i + 1), 4096), torch.bfloat16, seed=20 + i) * (i + 1) for i in range(5)]
    outs = []
    for x in xs:
        q = torch.empty(x.shape, dtype=torch.uint8, device="cuda")
        outs.append((q, _noalloc(x.cuda(), q, "e4m3")))
    torch.cuda.synchronize()
    for x, (q, s) in zip(xs, outs):
        codes, s_oracle = ofp8.quant_tensor(x.float().numpy(), "e4m3")
        assert_codes_equal(q, codes)
        assert_f32_bits_equal(s, s_oracle)


def test_rejects_size_beyond_int64_before_device_calls():
    lib = _lib()
    assert lib.launch_fp8_quant_tensor_noalloc_fwd(None, None, None, 1 << 40, 1 << 40, 2, 3, None) == 1
    assert lib.launch_fp8_quant_tensor_noalloc_fwd(None, None, None, 0, 8, 2, 3, None) == 0
    assert lib.launch_fp8_quant_tensor_noalloc_fwd(None, None, None, 4, 8, 9, 3, None) == 1
    assert lib.launch_fp8_quant_tensor_noalloc_fwd(None, None, None, 4, 8, 2, 7, None) == 1
