"""The FP8 activation format contract (custom_cuda_kernals_amd.fp8_format) on
CPU tensors: scale layouts (the reference's [ceil(M/128), ceil(N/128)] and [1],
custom_cuda/kernels/fp8_quant.py:53-63, plus per-token [M]), validation
errors, the torch._scaled_mm scale views, and dequantisation against its closed
form (every code decoded by the oracle's exact decoder times the broadcast scale)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from custom_cuda_kernals_amd import fp8_format as ff
from oracle import fp8 as ofp8


@pytest.mark.parametrize("m,n", [(1, 1), (128, 128), (129, 257), (2048, 4096), (5, 11008)])
def test_scale_shapes(m, n):
    assert ff.scale_shape("token", m, n) == (m,)
    assert ff.scale_shape("tensor", m, n) == (1,)
    assert ff.scale_shape("block", m, n) == (-(-m // 128), -(-n // 128))
    with pytest.raises(ValueError):
        ff.scale_shape("row", m, n)


def _codes(m, n, dtype=torch.float8_e4m3fn, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, 256, (m, n), generator=g, dtype=torch.uint8).view(dtype)


def test_check_pair_errors():
    c = _codes(4, 8)
    ff.check_pair(c, torch.ones(4), "token")
    ff.check_pair(c, torch.ones(1), "tensor")
    ff.check_pair(c, torch.ones(1, 1), "block")
    with pytest.raises(ValueError, match="2-D"):
        ff.check_pair(c.view(-1), torch.ones(4), "token")
    with pytest.raises(ValueError, match="float8"):
        ff.check_pair(c.view(torch.uint8), torch.ones(4), "token")
    with pytest.raises(ValueError, match="contiguous"):
        ff.check_pair(_codes(8, 4).t(), torch.ones(4), "token")
    with pytest.raises(ValueError, match="float32"):
        ff.check_pair(c, torch.ones(4, dtype=torch.float64), "token")
    with pytest.raises(ValueError, match=r"shape \(4,\)"):
        ff.check_pair(c, torch.ones(1), "token")
    with pytest.raises(ValueError, match=r"shape \(1, 1\)"):
        ff.check_pair(c, torch.ones(4), "block")


def test_scaled_mm_views():
    s = torch.arange(6, dtype=torch.float32)
    assert ff.scaled_mm_scale(s, "token", "a").shape == (6, 1)
    assert ff.scaled_mm_scale(s, "token", "b").shape == (1, 6)
    assert ff.scaled_mm_scale(torch.ones(1), "tensor", "a").shape == ()
    assert ff.scaled_mm_scale(s, "token", "a").data_ptr() == s.data_ptr()  # a view, no copy
    with pytest.raises(ValueError, match="128x128"):
        ff.scaled_mm_scale(torch.ones(1, 1), "block", "a")
    with pytest.raises(ValueError):
        ff.scaled_mm_scale(s, "token", "c")


def test_fp8_linear_rejects_before_the_gemm():
    x, w = _codes(4, 8), _codes(6, 8)
    with pytest.raises(ValueError, match="no torch._scaled_mm mode"):
        ff.fp8_linear(x, torch.ones(4), "token", w, torch.ones(1), "tensor")
    with pytest.raises(ValueError, match="no torch._scaled_mm mode"):
        ff.fp8_linear(x, torch.ones(1, 1), "block", w, torch.ones(1, 1), "block")
    with pytest.raises(ValueError, match="e4m3fn"):
        ff.fp8_linear(_codes(4, 8, torch.float8_e5m2), torch.ones(4), "token", w, torch.ones(6), "token")
    with pytest.raises(ValueError, match="inner dimensions"):
        ff.fp8_linear(x, torch.ones(1), "tensor", _codes(6, 9), torch.ones(1), "tensor")


@pytest.mark.parametrize("fmt,dtype", [("e4m3", torch.float8_e4m3fn), ("e5m2", torch.float8_e5m2)])
@pytest.mark.parametrize("gran", ["token", "tensor", "block"])
def test_dequantize_closed_form(fmt, dtype, gran):
    m, n = 300, 260  # ragged tiles in both dimensions
    c = _codes(m, n, dtype, seed=3)
    g = torch.Generator().manual_seed(4)
    scale = (torch.rand(ff.scale_shape(gran, m, n), generator=g) * 3 + 1e-3).float()
    out = ff.dequantize(c, scale, gran).numpy()
    vals = ofp8.decode(c.view(torch.uint8).numpy(), fmt).astype(np.float32)
    s = scale.numpy()
    if gran == "token":
        sb = np.broadcast_to(s[:, None], (m, n))
    elif gran == "tensor":
        sb = np.full((m, n), s[0], dtype=np.float32)
    else:
        sb = s[np.arange(m)[:, None] // 128, np.arange(n)[None, :] // 128]
    want = vals * sb
    assert np.array_equal(np.isnan(out), np.isnan(want))
    fin = ~np.isnan(want)
    assert np.array_equal(out[fin].view(np.uint32), want[fin].view(np.uint32))
