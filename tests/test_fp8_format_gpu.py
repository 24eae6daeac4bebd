"""FP8 activations from the HIP kernels consumed the documented ways
(custom_cuda_kernals_amd.fp8_format): dequantisation of every granularity
equals the dequantised oracle codes bit for bit, and torch._scaled_mm with the
documented scale views (tensor-wise; row-wise x per-output-channel) equals the
fp32 product of the dequantised operands within the bf16 output rounding."""

from __future__ import annotations

import pytest
import torch

from custom_cuda_kernals_amd import fp8_format as ff
from custom_cuda_kernals_amd.kernels import fp8_quant, rmsnorm_residual_fp8, swiglu_fp8
from oracle import inputs

pytestmark = pytest.mark.gpu


def _gen(m, n, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(m, n, generator=g).to(torch.bfloat16)


@pytest.mark.parametrize("gran,static", [("token", None), ("tensor", None), ("block", None), ("tensor", 0.05)])
@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_dequantize_matches_oracle_codes(gran, static, fmt):
    from oracle import fp8 as ofp8

    x = _gen(300, 520, seed=1)
    codes, scale = fp8_quant(x.cuda(), fmt, gran, scale=static)
    ff.check_pair(codes, scale, gran)
    x2 = x.float().numpy()
    if static is not None:
        ref_codes, ref_scale = ofp8.quant_static(x2, static, fmt), torch.tensor([static], dtype=torch.float32)
    elif gran == "token":
        c, s = ofp8.quant_token(x2, fmt)
        ref_codes, ref_scale = c, torch.from_numpy(s)
    elif gran == "tensor":
        c, s = ofp8.quant_tensor(x2, fmt)
        ref_codes, ref_scale = c, torch.from_numpy(s).reshape(1)
    else:
        c, s = ofp8.quant_block(x2, fmt)
        ref_codes, ref_scale = c, torch.from_numpy(s)
    ref = ff.dequantize(torch.from_numpy(ref_codes).view(codes.dtype), ref_scale.float(), gran)
    got = ff.dequantize(codes, scale, gran).cpu()
    assert torch.equal(got.view(torch.int32), ref.view(torch.int32))
    # Round trip: |deq - x| <= half a code step (2^-4 e4m3, 2^-3 e5m2 relative) + subnormal step.
    rel = 2.0 ** -4 if fmt == "e4m3" else 2.0 ** -3
    tiny = (2.0 ** -9 if fmt == "e4m3" else 2.0 ** -16)
    s_b = ff.dequantize(torch.ones_like(codes.cpu(), dtype=torch.float32).to(codes.dtype), scale.cpu(), gran)
    fin = torch.isfinite(got)
    err = (got - x.float()).abs()
    assert bool((err[fin] <= rel * (1 + 2.0 ** -20) * x.float().abs()[fin] + tiny * s_b[fin]).all())


def _ref_mm(xq, xs, xg, wq, ws, wg):
    return ff.dequantize(xq, xs, xg).double() @ ff.dequantize(wq, ws, wg).double().t()


def _assert_gemm_close(y, ref):
    y = y.double()
    assert torch.isfinite(y).all()
    # bf16 output: at most one rounding (2^-8 relative) on top of fp32 accumulation.
    err = (y - ref).abs()
    assert bool((err <= 2.0 ** -8 * ref.abs() + 1e-3 * ref.abs().max()).all()), float(err.max())


@pytest.mark.parametrize("m,k,n", [(256, 4096, 512), (100, 1024, 384)])
def test_rowwise_gemm_consumes_token_scales(m, k, n):
    x, w = _gen(m, k, 2).cuda(), (_gen(n, k, 3) * 0.02).cuda()
    xq, xs = fp8_quant(x, "e4m3", "token")
    wq, ws = fp8_quant(w, "e4m3", "token")  # a weight row is an output channel
    y = ff.fp8_linear(xq, xs, "token", wq, ws, "token")
    assert y.shape == (m, n) and y.dtype == torch.bfloat16
    _assert_gemm_close(y, _ref_mm(xq, xs, "token", wq, ws, "token"))


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_tensorwise_gemm_consumes_tensor_and_static_scales(fmt):
    x, w = _gen(128, 2048, 4).cuda(), (_gen(256, 2048, 5) * 0.02).cuda()
    wq, ws = fp8_quant(w, "e4m3", "tensor")
    for xq, xs in (fp8_quant(x, fmt, "tensor"), fp8_quant(x, fmt, "tensor", scale=0.05)):
        y = ff.fp8_linear(xq, xs, "tensor", wq, ws, "tensor")
        _assert_gemm_close(y, _ref_mm(xq, xs, "tensor", wq, ws, "tensor"))


def test_fused_outputs_feed_the_gemm():
    """The fused RMSNorm+FP8 and SwiGLU+FP8 outputs are FP8 activations of the
    'token' layout and feed the row-wise GEMM directly (the Llama-block wiring)."""
    x, r, wn = inputs.rmsnorm_inputs(64, 4096, torch.bfloat16, seed=6)
    hq, hs, _ = rmsnorm_residual_fp8(x.cuda(), r.cuda(), wn.cuda(), 1e-5)
    ff.check_pair(hq, hs, "token")
    g, u = inputs.swiglu_inputs(64, 14336, torch.bfloat16, seed=7)
    mq, ms = swiglu_fp8(g.cuda(), u.cuda(), "e4m3")
    ff.check_pair(mq, ms, "token")
    wq, ws = fp8_quant((_gen(512, 14336, 8) * 0.02).cuda(), "e4m3", "token")
    _assert_gemm_close(ff.fp8_linear(mq, ms, "token", wq, ws, "token"), _ref_mm(mq, ms, "token", wq, ws, "token"))
