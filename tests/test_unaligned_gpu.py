"""Inputs and outputs that do not start on a 16-byte boundary, for the ops
whose per-op tests cover only aligned buffers. The reference accepts them and
handles them with scalar kernels (swiglu.cu:135,155; rope.cu:294-330;
fp8_quant.cu:122,226); here each launcher checks alignment on the host and
takes its scalar kernel, and the result must meet the same bar as the aligned
path: the per-op tests' oracles and tolerances, reused.

A buffer is made unaligned by viewing a larger allocation from element 1
(2 bytes for bf16 / fp16, 4 for fp32, 1 for FP8 codes).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from custom_cuda_kernals_amd import _native as native
from custom_cuda_kernals_amd.kernels import rmsnorm_residual, swiglu
from oracle import eager, inputs, moe
from oracle import fp8 as ofp8
from tests._parity import assert_codes_equal, assert_f32_bits_equal, assert_ulp_close, bits_equal

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.float16, torch.bfloat16]
F8 = {"e4m3": torch.float8_e4m3fn, "e5m2": torch.float8_e5m2}


def _off(t_cpu: torch.Tensor, offset: int = 1) -> torch.Tensor:
    """A device copy of t_cpu that starts `offset` elements into its allocation."""
    flat = torch.empty(t_cpu.numel() + offset, dtype=t_cpu.dtype, device="cuda")
    view = flat[offset:].view(t_cpu.shape)
    view.copy_(t_cpu.cuda())
    assert view.data_ptr() % 16 != 0
    return view


def _empty_off(shape, dtype, offset: int = 1) -> torch.Tensor:
    n = int(np.prod(shape))
    view = torch.empty(n + offset, dtype=dtype, device="cuda")[offset:].view(shape)
    assert view.data_ptr() % 16 != 0
    return view


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("which", ["inputs", "output"])
def test_swiglu_unaligned(dtype, which):
    g, u = inputs.swiglu_inputs(37, 1000, dtype, seed=5)
    if which == "inputs":
        y = swiglu(_off(g), _off(u))
    else:
        y = _empty_off(g.shape, dtype)
        native.swiglu_fwd(g.cuda(), u.cuda(), y)
    assert_ulp_close(y.cpu(), eager.swiglu(g, u), "y")
    assert bits_equal(y.cpu(), swiglu(g.cuda(), u.cuda()).cpu()).all(), "scalar and vector paths differ"


@pytest.mark.parametrize("static", [None, 0.05])
@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
def test_swiglu_fp8_unaligned(dtype, static):
    g, u = inputs.swiglu_inputs(19, 1024, dtype, seed=6)
    q = _empty_off(g.shape, F8["e4m3"])
    s = torch.empty(g.shape[0] if static is None else 1, dtype=torch.float32, device="cuda")
    native.swiglu_fp8_fwd(_off(g), _off(u), q, s if static is None else None, "e4m3", static)
    y_k = swiglu(g.cuda(), u.cuda()).float().cpu().numpy()
    if static is None:
        codes, s_ref = ofp8.quant_token(y_k, "e4m3")
        assert_f32_bits_equal(s, s_ref)
    else:
        codes = ofp8.quant_static(y_k, static, "e4m3")
    assert_codes_equal(q, codes)


@pytest.mark.parametrize("static", [None, 0.05])
@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
def test_rmsnorm_fp8_unaligned(dtype, static):
    x, r, w = inputs.rmsnorm_inputs(23, 2048, dtype, seed=7)
    q = _empty_off(x.shape, F8["e5m2"])
    ro = _empty_off(x.shape, dtype)
    s = torch.empty(x.shape[0], dtype=torch.float32, device="cuda") if static is None else None
    native.rmsnorm_residual_fp8_fwd(_off(x), _off(r), w.cuda(), q, s, ro, 1e-5, "e5m2", static)
    y_k, ro_k = rmsnorm_residual(x.cuda(), r.cuda(), w.cuda(), 1e-5)
    assert bits_equal(ro.cpu(), ro_k.cpu()).all()
    y32 = y_k.float().cpu().numpy()
    if static is None:
        codes, s_ref = ofp8.quant_token(y32, "e5m2")
        assert_f32_bits_equal(s, s_ref)
    else:
        codes = ofp8.quant_static(y32, static, "e5m2")
    assert_codes_equal(q, codes)


@pytest.mark.parametrize("inplace", [False, True])
@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
def test_rope_unaligned(dtype, inplace):
    q, k, cos, sin = inputs.rope_inputs(2, 33, 4, 2, 64, dtype=dtype, seed=8, theta=10000.0)
    qd, kd = _off(q), _off(k)
    if inplace:
        native.rope_fwd(qd, kd, cos.cuda(), sin.cuda(), qd, kd)
        qo, ko = qd, kd
    else:
        qo, ko = _empty_off(q.shape, dtype), _empty_off(k.shape, dtype)
        native.rope_fwd(qd, kd, cos.cuda(), sin.cuda(), qo, ko)
    q_ref, k_ref = eager.rope(q, k, cos, sin)
    assert bits_equal(qo.cpu(), q_ref).all() and bits_equal(ko.cpu(), k_ref).all()


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
def test_token_gather_combine_unaligned(dtype):
    src, idx = inputs.gather_inputs(40, 70, 264, dtype, seed=9)
    dst = _empty_off((70, 264), dtype)
    native.token_gather_fwd(_off(src), idx.cuda(), dst)
    assert bits_equal(dst.cpu(), moe.token_gather(src, idx)).all()
    eo, ui, w = inputs.combine_inputs(30, 3, 264, dtype, seed=10)
    out = _empty_off((30, 264), dtype)
    native.token_combine_fwd(_off(eo), ui.cuda(), w.cuda(), out)
    assert bits_equal(out.cpu(), moe.token_combine_aten(eo, ui, w)).all()


@pytest.mark.parametrize("cols", [64, 1000, 2048, 4096, 11008])
@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
def test_rmsnorm_scalar_path_equals_vector_path(dtype, cols):
    """The scalar kernel sums the squares in the register-resident kernels'
    canonical order, so an unaligned pointer changes no output bit."""
    if cols % (4 if dtype == torch.float32 else 8):
        pytest.skip("no vector path for this row length")
    x, r, w = inputs.rmsnorm_inputs(5, cols, dtype, seed=cols)
    y_a, ro_a = rmsnorm_residual(x.cuda(), r.cuda(), w.cuda(), 1e-6)
    y_u, ro_u = rmsnorm_residual(_off(x), _off(r), w.cuda(), 1e-6)
    assert bits_equal(ro_u.cpu(), ro_a.cpu()).all()
    assert bits_equal(y_u.cpu(), y_a.cpu()).all(), "scalar and vector RMSNorm paths differ"
