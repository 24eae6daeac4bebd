"""Pins oracle.eager (CPU, no GPU needed).

* golden vectors written from the reference's own eager baselines
  (tests/golden/make_golden.py) - bit-exact, which pins the op order and the
  rounding points of every restated function;
* the fp64 ground truths within the reference's own tolerances
  (tests/test_rmsnorm_residual.py, test_swiglu.py, test_rope.py: bf16 1e-2,
  fp16 1e-2/1e-3, fp32 1e-4) on the reference's case shapes;
* invariants: residual_out is the once-rounded sum; RoPE preserves each
  rotated pair's norm (tests/test_rope.py:69-78) and is the identity at
  position 0; a dropped bf16 rounding point is detected by the goldens.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from oracle import eager, fp8
from oracle import inputs as oinputs

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "reference_eager.npz")
DT = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}


@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN, allow_pickle=False)


def _t(a: np.ndarray, dt: torch.dtype) -> torch.Tensor:
    if dt in (torch.bfloat16, torch.float16):
        return torch.from_numpy(a.view(np.int16).copy()).view(dt)
    return torch.from_numpy(a.view(np.int32).copy()).view(torch.float32)


def _bits(t: torch.Tensor) -> np.ndarray:
    return (t.contiguous().view(torch.int16) if t.element_size() == 2 else t.contiguous().view(torch.int32)).numpy()


@pytest.mark.parametrize("tag", list(DT))
def test_rmsnorm_matches_golden(golden, tag):
    for cols in (256, 100):
        k = f"rms_{tag}_{cols}"
        x, r, w = (_t(golden[f"{k}_{n}"], DT[tag]) for n in ("x", "r", "w"))
        y, ro = eager.rmsnorm_residual(x, r, w, 1e-5)
        np.testing.assert_array_equal(_bits(y), golden[f"{k}_y"].view(_bits(y).dtype))
        np.testing.assert_array_equal(_bits(ro), golden[f"{k}_ro"].view(_bits(ro).dtype))


@pytest.mark.parametrize("tag", list(DT))
def test_swiglu_matches_golden(golden, tag):
    g, u = (_t(golden[f"swiglu_{tag}_{n}"], DT[tag]) for n in ("gate", "up"))
    y = eager.swiglu(g, u)
    want = golden[f"swiglu_{tag}_y"].view(_bits(y).dtype)
    if tag != "f32":
        np.testing.assert_array_equal(_bits(y), want)
        return
    # The golden fp32 output was written by the reference's eager code on an
    # AVX-512 host, one thread: the first 1184 of its 1200 elements took
    # torch's vector path, the last 1200 mod 32 = 16 its scalar tail (libm
    # expf). The oracle states the vector path for every element.
    from oracle import sigmoid as osig

    body = g.numel() - g.numel() % 32
    np.testing.assert_array_equal(_bits(y).reshape(-1)[:body], want.reshape(-1)[:body])
    g32 = g.numpy().reshape(-1)
    tail = (g32[body:] * osig.sigmoid_scalar(g32[body:])).astype(np.float32) * u.numpy().reshape(-1)[body:]
    np.testing.assert_array_equal(tail.astype(np.float32).view(np.int32), want.reshape(-1)[body:])


def test_cos_sin_tables_match_golden(golden):
    cos, sin = eager.compute_cos_sin(16, 64, 500000.0)
    np.testing.assert_array_equal(_bits(cos), golden["rope_cos_16x64_t5e5"].view(np.int32))
    np.testing.assert_array_equal(_bits(sin), golden["rope_sin_16x64_t5e5"].view(np.int32))


@pytest.mark.parametrize("tag", list(DT))
def test_rope_matches_golden(golden, tag):
    cos, sin = eager.compute_cos_sin(16, 64, 500000.0)
    q, k = (_t(golden[f"rope_{tag}_{n}"], DT[tag]) for n in ("q", "k"))
    qo, ko = eager.rope(q, k, cos, sin)
    np.testing.assert_array_equal(_bits(qo), golden[f"rope_{tag}_qo"].view(_bits(qo).dtype))
    np.testing.assert_array_equal(_bits(ko), golden[f"rope_{tag}_ko"].view(_bits(ko).dtype))


@pytest.mark.parametrize("tag", list(DT))
def test_fp8_quant_matches_golden(golden, tag):
    x = _t(golden[f"fp8_{tag}_x"], DT[tag]).float().numpy()
    for fmt in ("e4m3", "e5m2"):
        for gran, f in (("tensor", fp8.quant_tensor), ("block", fp8.quant_block)):
            codes, scale = f(x, fmt)
            np.testing.assert_array_equal(codes, golden[f"fp8_{tag}_{fmt}_{gran}_codes"])
            np.testing.assert_array_equal(scale.reshape(-1).view(np.uint32), golden[f"fp8_{tag}_{fmt}_{gran}_scale"])


def test_golden_detects_a_dropped_rounding_point(golden):
    """A restatement that skips eager's bf16 rounding of `normed` before
    `* weight` must fail the golden comparison."""
    k = "rms_bf16_256"
    x, r, w = (_t(golden[f"{k}_{n}"], torch.bfloat16) for n in ("x", "r", "w"))
    ro = x + r
    r32 = ro.float()
    normed = r32 * torch.rsqrt(r32.pow(2).mean(-1, keepdim=True) + 1e-5)
    wrong = (normed * w.float()).to(torch.bfloat16)
    assert not np.array_equal(_bits(wrong), golden[f"{k}_y"].view(np.int16))


TOL = {torch.float32: (1e-4, 1e-4), torch.float16: (1e-2, 1e-3), torch.bfloat16: (1e-2, 1e-2)}


@pytest.mark.parametrize("dtype", list(TOL), ids=str)
@pytest.mark.parametrize("shape", [(4, 128, 768), (3, 17, 4096), (2, 64, 100), (1, 1, 128)])
def test_rmsnorm_close_to_fp64(shape, dtype):
    x, r, w = oinputs.rmsnorm_inputs(shape[0] * shape[1], shape[2], dtype, seed=1)
    y, ro = eager.rmsnorm_residual(x, r, w, 1e-6)
    y64, ro64 = eager.rmsnorm_residual_fp64(x, r, w, 1e-6)
    rtol, atol = TOL[dtype]
    torch.testing.assert_close(y.double(), y64, rtol=rtol, atol=atol)
    torch.testing.assert_close(ro.double(), ro64, rtol=rtol, atol=atol)
    assert torch.equal(ro, (x.float() + r.float()).to(dtype))  # one rounding of the sum


@pytest.mark.parametrize("dtype", list(TOL), ids=str)
def test_swiglu_close_to_fp64(dtype):
    g, u = oinputs.swiglu_inputs(64, 3072, dtype, seed=2)
    rtol, atol = TOL[dtype]
    torch.testing.assert_close(eager.swiglu(g, u).double(), eager.swiglu_fp64(g, u), rtol=rtol, atol=atol)


@pytest.mark.parametrize("dtype", list(TOL), ids=str)
def test_rope_close_to_fp64_and_norm_preserving(dtype):
    q, k, cos, sin = oinputs.rope_inputs(2, 64, 8, 2, 128, dtype, seed=3)
    qo, ko = eager.rope(q, k, cos, sin)
    q64, k64 = eager.rope_fp64(q, k, cos, sin)
    rtol, atol = TOL[dtype]
    torch.testing.assert_close(qo.double(), q64, rtol=rtol, atol=atol)
    torch.testing.assert_close(ko.double(), k64, rtol=rtol, atol=atol)

    def pair_norm(t):
        t = t.double()
        return t[..., :64] ** 2 + t[..., 64:] ** 2

    torch.testing.assert_close(pair_norm(q64), pair_norm(q), rtol=1e-6, atol=1e-6)  # cos^2+sin^2 = 1 to fp32 precision
    assert torch.equal(qo[:, 0], q[:, 0]) and torch.equal(ko[:, 0], k[:, 0])  # position 0: cos 1, sin 0


def test_fused_compositions_are_quantised_eager_outputs():
    x, r, w = oinputs.rmsnorm_inputs(8, 512, torch.bfloat16, seed=4)
    codes, scale, ro, y = eager.rmsnorm_residual_fp8(x, r, w, 1e-5)
    c2, s2 = fp8.quant_token(y.float().numpy(), "e4m3")
    np.testing.assert_array_equal(codes, c2)
    np.testing.assert_array_equal(scale, s2)
    g, u = oinputs.swiglu_inputs(8, 512, torch.bfloat16, seed=5)
    codes, scale, y = eager.swiglu_fp8(g, u, "e5m2", 0.05)
    np.testing.assert_array_equal(codes, fp8.quant_static(y.float().numpy(), 0.05, "e5m2"))
    assert scale is None


def test_config_generators_are_seeded_and_shaped():
    a = oinputs.fp8_token_input(64, 128, seed=7)
    b = oinputs.fp8_token_input(64, 128, seed=7)
    assert torch.equal(a, b) and a.dtype == torch.bfloat16 and a.shape == (64, 128)
    assert int((a.float().abs() > 8).sum()) >= 1  # outliers present
    assert oinputs.digest(a) == oinputs.digest(b)
