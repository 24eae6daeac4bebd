"""torch-CPU restatements of the reference's eager baselines, same op order and
rounding points, for the floating-point ops of the path.

* ``rmsnorm_residual``  <- baselines/rmsnorm_residual.py:123-136
* ``swiglu``            <- baselines/swiglu.py:107-112
* ``compute_cos_sin``   <- baselines/rope.py:103-115
* ``rope``              <- baselines/rope.py:129-145 (half-split)
* ``*_fp64``            <- the fp64 ``reference_fp64`` ground truths
                           (rmsnorm_residual.py:156-169, swiglu.py:127-132,
                           rope.py:161-176)
* fused compositions: the build's RMSNorm+FP8 / SwiGLU+FP8 are the eager op
  followed by the per-row quantisation of ``oracle.fp8`` on the op's output as
  stored in its dtype.

The arithmetic is torch's own CPU kernels (the reference oracle's
dependency), so it reproduces torch-CPU reduction order, rsqrt and sigmoid by
construction. Pinned by (tests/test_oracle_eager.py): the fp64 closed forms
within the reference's tolerances, the golden vectors under tests/golden/
written from the reference's own baselines, and invariants (RoPE preserves
each pair's norm, residual_out is the once-rounded sum, position 0 is the
identity rotation).
"""

from __future__ import annotations

import numpy as np
import torch

from oracle import fp8 as _fp8


def rmsnorm_residual(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float):
    dt = x.dtype
    residual_out = x + residual                       # rounded to dt
    r32 = residual_out.to(torch.float32)
    variance = r32.pow(2).mean(dim=-1, keepdim=True)  # fp32
    normed = r32 * torch.rsqrt(variance + eps)
    return normed.to(dt) * weight, residual_out        # normed rounded to dt, then * weight in dt


def sigmoid_f32_vectorised(g32: torch.Tensor) -> torch.Tensor:
    """torch.sigmoid of a float32 tensor as torch's vectorised loop evaluates
    it, for every element (oracle/sigmoid.py): torch itself on one thread
    over a body that is a whole number of double vectors (so no element falls
    into the loop's scalar tail), the restated vector path for the rest.
    Multi-threaded torch would evaluate up to 2W - 1 elements at the end of
    each thread's chunk with libm's expf instead."""
    from oracle import sigmoid as osig

    flat = g32.reshape(-1).contiguous()
    n = flat.numel()
    body = n - n % 64
    out = torch.empty_like(flat)
    if body:
        prev = torch.get_num_threads()
        torch.set_num_threads(1)
        try:
            out[:body] = torch.sigmoid(flat[:body])
        finally:
            torch.set_num_threads(prev)
    if body < n:
        out[body:] = torch.from_numpy(osig.sigmoid_vector(flat[body:].numpy()))
    return out.view(g32.shape)


def swiglu(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    g32 = gate.to(torch.float32)
    # fp32 keeps every bit of the sigmoid, so its evaluation path is pinned
    # (sigmoid_f32_vectorised); the narrower types round it away.
    sig = sigmoid_f32_vectorised(g32) if gate.dtype == torch.float32 else torch.sigmoid(g32)
    act = g32 * sig
    return act.to(gate.dtype) * up


def compute_cos_sin(seq_len: int, head_dim: int, theta: float = 10000.0):
    exponents = torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim
    inv_freq = 1.0 / (theta ** exponents)
    pos = torch.arange(seq_len, dtype=torch.float32)
    angles = torch.outer(pos, inv_freq)
    return angles.cos().contiguous(), angles.sin().contiguous()


def _rotate(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    x32 = x.to(torch.float32)
    half = x32.shape[-1] // 2
    a, b = x32[..., :half], x32[..., half:]
    c = cos[None, :, None, :]
    s = sin[None, :, None, :]
    return torch.cat([a * c - b * s, b * c + a * s], dim=-1).to(x.dtype)


def rope(q, k, cos, sin):
    return _rotate(q, cos, sin), _rotate(k, cos, sin)


# --- fp64 ground truths -------------------------------------------------------

def rmsnorm_residual_fp64(x, residual, weight, eps):
    r64 = x.double() + residual.double()
    inv = torch.rsqrt(r64.pow(2).mean(dim=-1, keepdim=True) + eps)
    return r64 * inv * weight.double(), r64


def swiglu_fp64(gate, up):
    g = gate.double()
    return g * torch.sigmoid(g) * up.double()


def rope_fp64(q, k, cos, sin):
    def rot(x):
        x64 = x.double()
        half = x64.shape[-1] // 2
        a, b = x64[..., :half], x64[..., half:]
        c = cos.double()[None, :, None, :]
        s = sin.double()[None, :, None, :]
        return torch.cat([a * c - b * s, b * c + a * s], dim=-1)

    return rot(q), rot(k)


# --- per-token FP8 with torch's own CPU cast ----------------------------------

_FP8_TORCH = {"e4m3": torch.float8_e4m3fn, "e5m2": torch.float8_e5m2}


def fp8_quant_token_torch(x: torch.Tensor, fmt: str = "e4m3"):
    """eager_fp8_quant's "tensor" formula (baselines/fp8_quant.py:162-178)
    applied per row of a [M, N] tensor with torch's CPU ops: amax, clamp(amax /
    FP8_MAX, min=1e-12), (x.float() / scale).to(fp8). Returns (codes as uint8
    [M, N], scale [M]). The CPU baseline times this (torch's cast, as the
    reference's eager path runs); oracle.fp8.quant_token is the exact-encoder
    restatement it is pinned against (tests/test_oracle_fp8.py)."""
    dt = _FP8_TORCH[fmt]
    x32 = x.to(torch.float32)
    amax = x32.abs().amax(dim=-1, keepdim=True)
    scale = torch.clamp(amax / torch.finfo(dt).max, min=1e-12)
    return (x32 / scale).to(dt).view(torch.uint8), scale.reshape(-1)


# --- fused compositions -------------------------------------------------------

def to_f32_numpy(t: torch.Tensor) -> np.ndarray:
    return t.to(torch.float32).numpy()


def rmsnorm_residual_fp8(x, residual, weight, eps, fmt="e4m3", static_scale=None):
    """(codes [rows, cols], scale [rows] or None, residual_out, y) with y the
    eager RMSNorm output in x's dtype."""
    y, residual_out = rmsnorm_residual(x, residual, weight, eps)
    y2 = to_f32_numpy(y).reshape(-1, y.shape[-1])
    if static_scale is None:
        codes, scale = _fp8.quant_token(y2, fmt)
    else:
        codes, scale = _fp8.quant_static(y2, static_scale, fmt), None
    return codes.reshape(y.shape), scale, residual_out, y


def swiglu_fp8(gate, up, fmt="e4m3", static_scale=None):
    """(codes, scale [rows] or None, y) with y the eager SwiGLU output."""
    y = swiglu(gate, up)
    y2 = to_f32_numpy(y).reshape(-1, y.shape[-1])
    if static_scale is None:
        codes, scale = _fp8.quant_token(y2, fmt)
    else:
        codes, scale = _fp8.quant_static(y2, static_scale, fmt), None
    return codes.reshape(y.shape), scale, y
