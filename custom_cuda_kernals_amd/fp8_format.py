"""The FP8 activation format this library writes, and its GEMM-consumer contract.

An FP8 activation is a pair ``(codes, scale)``:

* ``codes``: ``[M, N]`` row-major, one byte per element, torch dtype
  ``float8_e4m3fn`` (OCP e4m3fn, as on gfx950; not MI300's fnuz) or
  ``float8_e5m2``. A code decodes exactly to an fp32 value ``c``.
* ``scale``: float32, one of three layouts (the reference's two,
  custom_cuda/kernels/fp8_quant.py:53-63, plus the per-token one):

  ================  =============================  ===========================
  granularity       scale shape                    element (i, j) dequantises
  ================  =============================  ===========================
  ``"token"``       ``[M]``                        ``c[i, j] * scale[i]``
  ``"tensor"``      ``[1]`` (dynamic or static)    ``c[i, j] * scale[0]``
  ``"block"``       ``[ceil(M/128), ceil(N/128)]`` ``c[i, j] * scale[i//128, j//128]``
  ================  =============================  ===========================

  and ``scale = clamp(amax / FP8_MAX, min=1e-12)`` over the row / tensor /
  tile (baselines/fp8_quant.py:162-189), or the given static scale.

GEMM consumers. ``torch._scaled_mm`` on ROCm (hipBLASLt, gfx950) accepts two
scale modes, probed on MI355X with torch 2.10:

* tensor-wise: both scales singletons (any of ``()``, ``[1]``, ``[1, 1]``);
  e4m3fn or e5m2 activations;
* row-wise: ``scale_a`` ``[M, 1]`` with ``scale_b`` ``[1, N]`` (both operands
  row-wise, e4m3fn only; 1-D scales and mixed modes are rejected). A weight
  ``[N, K]`` quantised with ``granularity="token"`` has exactly this per-output-
  channel scale.

There is no ``_scaled_mm`` mode for 128x128 tiles on this stack: block-scaled
activations are dequantised (``dequantize``) or fed to a GEMM that applies tile
scales itself. ``fp8_linear`` maps the layouts above onto ``_scaled_mm`` and
raises ``ValueError`` for the combinations it cannot express.
"""

from __future__ import annotations

import math

import torch

__all__ = ["FP8_DTYPES", "GRANULARITIES", "TILE", "scale_shape", "check_pair", "scaled_mm_scale", "fp8_linear",
           "dequantize"]

FP8_DTYPES = (torch.float8_e4m3fn, torch.float8_e5m2)
GRANULARITIES = ("token", "tensor", "block")
TILE = 128


def scale_shape(granularity: str, m: int, n: int) -> tuple[int, ...]:
    """Shape of the float32 scale tensor for codes ``[m, n]``."""
    if granularity == "token":
        return (m,)
    if granularity == "tensor":
        return (1,)
    if granularity == "block":
        return (math.ceil(m / TILE), math.ceil(n / TILE))
    raise ValueError(f"granularity must be one of {GRANULARITIES}, got {granularity!r}")


def check_pair(codes: torch.Tensor, scale: torch.Tensor, granularity: str) -> None:
    """Raise ValueError unless (codes, scale) is a well-formed FP8 activation."""
    if codes.dim() != 2:
        raise ValueError(f"codes must be 2-D [M, N], got shape {tuple(codes.shape)}")
    if codes.dtype not in FP8_DTYPES:
        raise ValueError(f"codes must be float8_e4m3fn or float8_e5m2, got {codes.dtype}")
    if not codes.is_contiguous():
        raise ValueError("codes must be contiguous (row-major)")
    if scale.dtype != torch.float32:
        raise ValueError(f"scale must be float32, got {scale.dtype}")
    want = scale_shape(granularity, *codes.shape)
    if tuple(scale.shape) != want:
        raise ValueError(f"{granularity} scale must have shape {want}, got {tuple(scale.shape)}")
    if scale.device != codes.device:
        raise ValueError("codes and scale must be on the same device")


def scaled_mm_scale(scale: torch.Tensor, granularity: str, side: str) -> torch.Tensor:
    """View of ``scale`` in the layout ``torch._scaled_mm`` expects.

    ``side="a"`` for the activation operand ``[M, K]`` (row-wise -> ``[M, 1]``),
    ``side="b"`` for a weight quantised per output channel (row-wise -> ``[1, N]``).
    """
    if side not in ("a", "b"):
        raise ValueError(f"side must be 'a' or 'b', got {side!r}")
    if granularity == "tensor":
        return scale.reshape(())
    if granularity == "token":
        return scale.view(-1, 1) if side == "a" else scale.view(1, -1)
    if granularity == "block":
        raise ValueError("torch._scaled_mm has no 128x128-tile scale mode on ROCm: dequantize block-scaled "
                         "operands or use a GEMM that applies tile scales")
    raise ValueError(f"granularity must be one of {GRANULARITIES}, got {granularity!r}")


def fp8_linear(x_codes: torch.Tensor, x_scale: torch.Tensor, x_granularity: str, w_codes: torch.Tensor,
               w_scale: torch.Tensor, w_granularity: str, out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """``y = dequant(x) @ dequant(w).T`` for x ``[M, K]`` and a weight ``[N, K]``
    through ``torch._scaled_mm``.

    Supported: both ``"tensor"``; or x ``"token"`` with w ``"token"`` (per
    output channel), e4m3fn. Anything else raises ValueError before the GEMM.
    """
    check_pair(x_codes, x_scale, x_granularity)
    check_pair(w_codes, w_scale, w_granularity)
    if x_codes.shape[1] != w_codes.shape[1]:
        raise ValueError(f"inner dimensions differ: x {tuple(x_codes.shape)}, w {tuple(w_codes.shape)}")
    modes = (x_granularity, w_granularity)
    if modes == ("token", "token"):
        if x_codes.dtype != torch.float8_e4m3fn or w_codes.dtype != torch.float8_e4m3fn:
            raise ValueError("row-wise scaled GEMMs need float8_e4m3fn operands on this stack")
    elif modes != ("tensor", "tensor"):
        raise ValueError(f"no torch._scaled_mm mode for x {x_granularity!r} with w {w_granularity!r}: "
                         "use ('tensor', 'tensor') or ('token', 'token')")
    return torch._scaled_mm(x_codes, w_codes.t(), scale_a=scaled_mm_scale(x_scale, x_granularity, "a"),
                            scale_b=scaled_mm_scale(w_scale, w_granularity, "b"), out_dtype=out_dtype)


def dequantize(codes: torch.Tensor, scale: torch.Tensor, granularity: str,
               out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """``codes * scale`` broadcast per the layout, one fp32 multiply per element."""
    check_pair(codes, scale, granularity)
    c = codes.to(torch.float32)
    if granularity == "token":
        s = scale.view(-1, 1)
    elif granularity == "tensor":
        s = scale.view(1, 1)
    else:
        m, n = codes.shape
        s = scale.repeat_interleave(TILE, dim=0)[:m].repeat_interleave(TILE, dim=1)[:, :n]
    return (c * s).to(out_dtype)
