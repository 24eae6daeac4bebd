"""Dynamic / static FP8 quantisation.

Keeps the reference signature and defaults (custom_cuda/kernels/fp8_quant.py:28-63)
and adds ``granularity="token"`` (one scale per row) and a static ``scale``.
Semantics: ``scale = clamp(amax / FP8_MAX, min=1e-12)``,
``x_fp8 = (x.float() / scale).to(fp8)`` (baselines/fp8_quant.py:162-189).
"""

from __future__ import annotations

import math

import torch

from custom_cuda_kernals_amd._lib import native

__all__ = ["fp8_quant", "FP8_TORCH_DTYPES", "check_fp8_format"]

FP8_TORCH_DTYPES: dict[str, torch.dtype] = {
    "e4m3": torch.float8_e4m3fn,
    "e5m2": torch.float8_e5m2,
}

_BLOCK_SIZE = 128


def check_fp8_format(fp8_format: str) -> None:
    if fp8_format not in FP8_TORCH_DTYPES:
        raise ValueError(f"fp8_format must be 'e4m3' or 'e5m2', got {fp8_format!r}")


def fp8_quant(
    x: torch.Tensor,
    fp8_format: str = "e4m3",
    granularity: str = "block",
    scale: float | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Quantise a ``[M, N]`` float32/float16/bfloat16 device tensor to FP8.

    ``granularity``: ``"block"`` (one scale per 128x128 tile, scale
    ``[ceil(M/128), ceil(N/128)]``), ``"tensor"`` (one scale, ``[1]``) or
    ``"token"`` (one scale per row, ``[M]``). ``scale``: a static per-tensor
    scale (requires ``granularity="tensor"``); returned as a ``[1]`` tensor.
    Returns ``(x_fp8, scale)``.
    """
    check_fp8_format(fp8_format)
    if granularity not in ("block", "tensor", "token"):
        raise ValueError(f"granularity must be 'block', 'tensor' or 'token', got {granularity!r}")
    if scale is not None and granularity != "tensor":
        raise ValueError("a static scale is per-tensor: use granularity='tensor'")

    m, n = x.shape
    device = x.device
    x_fp8 = torch.empty((m, n), dtype=FP8_TORCH_DTYPES[fp8_format], device=device)

    if scale is not None:
        # The kernel stores the scale into the returned [1] tensor (one launch);
        # an empty x launches nothing, so its scale tensor is filled here.
        scales = torch.empty(1, dtype=torch.float32, device=device)
        native.fp8_quant_static_fwd(x, x_fp8, float(scale), fp8_format, scales)
        if x.numel() == 0:
            scales.fill_(float(scale))
        return x_fp8, scales

    if granularity == "block":
        scales = torch.empty(
            math.ceil(m / _BLOCK_SIZE), math.ceil(n / _BLOCK_SIZE), dtype=torch.float32, device=device
        )
        native.fp8_quant_block_fwd(x, x_fp8, scales, fp8_format)
        return x_fp8, scales

    if granularity == "token":
        scales = torch.empty(m, dtype=torch.float32, device=device)
        native.fp8_quant_token_fwd(x, x_fp8, scales, fp8_format)
        return x_fp8, scales

    # The reference zero-fills an int32 that receives the amax bits and then
    # drops it; None skips that word (and the fill launch) with the same codes
    # and scale.
    scales = torch.empty(1, dtype=torch.float32, device=device)
    native.fp8_quant_tensor_fwd(x, x_fp8, scales, None, fp8_format)
    return x_fp8, scales
