"""Fused residual add + RMSNorm, optionally fused with FP8 quantisation.

``rmsnorm_residual`` keeps the reference signature
(custom_cuda/kernels/rmsnorm_residual.py:17-28); ``rmsnorm_residual_fp8`` is
additive. Semantics: baselines/rmsnorm_residual.py:123-136.
"""

from __future__ import annotations

import torch

from custom_cuda_kernals_amd._lib import native
from custom_cuda_kernals_amd.kernels.fp8_quant import FP8_TORCH_DTYPES, check_fp8_format

__all__ = ["rmsnorm_residual", "rmsnorm_residual_fp8"]


def rmsnorm_residual(
    x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6
) -> tuple[torch.Tensor, torch.Tensor]:
    """``y, residual_out = RMSNorm(x + residual) * weight, x + residual``.

    x, residual: ``[..., hidden_dim]`` contiguous device tensors, same dtype
    (float32 / float16 / bfloat16). weight: ``[hidden_dim]``, same dtype.
    """
    y = torch.empty_like(x)
    residual_out = torch.empty_like(x)
    native.rmsnorm_residual_fwd(x, residual, weight, y, residual_out, eps)
    return y, residual_out


def rmsnorm_residual_fp8(
    x: torch.Tensor,
    residual: torch.Tensor,
    weight: torch.Tensor,
    eps: float = 1e-6,
    fp8_format: str = "e4m3",
    scale: float | None = None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """``residual_out = x + residual`` and the FP8 codes of
    ``y = RMSNorm(residual_out) * weight`` in one pass; ``y`` itself is not
    materialised.

    ``scale=None``: dynamic per-token scales ``clamp(amax_row(y)/FP8_MAX, 1e-12)``,
    returned with shape ``x.shape[:-1]``. ``scale=<float>``: static per-tensor
    scale, returned as a ``[1]`` tensor. Returns ``(y_fp8, scale, residual_out)``.
    """
    check_fp8_format(fp8_format)
    y_fp8 = torch.empty(x.shape, dtype=FP8_TORCH_DTYPES[fp8_format], device=x.device)
    residual_out = torch.empty_like(x)
    if scale is None:
        rows = x.numel() // x.shape[-1] if x.dim() > 0 and x.shape[-1] > 0 else 0
        scales = torch.empty(rows, dtype=torch.float32, device=x.device)
        native.rmsnorm_residual_fp8_fwd(x, residual, weight, y_fp8, scales, residual_out, eps, fp8_format, None)
        return y_fp8, scales.view(x.shape[:-1]), residual_out
    # The kernel stores the static scale into the returned [1] tensor (one
    # launch); an empty x launches nothing, so its scale tensor is filled here.
    scales = torch.empty(1, dtype=torch.float32, device=x.device)
    native.rmsnorm_residual_fp8_fwd(x, residual, weight, y_fp8, scales, residual_out, eps, fp8_format, float(scale))
    if x.numel() == 0:
        scales.fill_(float(scale))
    return y_fp8, scales, residual_out
