"""SwiGLU activation, optionally fused with FP8 quantisation.

``swiglu`` keeps the reference signature (custom_cuda/kernels/swiglu.py:16-20);
``swiglu_fp8`` is additive. Semantics: baselines/swiglu.py:107-112.
"""

from __future__ import annotations

import torch

from custom_cuda_kernals_amd._lib import native
from custom_cuda_kernals_amd.kernels.fp8_quant import FP8_TORCH_DTYPES, check_fp8_format

__all__ = ["swiglu", "swiglu_fp8"]


def swiglu(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """``y = SiLU(gate) * up``. gate, up: same-shape contiguous device tensors."""
    y = torch.empty_like(gate)
    native.swiglu_fwd(gate, up, y)
    return y


def swiglu_fp8(
    gate: torch.Tensor, up: torch.Tensor, fp8_format: str = "e4m3", scale: float | None = None
) -> tuple[torch.Tensor, torch.Tensor]:
    """FP8 codes of ``y = SiLU(gate) * up`` (y rounded to gate's dtype first),
    one pass over gate/up; ``y`` itself is not materialised.

    ``scale=None``: dynamic per-token scales over the last dimension, returned
    with shape ``gate.shape[:-1]``; ``scale=<float>``: static per-tensor scale,
    returned as a ``[1]`` tensor. Returns ``(y_fp8, scale)``.
    """
    check_fp8_format(fp8_format)
    y_fp8 = torch.empty(gate.shape, dtype=FP8_TORCH_DTYPES[fp8_format], device=gate.device)
    if scale is None:
        rows = gate.numel() // gate.shape[-1] if gate.dim() > 0 and gate.shape[-1] > 0 else 0
        scales = torch.empty(rows, dtype=torch.float32, device=gate.device)
        native.swiglu_fp8_fwd(gate, up, y_fp8, scales, fp8_format, None)
        return y_fp8, scales.view(gate.shape[:-1])
    # The kernel stores the static scale into the returned [1] tensor (one
    # launch); an empty gate launches nothing, so its scale tensor is filled here.
    scales = torch.empty(1, dtype=torch.float32, device=gate.device)
    native.swiglu_fp8_fwd(gate, up, y_fp8, scales, fp8_format, float(scale))
    if gate.numel() == 0:
        scales.fill_(float(scale))
    return y_fp8, scales
