"""MoE top-k router with softmax gating.

Keeps the reference signature (custom_cuda/kernels/moe_router.py:18-34).
Semantics (baselines/moe_router.py:117-128): ``probs = softmax(float(logits))``,
the ``k`` largest in descending order (ties to the lower expert index), and
``weights /= weights.sum(-1)`` when ``renormalize``.
"""

from __future__ import annotations

import torch

from custom_cuda_kernals_amd._lib import native

__all__ = ["moe_router"]


def moe_router(logits: torch.Tensor, k: int, renormalize: bool = True) -> tuple[torch.Tensor, torch.Tensor]:
    """logits: ``[T, E]`` contiguous device tensor, ``E <= 256``. Returns
    ``topk_weights [T, k]`` float32 and ``topk_indices [T, k]`` int64."""
    n_tokens = logits.shape[0]
    topk_weights = torch.empty((n_tokens, k), dtype=torch.float32, device=logits.device)
    topk_indices = torch.empty((n_tokens, k), dtype=torch.long, device=logits.device)
    native.moe_router_fwd(logits, topk_weights, topk_indices, renormalize)
    return topk_weights, topk_indices
