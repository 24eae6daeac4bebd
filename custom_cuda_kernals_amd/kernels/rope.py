"""Half-split rotary position embedding.

Keeps the reference signature (custom_cuda/kernels/rope.py:16-28) and adds an
``inplace`` keyword. Semantics: baselines/rope.py:129-145 with
``position_ids = arange(seq_len)``.
"""

from __future__ import annotations

import torch

from custom_cuda_kernals_amd._lib import native

__all__ = ["rope"]


def rope(
    q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, *, inplace: bool = False
) -> tuple[torch.Tensor, torch.Tensor]:
    """Rotate q/k with precomputed cos/sin tables.

    q: ``[B, S, Hq, D]``, k: ``[B, S, Hkv, D]``, same dtype, contiguous device
    tensors. cos, sin: ``[S, D/2]`` float32. With ``inplace=True`` q and k are
    overwritten and returned.
    """
    if inplace:
        q_out, k_out = q, k
    else:
        q_out = torch.empty_like(q)
        k_out = torch.empty_like(k)
    native.rope_fwd(q, k, cos, sin, q_out, k_out)
    return q_out, k_out
