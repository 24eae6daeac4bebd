"""MoE token permute (row gather) and unpermute (weighted combine).

``token_gather`` and ``token_combine`` keep the reference signatures
(custom_cuda/kernels/token_permute.py:19-44). ``compute_permutation`` is the
index bookkeeping the reference keeps beside them
(baselines/token_permute.py:55-70): a stable sort of the expert
assignments. Given ``num_experts`` it runs the HIP counting-sort kernel
(moe_permutation, one launch, three from 65536 entries); without it, the
reference's torch ops (a stable argsort and its inverse) on the device.

Additions: ``token_gather`` also moves FP8 rows (1-byte codes), and an
index outside the source rows yields a zero row (gather) or drops its term
(combine) instead of reading out of bounds.
"""

from __future__ import annotations

import torch

from custom_cuda_kernals_amd._lib import native

__all__ = ["token_gather", "token_combine", "compute_permutation"]


def token_gather(src: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
    """``dst[i] = src[indices[i]]``. src: ``[S, H]`` contiguous device tensor,
    indices: ``[N]`` int64. Returns ``dst: [N, H]``."""
    n = indices.shape[0]
    h = src.shape[1]
    dst = torch.empty((n, h), dtype=src.dtype, device=src.device)
    native.token_gather_fwd(src, indices, dst)
    return dst


def token_combine(expert_output: torch.Tensor, unpermute_index: torch.Tensor, weights: torch.Tensor) -> torch.Tensor:
    """``combined[t] = sum_j weights[t,j] * expert_output[unpermute_index[t,j]]``.

    expert_output: ``[N, H]`` contiguous device tensor; unpermute_index:
    ``[T, k]`` int64; weights: ``[T, k]`` float32. Returns ``[T, H]``."""
    t, _ = unpermute_index.shape
    h = expert_output.shape[1]
    combined = torch.empty((t, h), dtype=expert_output.dtype, device=expert_output.device)
    native.token_combine_fwd(expert_output, unpermute_index, weights, combined)
    return combined


def compute_permutation(topk_indices: torch.Tensor, num_experts: int | None = None
                        ) -> tuple[torch.Tensor, torch.Tensor]:
    """From ``topk_indices [T, k]`` (expert per token and slot): ``permute_index
    [T*k]`` (source token of each expert-sorted slot; ties keep token order)
    and ``unpermute_index [T, k]`` (the sorted slot each assignment went to).

    With ``num_experts`` (at most 256; ids outside ``[0, num_experts)`` are
    ordered after every expert) this is one HIP kernel, a stable counting sort;
    without it, the reference's torch ops (a stable argsort and its inverse,
    baselines/token_permute.py:55-70) on the tensor's device."""
    t, k = topk_indices.shape
    if num_experts is not None:
        permute_index = torch.empty(t * k, dtype=torch.int64, device=topk_indices.device)
        unpermute_index = torch.empty((t, k), dtype=torch.int64, device=topk_indices.device)
        native.moe_permutation_fwd(topk_indices, permute_index, unpermute_index, int(num_experts))
        return permute_index, unpermute_index
    order = torch.argsort(topk_indices.reshape(-1), stable=True)
    permute_index = order // k
    inverse = torch.empty_like(order)
    inverse[order] = torch.arange(t * k, device=topk_indices.device)
    return permute_index, inverse.reshape(t, k)
