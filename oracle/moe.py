"""CPU restatements of the reference's MoE dispatch baselines (test
infrastructure only; the product never imports this module).

* ``compute_permutation`` <- baselines/token_permute.py:55-70 (stable argsort
  of the flattened expert assignments and its inverse), in numpy
* ``token_gather``        <- baselines/token_permute.py:215-217 (index_select)
* ``token_combine``       <- baselines/token_permute.py:237-251
                             ((gathered.float() * w).sum(dim=1).to(dtype))
* ``moe_router``          <- baselines/moe_router.py:117-128
                             (softmax in fp32, topk, optional renormalisation)
* ``*_fp64``              <- the fp64 ground truths (token_permute.py:229-232,
                             254-260; moe_router.py:140-148)
* ``combine_sequential``  the combine with its sum written out: fp32
                          products added in j order onto +0.0, the order the
                          HIP kernel uses

The torch ops are the reference oracle's own CPU kernels. Pinned by
(tests/test_oracle_moe.py): golden vectors written from the reference's own
baselines (tests/golden/reference_moe.npz), the permutation invariants
(expert-sorted and stable, inverse of each other, round trip), the fp64
closed forms within the reference's tolerances, and, for rows whose length is
a multiple of 16, bit equality of ``token_combine`` and
``combine_sequential``.
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F


def compute_permutation(topk_indices: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """(permute_index [T*k], unpermute_index [T, k]) from topk_indices [T, k]."""
    topk_indices = np.asarray(topk_indices)
    t, k = topk_indices.shape
    order = np.argsort(topk_indices.reshape(-1), kind="stable")
    permute_index = order // k
    inverse = np.empty_like(order)
    inverse[order] = np.arange(t * k)
    return permute_index.astype(np.int64), inverse.reshape(t, k).astype(np.int64)


def token_gather(src: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
    return src.index_select(0, indices)


def token_combine(expert_output: torch.Tensor, unpermute_index: torch.Tensor, weights: torch.Tensor) -> torch.Tensor:
    if unpermute_index.numel() == 0:
        return torch.zeros(unpermute_index.shape[0], expert_output.shape[-1], dtype=expert_output.dtype)
    gathered = expert_output[unpermute_index]
    return (gathered.to(torch.float32) * weights.unsqueeze(-1)).sum(dim=1).to(expert_output.dtype)


def combine_sequential(expert_output: torch.Tensor, unpermute_index: torch.Tensor,
                       weights: torch.Tensor) -> torch.Tensor:
    """The same sum with an explicit order: acc = +0.0; acc += w_j * x_j for j = 0..k-1."""
    eo = expert_output.to(torch.float32).numpy()
    ui = unpermute_index.numpy()
    w = weights.numpy().astype(np.float32)
    acc = np.zeros((ui.shape[0], eo.shape[1]), dtype=np.float32)
    for j in range(ui.shape[1]):
        acc = (acc + (eo[ui[:, j]] * w[:, j:j + 1]).astype(np.float32)).astype(np.float32)
    return torch.from_numpy(acc).to(expert_output.dtype)


def moe_router(logits: torch.Tensor, k: int, renormalize: bool = True) -> tuple[torch.Tensor, torch.Tensor]:
    probs = F.softmax(logits.to(torch.float32), dim=-1)
    w, i = torch.topk(probs, k, dim=-1)
    if renormalize:
        w = w / w.sum(dim=-1, keepdim=True)
    return w, i


def softmax_probs(logits: torch.Tensor) -> torch.Tensor:
    """The router's fp32 probabilities (for tie / near-tie analysis in tests)."""
    return F.softmax(logits.to(torch.float32), dim=-1)


def token_gather_fp64(src: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
    return src.to(torch.float64).index_select(0, indices)


def token_combine_fp64(expert_output: torch.Tensor, unpermute_index: torch.Tensor,
                       weights: torch.Tensor) -> torch.Tensor:
    if unpermute_index.numel() == 0:
        return torch.zeros(unpermute_index.shape[0], expert_output.shape[-1], dtype=torch.float64)
    g = expert_output.to(torch.float64)[unpermute_index]
    return (g * weights.to(torch.float64).unsqueeze(-1)).sum(dim=1)


def moe_router_fp64(logits: torch.Tensor, k: int, renormalize: bool = True) -> tuple[torch.Tensor, torch.Tensor]:
    probs = F.softmax(logits.to(torch.float64), dim=-1)
    w, i = torch.topk(probs, k, dim=-1)
    if renormalize:
        w = w / w.sum(dim=-1, keepdim=True)
    return w, i
