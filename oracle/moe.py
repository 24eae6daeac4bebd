"""CPU restatements of the reference's MoE dispatch baselines (test
infrastructure only; the product never imports this module).

* ``compute_permutation`` <- baselines/token_permute.py:55-70 (stable argsort
  of the flattened expert assignments and its inverse), in numpy
* ``token_gather``        <- baselines/token_permute.py:215-217 (index_select)
* ``token_combine``       <- baselines/token_permute.py:237-251
                             ((gathered.float() * w).sum(dim=1).to(dtype))
* ``moe_router``          <- baselines/moe_router.py:117-128
                             (softmax in fp32, topk, optional renormalisation)
* ``softmax_avx512``      torch-CPU's float32 softmax over the last dim as
                          its AVX-512 kernel computes it (below)
* ``moe_router_avx512``   ``moe_router`` with that softmax and the
                          renormalising sum in ATen's row-sum order
                          (oracle/rowsum.py): what torch computes on an
                          AVX-512 host, whatever the test host is
* ``*_fp64``              <- the fp64 ground truths (token_permute.py:229-232,
                             254-260; moe_router.py:140-148)
* ``token_combine_aten``  the combine with torch-CPU's summation order
                          written out (the order the HIP kernel follows)

torch-CPU's float32 softmax (torch 2.10, ATen's vectorised last-dim kernel
with 16-float AVX-512 vectors, the oracle's third-party dependency), per row
of n values x:
  m = max(x) (NaN-propagating);  e_i = xexpf(x_i - m), SLEEF's 1-ulp expf
  (oracle/sigmoid.py);  the sum of e in 16 lane classes: for n >= 16 lane L
  starts at e_L and adds e_{L+16}, e_{L+32}, ... in order over the whole
  vectors, lanes L < n mod 16 then add the tail element 16 (n // 16) + L, and
  the 16 lanes are combined as lane L + lane (L xor 8), then xor 4, 2, 1,
  giving lane 0; for n < 16 the sum is e_0 + e_1 + ... in order;
  p_i = e_i * RN(1 / sum).
On an AVX2 host torch uses 8-float vectors (another order); the restatement
fixes the AVX-512 one, which the GPU kernel follows.

The torch ops are the reference oracle's own CPU kernels. Pinned by
(tests/test_oracle_moe.py): golden vectors written from the reference's own
baselines (tests/golden/reference_moe.npz), the permutation invariants
(expert-sorted and stable, inverse of each other, round trip), the fp64
closed forms within the reference's tolerances, and bit equality of
``token_combine`` and ``token_combine_aten`` over row lengths and top-k.
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
    """The reference's formula on torch-CPU, evaluated on one thread: with
    several threads torch may split a reduction of at least 32768 elements
    over the hidden columns (in 32-column ranges, when the token count is
    small), and a last range of 4 to 7 columns then sums its first 4 columns
    in j order instead of the scalar form, so those bits depend on the host's
    thread count. One thread gives the order every host shares."""
    if unpermute_index.numel() == 0:
        return torch.zeros(unpermute_index.shape[0], expert_output.shape[-1], dtype=expert_output.dtype)
    prev = torch.get_num_threads()
    torch.set_num_threads(1)
    try:
        gathered = expert_output[unpermute_index]
        return (gathered.to(torch.float32) * weights.unsqueeze(-1)).sum(dim=1).to(expert_output.dtype)
    finally:
        torch.set_num_threads(prev)


def combine_main_columns(h: int) -> int:
    """How many leading hidden columns torch-CPU's ``sum(dim=1)`` of a
    contiguous [T, k, h] float32 tensor reduces as vector lanes (32-column
    chunks; 4 columns for rows of 4 to 7); the rest take the scalar form."""
    if h >= 32:
        return h - h % 32
    if 4 <= h < 8:
        return 4
    return 0


def token_combine_aten(expert_output: torch.Tensor, unpermute_index: torch.Tensor,
                       weights: torch.Tensor) -> torch.Tensor:
    """``(gathered.float() * w).sum(dim=1).to(dtype)`` in torch-CPU's own
    order (torch 2.10 ATen, the oracle's third-party dependency): the products
    rounded to float32, then per output column
      * the leading ``combine_main_columns(h)`` columns: one running sum over
        j = 0..k-1 in ATen's block cascade (blocks of 2^P steps, P = max(4,
        ceil_log2(k) // 4), folded into a second, third and fourth
        accumulator; oracle/rowsum.py), i.e. plain j order for k <= 16;
      * the other columns: the scalar form, four slots of every fourth j
        (each slot in the same cascade), the k mod 4 leftovers added to slot
        0, then ((s0 + s1) + s2) + s3;
      * h == 1 (the reduced dimension is contiguous): the row sum over k.
    Pinned against torch by tests/test_oracle_moe.py."""
    from oracle import rowsum

    t, k = unpermute_index.shape
    h = expert_output.shape[-1]
    dt = expert_output.dtype
    if t == 0 or k == 0:
        return torch.zeros(t, h, dtype=dt)
    prod = (expert_output.to(torch.float32)[unpermute_index] * weights.to(torch.float32).unsqueeze(-1)).numpy()
    out = np.empty((t, h), np.float32)
    if h == 1:
        out[:, 0] = rowsum.row_sum(prod[:, :, 0])
        return torch.from_numpy(out).to(dt)
    cols = np.ascontiguousarray(prod.transpose(0, 2, 1))  # [t, h, k]
    mc = combine_main_columns(h)
    if mc:
        u = cols[:, :mc].reshape(t * mc, k, 1, 1)
        out[:, :mc] = rowsum._fold_slots(u)[:, 0, 0].reshape(t, mc)
    if mc < h:
        u = cols[:, mc:].reshape(t * (h - mc), k, 1)
        out[:, mc:] = (np.float32(0) + rowsum._slot_sum(u)[:, 0]).reshape(t, h - mc)
    return torch.from_numpy(out).to(dt)


def moe_router(logits: torch.Tensor, k: int, renormalize: bool = True) -> tuple[torch.Tensor, torch.Tensor]:
    probs = F.softmax(logits.to(torch.float32), dim=-1)
    w, i = torch.topk(probs, k, dim=-1)
    if renormalize:
        w = w / w.sum(dim=-1, keepdim=True)
    return w, i


def softmax_probs(logits: torch.Tensor) -> torch.Tensor:
    """The router's fp32 probabilities as torch computes them on an AVX-512
    host (for tie analysis in tests)."""
    return torch.from_numpy(softmax_avx512(logits.to(torch.float32).numpy()))


_LANES16 = 16


def softmax_avx512(x: np.ndarray) -> np.ndarray:
    """float32 [rows, n] -> float32 [rows, n]: torch-CPU's softmax over the
    last dim with 16-float vectors (module docstring)."""
    from oracle import sigmoid as osig

    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, n = x.shape
    if n == 0:
        return x.copy()
    with np.errstate(invalid="ignore", over="ignore"):
        m = np.max(x, axis=1)  # order-free; NaN-propagating like ATen's maximum
        e = osig.sleef_expf((x - m[:, None]).astype(np.float32))
        if n < _LANES16:
            total = e[:, 0].copy()
            for i in range(1, n):
                total = (total + e[:, i]).astype(np.float32)
        else:
            full = n // _LANES16
            acc = e[:, :_LANES16].copy()
            for v in range(1, full):
                acc = (acc + e[:, v * _LANES16:(v + 1) * _LANES16]).astype(np.float32)
            r = n - full * _LANES16
            if r:
                acc[:, :r] = (acc[:, :r] + e[:, full * _LANES16:]).astype(np.float32)
            lanes = np.arange(_LANES16)
            for step in (8, 4, 2, 1):
                acc = (acc + acc[:, lanes ^ step]).astype(np.float32)
            total = acc[:, 0]
        inv = (np.float32(1) / total).astype(np.float32)
        return (e * inv[:, None]).astype(np.float32)


def moe_router_avx512(logits: torch.Tensor, k: int, renormalize: bool = True) -> tuple[torch.Tensor, torch.Tensor]:
    """baselines/moe_router.py:117-128 as torch computes it on an AVX-512
    host: the restated softmax, torch's topk (its order among exactly equal
    probabilities is its own), and the renormalising sum in ATen's row-sum
    order followed by an IEEE division."""
    from oracle import rowsum

    probs = torch.from_numpy(softmax_avx512(logits.to(torch.float32).numpy()))
    w, i = torch.topk(probs, k, dim=-1)
    if renormalize and k > 0 and w.shape[0] > 0:
        wn = w.numpy()
        with np.errstate(invalid="ignore", divide="ignore"):
            w = torch.from_numpy((wn / rowsum.row_sum(wn)[:, None]).astype(np.float32))
    return w, i


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
