"""Seeded CPU input generators for the BASELINE.json configurations and the
small parity cases. Inputs are made on the CPU with a seeded
``torch.Generator`` and copied to the device, so the GPU kernel and the CPU
oracle see identical bits (the reference generates with a CUDA generator,
baselines/*.py ``make_inputs``, which a CPU run cannot reproduce).
"""

from __future__ import annotations

import hashlib

import torch

CONFIG_SHAPES = {
    # 1: per-token FP8 quant, X [2048, 4096] with 0.1 % outliers x50
    "fp8_token": (2048, 4096),
    # 2: RMSNorm + residual, Llama-3-8B width
    "rmsnorm": (8192, 4096),
    # 3: SwiGLU (and SwiGLU + per-token FP8)
    "swiglu": (8192, 14336),
    # 4: RoPE, Llama-3 GQA prefill: q [8,4096,32,128], k [8,4096,8,128], theta 5e5
    "rope": (8, 4096, 32, 8, 128),
    # 5: block chain at T = 16384 tokens
    "chain_rmsnorm": (16384, 4096),
    "chain_swiglu": (16384, 14336),
}
# MoE dispatch (the reference's standard cases, baselines/token_permute.py:128-146,
# baselines/moe_router.py:72-79): gather 2048 -> 4096 rows of 4096; combine
# T = 2048 at top-2 and top-6 over hidden 4096; router 2048 x 160 experts, top-6.
MOE_SHAPES = {
    "gather": (2048, 4096, 4096),      # (n_src_rows, n_dst_rows, hidden)
    "combine_k2": (2048, 2, 4096),     # (n_tokens, k, hidden)
    "combine_k6": (2048, 6, 4096),
    "router": (2048, 160, 6),          # (n_tokens, n_experts, k)
}
ROPE_THETA = 500000.0
RMS_EPS = 1e-5
STATIC_SCALE = 0.05
OUTLIER_FRACTION = 0.001
OUTLIER_GAIN = 50.0


def _gen(seed: int) -> torch.Generator:
    return torch.Generator(device="cpu").manual_seed(seed)


def randn(shape, dtype=torch.bfloat16, seed: int = 0, gen: torch.Generator | None = None) -> torch.Tensor:
    g = gen if gen is not None else _gen(seed)
    return torch.randn(shape, dtype=torch.float32, generator=g).to(dtype)


def fp8_token_input(m: int, n: int, dtype=torch.bfloat16, seed: int = 0) -> torch.Tensor:
    """N(0,1) with round(0.1 % of m*n) seeded entries multiplied by 50."""
    g = _gen(seed)
    x = torch.randn((m, n), dtype=torch.float32, generator=g)
    k = int(round(OUTLIER_FRACTION * m * n))
    if k:
        idx = torch.randperm(m * n, generator=g)[:k]
        x.view(-1)[idx] *= OUTLIER_GAIN
    return x.to(dtype)


def rmsnorm_inputs(rows: int, cols: int, dtype=torch.bfloat16, seed: int = 0):
    """x, residual ~ N(0,1); weight ~ N(1, 0.1)."""
    g = _gen(seed)
    x = torch.randn((rows, cols), dtype=torch.float32, generator=g).to(dtype)
    r = torch.randn((rows, cols), dtype=torch.float32, generator=g).to(dtype)
    w = (1.0 + 0.1 * torch.randn((cols,), dtype=torch.float32, generator=g)).to(dtype)
    return x, r, w


def swiglu_inputs(rows: int, cols: int, dtype=torch.bfloat16, seed: int = 0):
    g = _gen(seed)
    gate = torch.randn((rows, cols), dtype=torch.float32, generator=g).to(dtype)
    up = torch.randn((rows, cols), dtype=torch.float32, generator=g).to(dtype)
    return gate, up


def rope_inputs(b: int, s: int, hq: int, hkv: int, d: int, dtype=torch.bfloat16, seed: int = 0,
                theta: float = ROPE_THETA):
    from oracle.eager import compute_cos_sin

    g = _gen(seed)
    q = torch.randn((b, s, hq, d), dtype=torch.float32, generator=g).to(dtype)
    k = torch.randn((b, s, hkv, d), dtype=torch.float32, generator=g).to(dtype)
    cos, sin = compute_cos_sin(s, d, theta)
    return q, k, cos, sin


def digest(*tensors: torch.Tensor) -> str:
    h = hashlib.sha256()
    for t in tensors:
        h.update(t.contiguous().view(torch.uint8).numpy().tobytes() if t.numel() else b"")
    return h.hexdigest()[:16]


def gather_inputs(n_src: int, n_dst: int, hidden: int, dtype=torch.bfloat16, seed: int = 0):
    """src ~ N(0,1) [n_src, hidden]; indices uniform in [0, n_src), int64 [n_dst]."""
    g = _gen(seed)
    src = torch.randn((n_src, hidden), dtype=torch.float32, generator=g).to(dtype)
    idx = torch.randint(0, max(n_src, 1), (n_dst,), generator=g, dtype=torch.int64) if n_src else \
        torch.empty(n_dst, dtype=torch.int64)
    return src, idx


def combine_inputs(n_tokens: int, k: int, hidden: int, dtype=torch.bfloat16, seed: int = 0):
    """expert_output ~ N(0,1) [T*k, hidden]; unpermute_index a random permutation
    of range(T*k) as [T, k] (every expert row claimed once); weights U[0,1) fp32."""
    g = _gen(seed)
    eo = torch.randn((n_tokens * k, hidden), dtype=torch.float32, generator=g).to(dtype)
    w = torch.rand((n_tokens, k), dtype=torch.float32, generator=g)
    ui = torch.randperm(n_tokens * k, generator=g).reshape(n_tokens, k)
    return eo, ui, w


def router_inputs(n_tokens: int, n_experts: int, dtype=torch.float32, seed: int = 0) -> torch.Tensor:
    return torch.randn((n_tokens, n_experts), dtype=torch.float32, generator=_gen(seed)).to(dtype)
