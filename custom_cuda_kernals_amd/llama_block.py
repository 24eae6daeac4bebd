"""Llama-3-8B decoder block on the MI355X activation kernels - the path's
integration caller.

Same architecture and numbers as the reference's integration proof
(examples/llama_block.py:55-204): pre-norm, GQA 32/8 heads of 128, RoPE theta
500000, SwiGLU FFN 4096 -> 14336 -> 4096, rms eps 1e-5, bf16. Three variants
share one set of weights:

* ``"eager"`` - plain torch ops (the reference's BaselineLlamaBlock);
* ``"fused"`` - the reference's CustomCUDA_LlamaBlock with this library:
  fused RMSNorm + residual, in-place RoPE and SwiGLU; GEMMs in bf16;
* ``"fp8"``   - the MI355X FP8 path: RMSNorm + residual fused with per-token
  FP8 quantisation feeds FP8 q/k/v and gate/up GEMMs (torch._scaled_mm on
  hipBLASLt, OCP e4m3fn, row-wise activation scales x per-output-channel
  weight scales); SwiGLU fused with per-token FP8 feeds the FP8 down
  projection; the attention output is quantised per token for the FP8 o_proj.
  Weights are quantised once, per output channel, with this library's
  per-token quantiser (a weight row is an output channel).

Attention itself (scaled_dot_product_attention) is identical in all three.
"""

from __future__ import annotations

import dataclasses
import statistics

import torch
import torch.nn as nn
import torch.nn.functional as F

from custom_cuda_kernals_amd.fp8_format import fp8_linear
from custom_cuda_kernals_amd.kernels import (
    fp8_quant,
    rmsnorm_residual,
    rmsnorm_residual_fp8,
    rope,
    swiglu,
    swiglu_fp8,
)

__all__ = ["LlamaBlockConfig", "LlamaBlock", "rope_tables", "block_latency_ms", "MODES", "CONFIGS"]

MODES = ("eager", "fused", "fp8")


@dataclasses.dataclass(frozen=True)
class LlamaBlockConfig:
    """Llama-3-8B config.json values (reference examples/llama_block.py:55-71)."""

    hidden_size: int = 4096
    intermediate_size: int = 14336
    num_heads: int = 32
    num_kv_heads: int = 8
    rms_eps: float = 1e-5
    rope_theta: float = 500000.0

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_heads


# The reference's block (Llama-3-8B) and, as an addition, Llama-3-70B's layer
# shapes (config.json: hidden 8192, intermediate 28672, 64 heads, 8 KV heads).
CONFIGS = {
    "llama3-8b": LlamaBlockConfig(),
    "llama3-70b": LlamaBlockConfig(hidden_size=8192, intermediate_size=28672, num_heads=64, num_kv_heads=8),
}


def rope_tables(seq_len: int, head_dim: int, theta: float, device) -> tuple[torch.Tensor, torch.Tensor]:
    """fp32 [S, D/2] cos/sin tables, computed as the reference's
    compute_cos_sin (baselines/rope.py:103-115)."""
    exponents = torch.arange(0, head_dim, 2, dtype=torch.float32, device=device) / head_dim
    inv_freq = 1.0 / (theta ** exponents)
    angles = torch.outer(torch.arange(seq_len, dtype=torch.float32, device=device), inv_freq)
    return angles.cos().contiguous(), angles.sin().contiguous()


def _eager_rmsnorm_residual(x, residual, weight, eps):
    ro = x + residual
    r32 = ro.float()
    normed = r32 * torch.rsqrt(r32.pow(2).mean(-1, keepdim=True) + eps)
    return normed.to(x.dtype) * weight, ro


def _eager_rope(q, k, cos, sin):
    def rot(t):
        t32 = t.float()
        half = t32.shape[-1] // 2
        a, b = t32[..., :half], t32[..., half:]
        c, s = cos[None, :, None, :], sin[None, :, None, :]
        return torch.cat([a * c - b * s, b * c + a * s], dim=-1).to(t.dtype)

    return rot(q), rot(k)


def _eager_swiglu(gate, up):
    g32 = gate.float()
    return (g32 * torch.sigmoid(g32)).to(gate.dtype) * up


class _Fp8Linear:
    """A bf16 weight [N, K] quantised once to e4m3fn per output channel; the
    activation comes per token (row-wise x row-wise _scaled_mm)."""

    def __init__(self, weight: torch.Tensor) -> None:
        self.w_codes, self.w_scale = fp8_quant(weight.contiguous(), "e4m3", "token")

    def __call__(self, x_fp8: torch.Tensor, x_scale: torch.Tensor) -> torch.Tensor:
        return fp8_linear(x_fp8, x_scale, "token", self.w_codes, self.w_scale, "token")


class LlamaBlock(nn.Module):
    def __init__(self, seq_len: int, cfg: LlamaBlockConfig = LlamaBlockConfig(), mode: str = "fused",
                 dtype: torch.dtype = torch.bfloat16, device: str = "cuda") -> None:
        super().__init__()
        if mode not in MODES:
            raise ValueError(f"mode must be one of {MODES}, got {mode!r}")
        self.cfg, self.mode = cfg, mode
        h, i, d = cfg.hidden_size, cfg.intermediate_size, cfg.head_dim

        def linear(n_in, n_out):
            return nn.Linear(n_in, n_out, bias=False, dtype=dtype, device=device)

        self.input_layernorm_weight = nn.Parameter(torch.ones(h, dtype=dtype, device=device))
        self.post_attention_layernorm_weight = nn.Parameter(torch.ones(h, dtype=dtype, device=device))
        self.q_proj, self.k_proj = linear(h, cfg.num_heads * d), linear(h, cfg.num_kv_heads * d)
        self.v_proj, self.o_proj = linear(h, cfg.num_kv_heads * d), linear(cfg.num_heads * d, h)
        self.gate_proj, self.up_proj, self.down_proj = linear(h, i), linear(h, i), linear(i, h)
        cos, sin = rope_tables(seq_len, d, cfg.rope_theta, device)
        self.register_buffer("rope_cos", cos, persistent=False)
        self.register_buffer("rope_sin", sin, persistent=False)
        self._fp8 = None

    def prepare_fp8(self) -> None:
        """Quantise the projection weights (call after loading weights)."""
        self._fp8 = {name: _Fp8Linear(getattr(self, name).weight.detach())
                     for name in ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")}

    def _attention(self, q, k, v):
        b, s = q.shape[0], q.shape[1]
        rep = self.cfg.num_heads // self.cfg.num_kv_heads
        k = k.repeat_interleave(rep, dim=2)
        v = v.repeat_interleave(rep, dim=2)
        out = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), is_causal=True)
        return out.transpose(1, 2).reshape(b, s, -1)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        cfg = self.cfg
        b, s, hid = x.shape
        d = cfg.head_dim
        zero = torch.zeros_like(x)
        if self.mode == "fp8":
            return self._forward_fp8(x, zero)
        norm = _eager_rmsnorm_residual if self.mode == "eager" else rmsnorm_residual
        h, residual = norm(x, zero, self.input_layernorm_weight, cfg.rms_eps)
        q = self.q_proj(h).view(b, s, cfg.num_heads, d)
        k = self.k_proj(h).view(b, s, cfg.num_kv_heads, d)
        v = self.v_proj(h).view(b, s, cfg.num_kv_heads, d)
        if self.mode == "eager":
            q, k = _eager_rope(q, k, self.rope_cos, self.rope_sin)
        else:
            q, k = rope(q, k, self.rope_cos, self.rope_sin, inplace=True)
        attn = self.o_proj(self._attention(q, k, v))
        h2, residual2 = norm(attn, residual, self.post_attention_layernorm_weight, cfg.rms_eps)
        gate, up = self.gate_proj(h2), self.up_proj(h2)
        act = _eager_swiglu(gate, up) if self.mode == "eager" else swiglu(gate, up)
        return self.down_proj(act) + residual2

    def _forward_fp8(self, x: torch.Tensor, zero: torch.Tensor) -> torch.Tensor:
        if self._fp8 is None:
            self.prepare_fp8()
        cfg, w = self.cfg, self._fp8
        b, s, hid = x.shape
        d, t = cfg.head_dim, b * s
        hq, hs, residual = rmsnorm_residual_fp8(x, zero, self.input_layernorm_weight, cfg.rms_eps)
        hq, hs = hq.view(t, hid), hs.view(t)
        q = w["q_proj"](hq, hs).view(b, s, cfg.num_heads, d)
        k = w["k_proj"](hq, hs).view(b, s, cfg.num_kv_heads, d)
        v = w["v_proj"](hq, hs).view(b, s, cfg.num_kv_heads, d)
        q, k = rope(q, k, self.rope_cos, self.rope_sin, inplace=True)
        a = self._attention(q, k, v).reshape(t, -1)
        aq, as_ = fp8_quant(a, "e4m3", "token")
        attn = w["o_proj"](aq, as_).view(b, s, hid)
        h2q, h2s, residual2 = rmsnorm_residual_fp8(attn, residual, self.post_attention_layernorm_weight, cfg.rms_eps)
        h2q, h2s = h2q.view(t, hid), h2s.view(t)
        gate, up = w["gate_proj"](h2q, h2s), w["up_proj"](h2q, h2s)
        mq, ms = swiglu_fp8(gate, up, "e4m3")
        return w["down_proj"](mq, ms).view(b, s, hid) + residual2


def block_latency_ms(block: nn.Module, x: torch.Tensor, warmup: int = 5, iters: int = 20,
                     flush_bytes: int = 1 << 30) -> dict:
    """Median / IQR of block(x) in ms, with the reference's methodology
    (examples/llama_block.py:220-250): a cache flush before every measured
    iteration (1 GiB here, larger than MI355X's 256 MB Infinity Cache) and
    HIP events around the forward."""
    flush = torch.empty(flush_bytes // 4, dtype=torch.float32, device=x.device)
    times = []
    with torch.no_grad():
        for _ in range(warmup):
            block(x)
        torch.cuda.synchronize()
        for _ in range(iters):
            flush.fill_(1.0)
            torch.cuda.synchronize()
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record()
            block(x)
            end.record()
            torch.cuda.synchronize()
            times.append(start.elapsed_time(end))
        torch.cuda.reset_peak_memory_stats()
        block(x)
        torch.cuda.synchronize()
        peak = torch.cuda.max_memory_allocated()
    times.sort()
    return {"median_ms": round(statistics.median(times), 4),
            "iqr_ms": round(times[(3 * len(times)) // 4] - times[len(times) // 4], 4),
            "peak_mem_MB": round(peak / 2**20, 1)}
