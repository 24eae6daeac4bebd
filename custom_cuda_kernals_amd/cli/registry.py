"""What each op of this library is, as data for the CLI commands.

Mirrors the role of the reference's kernel registry
(custom_cuda/cli/registry.py): one record per op with its purpose, dtypes,
memory profile, design notes, target, files, tests, the bench.py ops that
time it, and a builder for one representative call (used by `profile` and
`compare`). Kept free of torch imports at module scope so `list`, `info` and
`help` start fast; the builders import lazily.
"""

from __future__ import annotations

import dataclasses
from collections.abc import Callable

__all__ = ["OpSpec", "Target", "REGISTRY", "get_op", "list_ops"]


@dataclasses.dataclass(frozen=True)
class Target:
    """A ready-to-call workload: the library's kernel and the reference's
    eager formula on the same device tensors."""

    kernel: Callable[[], object]
    eager: Callable[[], object]
    description: str
    nbytes: int  # algorithmic HBM bytes of one kernel call


@dataclasses.dataclass(frozen=True)
class OpSpec:
    id: str
    number: int
    title: str
    purpose: str
    formula: str
    dtypes: tuple[str, ...]
    memory_profile: str
    design: tuple[str, ...]
    target: str
    reference: tuple[str, ...]
    python_api: tuple[str, ...]
    c_entry_points: tuple[str, ...]
    sources: tuple[str, ...]
    test_files: tuple[str, ...]
    bench_ops: tuple[str, ...]
    build_target: Callable[[str], Target]


def _rn(shape, dtype, device, gen):
    import torch

    return torch.randn(shape, device=device, dtype=torch.float32, generator=gen).to(dtype)


def _gen(device):
    import torch

    return torch.Generator(device=device).manual_seed(0)


# --- representative calls (config shapes of BASELINE.json, bf16) -----------------------------------


def _t_rmsnorm(device: str) -> Target:
    import torch

    from custom_cuda_kernals_amd.kernels import rmsnorm_residual

    g = _gen(device)
    m, n = 8192, 4096
    x, r = _rn((m, n), torch.bfloat16, device, g), _rn((m, n), torch.bfloat16, device, g)
    w = (1.0 + 0.1 * torch.randn(n, device=device, generator=g)).to(torch.bfloat16)

    def eager():  # baselines/rmsnorm_residual.py:123-136
        ro = x + r
        up = ro.float()
        return (up * torch.rsqrt(up.pow(2).mean(-1, keepdim=True) + 1e-5)).to(x.dtype) * w, ro

    return Target(lambda: rmsnorm_residual(x, r, w, 1e-5), eager, "rmsnorm_residual bf16 [8192, 4096]",
                  m * n * 8 + n * 2)


def _t_swiglu(device: str) -> Target:
    import torch

    from custom_cuda_kernals_amd.kernels import swiglu

    g = _gen(device)
    m, n = 8192, 14336
    a, b = _rn((m, n), torch.bfloat16, device, g), _rn((m, n), torch.bfloat16, device, g)

    def eager():  # baselines/swiglu.py:107-112
        g32 = a.float()
        return (g32 * torch.sigmoid(g32)).to(a.dtype) * b

    return Target(lambda: swiglu(a, b), eager, "swiglu bf16 [8192, 14336]", m * n * 6)


def _t_rope(device: str) -> Target:
    import torch

    from custom_cuda_kernals_amd.kernels import rope

    g = _gen(device)
    B, S, HQ, HKV, D = 8, 4096, 32, 8, 128
    q, k = _rn((B, S, HQ, D), torch.bfloat16, device, g), _rn((B, S, HKV, D), torch.bfloat16, device, g)
    inv = 1.0 / (500000.0 ** (torch.arange(0, D, 2, dtype=torch.float32, device=device) / D))
    ang = torch.outer(torch.arange(S, dtype=torch.float32, device=device), inv)
    cos, sin = ang.cos().contiguous(), ang.sin().contiguous()

    def rot(t):  # baselines/rope.py:129-145
        t32 = t.float()
        h = t32.shape[-1] // 2
        c, s = cos[None, :, None, :], sin[None, :, None, :]
        return torch.cat([t32[..., :h] * c - t32[..., h:] * s, t32[..., h:] * c + t32[..., :h] * s], -1).to(t.dtype)

    return Target(lambda: rope(q, k, cos, sin, inplace=True), lambda: (rot(q), rot(k)),
                  "rope bf16 q [8, 4096, 32, 128] + k [8, 4096, 8, 128], in place", B * S * (HQ + HKV) * D * 4)


def _fp8_eager_rows(x):
    import torch

    x32 = x.float()
    s = torch.clamp(x32.abs().amax(-1, keepdim=True) / 448.0, min=1e-12)
    return (x32 / s).to(torch.float8_e4m3fn), s


def _t_fp8(device: str) -> Target:
    import torch

    from custom_cuda_kernals_amd.kernels import fp8_quant

    g = _gen(device)
    m, n = 2048, 4096
    x = _rn((m, n), torch.bfloat16, device, g)
    return Target(lambda: fp8_quant(x, "e4m3", "token"), lambda: _fp8_eager_rows(x),
                  "fp8_quant per-token e4m3 bf16 [2048, 4096]", m * n * 3 + m * 4)


def _t_rmsnorm_fp8(device: str) -> Target:
    import torch

    from custom_cuda_kernals_amd.kernels import rmsnorm_residual_fp8

    g = _gen(device)
    m, n = 16384, 4096
    x, r = _rn((m, n), torch.bfloat16, device, g), _rn((m, n), torch.bfloat16, device, g)
    w = (1.0 + 0.1 * torch.randn(n, device=device, generator=g)).to(torch.bfloat16)

    def eager():
        ro = x + r
        up = ro.float()
        y = (up * torch.rsqrt(up.pow(2).mean(-1, keepdim=True) + 1e-5)).to(x.dtype) * w
        return _fp8_eager_rows(y), ro

    return Target(lambda: rmsnorm_residual_fp8(x, r, w, 1e-5), eager,
                  "rmsnorm_residual_fp8 per-token bf16 [16384, 4096]", m * n * 7 + m * 4 + n * 2)


def _t_swiglu_fp8(device: str) -> Target:
    import torch

    from custom_cuda_kernals_amd.kernels import swiglu_fp8

    g = _gen(device)
    m, n = 8192, 14336
    a, b = _rn((m, n), torch.bfloat16, device, g), _rn((m, n), torch.bfloat16, device, g)

    def eager():
        g32 = a.float()
        return _fp8_eager_rows((g32 * torch.sigmoid(g32)).to(a.dtype) * b)

    return Target(lambda: swiglu_fp8(a, b), eager, "swiglu_fp8 per-token bf16 [8192, 14336]", m * n * 5 + m * 4)


def _t_token_permute(device: str) -> Target:
    import torch

    from custom_cuda_kernals_amd.kernels import token_gather

    g = _gen(device)
    src = _rn((2048, 4096), torch.bfloat16, device, g)
    idx = torch.randint(0, 2048, (4096,), device=device, generator=g)
    return Target(lambda: token_gather(src, idx), lambda: src[idx], "token_gather bf16 2048 -> 4096 rows x 4096",
                  4096 * 4096 * 4 + 4096 * 8)


def _t_moe_router(device: str) -> Target:
    import torch

    from custom_cuda_kernals_amd.kernels import moe_router

    g = _gen(device)
    logits = torch.randn((2048, 160), device=device, generator=g)

    def eager():  # baselines/moe_router.py:117-128
        w, i = torch.softmax(logits.float(), -1).topk(6, -1)
        return w / w.sum(-1, keepdim=True), i

    return Target(lambda: moe_router(logits, 6, True), eager, "moe_router f32 [2048, 160] top-6",
                  2048 * 160 * 4 + 2048 * 6 * 12)


_CSRC = "custom_cuda_kernals_amd/csrc/"

REGISTRY: dict[str, OpSpec] = {
    s.id: s
    for s in [
        OpSpec(
            id="rmsnorm_residual", number=1, title="Fused residual add + RMSNorm",
            purpose="residual_out = x + residual; y = RMSNorm(residual_out) * weight, one pass over HBM.",
            formula="ro = T(x + r); y = T(T(ro * rsqrt(mean(ro^2) + eps)) * w), the mean in torch-CPU's fp32 "
                    "summation order",
            dtypes=("float32", "float16", "bfloat16"),
            memory_profile="HBM-bound: 4 B in + 4 B out per bf16 element, plus the weight (config 2: 268 MB).",
            design=("one workgroup per row, the row held in registers between the reduction and the normalisation",
                    "row sum in torch-CPU's order: LDS-staged 64-vector regions folded by 32 lanes, one barrier",
                    "16-byte buffer-resource loads, SC1 / NT store policies measured per stream"),
            target=">= 75 % of 8 TB/s at [8192, 4096] bf16; y and residual_out bit-exact against eager",
            reference=("baselines/rmsnorm_residual.py:123-136", "csrc/kernels/rmsnorm_residual.cu",
                       "csrc/includes/rmsnorm_residual.h:17-27"),
            python_api=("rmsnorm_residual",), c_entry_points=("launch_rmsnorm_residual_fwd",),
            sources=(_CSRC + "rmsnorm_residual.hip", _CSRC + "aten_sum.hpp"),
            test_files=("tests/test_rmsnorm_residual_gpu.py", "tests/test_oracle_rowsum.py",
                        "tests/test_oracle_eager.py"),
            bench_ops=("rmsnorm_residual",), build_target=_t_rmsnorm),
        OpSpec(
            id="swiglu", number=2, title="SwiGLU activation",
            purpose="y = silu(gate) * up, elementwise.",
            formula="y = T(T(g * sigmoid(g)) * up), computed in fp32",
            dtypes=("float32", "float16", "bfloat16"),
            memory_profile="HBM-bound: 4 B in + 2 B out per bf16 element (config 3: 705 MB).",
            design=("512 threads x 2 vectors, at most 3 workgroups per CU",
                    "arithmetic SiLU: one v_exp_f32 with an exact exponent split, v_rcp_f32 + Newton"),
            target=">= 75 % of 8 TB/s at [8192, 14336] bf16; bit-exact against eager in bf16 / fp16",
            reference=("baselines/swiglu.py:107-112", "csrc/kernels/swiglu.cu", "csrc/includes/swiglu.h:16-22"),
            python_api=("swiglu",), c_entry_points=("launch_swiglu_fwd",),
            sources=(_CSRC + "swiglu.hip", _CSRC + "silu.hpp"),
            test_files=("tests/test_swiglu_gpu.py",), bench_ops=("swiglu",), build_target=_t_swiglu),
        OpSpec(
            id="rope", number=3, title="Rotary position embedding (half-split), in place or out of place",
            purpose="Rotate each (x1, x2) half-pair of q and k by the position's angle, with fp32 cos / sin tables.",
            formula="o1 = x1 c - x2 s; o2 = x2 c + x1 s, each product and difference rounded to fp32",
            dtypes=("float32", "float16", "bfloat16"),
            memory_profile="HBM-bound: 2 B in + 2 B out per bf16 element plus the tables (config 4: 673 MB).",
            design=("one workgroup per token, a thread per (head, chunk) for 33-128 heads (320 threads at "
                    "config 4's 40), cos / sin read once per chunk (staged in LDS while the grid fits one round)",
                    "per-token buffer-resource stores with SC1 | NT"),
            target=">= 75 % of 8 TB/s at q [8, 4096, 32, 128] + k [8, 4096, 8, 128] bf16; bit-exact",
            reference=("baselines/rope.py:103-145", "csrc/kernels/rope.cu", "csrc/includes/rope.h:23-36"),
            python_api=("rope",), c_entry_points=("launch_rope_fwd",), sources=(_CSRC + "rope.hip",),
            test_files=("tests/test_rope_gpu.py",), bench_ops=("rope_inplace",), build_target=_t_rope),
        OpSpec(
            id="fp8_quant", number=4, title="Dynamic / static FP8 quantisation (OCP e4m3fn / e5m2)",
            purpose="Quantise a [M, N] tensor to FP8 codes with one scale per row, per 128x128 tile, per tensor, "
                    "or a given static scale.",
            formula="scale = clamp(amax / FP8_MAX, min=1e-12); codes = (x.float() / scale).to(fp8)",
            dtypes=("float32", "float16", "bfloat16"),
            memory_profile="HBM-bound: 2 B in + 1 B out per bf16 element (config 1: 25 MB, launch-latency bound).",
            design=("row / tile held in registers; integer max of |x| bits (NaN-propagating)",
                    "division by the scale as three VALU ops (Markstein), v_cvt_pk_fp8_f32 with a sign-flip",
                    "per-tensor: partial, finish, cast; a no-allocation variant in two launches"),
            target="codes and scales bit-exact; per-token config 1 anchored on torch's own bf16->fp8 conversion",
            reference=("baselines/fp8_quant.py:126-189", "csrc/kernels/fp8_quant.cu", "csrc/includes/fp8_quant.h:41-60"),
            python_api=("fp8_quant",),
            c_entry_points=("launch_fp8_quant_block_fwd", "launch_fp8_quant_tensor_fwd",
                            "launch_fp8_quant_tensor_noalloc_fwd", "launch_fp8_quant_token_fwd",
                            "launch_fp8_quant_static_fwd"),
            sources=(_CSRC + "fp8_quant.hip", _CSRC + "fp8_codec.hpp", _CSRC + "cdna4.hpp"),
            test_files=("tests/test_fp8_quant_gpu.py", "tests/test_oracle_fp8.py", "tests/test_zz_no_alloc.py"),
            bench_ops=("fp8_quant_token", "fp8_quant_block", "fp8_quant_tensor", "fp8_quant_tensor_api",
                       "fp8_quant_tensor_noalloc", "fp8_quant_static"),
            build_target=_t_fp8),
        OpSpec(
            id="rmsnorm_residual_fp8", number=5, title="Fused residual add + RMSNorm + FP8 quantisation",
            purpose="residual_out and the FP8 codes of the bf16 RMSNorm output in one pass (y is not written).",
            formula="the rmsnorm_residual formula, then per-row (or static) FP8 of y as stored in its dtype",
            dtypes=("float32", "float16", "bfloat16"),
            memory_profile="HBM-bound: 4 B in + 2 B + 1 B out per bf16 element (config 5a: 470 MB).",
            design=("256 x 2 rows, y kept as fp32 in registers across the amax reduction",
                    "per-token rows of 1536+ vectors loop on a resident grid, the next row loaded across the amax "
                    "reduction"),
            target=">= 75 % of 8 TB/s at [16384, 4096] bf16; codes and scales bit-exact vs the composed eager op",
            reference=("baselines/rmsnorm_residual.py:123-136", "baselines/fp8_quant.py:162-178"),
            python_api=("rmsnorm_residual_fp8",), c_entry_points=("launch_rmsnorm_residual_fp8_fwd",),
            sources=(_CSRC + "rmsnorm_residual.hip",), test_files=("tests/test_fused_fp8_gpu.py",),
            bench_ops=("rmsnorm_residual_fp8_token", "rmsnorm_residual_fp8_static"), build_target=_t_rmsnorm_fp8),
        OpSpec(
            id="swiglu_fp8", number=6, title="Fused SwiGLU + FP8 quantisation",
            purpose="The FP8 codes of the bf16 SwiGLU output in one pass (y is not written).",
            formula="the swiglu formula, then per-row (or static) FP8 of y as stored in its dtype",
            dtypes=("float32", "float16", "bfloat16"),
            memory_profile="HBM-bound: 4 B in + 1 B out per bf16 element (config 3v: 587 MB, 5b: 1.17 GB).",
            design=("1024 x 2 rows; the bf16 SiLU tabulated in LDS (4864 entries) and looked up per gate",
                    "wider bf16 per-token rows park y in LDS on a looping grid, the next row loaded across the "
                    "amax reduction"),
            target=">= 75 % of 8 TB/s at [8192 | 16384, 14336] bf16; bit-exact vs the composed eager op",
            reference=("baselines/swiglu.py:107-112", "baselines/fp8_quant.py:162-178"),
            python_api=("swiglu_fp8",), c_entry_points=("launch_swiglu_fp8_fwd",), sources=(_CSRC + "swiglu.hip",),
            test_files=("tests/test_fused_fp8_gpu.py",),
            bench_ops=("swiglu_fp8_token", "swiglu_fp8_token_T16384", "swiglu_fp8_static_T16384"),
            build_target=_t_swiglu_fp8),
        OpSpec(
            id="token_permute", number=7, title="MoE token gather / weighted combine",
            purpose="Gather token rows into expert order, and combine expert outputs back with router weights.",
            formula="dst[i] = src[idx[i]]; out[t] = sum_j w[t, j] * eo[ui[t, j]] (fp32, j order)",
            dtypes=("float32", "float16", "bfloat16", "fp8 (gather)"),
            memory_profile="HBM-bound row moves (gather 67 MB, combine k = 2 50 MB at the reference's shapes).",
            design=("four or eight destination rows per gather workgroup; one vector per thread on a flat grid "
                    "for rows of more than 512 vectors and from 2^22 destination vectors",
                    "two expert rows in flight per combine step",
                    "the permutation bookkeeping as one stable counting-sort launch (compute_permutation with "
                    "num_experts)"),
            target="gather and the permutation bit-exact; combine equal to the j-order fp32 sum",
            reference=("baselines/token_permute.py:55-70, 215-251", "csrc/kernels/token_permute.cu",
                       "csrc/includes/token_permute.h:17-41"),
            python_api=("token_gather", "token_combine", "compute_permutation"),
            c_entry_points=("launch_token_gather_fwd", "launch_token_combine_fwd",
                            "launch_token_gather_checked_fwd", "launch_token_combine_checked_fwd",
                            "launch_moe_permutation_fwd"),
            sources=(_CSRC + "token_permute.hip",), test_files=("tests/test_token_permute_gpu.py",
                                                                 "tests/test_oracle_moe.py"),
            bench_ops=("token_gather", "token_combine_k2", "token_combine_k6", "moe_permutation"),
            build_target=_t_token_permute),
        OpSpec(
            id="moe_router", number=8, title="Softmax top-k MoE router",
            purpose="Per token: softmax over expert logits, the k largest probabilities, renormalised.",
            formula="probs = softmax(float(logits)); top-k descending, ties to the lower index; w / sum(w)",
            dtypes=("float32", "float16", "bfloat16"),
            memory_profile="latency-bound (1.3 MB at 2048 x 160).",
            design=("E <= 8: one lane per token, every step serial in its registers",
                    "9..32 experts (up to 64 from 4096 tokens): four lanes per token over 16-expert stripes",
                    "65..256 experts from 8192 / 12288 tokens: eight lanes per token",
                    "otherwise one wave per token, 4 experts per lane; wave arg-max per selection"),
            target="weights bit-exact against torch-CPU; indices equal the oracle's (exact ties aside)",
            reference=("baselines/moe_router.py:117-128", "csrc/kernels/moe_router.cu",
                       "csrc/includes/moe_router.h:20-29"),
            python_api=("moe_router",), c_entry_points=("launch_moe_router_fwd",), sources=(_CSRC + "moe_router.hip",),
            test_files=("tests/test_moe_router_gpu.py", "tests/test_oracle_moe.py"), bench_ops=("moe_router", "moe_router_e8"),
            build_target=_t_moe_router),
    ]
}


def get_op(op_id: str) -> OpSpec | None:
    return REGISTRY.get(op_id)


def list_ops() -> list[OpSpec]:
    return sorted(REGISTRY.values(), key=lambda s: s.number)
