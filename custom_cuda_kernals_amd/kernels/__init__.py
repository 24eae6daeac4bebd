"""Python entry points, one module per op, with the reference's signatures
(custom_cuda/kernels/{rmsnorm_residual,swiglu,rope,fp8_quant,token_permute,moe_router}.py)
plus the additive FP8 modes and fusions."""

from custom_cuda_kernals_amd.kernels.fp8_quant import fp8_quant
from custom_cuda_kernals_amd.kernels.moe_router import moe_router
from custom_cuda_kernals_amd.kernels.rmsnorm_residual import rmsnorm_residual, rmsnorm_residual_fp8
from custom_cuda_kernals_amd.kernels.rope import rope
from custom_cuda_kernals_amd.kernels.swiglu import swiglu, swiglu_fp8
from custom_cuda_kernals_amd.kernels.token_permute import compute_permutation, token_combine, token_gather

__all__ = ["fp8_quant", "rmsnorm_residual", "rmsnorm_residual_fp8", "rope", "swiglu", "swiglu_fp8",
           "token_gather", "token_combine", "compute_permutation", "moe_router"]
