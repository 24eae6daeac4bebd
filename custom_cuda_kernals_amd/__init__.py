"""MI355X-native (gfx950) Llama-block activation kernels.

Drop-in counterpart of the reference package ``custom_cuda`` for its
memory-bound activation path: fused RMSNorm + residual, SwiGLU, half-split
RoPE and dynamic / static FP8 quantisation (plus RMSNorm + FP8 and
SwiGLU + FP8 fusions). The Python API lives in
``custom_cuda_kernals_amd.kernels`` with the reference's signatures
(custom_cuda/kernels/*.py); the hand-written HIP kernels sit behind the C ABI
in ``include/custom_kernels_amd.h``.
"""

__version__ = "0.1.0"
