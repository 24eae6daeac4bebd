"""Kernels enqueued per Python API call, counted as the nodes of a HIP graph
that captures exactly one call (hipGraphGetNodes on the captured graph).

Static-scale calls are one kernel each: the op's own kernel stores the
static scale into the returned [1] tensor (no separate fill launch). The
dynamic ops are one kernel, except per-tensor FP8, whose launch count
depends on the input size (one-pass with its init launch, or the two-pass
forms). Every captured call is also replayed and checked against its
eager result.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from custom_cuda_kernals_amd.kernels import fp8_quant, rmsnorm_residual, rmsnorm_residual_fp8, swiglu, swiglu_fp8
from oracle import inputs

pytestmark = pytest.mark.gpu


def _hip():
    lib = ctypes.CDLL("libamdhip64.so.7")
    lib.hipGraphGetNodes.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.POINTER(ctypes.c_size_t)]
    lib.hipGraphGetNodes.restype = ctypes.c_int
    return lib


def _captured_nodes(call):
    """(node count, outputs of the captured call after one replay)."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call()  # warm-up outside the capture (allocator, one-time lookups)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph(keep_graph=True)
    with torch.cuda.graph(graph, stream=side):
        outs = call()
    n = ctypes.c_size_t(0)
    assert _hip().hipGraphGetNodes(ctypes.c_void_p(graph.raw_cuda_graph()), None, ctypes.byref(n)) == 0
    graph.replay()
    torch.cuda.synchronize()
    return n.value, outs


def _same(a: torch.Tensor, b: torch.Tensor) -> bool:
    return torch.equal(a.view(torch.uint8), b.view(torch.uint8))


@pytest.mark.parametrize("op", ["fp8_quant", "rmsnorm_residual_fp8", "swiglu_fp8"])
def test_static_scale_calls_are_one_kernel(op):
    x = inputs.randn((512, 4096), torch.bfloat16, seed=1).cuda()
    r = inputs.randn((512, 4096), torch.bfloat16, seed=2).cuda()
    w = inputs.randn((4096,), torch.bfloat16, seed=3).cuda()
    call = {
        "fp8_quant": lambda: fp8_quant(x, "e4m3", "tensor", scale=0.05),
        "rmsnorm_residual_fp8": lambda: rmsnorm_residual_fp8(x, r, w, 1e-5, scale=0.05),
        "swiglu_fp8": lambda: swiglu_fp8(x, r, scale=0.05),
    }[op]
    nodes, outs = _captured_nodes(call)
    assert nodes == 1, f"{op}: {nodes} kernels per static call"
    eager = call()
    torch.cuda.synchronize()
    for a, b in zip(outs, eager):
        assert _same(a, b)
    scale = outs[1]
    assert scale.shape == (1,) and scale.dtype == torch.float32
    assert np.array_equal(scale.cpu().numpy().view(np.uint32), np.array([0.05], dtype=np.float32).view(np.uint32))


def test_static_scale_of_an_empty_input():
    x = torch.empty((0, 4096), dtype=torch.bfloat16, device="cuda")
    q, s = fp8_quant(x, "e4m3", "tensor", scale=0.25)
    torch.cuda.synchronize()
    assert q.shape == (0, 4096) and float(s.item()) == 0.25


@pytest.mark.parametrize("case,expected", [
    ("rmsnorm_residual", 1), ("swiglu", 1), ("fp8_token", 1), ("fp8_block", 1),
    ("rmsnorm_residual_fp8_token", 1), ("swiglu_fp8_token", 1),
    ("fp8_tensor_one_workgroup", 1), ("fp8_tensor_one_pass", 2), ("fp8_tensor_two_pass_small", 2),
    ("fp8_tensor_two_pass_finish", 3),
])
def test_kernels_per_call(case, expected):
    x = inputs.randn((2048, 4096), torch.bfloat16, seed=4).cuda()
    r = inputs.randn((2048, 4096), torch.bfloat16, seed=5).cuda()
    w = inputs.randn((4096,), torch.bfloat16, seed=6).cuda()
    small = inputs.randn((512, 4096), torch.bfloat16, seed=7).cuda()
    tiny = inputs.randn((2, 4096), torch.bfloat16, seed=8).cuda()
    odd = inputs.randn((4099, 4097), torch.bfloat16, seed=9).cuda()
    call = {
        "rmsnorm_residual": lambda: rmsnorm_residual(x, r, w, 1e-5),
        "swiglu": lambda: (swiglu(x, r),),
        "fp8_token": lambda: fp8_quant(x, "e4m3", "token"),
        "fp8_block": lambda: fp8_quant(x, "e4m3", "block"),
        "rmsnorm_residual_fp8_token": lambda: rmsnorm_residual_fp8(x, r, w, 1e-5),
        "swiglu_fp8_token": lambda: swiglu_fp8(x, r),
        "fp8_tensor_one_workgroup": lambda: fp8_quant(tiny, "e4m3", "tensor"),
        "fp8_tensor_one_pass": lambda: fp8_quant(x, "e4m3", "tensor"),
        "fp8_tensor_two_pass_small": lambda: fp8_quant(small, "e4m3", "tensor"),
        "fp8_tensor_two_pass_finish": lambda: fp8_quant(odd, "e4m3", "tensor"),
    }[case]
    nodes, outs = _captured_nodes(call)
    assert nodes == expected, f"{case}: {nodes} kernels"
    eager = call()
    torch.cuda.synchronize()
    for a, b in zip(outs, eager):
        assert _same(a, b)
