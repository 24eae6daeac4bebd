"""The C-ABI boundary and the validating binding, on the CPU.

* libcustom_kernels_amd.so loads and exports every function that
  include/custom_kernels_amd.h declares, with that header's argument count;
* launchers return 0 for empty work and hipErrorInvalidValue (1) for an
  unknown dtype / format / mode tag, in both cases before any device call
  (reference csrc/kernels/rmsnorm_residual.cu:87-89, 113-114);
* the binding mirrors the reference's Rust checks (src/kernels/tensor.rs,
  error.rs, <op>.rs): ValueError for device type, contiguity, dtype, shape and
  format errors, in the reference's order. Tensors are stood in for by
  attribute-only fakes, so every case fails validation before a launch.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from tests import _cck

from custom_cuda_kernals_amd._lib import native  # noqa: E402
from custom_cuda_kernals_amd import kernels  # noqa: E402


def test_library_exports_every_declared_symbol():
    decls = _cck.declared_functions()
    assert len(decls) >= 11
    lib = ctypes.CDLL(_cck.LIB_PATH)
    for name in decls:
        assert hasattr(lib, name), name


# The reference's launchers, parameter by parameter, transcribed from its
# headers with its CUDA types mapped to this ABI's: cudaStream_t -> void*
# (the stream is an opaque pointer), cudaError_t (the return) -> int32_t.
REFERENCE_LAUNCHERS = {
    # csrc/includes/rmsnorm_residual.h:17-27
    "launch_rmsnorm_residual_fwd": ["const void*", "const void*", "const void*", "void*", "void*", "int64_t",
                                    "int64_t", "float", "int32_t", "void*"],
    # csrc/includes/swiglu.h:16-22
    "launch_swiglu_fwd": ["const void*", "const void*", "void*", "int64_t", "int32_t", "void*"],
    # csrc/includes/rope.h:23-36
    "launch_rope_fwd": ["const void*", "const void*", "const void*", "const void*", "void*", "void*", "int64_t",
                        "int64_t", "int64_t", "int64_t", "int64_t", "int32_t", "void*"],
    # csrc/includes/fp8_quant.h:41-49
    "launch_fp8_quant_block_fwd": ["const void*", "uint8_t*", "float*", "int64_t", "int64_t", "int32_t", "int32_t",
                                   "void*"],
    # csrc/includes/fp8_quant.h:51-60
    "launch_fp8_quant_tensor_fwd": ["const void*", "uint8_t*", "float*", "int32_t*", "int64_t", "int64_t",
                                    "int32_t", "int32_t", "void*"],
    # csrc/includes/token_permute.h:17-24
    "launch_token_gather_fwd": ["const void*", "const int64_t*", "void*", "int64_t", "int64_t", "int32_t",
                                "void*"],
    # csrc/includes/token_permute.h:32-41
    "launch_token_combine_fwd": ["const void*", "const int64_t*", "const float*", "void*", "int64_t", "int64_t",
                                 "int64_t", "int32_t", "void*"],
    # csrc/includes/moe_router.h:20-29
    "launch_moe_router_fwd": ["const void*", "float*", "int64_t*", "int64_t", "int64_t", "int64_t", "int32_t",
                              "int32_t", "void*"],
}


def test_reference_launchers_are_declared_with_reference_types():
    """Every reference launcher is declared in include/custom_kernels_amd.h
    with the reference's parameter types in the reference's order (and an
    int32_t return: the declaration parser only matches those)."""
    d = _cck.declared_functions()
    for name, params in REFERENCE_LAUNCHERS.items():
        assert name in d, name
        assert d[name] == params, f"{name}: header {d[name]} != reference {params}"


def test_parameter_type_parser_sees_a_changed_type():
    """The check above fails on a one-type change: the parser distinguishes
    the types it compares (a planted change to a copy of the header)."""
    import os
    import tempfile

    text = open(_cck.HEADER).read()
    changed = text.replace("void* y, void* residual_out, int64_t rows, int64_t cols,",
                           "void* y, void* residual_out, int64_t rows, int32_t cols,", 1)
    assert changed != text
    with tempfile.NamedTemporaryFile("w", suffix=".h", delete=False) as f:
        f.write(changed)
    try:
        saved = _cck.HEADER
        _cck.HEADER = f.name
        d = _cck.declared_functions()
    finally:
        _cck.HEADER = saved
        os.unlink(f.name)
    assert d["launch_rmsnorm_residual_fwd"] != REFERENCE_LAUNCHERS["launch_rmsnorm_residual_fwd"]


def test_empty_work_returns_success_without_device_calls():
    lib = _cck.load()
    assert lib.launch_rmsnorm_residual_fwd(None, None, None, None, None, 0, 4096, 1e-5, 2, None) == 0
    assert lib.launch_rmsnorm_residual_fwd(None, None, None, None, None, 8, 0, 1e-5, 2, None) == 0
    assert lib.launch_swiglu_fwd(None, None, None, 0, 2, None) == 0
    assert lib.launch_rope_fwd(None, None, None, None, None, None, 0, 16, 8, 8, 64, 2, None) == 0
    assert lib.launch_fp8_quant_block_fwd(None, None, None, 0, 16, 2, 3, None) == 0
    assert lib.launch_fp8_quant_tensor_fwd(None, None, None, None, 16, 0, 2, 3, None) == 0
    assert lib.launch_fp8_quant_token_fwd(None, None, None, 0, 16, 2, 3, None) == 0
    assert lib.launch_fp8_quant_static_fwd(None, None, 0.05, None, 0, 16, 2, 3, None) == 0
    assert lib.launch_rmsnorm_residual_fp8_fwd(None, None, None, None, None, None, 0, 16, 1e-5, 0.0, 0, 2, 3, None) == 0
    assert lib.launch_swiglu_fp8_fwd(None, None, None, None, 0, 16, 0.0, 0, 2, 3, None) == 0
    assert lib.launch_token_gather_fwd(None, None, None, 0, 4096, 2, None) == 0
    assert lib.launch_token_gather_fwd(None, None, None, 16, 0, 2, None) == 0
    assert lib.launch_token_gather_checked_fwd(None, None, None, 8, 0, 4096, 2, None) == 0
    assert lib.launch_token_combine_fwd(None, None, None, None, 0, 2, 4096, 2, None) == 0
    assert lib.launch_token_combine_fwd(None, None, None, None, 16, 0, 4096, 2, None) == 0
    assert lib.launch_token_combine_checked_fwd(None, None, None, None, 32, 16, 2, 0, 2, None) == 0
    assert lib.launch_moe_router_fwd(None, None, None, 0, 16, 2, 0, 1, None) == 0
    assert lib.launch_moe_router_fwd(None, None, None, 8, 16, 0, 0, 1, None) == 0
    assert lib.launch_moe_permutation_fwd(None, None, None, 0, 6, 160, None) == 0
    assert lib.launch_moe_permutation_fwd(None, None, None, 2048, 0, 160, None) == 0


def test_hbm_stream_rejects_bad_arguments_before_device_calls():
    lib = _cck.load()
    assert lib.cck_hbm_stream(0, None, None, None, None, 0, None) == 0
    assert lib.cck_hbm_stream(7, None, None, None, None, 0, None) == 0  # empty work first
    assert lib.cck_hbm_stream(7, None, None, None, None, 1024, None) == 1
    assert lib.cck_hbm_stream(-1, None, None, None, None, 1024, None) == 1
    assert lib.cck_hbm_stream(2, None, None, None, None, 1000, None) == 1  # partial 512-vector row
    assert lib.cck_hbm_stream(4, None, None, None, None, 1024, None) == 1  # partial 1792-vector row
    assert lib.cck_hbm_stream(5, None, None, None, None, 1000, None) == 1


def test_sigmoid_selftest_rejects_a_range_past_2_to_32_before_device_calls():
    lib = _cck.load()
    assert lib.cck_sigmoid_selftest(0, 0, None, None) == 0
    assert lib.cck_sigmoid_selftest((1 << 32) - 4, 8, None, None) == 1
    assert lib.cck_sigmoid_selftest(1 << 32, 1, None, None) == 1


def test_unknown_tags_return_invalid_value_before_device_calls():
    lib = _cck.load()
    assert lib.launch_rmsnorm_residual_fwd(None, None, None, None, None, 4, 8, 1e-5, 9, None) == 1
    assert lib.launch_swiglu_fwd(None, None, None, 8, 3, None) == 1  # fp8 is not a compute dtype
    assert lib.launch_rope_fwd(None, None, None, None, None, None, 1, 4, 2, 1, 8, 7, None) == 1
    assert lib.launch_rope_fwd(None, None, None, None, None, None, 1, 4, 2, 1, 7, 2, None) == 1  # odd head_dim
    assert lib.launch_fp8_quant_block_fwd(None, None, None, 4, 8, 2, 2, None) == 1  # bad fp8 format
    assert lib.launch_fp8_quant_token_fwd(None, None, None, 4, 8, 5, 3, None) == 1
    assert lib.launch_fp8_quant_tensor_fwd(None, None, None, None, 4, 8, 2, 9, None) == 1
    assert lib.launch_fp8_quant_tensor_noalloc_fwd(None, None, None, 4, 8, 2, 9, None) == 1
    assert lib.launch_fp8_quant_tensor_noalloc_fwd(None, None, None, 1 << 40, 1 << 40, 2, 3, None) == 1  # m*n > int64
    assert lib.launch_fp8_quant_static_fwd(None, None, 0.05, None, 4, 8, 2, 0, None) == 1
    assert lib.launch_rmsnorm_residual_fp8_fwd(None, None, None, None, None, None, 4, 8, 1e-5, 0.0, 2, 2, 3, None) == 1
    assert lib.launch_swiglu_fp8_fwd(None, None, None, None, 4, 8, 0.0, 7, 2, 3, None) == 1
    assert lib.cck_fp8_cvt_selftest(0, 16, 1, None, None) == 1
    assert lib.launch_token_gather_fwd(None, None, None, 4, 8, 7, None) == 1
    assert lib.launch_token_gather_checked_fwd(None, None, None, -1, 4, 8, 2, None) == 1
    assert lib.launch_token_combine_fwd(None, None, None, None, 4, 2, 8, 3, None) == 1  # fp8 is not a compute dtype
    assert lib.launch_token_combine_checked_fwd(None, None, None, None, -1, 4, 2, 8, 2, None) == 1
    assert lib.launch_moe_router_fwd(None, None, None, 4, 300, 2, 0, 1, None) == 1  # > 256 experts
    assert lib.launch_moe_router_fwd(None, None, None, 4, 8, 9, 0, 1, None) == 1  # k > experts
    assert lib.launch_moe_router_fwd(None, None, None, 4, 8, 2, 5, 1, None) == 1  # bad dtype
    assert lib.launch_moe_permutation_fwd(None, None, None, 4, 2, 0, None) == 1  # no experts
    assert lib.launch_moe_permutation_fwd(None, None, None, 4, 2, 257, None) == 1  # > 256 experts
    assert lib.launch_moe_permutation_fwd(None, None, None, 1 << 30, 8, 16, None) == 1  # positions past 32 bits
    assert lib.launch_moe_permutation_fwd(None, None, None, -1, 2, 16, None) == 1


class _Dev:
    def __init__(self, type_="cuda", index=0):
        self.type, self.index = type_, index


class FakeTensor:
    """Quacks like a torch.Tensor for the attributes the binding reads."""

    def __init__(self, shape, dtype=torch.bfloat16, device="cuda", contiguous=True):
        self.shape = torch.Size(shape)
        self.dtype = dtype
        self.device = _Dev(device)
        self._contig = contiguous

    def is_contiguous(self):
        return self._contig

    def data_ptr(self):
        return 0


def F(*shape, **kw):
    return FakeTensor(shape, **kw)


def _raises(fn, *args, match=None):
    with pytest.raises(ValueError, match=match):
        fn(*args)


def test_device_then_contiguity_then_dtype_order():
    # device type is checked first, even when the tensor is also non-contiguous
    _raises(native.swiglu_fwd, F(4, 8, device="cpu", contiguous=False), F(4, 8), F(4, 8), match="must be a CUDA tensor")
    _raises(native.swiglu_fwd, F(4, 8, contiguous=False), F(4, 8), F(4, 8), match="'gate' must be contiguous")
    _raises(native.swiglu_fwd, F(4, 8, dtype=torch.int64), F(4, 8), F(4, 8), match="unsupported dtype 'torch.int64'")
    # arguments are validated in order: a bad 'up' is reported before a bad 'y'
    _raises(native.swiglu_fwd, F(4, 8), F(4, 8, device="cpu"), F(4, 8, contiguous=False), match="'up' must be a CUDA")


def test_real_cpu_tensors_are_rejected_by_the_python_api():
    with pytest.raises(ValueError, match="must be a CUDA tensor, got device type 'cpu'"):
        kernels.swiglu(torch.randn(2, 8), torch.randn(2, 8))
    with pytest.raises(ValueError):
        kernels.rmsnorm_residual(torch.randn(2, 4, 8), torch.randn(2, 4, 8), torch.randn(8))
    with pytest.raises(ValueError):
        kernels.fp8_quant(torch.randn(4, 8), "e4m3", "block")
    with pytest.raises(ValueError):
        kernels.rope(torch.randn(1, 4, 2, 8), torch.randn(1, 4, 1, 8), torch.randn(4, 4), torch.randn(4, 4))


def test_rmsnorm_checks():
    ok = dict(x=F(2, 3, 8), r=F(2, 3, 8), w=F(8), y=F(2, 3, 8), ro=F(2, 3, 8))
    def call(**over):
        a = {**ok, **over}
        native.rmsnorm_residual_fwd(a["x"], a["r"], a["w"], a["y"], a["ro"], 1e-6)
    with pytest.raises(ValueError, match="dtype mismatch: 'residual' is F32 but expected BF16"):
        call(r=F(2, 3, 8, dtype=torch.float32))
    with pytest.raises(ValueError, match="'weight' is F16"):
        call(w=F(8, dtype=torch.float16))
    with pytest.raises(ValueError, match="shape mismatch: x/residual/y/residual_out must share"):
        call(y=F(2, 3, 9))
    with pytest.raises(ValueError, match=r"weight shape \[9\] must be \[8\]"):
        call(w=F(9))
    with pytest.raises(ValueError, match="at least 1 dimension"):
        call(x=F(), r=F(), y=F(), ro=F(), w=F(1))


def test_rope_checks():
    ok = dict(q=F(1, 4, 2, 8), k=F(1, 4, 1, 8), c=F(4, 4, dtype=torch.float32), s=F(4, 4, dtype=torch.float32),
              qo=F(1, 4, 2, 8), ko=F(1, 4, 1, 8))
    def call(**over):
        a = {**ok, **over}
        native.rope_fwd(a["q"], a["k"], a["c"], a["s"], a["qo"], a["ko"])
    with pytest.raises(ValueError, match="cos must be float32"):
        call(c=F(4, 4))
    with pytest.raises(ValueError, match="q must be 4-D"):
        call(q=F(4, 2, 8), qo=F(4, 2, 8))
    with pytest.raises(ValueError, match="q_out must match"):
        call(qo=F(1, 4, 2, 16))
    with pytest.raises(ValueError, match="share batch/seq_len/head_dim"):
        call(k=F(1, 5, 1, 8), ko=F(1, 5, 1, 8))
    with pytest.raises(ValueError, match="head_dim must be even"):
        call(q=F(1, 4, 2, 7), qo=F(1, 4, 2, 7), k=F(1, 4, 1, 7), ko=F(1, 4, 1, 7))
    with pytest.raises(ValueError, match=r"cos/sin must have shape \[4, 4\]"):
        call(c=F(4, 3, dtype=torch.float32))
    with pytest.raises(ValueError, match="'k_out' is F16"):
        call(ko=F(1, 4, 1, 8, dtype=torch.float16))


def test_fp8_checks():
    e4 = torch.float8_e4m3fn
    with pytest.raises(ValueError, match="fp8_format must be 'e4m3' or 'e5m2', got \"e4m4\""):
        native.fp8_quant_block_fwd(F(4, 8, device="cpu"), F(4, 8, dtype=e4), F(1, 1, dtype=torch.float32), "e4m4")
    with pytest.raises(ValueError, match="does not match requested fp8_format"):
        native.fp8_quant_block_fwd(F(4, 8), F(4, 8, dtype=torch.float8_e5m2), F(1, 1, dtype=torch.float32), "e4m3")
    with pytest.raises(ValueError, match="scale must be float32"):
        native.fp8_quant_block_fwd(F(4, 8), F(4, 8, dtype=e4), F(1, 1), "e4m3")
    with pytest.raises(ValueError, match="x must be 2-D"):
        native.fp8_quant_block_fwd(F(4, 8, 2), F(4, 8, 2, dtype=e4), F(1, 1, dtype=torch.float32), "e4m3")
    with pytest.raises(ValueError, match=r"scale shape \[1, 1\] must be \[2, 1\]"):
        native.fp8_quant_block_fwd(F(130, 8), F(130, 8, dtype=e4), F(1, 1, dtype=torch.float32), "e4m3")
    with pytest.raises(ValueError, match="amax_scratch must be int32"):
        native.fp8_quant_tensor_fwd(F(4, 8), F(4, 8, dtype=e4), F(1, dtype=torch.float32), F(1, dtype=torch.int64), "e4m3")
    with pytest.raises(ValueError, match="exactly 1 element"):
        native.fp8_quant_tensor_fwd(F(4, 8), F(4, 8, dtype=e4), F(1, dtype=torch.float32), F(2, dtype=torch.int32), "e4m3")
    # amax_scratch may be None; the other arguments are still checked in order
    with pytest.raises(ValueError, match="x_fp8 shape"):
        native.fp8_quant_tensor_fwd(F(4, 8), F(4, 9, dtype=e4), F(1, dtype=torch.float32), None, "e4m3")
    with pytest.raises(ValueError, match="scale must be float32"):
        native.fp8_quant_tensor_fwd(F(4, 8), F(4, 8, dtype=e4), F(1), None, "e4m3")
    with pytest.raises(ValueError, match=r"scale shape \[3\] must be \[4\]"):
        native.fp8_quant_token_fwd(F(4, 8), F(4, 8, dtype=e4), F(3, dtype=torch.float32), "e4m3")
    with pytest.raises(ValueError, match="x_fp8 shape"):
        native.fp8_quant_static_fwd(F(4, 8), F(4, 9, dtype=e4), 0.05, "e4m3")


def test_moe_permutation_checks():
    i64 = torch.int64
    with pytest.raises(ValueError, match="topk_indices must be 2-D"):
        native.moe_permutation_fwd(F(8, dtype=i64), F(8, dtype=i64), F(8, dtype=i64), 16)
    with pytest.raises(ValueError, match=r"permute_index shape \[7\] must be \[8\]"):
        native.moe_permutation_fwd(F(4, 2, dtype=i64), F(7, dtype=i64), F(4, 2, dtype=i64), 16)
    with pytest.raises(ValueError, match="unpermute_index shape"):
        native.moe_permutation_fwd(F(4, 2, dtype=i64), F(8, dtype=i64), F(2, 4, dtype=i64), 16)
    for bad in (0, 257):
        with pytest.raises(ValueError, match=r"num_experts \(\d+\) must be in \[1, 256\]"):
            native.moe_permutation_fwd(F(4, 2, dtype=i64), F(8, dtype=i64), F(4, 2, dtype=i64), bad)
    with pytest.raises(ValueError, match="must be int64"):
        native.moe_permutation_fwd(F(4, 2, dtype=torch.int32), F(8, dtype=i64), F(4, 2, dtype=i64), 16)
    with pytest.raises(ValueError, match="must be a CUDA tensor"):
        kernels.compute_permutation(torch.zeros(4, 2, dtype=i64), 16)


def test_fused_checks():
    e4 = torch.float8_e4m3fn
    with pytest.raises(ValueError, match="scale must be a float32 tensor"):
        native.rmsnorm_residual_fp8_fwd(F(2, 8), F(2, 8), F(8), F(2, 8, dtype=e4), None, F(2, 8), 1e-5, "e4m3", None)
    with pytest.raises(ValueError, match=r"scale shape \[3\] must be \[2\]"):
        native.rmsnorm_residual_fp8_fwd(F(2, 8), F(2, 8), F(8), F(2, 8, dtype=e4), F(3, dtype=torch.float32), F(2, 8),
                                        1e-5, "e4m3", None)
    with pytest.raises(ValueError, match="y_fp8 dtype"):
        native.swiglu_fp8_fwd(F(2, 8), F(2, 8), F(2, 8), None, "e4m3", 0.05)
    with pytest.raises(ValueError, match="dtype mismatch: 'up'"):
        native.swiglu_fp8_fwd(F(2, 8), F(2, 8, dtype=torch.float16), F(2, 8, dtype=e4), None, "e4m3", 0.05)
    with pytest.raises(ValueError):
        kernels.swiglu_fp8(torch.randn(2, 8), torch.randn(2, 8), "e4m3")
    with pytest.raises(ValueError, match="fp8_format"):
        kernels.rmsnorm_residual_fp8(torch.randn(2, 8), torch.randn(2, 8), torch.randn(8), fp8_format="x")


def test_python_api_argument_errors():
    with pytest.raises(ValueError, match="granularity must be"):
        kernels.fp8_quant(torch.randn(4, 8), "e4m3", "row")
    with pytest.raises(ValueError, match="static scale is per-tensor"):
        kernels.fp8_quant(torch.randn(4, 8), "e4m3", "token", scale=0.1)


def test_token_permute_checks():
    """src/kernels/token_permute.rs:45-201 validation branches, in order."""
    i64 = torch.int64
    _raises(native.token_gather_fwd, F(8, 16), F(4, dtype=torch.int32), F(4, 16), match="indices must be int64")
    _raises(native.token_gather_fwd, F(8, 16), F(4, dtype=i64), F(4, 16, dtype=torch.float16), match="dtype mismatch")
    _raises(native.token_gather_fwd, F(8, 16, 2), F(4, dtype=i64), F(4, 16), match="src and dst must be 2-D")
    _raises(native.token_gather_fwd, F(8, 16), F(4, dtype=i64), F(4, 15), match="hidden dim")
    _raises(native.token_gather_fwd, F(8, 16), F(5, dtype=i64), F(4, 16), match=r"indices shape \[5\] must be \[4\]")
    _raises(native.token_gather_fwd, F(8, 16), F(4, 1, dtype=i64), F(4, 16), match="indices shape")
    c = native.token_combine_fwd
    _raises(c, F(8, 16), F(4, 2, dtype=i64), F(4, 2, dtype=torch.float16), F(4, 16), match="weights must be float32")
    _raises(c, F(8, 16), F(4, 2, dtype=i64), F(4, 2, dtype=torch.float32), F(4, 16, dtype=torch.float32),
            match="dtype mismatch")
    _raises(c, F(8, 16, 1), F(4, 2, dtype=i64), F(4, 2, dtype=torch.float32), F(4, 16), match="must be 2-D")
    _raises(c, F(8, 16), F(4, 2, dtype=i64), F(4, 2, dtype=torch.float32), F(4, 8), match="hidden dim")
    _raises(c, F(8, 16), F(8, dtype=i64), F(4, 2, dtype=torch.float32), F(4, 16), match=r"must be 2-D \[T, k\]")
    _raises(c, F(8, 16), F(4, 2, dtype=i64), F(4, 3, dtype=torch.float32), F(4, 16), match="weights shape")
    _raises(c, F(8, 16), F(4, 2, dtype=i64), F(4, 2, dtype=torch.float32), F(5, 16), match="row count")


def test_moe_router_checks():
    """src/kernels/moe_router.rs:36-116 validation branches, in order."""
    r = native.moe_router_fwd
    i64 = torch.int64
    _raises(r, F(4, 8), F(4, 2, dtype=torch.float16), F(4, 2, dtype=i64), True, match="topk_weights must be float32")
    _raises(r, F(4, 8), F(4, 2, dtype=torch.float32), F(4, 2, dtype=torch.int32), True, match="must be int64")
    _raises(r, F(4, 8, 1), F(4, 2, dtype=torch.float32), F(4, 2, dtype=i64), True, match="logits must be 2-D")
    _raises(r, F(4, 8), F(3, 2, dtype=torch.float32), F(4, 2, dtype=i64), True, match=r"must be \[4, k\]")
    _raises(r, F(4, 8), F(4, 2, dtype=torch.float32), F(4, 3, dtype=i64), True, match="topk_indices shape")
    with pytest.raises(RuntimeError, match=r"k \(9\) must be <= num_experts \(8\)"):
        r(F(4, 8), F(4, 9, dtype=torch.float32), F(4, 9, dtype=i64), True)
    _raises(r, F(4, 300), F(4, 2, dtype=torch.float32), F(4, 2, dtype=i64), True, match="maximum of 256")


def test_header_is_plain_c_and_links(tmp_path):
    """A C99 program (the way cgo, a Rust -sys crate or any C host sees the
    boundary) includes the header, links libcustom_kernels_amd.so, and gets
    0 for empty work and 1 for an unknown tag from a few launchers, with no
    GPU: those paths return before any device call."""
    import os
    import shutil
    import subprocess

    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    src = tmp_path / "abi.c"
    src.write_text(r"""
#include <stdio.h>
#include "custom_kernels_amd.h"
int main(void) {
  int bad = 0;
  bad |= launch_rmsnorm_residual_fwd(0, 0, 0, 0, 0, 0, 4096, 1e-5f, CCK_DTYPE_BF16, 0) != 0;
  bad |= launch_swiglu_fwd(0, 0, 0, 0, CCK_DTYPE_BF16, 0) != 0;
  bad |= launch_fp8_quant_token_fwd(0, 0, 0, 0, 16, CCK_DTYPE_BF16, CCK_DTYPE_F8E4M3, 0) != 0;
  bad |= launch_swiglu_fp8_fwd(0, 0, 0, 0, 4, 16, 0.f, 7, CCK_DTYPE_BF16, CCK_DTYPE_F8E4M3, 0) != 1;
  bad |= launch_moe_router_fwd(0, 0, 0, 4, 300, 2, CCK_DTYPE_F32, 1, 0) != 1;
  printf("%s\n", bad ? "FAIL" : "OK");
  return bad;
}
""")
    lib_dir = os.path.dirname(_cck.LIB_PATH)
    include_dir = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include")
    exe = tmp_path / "abi"
    subprocess.run([cc, "-std=c99", "-Wall", "-Werror", f"-I{include_dir}", str(src), f"-L{lib_dir}",
                    "-lcustom_kernels_amd", f"-Wl,-rpath,{lib_dir}", "-o", str(exe)], check=True)
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert run.returncode == 0 and run.stdout.strip() == "OK", run.stdout + run.stderr


def test_noalloc_poll_limit_hook_is_host_state():
    """The one-pass per-tensor kernel's poll limit: a host-side setting (no
    device call), default 65536, returned on change and restorable."""
    lib = _cck.load()
    prev = lib.cck_fp8_tensor_noalloc_poll_limit(-1)
    assert prev == 2048
    assert lib.cck_fp8_tensor_noalloc_poll_limit(17) == prev
    assert lib.cck_fp8_tensor_noalloc_poll_limit(-1) == 17
    assert lib.cck_fp8_tensor_noalloc_poll_limit(prev) == 17
