"""Inputs past 2^31 elements, in buffers past 4 GiB: every op family at such a
size, against the CPU oracle on slices at the start, across element 2^31 and
at the end. The ops are elementwise or per row (per token), so a slice's
output depends only on the slice's inputs and the oracle runs on the slice
alone; the per-tensor maximum is planted past element 2^31, so the tensor's
scale is known without reducing it on the CPU. This is the "maximum sizes"
edge case: 64-bit offsets, grids capped and looping over rows or vectors.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from custom_cuda_kernals_amd.kernels import (fp8_quant, rmsnorm_residual, rmsnorm_residual_fp8, rope, swiglu,
                                             swiglu_fp8, token_combine, token_gather)
from oracle import eager, moe
from oracle import fp8 as ofp8
from tests._parity import assert_codes_equal, assert_f32_bits_equal, bits_equal

pytestmark = pytest.mark.gpu

BIG = 1 << 31


@pytest.fixture(autouse=True)
def _free_device_memory():
    yield
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def _randn(shape, seed, dtype=torch.bfloat16):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return torch.randn(shape, dtype=dtype, device="cuda", generator=g)


def _row_slices(rows: int, cols: int, width: int = 48) -> list[slice]:
    """Rows at the start, the rows holding element 2^31 and the last rows."""
    mid = BIG // cols
    return [slice(0, width), slice(mid - width // 2, mid + width // 2), slice(rows - width, rows)]


def _flat_slices(n: int, width: int = 1 << 16) -> list[slice]:
    return [slice(0, width), slice(BIG - width // 2, BIG + width // 2), slice(n - width, n)]


def _scale_bits(v: float) -> np.ndarray:
    return np.array([v], dtype=np.float32)


def test_swiglu_flat_past_2g():
    """One flat stream of 2^31 + 8005 elements: the vector grid loops, and a
    scalar tail follows the last whole vector."""
    n = BIG + 8 * 1000 + 5
    gate, up = _randn((n,), 1), _randn((n,), 2)
    y = swiglu(gate, up)
    torch.cuda.synchronize()
    for s in _flat_slices(n):
        ref = eager.swiglu(gate[s].cpu(), up[s].cpu())
        assert bits_equal(y[s].cpu(), ref).all(), s


@pytest.mark.parametrize("static", [None, 0.05], ids=["token", "static"])
def test_swiglu_fp8_rows_past_2g(static):
    rows, cols = 149_800, 14_336  # 2,147,532,800 elements
    gate, up = _randn((rows, cols), 3), _randn((rows, cols), 4)
    q, s = swiglu_fp8(gate, up, "e4m3", scale=static)
    torch.cuda.synchronize()
    for r in _row_slices(rows, cols):
        codes, s_ref, _ = eager.swiglu_fp8(gate[r].cpu(), up[r].cpu(), "e4m3", static)
        assert_codes_equal(q[r], codes, f"codes rows {r}")
        if static is None:
            assert_f32_bits_equal(s[r], s_ref, f"scales rows {r}")


def test_rmsnorm_residual_rows_past_2g():
    rows, cols = 524_300, 4096  # 2,147,532,800 elements; 65536-workgroup grid looping over rows
    x, r = _randn((rows, cols), 5), _randn((rows, cols), 6)
    w = (1.0 + 0.1 * _randn((cols,), 7, torch.float32)).to(torch.bfloat16)
    y, ro = rmsnorm_residual(x, r, w, 1e-5)
    torch.cuda.synchronize()
    w_cpu = w.cpu()
    for sl in _row_slices(rows, cols):
        y_ref, ro_ref = eager.rmsnorm_residual(x[sl].cpu(), r[sl].cpu(), w_cpu, 1e-5)
        assert bits_equal(ro[sl].cpu(), ro_ref).all(), f"residual_out rows {sl}"
        assert bits_equal(y[sl].cpu(), y_ref).all(), f"y rows {sl}"
    del y, ro
    q, s, ro = rmsnorm_residual_fp8(x, r, w, 1e-5, "e4m3")
    torch.cuda.synchronize()
    for sl in _row_slices(rows, cols):
        codes, s_ref, ro_ref, _ = eager.rmsnorm_residual_fp8(x[sl].cpu(), r[sl].cpu(), w_cpu, 1e-5, "e4m3")
        assert_codes_equal(q[sl], codes, f"codes rows {sl}")
        assert_f32_bits_equal(s[sl], s_ref, f"scales rows {sl}")
        assert bits_equal(ro[sl].cpu(), ro_ref).all(), f"residual_out rows {sl}"


def test_fp8_token_rows_past_2g():
    rows, cols = 524_300, 4096
    x = _randn((rows, cols), 8)
    q, s = fp8_quant(x, "e4m3", "token")
    torch.cuda.synchronize()
    for sl in _row_slices(rows, cols):
        codes, s_ref = ofp8.quant_token(x[sl].float().cpu().numpy(), "e4m3")
        assert_codes_equal(q[sl], codes, f"codes rows {sl}")
        assert_f32_bits_equal(s[sl], s_ref, f"scales rows {sl}")


def test_fp8_tensor_and_static_past_2g():
    """One dynamic scale over 2^31 + 49152 elements with the maximum planted
    past element 2^31: the Python API (no amax word), the reference ABI (the
    caller's int32 left holding the amax bits), the no-allocation entry point
    (the one-pass form streaming what its registers do not hold), and a
    static scale."""
    from tests import _cck

    rows, cols = 524_300, 4096
    x = _randn((rows, cols), 9)
    x[rows - 3, 7] = -1000.0
    s_ref = np.float32(1000.0) / np.float32(448.0)
    checks = _row_slices(rows, cols)

    def check(q, scale, what):
        assert_f32_bits_equal(scale, _scale_bits(s_ref), f"{what} scale")
        for sl in checks:
            assert_codes_equal(q[sl], ofp8.quant_static(x[sl].float().cpu().numpy(), float(s_ref), "e4m3"),
                               f"{what} codes rows {sl}")

    q, s = fp8_quant(x, "e4m3", "tensor")
    torch.cuda.synchronize()
    check(q, s, "python API")
    del q
    lib = _cck.load()
    stream = torch.cuda.current_stream().cuda_stream
    q = torch.empty((rows, cols), dtype=torch.uint8, device="cuda")
    s = torch.empty(1, dtype=torch.float32, device="cuda")
    word = torch.zeros(1, dtype=torch.int32, device="cuda")
    assert lib.launch_fp8_quant_tensor_fwd(x.data_ptr(), q.data_ptr(), s.data_ptr(), word.data_ptr(), rows, cols, 2, 3,
                                           stream) == 0
    torch.cuda.synchronize()
    check(q, s, "reference ABI")
    assert int(word.item()) == int(np.array([1000.0], dtype=np.float32).view(np.int32)[0])
    q.fill_(0)
    assert lib.launch_fp8_quant_tensor_noalloc_fwd(x.data_ptr(), q.data_ptr(), s.data_ptr(), rows, cols, 2, 3,
                                                   stream) == 0
    torch.cuda.synchronize()
    check(q, s, "no-allocation entry point")
    del q
    qs, _ = fp8_quant(x, "e4m3", "tensor", scale=0.05)
    torch.cuda.synchronize()
    for sl in checks:
        assert_codes_equal(qs[sl], ofp8.quant_static(x[sl].float().cpu().numpy(), 0.05, "e4m3"), f"static rows {sl}")


def test_rope_in_place_past_2g():
    """q of 2^31 + 65536 elements ([16, 32769, 32, 128]), rotated in place."""
    b, s, hq, hkv, d = 16, 32_769, 32, 8, 128
    q, k = _randn((b, s, hq, d), 10), _randn((b, s, hkv, d), 11)
    cos, sin = eager.compute_cos_sin(s, d, 500000.0)
    # (batch, positions): the first tokens, the tokens holding q's element 2^31, the last tokens
    t_mid = BIG // (hq * d)
    b_mid, s_mid = divmod(t_mid, s)
    spans = [(0, slice(0, 32)), (b_mid, slice(s_mid - 32, min(s, s_mid + 16))), (b - 1, slice(s - 32, s))]
    before = [(bi, sl, q[bi, sl].cpu(), k[bi, sl].cpu()) for bi, sl in spans]
    rope(q, k, cos.cuda(), sin.cuda(), inplace=True)
    torch.cuda.synchronize()
    for bi, sl, q0, k0 in before:
        q_ref, k_ref = eager.rope(q0[None], k0[None], cos[sl], sin[sl])
        assert bits_equal(q[bi, sl].cpu(), q_ref[0]).all(), f"q batch {bi} positions {sl}"
        assert bits_equal(k[bi, sl].cpu(), k_ref[0]).all(), f"k batch {bi} positions {sl}"


def test_token_gather_and_combine_past_2g():
    """Destination / expert-output buffers of 2,457,600,000 elements (600,000
    rows of 4096 bf16)."""
    n_src, n_dst, h = 300_000, 600_000, 4096
    g = torch.Generator(device="cuda").manual_seed(12)
    src = _randn((n_src, h), 13)
    idx = torch.randint(0, n_src, (n_dst,), device="cuda", dtype=torch.int64, generator=g)
    dst = token_gather(src, idx)
    torch.cuda.synchronize()
    src_cpu, idx_cpu = src.cpu(), idx.cpu()
    for sl in _row_slices(n_dst, h):
        assert bits_equal(dst[sl].cpu(), moe.token_gather(src_cpu, idx_cpu[sl])).all(), f"gather rows {sl}"
    del src, src_cpu
    t, k = n_dst // 2, 2
    unperm = torch.randperm(n_dst, device="cuda", generator=g).view(t, k)
    wts = torch.rand((t, k), device="cuda", dtype=torch.float32, generator=g)
    out = token_combine(dst, unperm, wts)
    torch.cuda.synchronize()
    eo_cpu, u_cpu, w_cpu = dst.cpu(), unperm.cpu(), wts.cpu()
    spans = [slice(0, 48), slice(t // 2 - 24, t // 2 + 24), slice(t - 48, t)]
    assert all((u_cpu[sl] >= BIG // h).any() for sl in spans), "each span reads expert rows past element 2^31"
    for sl in spans:
        # rows of 4096 elements, k = 2: torch's CPU sum adds in j order, as the kernel does
        ref = moe.token_combine(eo_cpu, u_cpu[sl], w_cpu[sl])
        assert bits_equal(out[sl].cpu(), ref).all(), f"combine tokens {sl}"
