"""Fused RMSNorm+FP8 and SwiGLU+FP8 kernels against the composed eager oracle
(the eager op of baselines/rmsnorm_residual.py:123-136 or baselines/swiglu.py:107-112,
then the per-row or static quantisation of baselines/fp8_quant.py:162-178
applied to its output as stored in its dtype).

* RMSNorm+FP8, every dtype: codes and scales bit-exact against the composed
  eager oracle (the kernel's y equals the eager y bit for bit), and
  residual_out bit-exact;
* SwiGLU+FP8, every dtype: codes and scales bit-exact against the composed
  eager oracle (fp32 with torch-CPU's vectorised float32 sigmoid,
  oracle/sigmoid.py).
Workloads: BASELINE configs 3v and 5 (per-token and static 0.05) at full size,
plus small and ragged shapes in all dtypes / formats.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from custom_cuda_kernals_amd.kernels import rmsnorm_residual, rmsnorm_residual_fp8, swiglu, swiglu_fp8
from oracle import eager, inputs
from oracle import fp8 as ofp8
from tests._parity import assert_codes_equal, assert_f32_bits_equal, bits_equal, codes_np

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.float16, torch.bfloat16]


def _quant(y: torch.Tensor, fmt, static):
    y2 = y.float().cpu().numpy().reshape(-1, y.shape[-1])
    if static is None:
        return ofp8.quant_token(y2, fmt)
    return ofp8.quant_static(y2, static, fmt), np.array([static], dtype=np.float32)


def _scales_ref(s_ref, static):
    return s_ref if static is None else np.array([static], dtype=np.float32)


def _check_rms(x, r, w, eps, fmt, static):
    xd, rd, wd = x.cuda(), r.cuda(), w.cuda()
    q, s, ro = rmsnorm_residual_fp8(xd, rd, wd, eps, fp8_format=fmt, scale=static)
    strict, s_ref, ro_ref, _ = eager.rmsnorm_residual_fp8(x, r, w, eps, fmt, static)
    n_bad = int((codes_np(q).reshape(strict.shape) != strict).sum())
    print(f"\nrmsnorm+fp8 {tuple(x.shape)} {x.dtype} {fmt} static={static}: "
          f"{n_bad} of {strict.size} codes differ from the composed eager oracle")
    assert_codes_equal(q, strict.reshape(q.shape))
    s_ref = _scales_ref(s_ref, static)
    assert_f32_bits_equal(s, s_ref.reshape(s.shape) if static is None else s_ref)
    assert bits_equal(ro, ro_ref).all()


def _check_swiglu(g, u, fmt, static):
    gd, ud = g.cuda(), u.cuda()
    q, s = swiglu_fp8(gd, ud, fp8_format=fmt, scale=static)
    strict, s_strict, y_ref = eager.swiglu_fp8(g, u, fmt, static)
    qn = codes_np(q).reshape(strict.shape)
    n_bad = int((qn != strict).sum())
    print(f"\nswiglu+fp8 {tuple(g.shape)} {g.dtype} {fmt} static={static}: "
          f"{n_bad} of {strict.size} codes differ from the composed eager oracle")
    assert_codes_equal(q, strict.reshape(q.shape))
    s_strict = _scales_ref(s_strict, static)
    assert_f32_bits_equal(s, s_strict.reshape(s.shape) if static is None else s_strict)


@pytest.mark.parametrize("static", [None, 0.05])
@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("shape", [(64, 4096), (17, 100), (3, 40000), (5, 11008)], ids=lambda s: f"{s[0]}x{s[1]}")
def test_rmsnorm_fp8_small(shape, dtype, fmt, static):
    x, r, w = inputs.rmsnorm_inputs(*shape, dtype, seed=shape[1])
    _check_rms(x, r, w, 1e-5, fmt, static)


@pytest.mark.parametrize("static", [None, 0.05])
@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("shape", [(64, 14336), (17, 100), (3, 40000), (5, 11008)], ids=lambda s: f"{s[0]}x{s[1]}")
def test_swiglu_fp8_small(shape, dtype, fmt, static):
    g, u = inputs.swiglu_inputs(*shape, dtype, seed=shape[1])
    if static is not None:
        g = g * 3  # push some |y| / 0.05 past the e4m3 range (NaN codes)
    _check_swiglu(g, u, fmt, static)


# Row lengths that reach every register-resident shape of both kernels (the
# largest row each shape holds, and one vector past some of them).
BUCKET_COLS = [64, 512, 1024, 2048, 2056, 2560, 3072, 3584, 4096, 5120, 6144, 6152, 7176, 8192, 9216, 10240, 12288,
               16384, 20480, 24576, 28672, 32768, 40960, 53248, 65536]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16], ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("cols", BUCKET_COLS)
def test_every_row_shape_bucket(cols, dtype):
    x, r, w = inputs.rmsnorm_inputs(3, cols, dtype, seed=cols)
    _check_rms(x, r, w, 1e-5, "e4m3", None)
    _check_rms(x, r, w, 1e-5, "e4m3", 0.05)
    g, u = inputs.swiglu_inputs(3, cols, dtype, seed=cols + 1)
    _check_swiglu(g, u, "e4m3", None)


@pytest.mark.parametrize("shape", [(513, 20480), (512, 20480), (600, 22528), (600, 22536), (257, 30720),
                                   (257, 30728), (256, 28672)], ids=lambda s: f"{s[0]}x{s[1]}")
def test_swiglu_fp8_parked_row_edges(shape):
    """bf16 per-token rows of 1024 x 3 and 1024 x 4 vectors park y in LDS
    on a looping grid only when there are more rows than resident
    workgroups and at most 3/4 of the threads hold a last vector: row counts
    and lengths on both sides of those two edges."""
    g, u = inputs.swiglu_inputs(*shape, torch.bfloat16, seed=shape[1] + shape[0])
    _check_swiglu(g, u, "e4m3", None)


def _nan_aware_equal(got: np.ndarray, want: np.ndarray, nan_of) -> None:
    """Equal bit for bit, except that NaNs (as `nan_of` tells them) only need
    to be NaN on both sides: the sign of a NaN is not pinned (see the test
    below)."""
    gn, wn = nan_of(got), nan_of(want)
    assert np.array_equal(gn, wn), "NaN positions differ"
    assert np.array_equal(got[~wn], want[~wn]), "non-NaN values differ"


@pytest.mark.parametrize("shape", [(1200, 12288), (64, 4096)], ids=lambda s: f"{s[0]}x{s[1]}")
def test_rmsnorm_fp8_non_finite_rows(shape):
    """Per-token RMSNorm + FP8 with NaN and infinite inputs / residuals in a few
    rows (rows looping on a resident grid, and one workgroup per row): codes,
    scales and residual_out equal the composed eager oracle bit for bit, NaNs
    compared as NaN."""
    x, r, w = inputs.rmsnorm_inputs(*shape, torch.bfloat16, seed=shape[1] + 11)
    x[2, 7] = float("nan")
    r[4, 100] = float("inf")
    x[6, 3] = float("-inf")
    q, s, ro = rmsnorm_residual_fp8(x.cuda(), r.cuda(), w.cuda(), 1e-5, fp8_format="e4m3")
    strict, s_ref, ro_ref, _ = eager.rmsnorm_residual_fp8(x, r, w, 1e-5, "e4m3", None)
    _nan_aware_equal(codes_np(q).reshape(strict.shape), strict, lambda c: (c & 0x7F) == 0x7F)
    _nan_aware_equal(s.cpu().numpy().view(np.uint32), np.asarray(s_ref, dtype=np.float32).reshape(-1).view(np.uint32),
                     lambda b: (b & 0x7FFFFFFF) > 0x7F800000)
    _nan_aware_equal(ro.cpu().view(torch.int16).numpy(), ro_ref.view(torch.int16).numpy(),
                     lambda b: (b & 0x7FFF) > 0x7F80)
    assert ((codes_np(q).reshape(strict.shape) & 0x7F) == 0x7F).any(axis=1).sum() >= 3


@pytest.mark.parametrize("shape", [(600, 22528), (64, 14336)], ids=lambda s: f"{s[0]}x{s[1]}")
def test_swiglu_fp8_non_finite_rows(shape):
    """Per-token SwiGLU + FP8 with NaN and infinite gates / ups in a few rows
    (parked rows on a looping grid, and register rows): codes and scales equal
    the composed eager oracle bit for bit, the non-finite rows included."""
    g, u = inputs.swiglu_inputs(*shape, torch.bfloat16, seed=shape[1] + 7)
    g[3, 100] = float("nan")
    u[5, 2000] = float("inf")
    g[9, 17] = float("-inf")
    g[11, shape[1] - 1] = float("inf")
    u[11, 5] = 0.0
    q, s = swiglu_fp8(g.cuda(), u.cuda(), fp8_format="e4m3")
    strict, s_ref, _ = eager.swiglu_fp8(g, u, "e4m3", None)
    got = codes_np(q).reshape(strict.shape)
    # NaN codes: the sign of a NaN y is not pinned (torch-CPU writes a NaN bf16
    # as 0xffff in its vectorised conversion and 0x7fc0 in its scalar one), so
    # NaN codes (0x7f / 0xff) compare as NaN; every other code bit for bit.
    want_nan = (strict & 0x7F) == 0x7F
    assert np.array_equal((got & 0x7F) == 0x7F, want_nan)
    assert np.array_equal(got[~want_nan], strict[~want_nan])
    assert int(want_nan.sum()) > 0 and (want_nan.sum(axis=1) > 0).sum() >= 3
    s_got, s_want = s.cpu().numpy(), np.asarray(s_ref, dtype=np.float32).reshape(-1)
    assert np.array_equal(np.isnan(s_got), np.isnan(s_want))
    fin = ~np.isnan(s_want)
    assert np.array_equal(s_got[fin].view(np.uint32), s_want[fin].view(np.uint32))


def test_config3v_swiglu_fp8_full_size():
    g, u = inputs.swiglu_inputs(*inputs.CONFIG_SHAPES["swiglu"], torch.bfloat16, seed=0)
    _check_swiglu(g, u, "e4m3", None)


@pytest.mark.parametrize("static", [None, inputs.STATIC_SCALE])
def test_config5_chain_full_size(static):
    x, r, w = inputs.rmsnorm_inputs(*inputs.CONFIG_SHAPES["chain_rmsnorm"], torch.bfloat16, seed=0)
    _check_rms(x, r, w, inputs.RMS_EPS, "e4m3", static)
    del x, r, w
    g, u = inputs.swiglu_inputs(*inputs.CONFIG_SHAPES["chain_swiglu"], torch.bfloat16, seed=1)
    _check_swiglu(g, u, "e4m3", static)


def test_fused_rejections():
    x = torch.randn(4, 8, device="cuda")
    with pytest.raises(ValueError):
        rmsnorm_residual_fp8(x, x, torch.randn(8, device="cuda"), fp8_format="e3m4")
    with pytest.raises(ValueError):
        swiglu_fp8(x, torch.randn(4, 8, device="cuda", dtype=torch.float16))


def test_every_bf16_gate_fused_table_rows():
    """Rows of 16384 (the LDS-table resident kernel) holding every finite bf16
    gate value, shuffled, with random up: codes and scales equal the
    quantised unfused output, per-token and static."""
    import numpy as np

    bits = np.arange(1 << 16, dtype=np.uint16)
    bits[(bits & 0x7FFF) >= 0x7F80] = 0  # finite gates only, so row scales stay finite
    g = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16)
    gen = torch.Generator().manual_seed(11)
    g = g.repeat(4)[torch.randperm(4 << 16, generator=gen)].view(16, 16384)
    u = torch.randn(16, 16384, generator=gen).to(torch.bfloat16)
    for static in (None, 0.05):
        _check_swiglu(g, u, "e4m3", static)


@pytest.mark.parametrize("static", [None, 0.05])
@pytest.mark.parametrize("dtype,shape", [
    (torch.bfloat16, (1000, 12288)), (torch.bfloat16, (700, 16384)), (torch.bfloat16, (600, 24576)),
    (torch.bfloat16, (300, 32768)), (torch.float16, (700, 16384)), (torch.float32, (900, 8192)),
    (torch.float32, (500, 16384))], ids=lambda v: str(v).split(".")[-1] if isinstance(v, torch.dtype) else f"{v[0]}x{v[1]}")
def test_rmsnorm_fp8_wide_rows_every_row(dtype, shape, static):
    """Wide RMSNorm + FP8 rows run on a grid of the workgroups the device
    holds at once, each looping over rows with the weight held: every row
    checked, with grids that loop once or more and a partial last round."""
    x, r, w = inputs.rmsnorm_inputs(*shape, dtype, seed=shape[1] + 1)
    _check_rms(x, r, w, 1e-5, "e4m3", static)


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("shape", [(600, 40960), (300, 65536), (257, 53248), (1000, 36872)],
                         ids=lambda s: f"{s[0]}x{s[1]}")
def test_swiglu_fp8_bf16_lds_rows_every_row(shape, fmt):
    """bf16 rows with y parked in LDS run on a grid of the workgroups the
    device holds at once (one per CU), each looping over rows with the next
    row's loads issued before the amax reduction: every row checked, grids
    that loop once, twice and with a partial last round."""
    g, u = inputs.swiglu_inputs(*shape, torch.bfloat16, seed=shape[0])
    _check_swiglu(g, u, fmt, None)


@pytest.mark.parametrize("static", [None, 0.05])
@pytest.mark.parametrize("shape", [(77, 14336), (9, 20008), (130, 8200)], ids=lambda s: f"{s[0]}x{s[1]}")
def test_swiglu_fp8_table_paths_ragged(shape, static):
    """bf16 shapes on the LDS-table kernels with partial tiles: rows of
    1024 x 2 and 1024 x 4 vectors (per-token) and a static stream whose length
    is not a multiple of the 16384-element tile."""
    g, u = inputs.swiglu_inputs(*shape, torch.bfloat16, seed=shape[1])
    _check_swiglu(g, u, "e4m3", static)
