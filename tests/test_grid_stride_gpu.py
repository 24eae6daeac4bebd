"""More rows (tokens) than the row kernels' workgroup cap, kMaxRowGroups =
65536 (custom_cuda_kernals_amd/csrc/launch.hpp), so that workgroups loop over
rows blockIdx.x, blockIdx.x + 65536, ...: the loop itself, the next-row
prefetch of the FP8 kernels and the alternating LDS reduction buffers all
run. With 2 * 65536 + 37 rows the first 37 workgroups take three rows.

Two checks per op:
* narrow rows against the oracle, with the per-op tests' helpers and bars;
* the config row length (so the config's register-resident kernel loops),
  bit for bit against the same op run over row slices of at most 65536 rows,
  where every workgroup takes one row: the assignment of rows to workgroups
  must not change an output bit.
"""

from __future__ import annotations

import pytest
import torch

from custom_cuda_kernals_amd.kernels import (fp8_quant, moe_router, rmsnorm_residual, rmsnorm_residual_fp8, rope,
                                             swiglu_fp8, token_combine, token_gather)
from oracle import inputs, moe
from tests._parity import bits_equal
from tests.test_fp8_quant_gpu import _check as check_fp8
from tests.test_fused_fp8_gpu import _check_rms, _check_swiglu
from tests.test_moe_router_gpu import _check as check_router
from tests.test_rmsnorm_residual_gpu import _run as run_rmsnorm
from tests.test_rope_gpu import _run as run_rope
from tests.test_token_permute_gpu import _check_combine

pytestmark = pytest.mark.gpu

CAP = 65536
ROWS = 2 * CAP + 37
BF16 = torch.bfloat16


def _slices(n: int):
    return [(a, min(a + CAP, n)) for a in range(0, n, CAP)]


_INT_OF_SIZE = {1: torch.uint8, 2: torch.int16, 4: torch.int32, 8: torch.int64}


def _same(a: torch.Tensor, b: torch.Tensor) -> bool:
    """Bit equality (NaN payloads included)."""
    return a.shape == b.shape and torch.equal(a.detach().view(_INT_OF_SIZE[a.element_size()]),
                                              b.detach().view(_INT_OF_SIZE[b.element_size()]))


def _randn(*shape, dtype=BF16, seed=0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return torch.randn(shape, device="cuda", dtype=torch.float32, generator=g).to(dtype)


@pytest.mark.parametrize("dtype", [BF16, torch.float32], ids=["bfloat16", "float32"])
def test_rmsnorm_oracle(dtype):
    x, r, w = inputs.rmsnorm_inputs(ROWS, 64, dtype, seed=11)
    run_rmsnorm(x, r, w, 1e-6)


@pytest.mark.parametrize("static", [None, 0.05])
def test_rmsnorm_fp8_oracle(static):
    x, r, w = inputs.rmsnorm_inputs(ROWS, 64, BF16, seed=12)
    _check_rms(x, r, w, 1e-5, "e4m3", static)


@pytest.mark.parametrize("mode", ["plain", "token", "static"])
def test_rmsnorm_config_rows_equal_sliced(mode):
    cols = 4096
    x, r = _randn(ROWS, cols, seed=1), _randn(ROWS, cols, seed=2)
    w = (1.0 + 0.1 * _randn(cols, dtype=torch.float32, seed=3)).to(BF16)

    def op(a, b):
        if mode == "plain":
            return rmsnorm_residual(a, b, w, 1e-5)
        return rmsnorm_residual_fp8(a, b, w, 1e-5, fp8_format="e4m3", scale=0.05 if mode == "static" else None)

    whole = op(x, r)
    parts = [op(x[a:b], r[a:b]) for a, b in _slices(ROWS)]
    for i, t in enumerate(whole):
        if mode == "static" and i == 1:
            continue  # the static scale is returned as given
        joined = torch.cat([p[i] for p in parts])
        assert _same(t, joined), f"output {i} depends on the row-to-workgroup assignment"


def test_fp8_token_oracle():
    x = inputs.randn((ROWS, 64), BF16, seed=13)
    check_fp8(x, "e4m3", "token")


def test_fp8_token_config_rows_equal_sliced():
    x = _randn(ROWS, 4096, seed=4)
    x.view(-1)[:: 997] *= 50
    q, s = fp8_quant(x, "e4m3", "token")
    parts = [fp8_quant(x[a:b], "e4m3", "token") for a, b in _slices(ROWS)]
    assert _same(q, torch.cat([p[0] for p in parts]))
    assert _same(s, torch.cat([p[1] for p in parts]))


@pytest.mark.parametrize("static", [None, 0.05])
def test_swiglu_fp8_oracle(static):
    g, u = inputs.swiglu_inputs(ROWS, 64, BF16, seed=14)
    _check_swiglu(g, u, "e4m3", static)


@pytest.mark.parametrize("static", [None, 0.05])
def test_swiglu_fp8_config_rows_equal_sliced(static):
    rows, cols = CAP + 37, 14336
    g, u = _randn(rows, cols, seed=5), _randn(rows, cols, seed=6)
    q, s = swiglu_fp8(g, u, fp8_format="e4m3", scale=static)
    parts = [swiglu_fp8(g[a:b], u[a:b], fp8_format="e4m3", scale=static) for a, b in _slices(rows)]
    assert _same(q, torch.cat([p[0] for p in parts]))
    if static is None:
        assert _same(s, torch.cat([p[1] for p in parts]))


def test_rope_oracle():
    run_rope((1, ROWS, 1, 1, 128), BF16, 500000.0, inplace=True, seed=15)


def test_rope_config_heads_equal_sliced():
    hq, hkv, d = 32, 8, 128
    q, k = _randn(1, ROWS, hq, d, seed=7), _randn(1, ROWS, hkv, d, seed=8)
    cos, sin = _randn(ROWS, d // 2, dtype=torch.float32, seed=9), _randn(ROWS, d // 2, dtype=torch.float32, seed=10)
    qo, ko = rope(q, k, cos, sin)
    for a, b in _slices(ROWS):
        qs, ks = rope(q[:, a:b], k[:, a:b], cos[a:b], sin[a:b])
        assert _same(qo[:, a:b], qs) and _same(ko[:, a:b], ks)


def test_token_gather_oracle():
    # The gather takes four destination rows per workgroup: 4 * 65536 + 151
    # rows make it loop, and leave a partial group of three at the end.
    src, idx = inputs.gather_inputs(1000, 4 * CAP + 151, 64, BF16, seed=16)
    out = token_gather(src.cuda(), idx.cuda()).cpu()
    assert bits_equal(out, moe.token_gather(src, idx)).all()


def test_token_combine_oracle():
    eo, ui, w = inputs.combine_inputs(ROWS, 2, 64, BF16, seed=17)
    _check_combine(eo, ui, w)


def test_moe_router_oracle():
    check_router(inputs.router_inputs(4 * CAP + 37, 16, torch.float32, seed=18), 2, True)
