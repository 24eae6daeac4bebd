"""The HBM calibration streams (cck_hbm_stream) move the bytes they claim to:
each pattern's outputs are checked against the same function of its inputs
on the host, so the ceilings bench.py reports are ceilings of real traffic."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests import _cck

pytestmark = pytest.mark.gpu


def _u32(n_vec: int, seed: int) -> torch.Tensor:
    g = torch.Generator(device="cuda").manual_seed(seed)
    return torch.randint(0, 1 << 31, (n_vec * 4,), generator=g, device="cuda", dtype=torch.int64).to(torch.int32)


def _run(pattern, a, b, c, d, n_vec):
    lib = _cck.load()
    ptr = lambda t: None if t is None else t.data_ptr()
    rc = lib.cck_hbm_stream(pattern, ptr(a), ptr(b), ptr(c), ptr(d), n_vec, torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()


@pytest.mark.parametrize("n_vec", [1, 1000, 512 * 300])
def test_copy_and_two_read_streams(n_vec):
    a, b = _u32(n_vec, 1), _u32(n_vec, 2)
    c = torch.empty_like(a)
    _run(0, a, None, c, None, n_vec)
    assert torch.equal(c, a)
    _run(1, a, b, c, None, n_vec)
    assert torch.equal(c, a ^ b)


@pytest.mark.parametrize("rows", [1, 37, 70000])
def test_rows_with_barrier(rows):
    n_vec = 512 * rows
    a, b = _u32(n_vec, 3), _u32(n_vec, 4)
    c, d = torch.empty_like(a), torch.empty_like(a)
    _run(2, a, b, c, d, n_vec)
    an, bn = a.cpu().numpy().view(np.uint32), b.cpu().numpy().view(np.uint32)
    assert np.array_equal(c.cpu().numpy().view(np.uint32), an + bn)  # wraps mod 2^32 like the kernel
    # d = a ^ b ^ (word 0 of the first vector of the partner wave, 64 threads away)
    words = an.reshape(rows, 8, 64, 4)[:, :, 0, 0]  # [row, wave]
    partner = words[:, np.arange(8) ^ 1]
    expect = (an ^ bn).reshape(rows, 8, 64, 4) ^ partner[:, :, None, None]
    assert np.array_equal(d.cpu().numpy().view(np.uint32).reshape(rows, 8, 64, 4), expect)


def test_read16_write8_stream():
    n_vec = 4096
    a = _u32(n_vec, 5)
    c = torch.empty(n_vec * 2, dtype=torch.int32, device="cuda")
    _run(3, a, None, c, None, n_vec)
    an = a.cpu().numpy().view(np.uint32).reshape(n_vec, 4)
    expect = np.stack([an[:, 0] ^ an[:, 1], an[:, 2] ^ an[:, 3]], axis=1)
    assert np.array_equal(c.cpu().numpy().view(np.uint32).reshape(n_vec, 2), expect)
