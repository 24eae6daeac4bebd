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


def test_long_rows_two_reads_one_eight_byte_write():
    rows = 37
    n_vec = 1792 * rows
    a, b = _u32(n_vec, 6), _u32(n_vec, 7)
    c = torch.empty(n_vec * 2, dtype=torch.int32, device="cuda")
    _run(4, a, b, c, None, n_vec)
    x = (a.cpu().numpy().view(np.uint32) ^ b.cpu().numpy().view(np.uint32)).reshape(rows, 1792, 4)
    # partner word: word 0 of the first vector of wave (w ^ 1) of the first vector block (k = 0)
    t = np.arange(1024)
    words = x[:, (np.arange(16) * 64), 0]  # [row, wave]
    w = words[:, (t >> 6) ^ 1]  # [row, thread]
    expect = np.empty((rows, 1792, 2), dtype=np.uint32)
    for k in range(2):
        v = t + 1024 * k
        ok = v < 1792
        expect[:, v[ok], 0] = x[:, v[ok], 0] ^ w[:, ok]
        expect[:, v[ok], 1] = x[:, v[ok], 2]
    assert np.array_equal(c.cpu().numpy().view(np.uint32).reshape(rows, 1792, 2), expect)


@pytest.mark.parametrize("rows", [1, 37, 65573])
def test_rows_two_reads_two_writes_of_sixteen_and_eight_bytes(rows):
    n_vec = 512 * rows
    a, b = _u32(n_vec, 8), _u32(n_vec, 9)
    c = torch.empty_like(a)
    d = torch.empty(n_vec * 2, dtype=torch.int32, device="cuda")
    _run(5, a, b, c, d, n_vec)
    an = a.cpu().numpy().view(np.uint32).reshape(rows, 512, 4)
    bn = b.cpu().numpy().view(np.uint32).reshape(rows, 512, 4)
    assert np.array_equal(c.cpu().numpy().view(np.uint32).reshape(rows, 512, 4), an + bn)
    t = np.arange(256)
    words = an[:, np.arange(4) * 64, 0]  # [row, wave]: thread 64w's first vector (i0)
    w = words[:, (t >> 6) ^ 1]  # [row, thread]
    expect = np.empty((rows, 512, 2), dtype=np.uint32)
    for half in range(2):
        v = t + 256 * half
        expect[:, v, 0] = an[:, v, 0] ^ w
        expect[:, v, 1] = bn[:, v, 1]
    assert np.array_equal(d.cpu().numpy().view(np.uint32).reshape(rows, 512, 2), expect)
