"""Pins oracle.rowsum, the stated fp32 order of torch-CPU's row sum (CPU only).

* bit equality with torch's own ``x.sum(-1)`` and ``x.pow(2).mean(-1)`` on
  rows whose addends span many binades (so any other order shows), for every
  row length 1..80 and lengths that exercise each part of the order: the
  8-lane vectors and their scalar tail, the four slots and their leftovers,
  the 16-step blocks, the acc2 level (>= 256 steps) and the acc3 level
  (>= 4096 steps);
* a planted mistake (16-lane vectors, or the slots combined before the
  leftovers) disagrees with torch;
* the closed form on integer-valued addends (exact in any order): the sum of
  every element, so a dropped or repeated term fails.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import rowsum

LENGTHS = list(range(1, 81)) + [100, 127, 255, 256, 257, 511, 1000, 2048, 4095, 4096, 4104, 5120,
                                8192, 8200, 11008, 14336, 16384, 40000, 131072, 140008]


def _wide(rows: int, n: int, seed: int) -> np.ndarray:
    g = np.random.default_rng(seed)
    return (g.standard_normal((rows, n)) * np.exp(3.0 * g.standard_normal((rows, n)))).astype(np.float32)


def _torch_sum(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(x).sum(dim=-1).numpy()


@pytest.mark.parametrize("n", LENGTHS)
def test_row_sum_equals_torch(n):
    rows = 3 if n < 100000 else 2
    x = _wide(rows, n, seed=n)
    np.testing.assert_array_equal(rowsum.row_sum(x).view(np.uint32), _torch_sum(x).view(np.uint32))


@pytest.mark.parametrize("n", [7, 100, 4096, 14336])
def test_mean_of_squares_equals_torch(n):
    x = torch.randn(4, n, generator=torch.Generator().manual_seed(n)) * 3
    ref = x.pow(2).mean(dim=-1).numpy()
    mine = rowsum.sum_of_squares(x.numpy()) / np.float32(n)
    np.testing.assert_array_equal(mine.view(np.uint32), ref.view(np.uint32))


def test_planted_mistakes_disagree():
    x = _wide(8, 4096, seed=1)
    want = _torch_sum(x)

    def sixteen_lanes(a):
        nv = a.shape[1] // 16
        lanes = rowsum._slot_sum(a[:, : nv * 16].reshape(a.shape[0], nv, 16))
        t = np.zeros(a.shape[0], dtype=np.float32)
        for l in range(16):
            t = t + lanes[:, l]
        return t

    assert (sixteen_lanes(x) != want).any()
    y = _wide(8, 4096 + 24, seed=2)
    want_y = _torch_sum(y)

    def leftovers_last(a):
        rows = a.shape[0]
        nv = a.shape[1] // 8
        u = a[:, : nv * 8].reshape(rows, nv, 8)
        s = nv // 4
        p = rowsum._fold_slots(u[:, : s * 4].reshape(rows, s, 4, 8))
        p0 = ((p[:, 0] + p[:, 1]) + p[:, 2]) + p[:, 3]
        for v in range(s * 4, nv):
            p0 = p0 + u[:, v]
        t = np.zeros(rows, dtype=np.float32)
        for l in range(8):
            t = t + p0[:, l]
        return t

    assert (leftovers_last(y) != want_y).any()


@pytest.mark.parametrize("n", [5, 99, 4096, 40000])
def test_integer_addends_sum_exactly(n):
    g = np.random.default_rng(n)
    x = g.integers(-1000, 1000, size=(3, n)).astype(np.float32)
    np.testing.assert_array_equal(rowsum.row_sum(x), x.astype(np.float64).sum(axis=1).astype(np.float32))
