"""The fp32 row-sum order of torch's CPU ``sum`` / ``mean`` over a contiguous
last dimension, restated in numpy. TEST INFRASTRUCTURE ONLY.

The reference's RMSNorm takes ``upcast.pow(2).mean(dim=-1, keepdim=True)``
(baselines/rmsnorm_residual.py:133). On the CPU, ``mean`` of a float tensor is
``sum`` followed by an in-place division by the row length, and ``sum`` of
float32 accumulates in float32 in a fixed, data-independent order. That order
decides the last bits of the variance, hence of ``rsqrt`` and of every output
element of the row, so the GPU kernel reproduces it; this module states it so
the tests can pin it against torch itself (tests/test_oracle_rowsum.py) and
so the kernel has a written specification.

The order (a fixed function of the row length n; x are the fp32 addends):

* vectors of W = 8 lanes: element e is lane e % 8 of vector V = e // 8, for
  the nv = n // 8 whole vectors (torch's 256-bit vectors: the sum kernel is
  dispatched at AVX2 width on AVX-512 hosts too);
* vector V = 4 i + k is step i of slot k (four independent accumulators),
  for i < s = nv // 4;
* per (slot, lane), steps are folded into acc0 from zero in blocks of
  2^P steps, P = max(4, ceil_log2(s) // 4) (ceil_log2(m) = 1 for m <= 2);
  after each whole block acc1 += acc0, acc0 = 0; after every 2^P blocks
  acc2 += acc1, acc1 = 0; after every 2^(2P) blocks acc3 += acc2, acc2 = 0;
  the trailing s % 2^P steps fold into acc0; then
  p = ((acc0 + acc1) + acc2) + acc3;
* the nv % 4 leftover vectors are added to slot 0 in order, then
  p0 = ((p0 + p1) + p2) + p3 (lane-wise);
* total = (((0 + the n % 8 trailing scalars, in order) + lane 0) + ...) + lane 7.

Rows shorter than 8 elements are summed as scalars with the same slot / fold
structure (4 slots of single elements, leftovers into slot 0).
"""

from __future__ import annotations

import numpy as np

F32 = np.float32
LANES = 8
SLOTS = 4


def ceil_log2(m: int) -> int:
    return 1 if m <= 2 else int(m - 1).bit_length()


def level_power(steps: int) -> int:
    return max(4, ceil_log2(steps) // 4)


def _fold_slots(vals: np.ndarray) -> np.ndarray:
    """vals [rows, steps, SLOTS, L] -> per-slot cascade sums [rows, SLOTS, L]."""
    rows, steps, slots, lanes = vals.shape
    p = level_power(steps)
    blk = 1 << p
    acc = np.zeros((4, rows, slots, lanes), dtype=F32)
    i = 0
    while i + blk <= steps:
        for _ in range(blk):
            acc[0] = acc[0] + vals[:, i]
            i += 1
        for lvl in range(1, 4):
            acc[lvl] = acc[lvl] + acc[lvl - 1]
            acc[lvl - 1] = 0
            if i & (((1 << p) - 1) << (lvl * p)):
                break
    while i < steps:
        acc[0] = acc[0] + vals[:, i]
        i += 1
    out = acc[0]
    for lvl in range(1, 4):
        out = out + acc[lvl]
    return out


def _slot_sum(units: np.ndarray) -> np.ndarray:
    """units [rows, m, L]: ATen's row_sum over m units with 4 slots -> [rows, L]."""
    rows, m, lanes = units.shape
    s = m // SLOTS
    p = _fold_slots(units[:, : s * SLOTS].reshape(rows, s, SLOTS, lanes))
    p0 = p[:, 0]
    for v in range(s * SLOTS, m):
        p0 = p0 + units[:, v]
    for k in range(1, SLOTS):
        p0 = p0 + p[:, k]
    return p0


def row_sum(x: np.ndarray) -> np.ndarray:
    """float32 [rows, n] -> float32 [rows], in torch-CPU's order (above)."""
    x = np.ascontiguousarray(x, dtype=F32)
    rows, n = x.shape
    if n < LANES:
        return F32(0) + _slot_sum(x.reshape(rows, n, 1))[:, 0]
    nv = n // LANES
    lanes = _slot_sum(x[:, : nv * LANES].reshape(rows, nv, LANES))
    total = np.zeros(rows, dtype=F32)
    for e in range(nv * LANES, n):
        total = total + x[:, e]
    for l in range(LANES):
        total = total + lanes[:, l]
    return total


def sum_of_squares(x: np.ndarray) -> np.ndarray:
    """Row sums of the fp32-rounded squares (``x.pow(2).sum(-1)``)."""
    x = np.asarray(x, dtype=F32)
    return row_sum(x * x)
