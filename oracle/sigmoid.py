"""torch-CPU's float32 sigmoid, restated in numpy. TEST INFRASTRUCTURE ONLY.

The reference's SwiGLU takes ``g32 * torch.sigmoid(g32)`` on a float32 copy
of the gate for every input dtype (baselines/swiglu.py:107-112), so its fp32
output is exactly torch's float32 sigmoid followed by two fp32 products. On
the CPU, torch evaluates sigmoid element-wise through ATen's vectorised loop
(the oracle's dependency: torch, here 2.10, ATen's CPU sigmoid kernel and the
SLEEF library it calls):

* vector path: ``r = 1 / (1 + exp(0 - x))`` with SLEEF's single-precision
  ``expf`` of 1.0-ulp accuracy (``xexpf``, the u10 variant, built with fused
  multiply-adds for AVX2 and AVX-512), the add and an IEEE division, lane by
  lane;
* scalar path: the elements a loop leaves over, ``n mod 2W`` at the end of
  each thread's chunk for a vector of W floats (16 with AVX-512, 8 with AVX2),
  take ``1 / (1 + std::exp(-x))``: libm's ``expf``, stated here as the
  correctly rounded exponential. glibc's ``expf`` is within 0.502 ulp, so it
  rounds the other way on a few inputs (measured: 20 of 93,000 sigmoids,
  0.02 %): this path is not pinned bit for bit ("parity unpinned" for those
  tail elements), only to that agreement.

SLEEF's ``xexpf`` (published in SLEEF's sources, ``sleefsimdsp.c``):
  q = rint(d * R_LN2);  s = fma(q, -L2U, d);  s = fma(q, -L2L, s);
  u = P(s) by Horner with fma, coefficients C0..C5;
  u = 1 + fma(s * s, u, s);  u = u * 2^(q >> 1) * 2^(q - (q >> 1));
  0 for d < -104, +inf for d > 100.
Every step is an IEEE float32 operation; ``fma32`` gives the correctly
rounded fused multiply-add through Boldo and Melquiond's round-to-odd: the
product of two floats is exact in float64, the float64 sum is made odd when
inexact, and rounding that to float32 is the correctly rounded result.

NaN inputs give NaN (their payload is not stated: a NaN gate propagates
itself through ``g * sigmoid(g)`` in torch, whatever the sigmoid's NaN is).

Pinned by tests/test_oracle_sigmoid.py: ``sigmoid_vector`` equals
``torch.sigmoid`` bit for bit on whole vectors over every float32 exponent
range, both signs, the special values and the thresholds; ``fma32`` equals
exact rational arithmetic; planted mistakes (separate multiply and add
instead of fma, the low part of ln 2 dropped) disagree with torch. The split
of a length-n input is checked against torch: the body bit for bit on the
vector path, the tail on the scalar path (which the vector path is not);
``sigmoid_scalar`` agrees with torch on at least 99.9 % of short inputs.
The GPU kernels follow the vector path for every element.
"""

from __future__ import annotations

import numpy as np

F32 = np.float32

# SLEEF xexpf constants (float32 literals)
R_LN2 = F32(1.442695040888963407359924681001892137426645954152985934135449406931)
L2U = F32(0.693145751953125)
L2L = F32(1.428606765330187045e-06)
POLY = (F32(0.000198527617612853646278381), F32(0.00139304355252534151077271), F32(0.00833336077630519866943359),
        F32(0.0416664853692054748535156), F32(0.166666671633720397949219), F32(0.5))


def fma32(a, b, c) -> np.ndarray:
    """Correctly rounded float32 a * b + c, element-wise."""
    a = np.asarray(a, F32).astype(np.float64)
    b = np.asarray(b, F32).astype(np.float64)
    c = np.asarray(c, F32).astype(np.float64)
    p = a * b  # exact: two 24-bit significands
    with np.errstate(over="ignore", invalid="ignore"):
        s = p + c
        bb = s - p
        err = (p - (s - bb)) + (c - bb)  # s + err == p + c exactly (TwoSum)
    bits = np.atleast_1d(s).view(np.uint64).copy()
    err = np.atleast_1d(err)
    s1 = np.atleast_1d(s)
    inexact_even = (err != 0) & np.isfinite(s1) & ((bits & np.uint64(1)) == 0)
    away = (err > 0) == (s1 > 0)  # the exact sum lies further from zero than s
    bits[inexact_even & away] += np.uint64(1)
    bits[inexact_even & ~away] -= np.uint64(1)
    out = bits.view(np.float64).astype(F32)
    return out.reshape(np.shape(s))


def _pow2i(q: np.ndarray) -> np.ndarray:
    return ((q.astype(np.int64) + 127) << 23).astype(np.uint32).view(F32)


def sleef_expf(d) -> np.ndarray:
    """SLEEF's xexpf (u10) on float32 d, element-wise."""
    d = np.asarray(d, F32)
    with np.errstate(over="ignore", invalid="ignore", under="ignore"):
        qf = np.rint((d * R_LN2).astype(F32))
        # q only matters where -104 <= d <= 100 (|q| <= 150); elsewhere the
        # result is replaced below, so q is clamped to stay representable.
        q = np.clip(np.where(np.isfinite(qf), qf, 0), -200, 200).astype(np.int64)
        qf = q.astype(F32)
        s = fma32(qf, -L2U, d)
        s = fma32(qf, -L2L, s)
        u = np.full(d.shape, POLY[0], dtype=F32)
        for c in POLY[1:]:
            u = fma32(u, s, c)
        u = (F32(1) + fma32((s * s).astype(F32), u, s)).astype(F32)
        h = q >> 1
        u = (u * _pow2i(h)).astype(F32)
        u = (u * _pow2i(q - h)).astype(F32)
        u = np.where(d < F32(-104), F32(0), u)
        u = np.where(F32(100) < d, F32(np.inf), u)
    return u.astype(F32)


def sigmoid_vector(x) -> np.ndarray:
    """torch-CPU's vector path: 1 / (1 + xexpf(0 - x)) in float32."""
    x = np.asarray(x, F32)
    with np.errstate(over="ignore", invalid="ignore"):
        e = sleef_expf((F32(0) - x).astype(F32))
        return (F32(1) / (F32(1) + e).astype(F32)).astype(F32)


def sigmoid_scalar(x) -> np.ndarray:
    """torch-CPU's scalar path: 1 / (1 + expf(-x)), expf correctly rounded."""
    x = np.asarray(x, F32)
    with np.errstate(over="ignore", invalid="ignore"):
        e = np.exp((-x).astype(np.float64)).astype(F32)
        return (F32(1) / (F32(1) + e).astype(F32)).astype(F32)


def sigmoid_torch(x, vector_floats: int) -> np.ndarray:
    """torch.sigmoid of a contiguous float32 array as one thread evaluates it:
    the vector path in steps of 2 * vector_floats elements, the scalar path
    for the rest."""
    flat = np.asarray(x, F32).reshape(-1)
    cut = len(flat) - len(flat) % (2 * vector_floats)
    out = np.empty_like(flat)
    out[:cut] = sigmoid_vector(flat[:cut])
    out[cut:] = sigmoid_scalar(flat[cut:])
    return out.reshape(np.shape(x))


def silu_vector(g) -> np.ndarray:
    """g * sigmoid(g) with the vector-path sigmoid (float32)."""
    g = np.asarray(g, F32)
    with np.errstate(over="ignore", invalid="ignore"):
        return (g * sigmoid_vector(g)).astype(F32)
