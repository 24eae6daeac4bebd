"""Pins oracle/sigmoid.py (torch-CPU's float32 sigmoid: SLEEF's xexpf on the
vector path, correctly rounded expf on the scalar tail) against torch itself,
and its exact fused multiply-add against rational arithmetic. Planted
mistakes must disagree with torch."""

from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import sigmoid as osig

F32 = np.float32
WIDTH = {"AVX512": 16, "AVX2": 8}


@pytest.fixture(scope="module")
def vector_floats():
    cap = torch.backends.cpu.get_cpu_capability()
    if cap not in WIDTH:
        pytest.skip(f"torch CPU capability {cap}: sigmoid is not vectorised with SLEEF here")
    return WIDTH[cap]


def _torch_sigmoid(x: np.ndarray) -> np.ndarray:
    """One thread, so the whole input is one chunk of the vectorised loop."""
    prev = torch.get_num_threads()
    torch.set_num_threads(1)
    try:
        return torch.sigmoid(torch.from_numpy(np.ascontiguousarray(x, F32))).numpy()
    finally:
        torch.set_num_threads(prev)


def _bits(a):
    return np.asarray(a, F32).view(np.uint32)


def _same(a, b):
    a, b = np.asarray(a, F32), np.asarray(b, F32)
    return (_bits(a) == _bits(b)) | (np.isnan(a) & np.isnan(b))


def _pad(x, vector_floats):
    k = 2 * vector_floats
    return np.concatenate([x, np.zeros((-len(x)) % k, F32)])


def _every_exponent(rng, per=64):
    parts = []
    for biased in range(0, 255):  # subnormals (0) through the largest finite exponent
        m = rng.integers(1 if biased == 0 else 0, 1 << 23, size=per, dtype=np.uint32)
        v = ((np.uint32(biased) << 23) | m).view(F32)
        parts += [v, -v]
    return np.concatenate(parts)


def _round_to_f32(fr: Fraction) -> np.float32:
    c = F32(float(fr))
    cands = [np.nextafter(c, F32(-np.inf)), c, np.nextafter(c, F32(np.inf))]
    best = min(cands, key=lambda v: (abs(Fraction(float(v)) - fr), int(_bits(v)) & 1))
    return F32(best)


def test_fma32_is_the_correctly_rounded_fused_multiply_add():
    rng = np.random.default_rng(1)
    n = 3000
    a = (rng.standard_normal(n) * np.exp2(rng.integers(-30, 30, n))).astype(F32)
    b = (rng.standard_normal(n) * np.exp2(rng.integers(-30, 30, n))).astype(F32)
    c = (rng.standard_normal(n) * np.exp2(rng.integers(-60, 60, n))).astype(F32)
    # cancellations and sums that land next to a float32 rounding boundary
    c[:500] = (-(a[:500].astype(np.float64) * b[:500])).astype(F32)
    got = osig.fma32(a, b, c)
    for i in range(n):
        want = _round_to_f32(Fraction(float(a[i])) * Fraction(float(b[i])) + Fraction(float(c[i])))
        assert _bits(got[i]) == _bits(want), (a[i], b[i], c[i], got[i], want)


def test_vector_path_matches_torch_over_every_exponent(vector_floats):
    rng = np.random.default_rng(2)
    x = np.concatenate([_every_exponent(rng), (rng.standard_normal(1 << 18) * 6).astype(F32)])
    x = _pad(x, vector_floats)
    ref = _torch_sigmoid(x)
    got = osig.sigmoid_vector(x)
    bad = np.nonzero(~_same(got, ref))[0]
    assert len(bad) == 0, [(x[i], ref[i], got[i]) for i in bad[:5]]


def test_vector_path_special_values_and_thresholds(vector_floats):
    base = [0.0, -0.0, np.inf, -np.inf, np.nan, 1e-45, -1e-45, 1.1754942e-38, -1.1754942e-38, 3e38, -3e38,
            16.635532, -16.635532, 17.0, -17.0, 87.33655, -87.33655, 88.72284, -88.72284]
    edges = []
    for t in (100.0, -100.0, 104.0, -104.0, 88.0, -88.0, 87.0, -87.0):
        v = F32(t)
        edges += [np.nextafter(v, F32(-np.inf)), v, np.nextafter(v, F32(np.inf))]
    x = _pad(np.array(base + edges, F32), vector_floats)
    assert _same(osig.sigmoid_vector(x), _torch_sigmoid(x)).all()


def _short_rows(vector_floats, rows=3000):
    """Inputs shorter than one double vector: torch takes the scalar path for
    all of them."""
    rng = np.random.default_rng(3)
    xs = (rng.standard_normal((rows, 2 * vector_floats - 1)) * 8).astype(F32)
    xs[:, 0] = np.array([0.0, -0.0, 30.0, -30.0, 90.0, -90.0] * (rows // 6), F32)
    return xs, np.stack([_torch_sigmoid(row) for row in xs])


def test_scalar_path_agrees_with_torch_on_short_inputs(vector_floats):
    """Correctly rounded expf against glibc's (0.502 ulp): equal on at least
    99.9 % of the sigmoids; the vector path, by contrast, differs on a few
    percent of the same inputs, so these rows did take the scalar path."""
    xs, ref = _short_rows(vector_floats)
    scalar = _same(osig.sigmoid_scalar(xs), ref).mean()
    vector = _same(osig.sigmoid_vector(xs), ref).mean()
    assert scalar >= 0.999, scalar
    assert vector < 0.99, vector


@pytest.mark.parametrize("tail", [0, 1, 7, 31])
def test_torch_splits_vector_body_and_scalar_tail(vector_floats, tail):
    """A single-thread input of 2W * k + r elements: the first 2W * k through
    the vector path (bit for bit), the last r (r < 2W) through the scalar
    path."""
    tail = tail % (2 * vector_floats)
    rng = np.random.default_rng(4 + tail)
    body = 2 * vector_floats * 4000
    x = (rng.standard_normal(body + tail) * 8).astype(F32)
    ref = _torch_sigmoid(x)
    got = osig.sigmoid_torch(x, vector_floats)
    assert _same(got[:body], ref[:body]).all()
    assert _same(got[body:], osig.sigmoid_scalar(x[body:])).all()
    if tail:
        assert _same(got[body:], ref[body:]).mean() >= 0.9


def test_the_two_paths_differ_so_the_split_matters():
    """The vector path (SLEEF, 1 ulp) and the scalar path (correctly rounded)
    disagree on a few percent of inputs: which path torch took decides bits."""
    x = (np.random.default_rng(5).standard_normal(1 << 16) * 8).astype(F32)
    differ = (~_same(osig.sigmoid_vector(x), osig.sigmoid_scalar(x))).mean()
    assert 0.005 < differ < 0.2, differ


def _sleef_variant(d, use_fma: bool, low_ln2: bool):
    d = np.asarray(d, F32)
    with np.errstate(all="ignore"):
        qf = np.rint((d * osig.R_LN2).astype(F32))
        q = np.clip(np.where(np.isfinite(qf), qf, 0), -200, 200).astype(np.int64)
        qf = q.astype(F32)

        def mla(a, b, c):
            return osig.fma32(a, b, c) if use_fma else ((np.asarray(a, F32) * b).astype(F32) + c).astype(F32)

        s = mla(qf, -osig.L2U, d)
        if low_ln2:
            s = mla(qf, -osig.L2L, s)
        u = np.full(d.shape, osig.POLY[0], F32)
        for c in osig.POLY[1:]:
            u = mla(u, s, c)
        u = (F32(1) + mla((s * s).astype(F32), u, s)).astype(F32)
        h = q >> 1
        return ((u * osig._pow2i(h)).astype(F32) * osig._pow2i(q - h)).astype(F32)


@pytest.mark.parametrize("use_fma,low_ln2", [(False, True), (True, False)], ids=["no-fma", "no-low-ln2"])
def test_planted_mistakes_disagree_with_torch(vector_floats, use_fma, low_ln2):
    x = _pad((np.random.default_rng(6).standard_normal(1 << 16) * 6).astype(F32), vector_floats)
    with np.errstate(all="ignore"):
        wrong = (F32(1) / (F32(1) + _sleef_variant((F32(0) - x).astype(F32), use_fma, low_ln2))).astype(F32)
    assert (~_same(wrong, _torch_sigmoid(x))).sum() > 50
