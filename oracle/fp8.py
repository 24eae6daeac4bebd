"""numpy restatement of the reference's dynamic FP8 quantisation.

Reference algorithm (baselines/fp8_quant.py):
* ``eager_fp8_quant`` (:162-189): ``x32 = x.float()``; ``scale =
  clamp(amax / FP8_MAX, min=1e-12)``; ``x_fp8 = (x32 / scale).to(fp8)``;
* ``block_amax`` (:137-149): per-128x128-tile amax with zero padding of ragged
  edge tiles;
* ``expand_block_scale`` (:152-154).
FP8_MAX is ``torch.finfo(fp8).max`` (448 for e4m3fn, 57344 for e5m2, :166).

The cast ``.to(float8_*)`` is PyTorch's (third-party: torch, unpinned
``torch>=2.3`` in the reference's pyproject.toml:25; 2.10.0 here). It is
restated from the format definitions as round-to-nearest-even, with PyTorch's
overflow conventions: e4m3fn has no infinity, so magnitudes that round above
448 (|v| > 464), +-inf and NaN give NaN (0x7f | sign); e5m2 overflows
(|v| >= 61440) and +-inf to infinity (0x7c | sign), NaN to 0x7f | sign.

Pinned by (tests/test_oracle_fp8.py): exhaustive comparison of ``encode``
with torch's cast over every bf16- and fp16-representable value, a large
random + boundary fp32 sample (and all 2^32 patterns in the slow suite);
torch-CPU ``eager``-formula quantisation on the same inputs (the reference's
own tensor / block code path run with torch); closed forms (amax and one
IEEE division for the scale); the reference's invariant tests
(tests/test_fp8_quant.py:56-94: zero input, round-trip bound).

Divisions are numpy float32 divisions, i.e. IEEE-754 with the host's (x86)
NaN conventions, which is what torch's CPU kernels compute.
"""

from __future__ import annotations

import numpy as np

FP8_MAX = {"e4m3": 448.0, "e5m2": 57344.0}
MIN_SCALE = np.float32(1e-12)  # baselines/fp8_quant.py:59 (_EPS), rounded to float32
BLOCK = 128  # baselines/fp8_quant.py:58

# (mantissa bits, exponent bias, min normal exponent)
_FORMATS = {"e4m3": (3, 7, -6), "e5m2": (2, 15, -14)}


def encode(v: np.ndarray, fmt: str) -> np.ndarray:
    """Exact fp32 -> fp8 codes (uint8) with PyTorch's conventions."""
    v = np.asarray(v, dtype=np.float32)
    mbits, bias, emin = _FORMATS[fmt]
    bits = v.view(np.uint32)
    sign = ((bits >> np.uint32(24)) & np.uint32(0x80)).astype(np.uint8)
    with np.errstate(invalid="ignore"):
        a = np.abs(v.astype(np.float64))
    finite = np.isfinite(a)
    a_f = np.where(finite, a, 0.0)

    # a = f * 2^k with f in [0.5, 1): floor(log2 a) = k - 1 (exact, no log).
    _, k = np.frexp(a_f)
    e = np.maximum(k.astype(np.int64) - 1, emin)  # subnormals share the min exponent
    quantum = np.ldexp(1.0, e - mbits)
    m = np.rint(a_f / quantum)  # a/quantum is exact; rint is ties-to-even
    carry = m >= (1 << (mbits + 1))  # rounded up into the next binade
    e = np.where(carry, e + 1, e)
    m = np.where(carry, m / 2, m).astype(np.int64)
    value = m * np.ldexp(1.0, e - mbits)

    normal = m >= (1 << mbits)
    code = np.where(normal, ((e + bias) << mbits) | (m - (1 << mbits)), m).astype(np.int64)

    if fmt == "e4m3":
        special = (~finite) | (value > 448.0)
        code = np.where(special, 0x7F, code)
    else:
        overflow = (value > 57344.0) | np.isinf(a)
        code = np.where(overflow, 0x7C, code)
        code = np.where(np.isnan(a), 0x7F, code)
    return code.astype(np.uint8) | sign


def decode(codes: np.ndarray, fmt: str) -> np.ndarray:
    """fp8 codes -> float32 values (NaN for NaN codes, +-inf for e5m2 inf)."""
    c = np.asarray(codes, dtype=np.uint8).astype(np.int64)
    mbits, bias, _ = _FORMATS[fmt]
    sign = np.where(c & 0x80, -1.0, 1.0)
    ebits = 7 - mbits
    e = (c >> mbits) & ((1 << ebits) - 1)
    m = c & ((1 << mbits) - 1)
    mag = np.where(e == 0, m * 2.0 ** (1 - bias - mbits), (1.0 + m / (1 << mbits)) * np.ldexp(1.0, e - bias))
    if fmt == "e4m3":
        mag = np.where((c & 0x7F) == 0x7F, np.nan, mag)
    else:
        mag = np.where(e == 31, np.where(m == 0, np.inf, np.nan), mag)
    return (sign * mag).astype(np.float32)


def _scale_from_amax(amax: np.ndarray, fmt: str) -> np.ndarray:
    s = np.asarray(amax, dtype=np.float32) / np.float32(FP8_MAX[fmt])
    # torch.clamp(min=...) keeps NaN: NaN < MIN_SCALE is False.
    return np.where(s < MIN_SCALE, MIN_SCALE, s).astype(np.float32)


def _amax(x32: np.ndarray, axis=None) -> np.ndarray:
    # |x| max with NaN propagation (torch's max does propagate NaN).
    return np.max(np.abs(x32), axis=axis)


def quant_token(x32: np.ndarray, fmt: str) -> tuple[np.ndarray, np.ndarray]:
    """Per-row dynamic quantisation: eager_fp8_quant's "tensor" formula applied
    to each row of a [M, N] float32 array. Returns (codes [M, N], scale [M]).
    Rows are processed in chunks to bound the encoder's temporaries."""
    x32 = np.asarray(x32, dtype=np.float32)
    scale = _scale_from_amax(_amax(x32, axis=-1), fmt)
    codes = np.empty(x32.shape, dtype=np.uint8)
    step = max(1, (1 << 24) // max(1, x32.shape[-1]))
    for i in range(0, x32.shape[0], step):
        with np.errstate(all="ignore"):
            q = x32[i:i + step] / scale[i:i + step, None]
        codes[i:i + step] = encode(q, fmt)
    return codes, scale


def quant_tensor(x32: np.ndarray, fmt: str) -> tuple[np.ndarray, np.ndarray]:
    """baselines/fp8_quant.py:172-178. Returns (codes, scale as a [1] array)."""
    x32 = np.asarray(x32, dtype=np.float32)
    scale = _scale_from_amax(_amax(x32), fmt).reshape(1)
    with np.errstate(all="ignore"):
        q = x32 / scale[0]
    return encode(q, fmt), scale


def quant_static(x32: np.ndarray, scale: float, fmt: str) -> np.ndarray:
    """codes = fp8(x / scale) with a given float32 scale."""
    x32 = np.asarray(x32, dtype=np.float32)
    flat = x32.reshape(-1)
    codes = np.empty(flat.shape, dtype=np.uint8)
    step = 1 << 24
    for i in range(0, flat.size, step):
        with np.errstate(all="ignore"):
            q = flat[i:i + step] / np.float32(scale)
        codes[i:i + step] = encode(q, fmt)
    return codes.reshape(x32.shape)


def quant_block(x32: np.ndarray, fmt: str, block: int = BLOCK) -> tuple[np.ndarray, np.ndarray]:
    """baselines/fp8_quant.py:180-189 with block_amax (:137-149) and
    expand_block_scale (:152-154). Returns (codes [M, N], scale [ceil(M/b), ceil(N/b)])."""
    x32 = np.asarray(x32, dtype=np.float32)
    m, n = x32.shape
    pm, pn = -(-m // block) * block, -(-n // block) * block
    padded = np.zeros((pm, pn), dtype=np.float32)
    padded[:m, :n] = np.abs(x32)
    tiles = padded.reshape(pm // block, block, pn // block, block)
    amax = tiles.max(axis=(1, 3))
    scale = _scale_from_amax(amax, fmt)
    expanded = np.repeat(np.repeat(scale, block, axis=0), block, axis=1)[:m, :n]
    with np.errstate(all="ignore"):
        q = x32 / expanded
    return encode(q, fmt), scale


# --- bf16 helpers (numpy has no bfloat16) -----------------------------------

def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)
