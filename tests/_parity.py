"""Comparison helpers shared by the GPU parity tests."""

from __future__ import annotations

import numpy as np
import torch

BF16_REL = 2.0 ** -7  # one bf16 ulp, relative


def codes_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().view(torch.uint8).cpu().numpy()


def assert_codes_equal(actual: torch.Tensor, expected: np.ndarray, what: str = "codes") -> None:
    a = codes_np(actual).reshape(expected.shape)
    bad = np.nonzero(a != expected)
    n = len(bad[0])
    if n:
        first = tuple(int(b[0]) for b in bad)
        raise AssertionError(
            f"{what}: {n} of {a.size} differ; first at {first}: got {a[first]:#04x}, want {expected[first]:#04x}"
        )


def assert_f32_bits_equal(actual: torch.Tensor, expected: np.ndarray, what: str = "scale") -> None:
    a = actual.detach().float().cpu().numpy().reshape(np.shape(expected)).astype(np.float32)
    e = np.asarray(expected, dtype=np.float32)
    same = (a.view(np.uint32) == e.view(np.uint32)) | (np.isnan(a) & np.isnan(e))
    if not same.all():
        i = np.argwhere(~same)[0]
        raise AssertionError(f"{what}: {int((~same).sum())} differ; first at {tuple(i)}: got {a[tuple(i)]!r}, want {e[tuple(i)]!r}")


def bits_equal(actual: torch.Tensor, expected: torch.Tensor) -> np.ndarray:
    a = actual.detach().cpu().contiguous()
    e = expected.detach().cpu().contiguous()
    ai = a.view(torch.int16 if a.element_size() == 2 else torch.int32).numpy()
    ei = e.view(torch.int16 if e.element_size() == 2 else torch.int32).numpy()
    return (ai == ei) | (np.isnan(a.float().numpy()) & np.isnan(e.float().numpy()))


# Per storage type: (one ulp relative, hard cap, allowed fraction above one
# ulp). The north-star bound is one ulp for every element (bf16 2^-7, fp16
# 2^-10, fp32 1e-5 relative), so nothing may exceed it.
ULP_TOL = {
    torch.bfloat16: (2.0 ** -7, 2.0 ** -7, 0.0),
    torch.float16: (2.0 ** -10, 2.0 ** -10, 0.0),
    torch.float32: (1e-5, 1e-5, 0.0),
}


def assert_ulp_close(actual: torch.Tensor, expected: torch.Tensor, what: str) -> dict:
    rel, hard, frac = ULP_TOL[expected.dtype]
    assert_within_rel(actual, expected, hard, what + " (hard cap)")
    return assert_within_rel(actual, expected, rel, what, max_outlier_fraction=frac)


def assert_within_rel(actual: torch.Tensor, expected: torch.Tensor, rel: float, what: str,
                      max_outlier_fraction: float = 0.0, atol: float = 0.0) -> dict:
    """|actual - expected| <= rel * max(|actual|, |expected|) + atol elementwise,
    allowing at most `max_outlier_fraction` violations. Returns stats."""
    a = actual.detach().double().cpu()
    e = expected.detach().double().cpu()
    diff = (a - e).abs()
    bound = rel * torch.maximum(a.abs(), e.abs()) + atol
    nan_ok = torch.isnan(a) & torch.isnan(e)
    viol = (diff > bound) & ~nan_ok
    n = int(viol.sum())
    exact = float(bits_equal(actual, expected).mean()) if actual.numel() else 1.0
    stats = {"n": actual.numel(), "violations": n, "bit_exact_fraction": exact,
             "max_rel": float((diff / e.abs().clamp_min(1e-30))[~nan_ok].max()) if actual.numel() else 0.0}
    if n > max_outlier_fraction * actual.numel():
        idx = torch.nonzero(viol)[0].tolist()
        raise AssertionError(f"{what}: {n} of {actual.numel()} beyond rel {rel}; first {idx}: "
                             f"got {a[tuple(idx)].item()!r}, want {e[tuple(idx)].item()!r}; stats {stats}")
    return stats
