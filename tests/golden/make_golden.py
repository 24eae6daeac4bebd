"""Writes tests/golden/reference_eager.npz: input/output vectors of the
reference's own eager baselines, for the functions whose bit-level results no
closed form pins (their fp32/bf16 rounding chains run through torch-CPU
reductions, rsqrt, sigmoid, pow, cos/sin).

Run in the build container (the reference is mounted there, read-only):
    python tests/golden/make_golden.py /root/reference
It imports baselines/{rmsnorm_residual,swiglu,rope,fp8_quant}.py from that
tree, feeds them small seeded CPU inputs, and stores inputs and outputs as
raw bit patterns. Nothing from the reference is copied into this repository
except these data vectors.
"""

from __future__ import annotations

import importlib.util
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def _load(ref_root: str, name: str):
    path = os.path.join(ref_root, "baselines", f"{name}.py")
    spec = importlib.util.spec_from_file_location(f"ref_baselines_{name}", path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[spec.name] = mod  # dataclasses resolve annotations through sys.modules
    spec.loader.exec_module(mod)
    return mod


def _bits(t: torch.Tensor) -> np.ndarray:
    t = t.contiguous()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.dtype == torch.float32:
        return t.view(torch.int32).numpy().view(np.uint32)
    if t.dtype in (torch.float8_e4m3fn, torch.float8_e5m2):
        return t.view(torch.uint8).numpy()
    raise TypeError(t.dtype)


DTYPES = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}


def main(ref_root: str) -> None:
    rms = _load(ref_root, "rmsnorm_residual")
    swi = _load(ref_root, "swiglu")
    rope = _load(ref_root, "rope")
    fp8 = _load(ref_root, "fp8_quant")
    g = torch.Generator().manual_seed(20261201)
    out: dict[str, np.ndarray] = {}
    for tag, dt in DTYPES.items():
        # RMSNorm + residual: [3, 5, 256] and a non-multiple-of-8 hidden size.
        for cols in (256, 100):
            x = torch.randn(3, 5, cols, generator=g).to(dt)
            r = torch.randn(3, 5, cols, generator=g).to(dt)
            w = (1.0 + 0.1 * torch.randn(cols, generator=g)).to(dt)
            y, ro = rms.eager_rmsnorm_residual(x, r, w, 1e-5)
            key = f"rms_{tag}_{cols}"
            out.update({f"{key}_x": _bits(x), f"{key}_r": _bits(r), f"{key}_w": _bits(w),
                        f"{key}_y": _bits(y), f"{key}_ro": _bits(ro)})
        # SwiGLU: [4, 300], includes large-magnitude gates.
        gate = (torch.randn(4, 300, generator=g) * 6).to(dt)
        up = torch.randn(4, 300, generator=g).to(dt)
        y = swi.eager_swiglu(gate, up)
        out.update({f"swiglu_{tag}_gate": _bits(gate), f"swiglu_{tag}_up": _bits(up), f"swiglu_{tag}_y": _bits(y)})
        # RoPE: tables at theta = 5e5 and a GQA pair.
        cos, sin = rope.compute_cos_sin(16, 64, 500000.0, device="cpu")
        q = torch.randn(2, 16, 4, 64, generator=g).to(dt)
        k = torch.randn(2, 16, 2, 64, generator=g).to(dt)
        qo, ko = rope.eager_rope(q, k, cos, sin)
        out.update({f"rope_{tag}_q": _bits(q), f"rope_{tag}_k": _bits(k), f"rope_{tag}_qo": _bits(qo),
                    f"rope_{tag}_ko": _bits(ko)})
        if tag == "f32":
            out.update({"rope_cos_16x64_t5e5": _bits(cos), "rope_sin_16x64_t5e5": _bits(sin)})
        # FP8: tensor and block granularity, both formats, ragged shape with outliers.
        xq = torch.randn(131, 259, generator=g)
        xq.view(-1)[torch.randperm(xq.numel(), generator=g)[:40]] *= 50
        xq = xq.to(dt)
        out[f"fp8_{tag}_x"] = _bits(xq)
        for fmt in ("e4m3", "e5m2"):
            for gran in ("tensor", "block"):
                codes, scale = fp8.eager_fp8_quant(xq, fmt, gran)
                out[f"fp8_{tag}_{fmt}_{gran}_codes"] = _bits(codes)
                out[f"fp8_{tag}_{fmt}_{gran}_scale"] = _bits(scale.reshape(-1).float())
    out["torch_version"] = np.frombuffer(torch.__version__.encode(), dtype=np.uint8)
    path = os.path.join(HERE, "reference_eager.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path}: {len(out)} arrays, {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
