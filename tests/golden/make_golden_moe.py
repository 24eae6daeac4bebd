"""Writes tests/golden/reference_moe.npz: input/output vectors of the
reference's own eager MoE baselines (baselines/token_permute.py:
compute_permutation, eager_token_gather, eager_token_combine;
baselines/moe_router.py: eager_moe_router).

Run in the build container (the reference is mounted there, read-only):
    python tests/golden/make_golden_moe.py /root/reference
It imports those two modules, feeds them small seeded CPU inputs and stores
inputs and outputs as raw bit patterns. Nothing from the reference is copied
into this repository except these data vectors.
"""

from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
from make_golden import DTYPES, _bits, _load  # noqa: E402


def main(ref_root: str) -> None:
    tp = _load(ref_root, "token_permute")
    mr = _load(ref_root, "moe_router")
    g = torch.Generator().manual_seed(20261202)
    out: dict[str, np.ndarray] = {}
    # Permutation bookkeeping: 37 tokens, top-3 of 8 experts (many ties per expert).
    topk = torch.randint(0, 8, (37, 3), generator=g)
    perm, unperm = tp.compute_permutation(topk)
    out.update({"perm_topk": topk.numpy(), "perm_permute": perm.numpy(), "perm_unpermute": unperm.numpy()})
    for tag, dt in DTYPES.items():
        src = torch.randn(50, 100, generator=g).to(dt)
        idx = torch.randint(0, 50, (70,), generator=g)
        out.update({f"gather_{tag}_src": _bits(src), f"gather_{tag}_idx": idx.numpy(),
                    f"gather_{tag}_dst": _bits(tp.eager_token_gather(src, idx))})
        for k, h in ((2, 128), (6, 128), (3, 100)):
            t = 33
            eo = torch.randn(t * k, h, generator=g).to(dt)
            ui = torch.randperm(t * k, generator=g).reshape(t, k)
            w = torch.rand(t, k, generator=g)
            key = f"combine_{tag}_k{k}_h{h}"
            out.update({f"{key}_eo": _bits(eo), f"{key}_ui": ui.numpy(), f"{key}_w": _bits(w),
                        f"{key}_out": _bits(tp.eager_token_combine(eo, ui, w))})
        for e, k, renorm in ((8, 2, True), (160, 6, True), (32, 4, False)):
            logits = torch.randn(40, e, generator=g)
            logits[:5] = torch.round(logits[:5] * 2) / 2  # exact ties in the first rows
            logits = logits.to(dt)
            wts, ids = mr.eager_moe_router(logits, k, renorm)
            key = f"router_{tag}_e{e}_k{k}_r{int(renorm)}"
            out.update({f"{key}_logits": _bits(logits), f"{key}_w": _bits(wts), f"{key}_i": ids.numpy()})
    out["torch_version"] = np.frombuffer(torch.__version__.encode(), dtype=np.uint8)
    path = os.path.join(HERE, "reference_moe.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path}: {len(out)} arrays, {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
