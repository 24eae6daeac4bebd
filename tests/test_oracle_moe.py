"""The MoE oracle (oracle/moe.py) pinned before it is trusted:
* golden vectors written from the reference's own baselines
  (tests/golden/reference_moe.npz; tests/golden/make_golden_moe.py): bit-exact;
* permutation invariants: expert-sorted and stable (token order kept within
  an expert), permute/unpermute inverse of each other, and the gather ->
  combine round trip with unit weights is the identity
  (tests/test_token_permute.py:88-126 in the reference);
* fp64 closed forms within the reference's tolerances (its TOLERANCES tables);
* the combine's summation order: for rows whose length is a multiple of 16,
  torch's (gathered.float() * w).sum(dim=1) equals fp32 products added in j
  order onto +0.0 (the order the HIP kernel uses), bit for bit;
* the router: probabilities sum to 1, weights descend, renormalised weights
  sum to 1, and a planted mistake (the softmax taken in the storage dtype)
  is caught by the golden vectors.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from oracle import inputs, moe

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "reference_moe.npz")
TAGS = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLDEN)


def _t(bits: np.ndarray, dtype: torch.dtype) -> torch.Tensor:
    if dtype == torch.float32:
        return torch.from_numpy(bits.view(np.float32).copy())
    return torch.from_numpy(bits.view(np.int16).copy()).view(dtype)


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int32 if t.dtype == torch.float32 else torch.int16).numpy()


def test_permutation_golden(gold):
    perm, unperm = moe.compute_permutation(gold["perm_topk"])
    assert np.array_equal(perm, gold["perm_permute"])
    assert np.array_equal(unperm, gold["perm_unpermute"])


@pytest.mark.parametrize("t,k,e", [(37, 3, 8), (2048, 6, 160), (1, 1, 1), (64, 8, 8)])
def test_permutation_invariants(t, k, e):
    rng = np.random.default_rng(t * 31 + k)
    topk = rng.integers(0, e, size=(t, k))
    perm, unperm = moe.compute_permutation(topk)
    flat = topk.reshape(-1)
    order = unperm.reshape(-1).argsort()  # flat assignment at each sorted slot
    sorted_experts = flat[order]
    assert np.all(np.diff(sorted_experts) >= 0)  # grouped by expert
    for ex in np.unique(flat):  # stable: token order kept inside an expert
        toks = perm[sorted_experts == ex]
        assert np.all(np.diff(toks) >= 0)
    # permute_index[unpermute_index[t, j]] == t
    assert np.array_equal(perm[unperm], np.repeat(np.arange(t)[:, None], k, axis=1))


def test_round_trip_identity():
    hidden = torch.randn(19, 32)
    topk = torch.from_numpy(np.random.default_rng(3).integers(0, 5, size=(19, 1)))
    perm, unperm = moe.compute_permutation(topk.numpy())
    permuted = moe.token_gather(hidden, torch.from_numpy(perm))
    back = moe.token_combine(permuted, torch.from_numpy(unperm), torch.ones(19, 1))
    assert torch.equal(back, hidden)


@pytest.mark.parametrize("tag", list(TAGS))
def test_gather_golden(gold, tag):
    dt = TAGS[tag]
    src = _t(gold[f"gather_{tag}_src"], dt)
    idx = torch.from_numpy(gold[f"gather_{tag}_idx"])
    out = moe.token_gather(src, idx)
    assert np.array_equal(_bits(out), gold[f"gather_{tag}_dst"].view(_bits(out).dtype))
    assert torch.equal(out, src[idx])  # closed form


@pytest.mark.parametrize("tag", list(TAGS))
@pytest.mark.parametrize("k,h", [(2, 128), (6, 128), (3, 100)])
def test_combine_golden_and_order(gold, tag, k, h):
    dt = TAGS[tag]
    key = f"combine_{tag}_k{k}_h{h}"
    eo, ui, w = _t(gold[f"{key}_eo"], dt), torch.from_numpy(gold[f"{key}_ui"]), _t(gold[f"{key}_w"], torch.float32)
    out = moe.token_combine(eo, ui, w)
    assert np.array_equal(_bits(out), gold[f"{key}_out"].view(_bits(out).dtype))
    if h % 16 == 0:
        assert torch.equal(moe.combine_sequential(eo, ui, w).view(torch.int16 if dt != torch.float32 else torch.int32),
                           out.view(torch.int16 if dt != torch.float32 else torch.int32))


@pytest.mark.parametrize("dt,rtol,atol", [(torch.float32, 1e-4, 1e-4), (torch.float16, 1e-2, 1e-2),
                                          (torch.bfloat16, 1e-2, 2e-2)])
def test_combine_fp64(dt, rtol, atol):
    eo, ui, w = inputs.combine_inputs(64, 6, 256, dt, seed=5)
    torch.testing.assert_close(moe.token_combine(eo, ui, w).double(), moe.token_combine_fp64(eo, ui, w),
                               rtol=rtol, atol=atol)


@pytest.mark.parametrize("tag", list(TAGS))
@pytest.mark.parametrize("e,k,renorm", [(8, 2, True), (160, 6, True), (32, 4, False)])
def test_router_golden(gold, tag, e, k, renorm):
    dt = TAGS[tag]
    key = f"router_{tag}_e{e}_k{k}_r{int(renorm)}"
    logits = _t(gold[f"{key}_logits"], dt)
    w, i = moe.moe_router(logits, k, renorm)
    assert np.array_equal(w.view(torch.int32).numpy(), gold[f"{key}_w"].view(np.int32))
    assert np.array_equal(i.numpy(), gold[f"{key}_i"])
    # Planted mistake: softmax in the storage dtype changes the bits for half types.
    if dt != torch.float32:
        wrong = torch.softmax(logits, dim=-1).float()
        ww, _ = torch.topk(wrong, k, dim=-1)
        if renorm:
            ww = ww / ww.sum(-1, keepdim=True)
        assert not np.array_equal(ww.view(torch.int32).numpy(), gold[f"{key}_w"].view(np.int32))


@pytest.mark.parametrize("renorm", [True, False])
def test_router_invariants_and_fp64(renorm):
    logits = inputs.router_inputs(256, 160, torch.float32, seed=9)
    p = moe.softmax_probs(logits)
    torch.testing.assert_close(p.sum(-1), torch.ones(256), rtol=0, atol=1e-5)
    w, i = moe.moe_router(logits, 6, renorm)
    assert bool((w[:, :-1] >= w[:, 1:]).all())
    assert torch.equal(torch.gather(p, 1, i) if not renorm else torch.gather(p, 1, i) / torch.gather(p, 1, i).sum(-1, keepdim=True), w)
    if renorm:
        torch.testing.assert_close(w.sum(-1), torch.ones(256), rtol=0, atol=1e-6)
    w64, i64 = moe.moe_router_fp64(logits, 6, renorm)
    assert torch.equal(i, i64)
    torch.testing.assert_close(w.double(), w64, rtol=1e-5, atol=1e-7)
