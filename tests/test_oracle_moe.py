"""The MoE oracle (oracle/moe.py) pinned before it is trusted:
* golden vectors written from the reference's own baselines
  (tests/golden/reference_moe.npz; tests/golden/make_golden_moe.py): bit-exact;
* permutation invariants: expert-sorted and stable (token order kept within
  an expert), permute/unpermute inverse of each other, and the gather ->
  combine round trip with unit weights is the identity
  (tests/test_token_permute.py:88-126 in the reference);
* fp64 closed forms within the reference's tolerances (its TOLERANCES tables);
* the combine's summation order (``token_combine_aten``, the order the HIP
  kernel follows) equals torch's (gathered.float() * w).sum(dim=1) bit for
  bit on the golden vectors and over row lengths 1-69 and 4096-4127 and top-k
  1-600, and planted mistakes (j order on every column, the four-slot form on
  every column, no block cascade) disagree with torch;
* the router: probabilities sum to 1, weights descend, renormalised weights
  sum to 1, and a planted mistake (the softmax taken in the storage dtype)
  is caught by the golden vectors;
* the restated AVX-512 softmax and router (``softmax_avx512``,
  ``moe_router_avx512``, the forms the HIP kernel follows) equal torch's own
  bit for bit on an AVX-512 host: every row length from 1 to 300, values over
  many scales, -inf / NaN entries, the router case table in three dtypes and
  the golden vectors; planted mistakes (8-lane vectors, lanes combined in
  order instead of the xor tree, a division by the sum instead of the
  reciprocal's product, a correctly rounded exp instead of SLEEF's) disagree
  with torch; and the serial form of ATen's row sum the kernel uses for the
  renormalising sum (non-negative addends, n < 512) equals the stated order.
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
    aten = moe.token_combine_aten(eo, ui, w)
    assert np.array_equal(_bits(aten), gold[f"{key}_out"].view(_bits(out).dtype))


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


@pytest.fixture(scope="module")
def avx512():
    if torch.backends.cpu.get_cpu_capability() != "AVX512":
        pytest.skip("torch's softmax runs with 16-float vectors only on AVX-512 hosts")


def _bits_equal(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    return (a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))


def test_softmax_avx512_equals_torch_for_every_length(avx512):
    rng = np.random.default_rng(21)
    for n in range(1, 301):
        scale = [0.1, 1.0, 4.0, 30.0][n % 4]
        x = (rng.standard_normal((8, n)) * scale).astype(np.float32)
        got = moe.softmax_avx512(x)
        ref = torch.softmax(torch.from_numpy(x), dim=-1).numpy()
        assert _bits_equal(got, ref).all(), n


def test_softmax_avx512_special_values(avx512):
    rng = np.random.default_rng(22)
    x = (rng.standard_normal((6, 160)) * 3).astype(np.float32)
    x[0, 5] = -np.inf
    x[1, :] = -np.inf          # all -inf: NaN row
    x[2, 7] = np.nan
    x[3, 100:] = -np.inf
    x[4, 9] = 1e30             # one dominant logit
    x[5, :] = 0.0              # all equal
    got = moe.softmax_avx512(x)
    ref = torch.softmax(torch.from_numpy(x), dim=-1).numpy()
    assert _bits_equal(got, ref).all()


ROUTER_CASES = [(2048, 8, 2, True), (2048, 160, 6, True), (1024, 32, 4, True), (257, 16, 2, True),
                (64, 1, 1, True), (128, 256, 8, True), (256, 16, 2, False), (96, 256, 256, True),
                (300, 100, 4, True), (50, 17, 3, True)]


@pytest.mark.parametrize("dt", list(TAGS.values()), ids=list(TAGS))
@pytest.mark.parametrize("case", ROUTER_CASES, ids=lambda c: "x".join(map(str, c)))
def test_router_avx512_equals_torch(avx512, case, dt):
    t, e, k, renorm = case
    logits = inputs.router_inputs(t, e, dt, seed=t + e + k)
    w, i = moe.moe_router_avx512(logits, k, renorm)
    w_ref, i_ref = moe.moe_router(logits, k, renorm)
    assert torch.equal(w.view(torch.int32), w_ref.view(torch.int32))
    assert torch.equal(i, i_ref)


@pytest.mark.parametrize("tag", list(TAGS))
@pytest.mark.parametrize("e,k,renorm", [(8, 2, True), (160, 6, True), (32, 4, False)])
def test_router_avx512_golden(gold, tag, e, k, renorm):
    key = f"router_{tag}_e{e}_k{k}_r{int(renorm)}"
    w, i = moe.moe_router_avx512(_t(gold[f"{key}_logits"], TAGS[tag]), k, renorm)
    assert np.array_equal(w.view(torch.int32).numpy(), gold[f"{key}_w"].view(np.int32))
    assert np.array_equal(i.numpy(), gold[f"{key}_i"])


def _softmax_variant(x, lanes=16, tree=True, divide=False, exact_exp=False):
    from oracle import sigmoid as osig

    x = x.astype(np.float32)
    m = x.max(axis=1)
    d = (x - m[:, None]).astype(np.float32)
    e = np.exp(d.astype(np.float64)).astype(np.float32) if exact_exp else osig.sleef_expf(d)
    n = x.shape[1]
    full = n // lanes
    acc = e[:, :lanes].copy()
    for v in range(1, full):
        acc = (acc + e[:, v * lanes:(v + 1) * lanes]).astype(np.float32)
    r = n - full * lanes
    if r:
        acc[:, :r] = (acc[:, :r] + e[:, full * lanes:]).astype(np.float32)
    if tree:
        idx = np.arange(lanes)
        step = lanes // 2
        while step:
            acc = (acc + acc[:, idx ^ step]).astype(np.float32)
            step //= 2
        total = acc[:, 0]
    else:
        total = acc[:, 0].copy()
        for j in range(1, lanes):
            total = (total + acc[:, j]).astype(np.float32)
    if divide:
        return (e / total[:, None]).astype(np.float32)
    return (e * (np.float32(1) / total)[:, None]).astype(np.float32)


@pytest.mark.parametrize("mistake", [dict(lanes=8), dict(tree=False), dict(divide=True), dict(exact_exp=True)],
                         ids=["8-lane", "lanes-in-order", "divide", "exact-exp"])
def test_softmax_planted_mistakes_disagree_with_torch(avx512, mistake):
    x = (np.random.default_rng(23).standard_normal((2048, 160)) * 3).astype(np.float32)
    ref = torch.softmax(torch.from_numpy(x), dim=-1).numpy()
    assert _bits_equal(_softmax_variant(x), ref).all()  # the stated form itself
    wrong = _softmax_variant(x, **mistake)
    assert (~_bits_equal(wrong, ref)).sum() > 100


def _small_row_sum_serial(v):
    """The router kernel's serial form of ATen's row sum for n < 512
    non-negative addends: 8-lane vectors in 4 slots, each slot one running
    sum from zero (no 16-step block completes below 512), leftover vectors
    into slot 0, then the trailing scalars and the 8 lanes; rows under 8 as
    scalars in 4 slots."""
    f = np.float32
    n = len(v)
    if n < 8:
        s = n >> 2
        p = [f(v[k]) if s else f(0) for k in range(4)]
        for u in range(4 * s, n):
            p[0] = f(p[0] + v[u])
        return f(f(f(p[0] + p[1]) + p[2]) + p[3])
    nv, total = n >> 3, f(0)
    s = nv >> 2
    for e in range(nv * 8, n):
        total = f(total + v[e])
    for lane in range(8):
        p = [f(0)] * 4
        for i in range(s):
            for k in range(4):
                p[k] = f(p[k] + v[(4 * i + k) * 8 + lane])
        for vec in range(4 * s, nv):
            p[0] = f(p[0] + v[vec * 8 + lane])
        total = f(total + f(f(f(p[0] + p[1]) + p[2]) + p[3]))
    return total


def test_small_row_sum_serial_form_equals_the_stated_order():
    from oracle import rowsum

    rng = np.random.default_rng(24)
    for n in list(range(1, 80)) + [100, 127, 128, 129, 255, 256, 257, 384, 511]:
        v = (rng.random((4, n)) * np.exp2(rng.integers(-20, 20, (4, n)))).astype(np.float32)
        want = rowsum.row_sum(v)
        got = np.array([_small_row_sum_serial(row) for row in v], np.float32)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), n


def _combine_variant(eo, ui, w, mode):
    """Planted mistakes of the combine order: "seq" (j order on every
    column), "slot4" (the four-slot form on every column), "flat" (no block
    cascade on the vector columns)."""
    from oracle import rowsum

    prod = (eo.float()[ui] * w.unsqueeze(-1)).numpy()
    t, k, h = prod.shape
    cols = np.ascontiguousarray(prod.transpose(0, 2, 1))
    if mode == "seq" or mode == "flat":
        acc = np.zeros((t, h), np.float32)
        for j in range(k):
            acc = (acc + cols[:, :, j]).astype(np.float32)
        if mode == "flat":
            mc = moe.combine_main_columns(h)
            u = cols[:, mc:].reshape(t * (h - mc), k, 1)
            acc[:, mc:] = (np.float32(0) + rowsum._slot_sum(u)[:, 0]).reshape(t, h - mc)
        return acc
    u = cols.reshape(t * h, k, 1)
    return (np.float32(0) + rowsum._slot_sum(u)[:, 0]).reshape(t, h)


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_combine_aten_order_equals_torch(dt):
    rng = np.random.default_rng(31)
    for h in list(range(1, 70)) + [96, 100, 4096, 4104, 4127]:
        for k in (1, 2, 3, 4, 6, 8, 16, 17, 64, 65, 257, 600):
            if h * k > 160000:
                continue
            t = 6
            eo = torch.from_numpy((rng.standard_normal((t * k, h)) * np.exp2(rng.integers(-6, 6, (t * k, h))))
                                  .astype(np.float32)).to(dt)
            ui = torch.from_numpy(rng.permutation(t * k).reshape(t, k))
            w = torch.from_numpy(rng.random((t, k)).astype(np.float32))
            assert np.array_equal(_bits(moe.token_combine_aten(eo, ui, w)), _bits(moe.token_combine(eo, ui, w))), (h, k)


@pytest.mark.parametrize("mode,h,k", [("seq", 100, 6), ("seq", 16, 8), ("slot4", 4096, 6), ("flat", 4096, 40)])
def test_combine_planted_order_mistakes_disagree_with_torch(mode, h, k):
    rng = np.random.default_rng(32)
    t = 64
    eo = torch.from_numpy((rng.standard_normal((t * k, h)) * np.exp2(rng.integers(-8, 8, (t * k, h))))
                          .astype(np.float32))
    ui = torch.from_numpy(rng.permutation(t * k).reshape(t, k))
    w = torch.from_numpy(rng.random((t, k)).astype(np.float32))
    ref = moe.token_combine(eo, ui, w).numpy()
    wrong = _combine_variant(eo, ui, w, mode)
    assert (wrong.view(np.uint32) != ref.view(np.uint32)).sum() > 20
