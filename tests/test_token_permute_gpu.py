"""MoE token permute / unpermute kernels vs the CPU oracle (oracle/moe.py,
restating baselines/token_permute.py:55-70, 215-217, 237-251).

* gather is byte movement: bit-exact for every dtype (and FP8 rows);
* combine: bit-exact for every row length, top-k and dtype, against torch's
  own sum and against its stated order (oracle/moe.py token_combine_aten: j
  order with ATen's block cascade on the columns torch reduces as vector
  lanes, its four-slot scalar form on the rest);
* the reference's case tables (baselines/token_permute.py:128-167) in three
  dtypes, its vector-tail sweep (tests/test_token_permute_kernel.py:107-137),
  the permute -> unpermute round trip, and index hygiene (out-of-range
  indices give zero rows / dropped terms).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from custom_cuda_kernals_amd.kernels import compute_permutation, token_combine, token_gather
from oracle import inputs, moe
from tests._parity import assert_ulp_close, bits_equal

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.float16, torch.bfloat16]
GATHER_CASES = [(2048, 4096, 4096), (2048, 4096, 11008), (257, 513, 100), (1, 1, 256), (64, 0, 256),
                (128, 256, 16)]
COMBINE_CASES = [(2048, 2, 4096), (2048, 6, 4096), (256, 1, 512), (256, 8, 512), (257, 3, 100), (1, 2, 256),
                 (0, 2, 256), (128, 4, 16),
                 # few tokens, rows of >= 512 vectors (one 512-thread pass, or two at fp32 hidden 16384); the
                 # boundary at 1024 tokens and k = 16; one 256-thread pass of 1024-vector rows at top-1/2
                 (512, 2, 4096), (300, 6, 7168), (100, 3, 16384), (1024, 16, 4096), (1025, 2, 4096),
                 (1536, 2, 4096), (1100, 1, 8192)]


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("case", GATHER_CASES, ids=lambda c: "x".join(map(str, c)))
def test_gather_matches_oracle(case, dtype):
    s, n, h = case
    src, idx = inputs.gather_inputs(s, n, h, dtype, seed=s + n + h)
    out = token_gather(src.cuda(), idx.cuda()).cpu()
    assert out.shape == (n, h) and out.dtype == dtype
    assert bits_equal(out, moe.token_gather(src, idx)).all()


@pytest.mark.parametrize("fmt", [torch.float8_e4m3fn, torch.float8_e5m2])
@pytest.mark.parametrize("h, n_dst", [(4096, 777), (100, 777), (7, 777), (4096, 16400)])
def test_gather_fp8_rows(fmt, h, n_dst):
    """FP8 code rows move as bytes; 16400 rows of 4096 codes take the flat
    form (2^22 destination vectors and more)."""
    src = torch.randint(0, 256, (300, h), dtype=torch.uint8).view(fmt)
    idx = torch.randint(0, 300, (n_dst,))
    out = token_gather(src.cuda(), idx.cuda()).cpu()
    assert torch.equal(out.view(torch.uint8), src.view(torch.uint8)[idx])


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
def test_gather_vector_tails(dtype):
    for h in list(range(1, 40)) + [63, 64, 65, 127, 128, 129]:
        src, idx = inputs.gather_inputs(33, 45, h, dtype, seed=h)
        out = token_gather(src.cuda(), idx.cuda()).cpu()
        assert bits_equal(out, moe.token_gather(src, idx)).all(), h


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("n_src, n_dst, h", [(3000, 4095, 512), (3000, 4097, 512), (5000, 100003, 64),
                                             (700, 70001, 8), (300, 1031, 8200), (300, 517, 4100),
                                             (3000, 4099, 8200), (5000, 65537, 512)])
def test_gather_row_forms(n_src, n_dst, h, dtype):
    """The gather's launch forms: 4 and 8 rows per workgroup step around 4096
    destination rows, the resident grid with prefetched indices (many short
    rows), and the flat form (rows of more than 512 vectors at any size, and
    from 2^22 destination vectors: waves that span two rows, a partial last
    wave, rows of exactly 64 vectors); a few indices out of range in each."""
    src, idx = inputs.gather_inputs(n_src, n_dst, h, dtype, seed=n_dst + h)
    idx[::997] = n_src  # out of range: zero rows
    out = token_gather(src.cuda(), idx.cuda()).cpu()
    bad = idx >= n_src
    assert torch.equal(out[bad], torch.zeros(int(bad.sum()), h, dtype=dtype))
    assert bits_equal(out[~bad], src[idx[~bad]]).all()


def test_gather_out_of_range_rows_are_zero():
    src, idx = inputs.gather_inputs(50, 64, 256, torch.bfloat16, seed=1)
    idx[3], idx[10], idx[40] = 50, -1, 1 << 40
    out = token_gather(src.cuda(), idx.cuda()).cpu()
    bad = torch.tensor([3, 10, 40])
    assert torch.equal(out[bad], torch.zeros(3, 256, dtype=torch.bfloat16))
    good = torch.ones(64, dtype=torch.bool)
    good[bad] = False
    assert bits_equal(out[good], src[idx[good]]).all()


def _check_combine(eo, ui, w):
    """Bit-exact against torch's (gathered.float() * w).sum(dim=1) and
    against its stated order (oracle/moe.py token_combine_aten), one rounding
    to the storage type."""
    out = token_combine(eo.cuda(), ui.cuda(), w.cuda()).cpu()
    ref = moe.token_combine(eo, ui, w)
    assert out.shape == ref.shape and out.dtype == eo.dtype
    if out.numel() == 0:
        return None
    assert bits_equal(out, moe.token_combine_aten(eo, ui, w)).all(), "kernel differs from ATen's order"
    assert bits_equal(out, ref).all(), "kernel differs from torch's sum"
    return 1.0


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("case", COMBINE_CASES, ids=lambda c: "x".join(map(str, c)))
def test_combine_matches_oracle(case, dtype):
    t, k, h = case
    eo, ui, w = inputs.combine_inputs(t, k, h, dtype, seed=t + k + h)
    _check_combine(eo, ui, w)


@pytest.mark.parametrize("k", [3, 6, 8])
@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
def test_combine_vector_tails(dtype, k):
    """Row lengths around every vector and 32-column boundary: the scalar
    four-slot columns (k >= 4 orders them differently from j order)."""
    for h in list(range(1, 20)) + [24, 31, 32, 33, 40, 63, 64, 65, 127, 128, 129, 4104]:
        eo, ui, w = inputs.combine_inputs(17, k, h, dtype, seed=h + k)
        _check_combine(eo, ui, w)


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("t,k,h", [(64, 17, 4096), (32, 20, 4104), (32, 65, 512), (16, 256, 136), (8, 300, 40),
                                   (16, 9, 1), (8, 40, 1), (4, 600, 1), (8, 1100, 64)])
def test_combine_deep_topk_block_cascade(t, k, h, dtype):
    """k > 16: ATen folds each running sum in 16-step blocks (the vector
    columns) and each of the four slots in 16-step blocks (the scalar
    columns); h == 1 sums each token's k terms as a contiguous row."""
    eo, ui, w = inputs.combine_inputs(t, k, h, dtype, seed=t + k + h)
    _check_combine(eo, ui, w)


def test_combine_out_of_range_terms_are_dropped():
    eo, ui, w = inputs.combine_inputs(64, 4, 256, torch.bfloat16, seed=2)
    ui[5, 1], ui[9, 0], ui[9, 3] = 256, -7, 1 << 40
    out = token_combine(eo.cuda(), ui.cuda(), w.cuda()).cpu()
    w_ref, ui_ref = w.clone(), ui.clone()
    for t, j in ((5, 1), (9, 0), (9, 3)):
        w_ref[t, j], ui_ref[t, j] = 0.0, 0
    assert bits_equal(out, moe.token_combine(eo, ui_ref, w_ref)).all()


def test_dispatch_round_trip():
    """Router assignments -> compute_permutation -> gather -> (identity experts)
    -> combine with the renormalised weights gives back the tokens: the MoE
    dispatch path of the reference (tests/test_token_permute_kernel.py:89-104)."""
    t, k, e, h = 512, 2, 8, 1024
    g = torch.Generator().manual_seed(4)
    hidden = torch.randn(t, h, generator=g)
    topk = torch.stack([torch.randperm(e, generator=g)[:k] for _ in range(t)])
    perm, unperm = compute_permutation(topk.cuda())
    p_ref, u_ref = moe.compute_permutation(topk.numpy())
    assert np.array_equal(perm.cpu().numpy(), p_ref) and np.array_equal(unperm.cpu().numpy(), u_ref)
    permuted = token_gather(hidden.cuda(), perm)
    w = torch.full((t, k), 1.0 / k)
    back = token_combine(permuted, unperm, w.cuda()).cpu()
    torch.testing.assert_close(back, hidden, rtol=1e-6, atol=1e-6)


# ---- The permutation bookkeeping as one kernel (compute_permutation with
# num_experts): a stable counting sort, bit-exact against the oracle's stable
# argsort (oracle/moe.py compute_permutation, pinned by the reference's own
# compute_permutation outputs in tests/golden).

def _expected_permutation(topk: np.ndarray, e: int):
    """The oracle's order with ids outside [0, e) mapped to one bucket after
    every expert (their relative order, by flat index, is kept)."""
    ids = np.where((topk >= 0) & (topk < e), topk, e)
    return moe.compute_permutation(ids)


def test_permutation_kernel_golden():
    import os

    gold = np.load(os.path.join(os.path.dirname(__file__), "golden", "reference_moe.npz"))
    topk = gold["perm_topk"]
    perm, unperm = compute_permutation(torch.from_numpy(topk).cuda(), int(topk.max()) + 1)
    assert np.array_equal(perm.cpu().numpy(), gold["perm_permute"])
    assert np.array_equal(unperm.cpu().numpy(), gold["perm_unpermute"])


@pytest.mark.parametrize("t,k,e", [
    (2048, 6, 160),    # the router bench shape: 12 workgroups, one tile each
    (8191, 8, 256),    # 65528 entries, the largest one-launch size: 64 workgroups
    (65535, 1, 3),     # the largest one-launch size with k = 1 (wave-combined counts)
    (8192, 8, 256),    # 65536 entries, the smallest three-launch size: 32 chunks of 2048
    (40000, 8, 256),   # 320000 entries (three launches): a partial last chunk, every bucket of the maximum expert count
    (131072, 8, 256),  # 1048576 entries: 256 chunks of 4096
    (70001, 2, 8),     # three launches, k = 2, few experts
    (257, 3, 8),       # a partial last tile, few experts (long runs of one bucket in a wave)
    (1, 1, 1), (3, 2, 1), (1025, 1, 2), (64, 8, 64), (511, 4, 255), (30000, 2, 8),
])
def test_permutation_kernel_matches_oracle(t, k, e):
    rng = np.random.default_rng(t * 7 + k * 3 + e)
    topk = rng.integers(0, e, size=(t, k))
    perm, unperm = compute_permutation(torch.from_numpy(topk).cuda(), e)
    p_ref, u_ref = moe.compute_permutation(topk)
    assert perm.dtype == torch.int64 and unperm.shape == (t, k)
    assert np.array_equal(perm.cpu().numpy(), p_ref)
    assert np.array_equal(unperm.cpu().numpy(), u_ref)


def test_permutation_kernel_skewed_and_router_assignments():
    """All tokens on one expert (one bucket per wave, the longest runs), most
    tokens on one expert, at one- and three-launch sizes and k = 1 / 2 / 4, and
    real router output (distinct experts per token)."""
    rng = np.random.default_rng(3)
    for t, k, e in ((3000, 4, 64), (3000, 1, 64), (12000, 2, 8), (90000, 1, 64), (40000, 4, 64)):
        topk = np.full((t, k), 17 % e, dtype=np.int64)
        mixed = np.where(rng.random((t, k)) < 0.9, 5, rng.integers(0, e, size=(t, k)))
        for ids in (topk, mixed):
            perm, unperm = compute_permutation(torch.from_numpy(ids).cuda(), e)
            p_ref, u_ref = moe.compute_permutation(ids)
            assert np.array_equal(perm.cpu().numpy(), p_ref), (t, k, e)
            assert np.array_equal(unperm.cpu().numpy(), u_ref), (t, k, e)
    from custom_cuda_kernals_amd.kernels import moe_router

    logits = inputs.router_inputs(2048, 160, torch.float32, seed=5)
    _, idx = moe_router(logits.cuda(), 6)
    perm, unperm = compute_permutation(idx, 160)
    p_ref, u_ref = moe.compute_permutation(idx.cpu().numpy())
    assert np.array_equal(perm.cpu().numpy(), p_ref) and np.array_equal(unperm.cpu().numpy(), u_ref)


def test_permutation_kernel_out_of_range_ids():
    """Ids outside [0, num_experts) (negative, too large) are ordered after
    every expert, by flat index: the outputs stay a permutation, so the gather
    and combine they feed stay in bounds."""
    rng = np.random.default_rng(9)
    for t, k, e in ((700, 3, 16), (30000, 3, 16)):  # one launch, three launches
        topk = rng.integers(0, e, size=(t, k))
        topk[5, 1], topk[77, 0], topk[300, 2], topk[699, 2] = -1, 16, 1 << 40, -(1 << 50)
        if t > 700:
            topk[rng.random((t, k)) < 0.01] = e + 3
        perm, unperm = compute_permutation(torch.from_numpy(topk).cuda(), e)
        p_ref, u_ref = _expected_permutation(topk, e)
        assert np.array_equal(perm.cpu().numpy(), p_ref) and np.array_equal(unperm.cpu().numpy(), u_ref)
        assert np.array_equal(np.sort(unperm.cpu().numpy().reshape(-1)), np.arange(t * k))


def test_permutation_kernel_rejects_bad_arguments():
    from custom_cuda_kernals_amd._lib import native

    topk = torch.zeros((4, 2), dtype=torch.int64, device="cuda")
    p = torch.empty(8, dtype=torch.int64, device="cuda")
    u = torch.empty((4, 2), dtype=torch.int64, device="cuda")
    for bad in (0, 257):
        with pytest.raises(ValueError):
            native.moe_permutation_fwd(topk, p, u, bad)
    with pytest.raises(ValueError):
        native.moe_permutation_fwd(topk, p[:7], u, 8)
    empty = torch.empty((0, 2), dtype=torch.int64, device="cuda")
    perm, unperm = compute_permutation(empty, 8)
    assert perm.numel() == 0 and unperm.shape == (0, 2)


@pytest.mark.parametrize("t,k,e,h", [(512, 8, 64, 7168), (300, 2, 8, 4096), (97, 6, 160, 1000)])
def test_fp8_dispatch_quantise_once_then_gather(t, k, e, h):
    """The FP8 MoE dispatch: router -> permutation -> per-token FP8 of the T
    token rows -> gather of their code rows and scales. Equal, bit for bit, to
    per-token FP8 of the gathered bf16 rows (the scale of a row depends on the
    row alone), at 3·T·H + 2·k·T·H bytes instead of 3·k·T·H."""
    from custom_cuda_kernals_amd.kernels import fp8_quant, moe_router
    from oracle import fp8 as ofp8

    g = torch.Generator().manual_seed(t * k + h)
    x = torch.randn(t, h, generator=g).to(torch.bfloat16).cuda()
    logits = torch.randn(t, e, generator=g).cuda()
    _, ids = moe_router(logits, k)
    perm, _ = compute_permutation(ids, e)
    codes, scales = fp8_quant(x, "e4m3", "token")
    g_codes = token_gather(codes, perm)
    g_scales = token_gather(scales.view(t, 1), perm).view(-1)
    ref_codes, ref_scales = ofp8.quant_token(x.cpu()[perm.cpu()].float().numpy(), "e4m3")
    assert np.array_equal(g_codes.cpu().view(torch.uint8).numpy(), ref_codes)
    assert np.array_equal(g_scales.cpu().numpy().view(np.uint32), ref_scales.view(np.uint32))


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("k,h", [(2, 4096), (8, 7168), (2, 16384), (6, 4096), (8, 5120)])
def test_combine_many_tokens(k, h, dtype):
    """4100 tokens: the 512-thread one-pass shape for rows of 4096-16384
    elements (and the default shapes beside it), checked on token slices at
    the start, the middle and the end against ATen's order."""
    t = 4100
    g = torch.Generator(device="cuda").manual_seed(k * h)
    eo = torch.randn(t * k, h, device="cuda", generator=g).to(dtype)
    ui = torch.randperm(t * k, device="cuda", generator=g).view(t, k)
    w = torch.rand(t, k, device="cuda", generator=g)
    out = token_combine(eo, ui, w)
    torch.cuda.synchronize()
    for sl in (slice(0, 24), slice(2000, 2024), slice(t - 24, t)):
        rows = ui[sl].reshape(-1)
        local = torch.arange(rows.numel()).view(-1, k)
        ref = moe.token_combine_aten(eo[rows].cpu(), local, w[sl].cpu())
        assert bits_equal(out[sl].cpu(), ref).all(), sl
