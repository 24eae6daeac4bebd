"""MoE top-k router kernel vs the CPU oracle (oracle/moe.py, restating
baselines/moe_router.py:117-128) on the reference's case table
(baselines/moe_router.py:72-95) in three dtypes.

The kernel follows torch-CPU's fp32 softmax as its AVX-512 kernel computes it
(SLEEF's expf, the 16-lane summation order, the reciprocal's product) and the
renormalising sum in ATen's row-sum order, so the weights equal the oracle's
``moe_router_avx512`` bit for bit (that restatement equals torch's own on an
AVX-512 host, tests/test_oracle_moe.py). Expert selections are compared
through the oracle's probabilities: the probability of each selected expert
must equal the oracle's top-k at that position, bit for bit, so a different
expert is accepted only at an exact tie (torch's topk orders those its own
way; the kernel takes the lower expert index).

Up to 8 experts one lane holds a token; a group of four lanes (16-expert
stripes) holds one of 9 to 32 experts, and of up to 64 from 4096 tokens on;
a group of eight lanes one of 65 to 256 experts from 8192 tokens (up to 128
experts) or 12288; otherwise a wave does: the cases cover each form's edges
(expert counts around 8, 16, 32, 64, 128 and 256, k = E, token counts that
leave a partial workgroup or cross the thresholds) and rows that are not
16-byte aligned.
"""

from __future__ import annotations

import pytest
import torch

from custom_cuda_kernals_amd.kernels import moe_router
from oracle import inputs, moe

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.float16, torch.bfloat16]
CASES = [(2048, 8, 2, True), (2048, 160, 6, True), (1024, 32, 1, True), (1024, 32, 2, True), (1024, 32, 4, True),
         (1024, 32, 8, True), (256, 100, 4, True), (257, 16, 2, True), (64, 1, 1, True), (64, 8, 8, True),
         (128, 256, 8, True), (256, 16, 2, False), (1, 16, 2, True), (0, 16, 2, True), (96, 256, 256, True),
         (5, 9, 3, True), (100, 12, 12, True), (333, 17, 3, True), (65, 24, 5, False), (130, 31, 31, True),
         (3, 33, 33, False), (77, 48, 7, True), (50, 64, 64, True), (129, 65, 9, True), (31, 127, 5, True),
         (97, 128, 16, True), (40, 129, 8, True), (4100, 8, 2, True), (1000, 32, 8, False), (4095, 48, 6, True),
         (4096, 48, 6, True), (4101, 64, 64, False), (4097, 33, 5, True), (33, 5, 5, True), (70, 3, 2, False),
         (200, 13, 4, False), (64, 15, 15, True), (129, 10, 1, True),
         (8192, 65, 5, True), (8193, 100, 8, False), (8191, 128, 8, True), (12288, 160, 6, True),
         (12289, 256, 8, True), (12290, 129, 129, False)]


def _check(logits, k, renorm):
    w, i = moe_router(logits.cuda(), k, renorm)
    w, i = w.cpu(), i.cpu()
    t = logits.shape[0]
    assert w.shape == (t, k) and i.shape == (t, k) and w.dtype == torch.float32 and i.dtype == torch.int64
    if t == 0:
        return
    w_ref, i_ref = moe.moe_router_avx512(logits, k, renorm)
    assert torch.equal(w.view(torch.int32), w_ref.view(torch.int32)), "weights differ from the oracle's bits"
    p = moe.softmax_probs(logits)
    p_sel = torch.gather(p, 1, i)
    p_top = torch.gather(p, 1, i_ref)
    assert torch.equal(p_sel.view(torch.int32), p_top.view(torch.int32)), "a selection is not an exact tie"
    assert bool(((i >= 0) & (i < logits.shape[1])).all())
    assert all(len(set(row.tolist())) == k for row in i)  # distinct experts
    tie = w[:, 1:] == w[:, :-1]
    assert bool((i[:, 1:][tie] > i[:, :-1][tie]).all())  # ties: lower index first
    if renorm:
        torch.testing.assert_close(w.sum(-1), torch.ones(t), rtol=0, atol=2e-6)


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c)))
def test_router_matches_oracle(case, dtype):
    t, e, k, renorm = case
    _check(inputs.router_inputs(t, e, dtype, seed=t + e + k), k, renorm)


def test_router_exact_ties_pick_lower_index():
    logits = torch.zeros(8, 16)
    logits[:, [3, 5, 9]] = 2.0  # three equal maxima
    w, i = moe_router(logits.cuda(), 4)
    assert torch.equal(i.cpu()[:, :3], torch.tensor([[3, 5, 9]] * 8))
    assert bool((i.cpu()[:, 3] == 0).all())  # next: the lowest of the equal zeros


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("e", [8, 12, 16, 32, 64, 128])
def test_router_unaligned_rows(e, dtype):
    """Logits one element past a 16-byte boundary: the kernels take element loads."""
    t, k = 4100, min(e, 6)
    logits = inputs.router_inputs(t, e, dtype, seed=e)
    flat = torch.empty(t * e + 1, dtype=dtype, device="cuda")
    dev = flat[1:].view(t, e)
    dev.copy_(logits.cuda())
    assert dev.data_ptr() % 16 != 0
    w, i = moe_router(dev, k)
    w_ref, _ = moe.moe_router_avx512(logits, k)
    assert torch.equal(w.cpu().view(torch.int32), w_ref.view(torch.int32))
    p = moe.softmax_probs(logits)
    assert torch.equal(torch.gather(p, 1, i.cpu()), torch.gather(p, 1, torch.topk(p, k).indices))


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("e", [72, 160, 256])
def test_router_eight_lane_groups_unaligned(e, dtype):
    """The eight-lane form on rows one element past a 16-byte boundary (element loads)."""
    t, k = 12300, 6
    logits = inputs.router_inputs(t, e, dtype, seed=e + 1)
    flat = torch.empty(t * e + 1, dtype=dtype, device="cuda")
    dev = flat[1:].view(t, e)
    dev.copy_(logits.cuda())
    w, i = moe_router(dev, k)
    w_ref, _ = moe.moe_router_avx512(logits, k)
    assert torch.equal(w.cpu().view(torch.int32), w_ref.view(torch.int32))
    p = moe.softmax_probs(logits)
    assert torch.equal(torch.gather(p, 1, i.cpu()), torch.gather(p, 1, torch.topk(p, k).indices))


@pytest.mark.parametrize("e", [12, 32, 100, 200])
def test_router_ties_across_lanes_and_minus_inf(e):
    """Equal maxima held by different lanes of a token's group, and -inf
    logits (probability +0, picked last, lowest index first)."""
    t = 9 if e <= 64 else 12289  # past the eight-lane threshold
    logits = torch.full((t, e), -float("inf"))
    picks = [1, e // 2 - 1, e // 2 + 3, e - 2]
    logits[:, picks] = 1.5
    logits[:, 0] = 0.25
    w, i = moe_router(logits.cuda(), 6)
    i = i.cpu()
    assert torch.equal(i[:, :5], torch.tensor([picks + [0]] * t))
    assert bool((i[:, 5] == 2).all())  # the lowest index among the +0 probabilities
    w_ref, _ = moe.moe_router_avx512(logits, 6)
    assert torch.equal(w.cpu().view(torch.int32), w_ref.view(torch.int32))


def test_router_rejections():
    logits = torch.randn(4, 8, device="cuda")
    with pytest.raises(RuntimeError):
        moe_router(logits, k=16)
    with pytest.raises(ValueError):
        moe_router(torch.randn(4, 300, device="cuda"), k=2)
    with pytest.raises(ValueError):
        moe_router(torch.randn(4, 8), k=2)
