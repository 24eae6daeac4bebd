"""Integration caller: a Llama-3-8B decoder block on this library's kernels
(custom_cuda_kernals_amd/llama_block.py) against the same block in plain torch
ops, with identical weights - the reference's integration gate
(examples/llama_block.py:271-283: rtol 1e-2, atol 2e-2, outlier fraction 1e-5)
for the bf16 fused block; the FP8 block (FP8 GEMMs fed by the fused
RMSNorm+FP8 / SwiGLU+FP8 outputs) is held to a relative-error bound."""

from __future__ import annotations

import pytest
import torch

from custom_cuda_kernals_amd.llama_block import LlamaBlock

pytestmark = pytest.mark.gpu

SEQ = 512


def _blocks():
    torch.manual_seed(0)
    ref = LlamaBlock(SEQ, mode="eager").eval()
    out = {"eager": ref}
    for mode in ("fused", "fp8"):
        blk = LlamaBlock(SEQ, mode=mode).eval()
        blk.load_state_dict(ref.state_dict())
        out[mode] = blk
    g = torch.Generator(device="cuda").manual_seed(0)
    x = torch.randn(1, SEQ, 4096, dtype=torch.bfloat16, device="cuda", generator=g) * 0.02
    return out, x


def _assert_close_with_outliers(actual, expected, rtol, atol, frac):
    diff = (actual.double() - expected.double()).abs()
    bad = diff > atol + rtol * expected.double().abs()
    assert bad.float().mean().item() <= frac, f"{int(bad.sum())} elements beyond rtol {rtol} / atol {atol}"


def test_fused_block_matches_eager_block():
    blocks, x = _blocks()
    with torch.no_grad():
        ref = blocks["eager"](x)
        out = blocks["fused"](x)
    assert out.shape == ref.shape and out.dtype == torch.bfloat16
    _assert_close_with_outliers(out, ref, 1e-2, 2e-2, 1e-5)


def test_fp8_block_tracks_eager_block():
    blocks, x = _blocks()
    with torch.no_grad():
        ref = blocks["eager"](x).float()
        out = blocks["fp8"](x).float()
        resid = x.float()
    assert torch.isfinite(out).all()
    # Relative error of the block's update (output - input): FP8 e4m3 carries
    # 3 mantissa bits, so a few percent is the expected quantisation error.
    upd_ref, upd = ref - resid, out - resid
    rel = ((upd - upd_ref).norm() / upd_ref.norm()).item()
    cos = torch.nn.functional.cosine_similarity(upd.flatten(), upd_ref.flatten(), dim=0).item()
    print(f"\nfp8 block: relative error of the update {rel:.4f}, cosine {cos:.6f}")
    assert rel < 0.12 and cos > 0.995


def test_fp8_block_activations_are_the_fused_kernels_codes():
    """The FP8 block's first GEMM input is exactly rmsnorm_residual_fp8's
    output, i.e. the quantisation of the fused bf16 block's normalised
    activation (same kernels, same rows)."""
    from custom_cuda_kernals_amd.kernels import fp8_quant, rmsnorm_residual, rmsnorm_residual_fp8

    blocks, x = _blocks()
    w = blocks["fp8"].input_layernorm_weight
    zero = torch.zeros_like(x)
    q, s, ro = rmsnorm_residual_fp8(x, zero, w, 1e-5)
    y, ro2 = rmsnorm_residual(x, zero, w, 1e-5)
    q2, s2 = fp8_quant(y.view(-1, y.shape[-1]), "e4m3", "token")
    assert torch.equal(q.view(torch.uint8).view(-1, 4096), q2.view(torch.uint8))
    assert torch.equal(s.view(-1), s2) and torch.equal(ro, ro2)


def test_llama3_70b_shaped_blocks_track_eager():
    """The same gates at Llama-3-70B's layer shapes (hidden 8192, FFN 28672,
    64 / 8 heads), which take the wide row shapes of the RMSNorm (+ FP8) and
    SwiGLU (+ FP8) launchers and RoPE with 64 query heads."""
    from custom_cuda_kernals_amd.llama_block import CONFIGS

    cfg, seq = CONFIGS["llama3-70b"], 256
    torch.manual_seed(1)
    ref = LlamaBlock(seq, cfg, mode="eager").eval()
    g = torch.Generator(device="cuda").manual_seed(1)
    x = torch.randn(1, seq, cfg.hidden_size, dtype=torch.bfloat16, device="cuda", generator=g) * 0.02
    with torch.no_grad():
        want = ref(x)
        for mode in ("fused", "fp8"):
            blk = LlamaBlock(seq, cfg, mode=mode).eval()
            blk.load_state_dict(ref.state_dict())
            got = blk(x)
            if mode == "fused":
                _assert_close_with_outliers(got, want, 1e-2, 2e-2, 1e-5)
            else:
                upd_ref, upd = want.float() - x.float(), got.float() - x.float()
                rel = ((upd - upd_ref).norm() / upd_ref.norm()).item()
                cos = torch.nn.functional.cosine_similarity(upd.flatten(), upd_ref.flatten(), dim=0).item()
                print(f"\nllama3-70b fp8 block: relative error of the update {rel:.4f}, cosine {cos:.6f}")
                assert rel < 0.12 and cos > 0.995
            del blk
            torch.cuda.empty_cache()


@pytest.mark.parametrize("mode", ["fused", "fp8"])
def test_block_replays_from_a_hip_graph(mode):
    """The whole block captured once in a HIP graph (this library's kernels,
    hipBLASLt GEMMs, attention) and replayed three times, with the block run
    eagerly between replays: every replay equals the eager output bit for bit,
    so the path runs under graph capture with no host work between kernels."""
    blocks, x = _blocks()
    blk = blocks[mode]
    with torch.no_grad():
        if mode == "fp8":
            blk.prepare_fp8()
        ref = blk(x).clone()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            blk(x)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = blk(x)
        for _ in range(3):
            out.fill_(0)
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, ref)
            assert torch.equal(blk(x), ref)
