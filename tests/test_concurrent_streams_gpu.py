"""The reference-ABI launchers keep no state between calls (reference
src/kernels/fp8_quant.rs passes every buffer in), so calls queued on several
streams at once may overlap freely. Per-tensor FP8 (its two-pass and one-pass
forms and the caller's scratch), per-token FP8, RMSNorm+FP8 and SwiGLU+FP8 are launched
round-robin on four streams with different inputs and sizes, without
synchronising between launches; every result must equal the oracle's.
Overlap itself is up to the runtime (streams may share hardware queues), so
this guards against state shared between calls rather than proving overlap.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from custom_cuda_kernals_amd.kernels import fp8_quant, rmsnorm_residual_fp8, swiglu_fp8
from oracle import eager, inputs
from oracle import fp8 as ofp8

pytestmark = pytest.mark.gpu


def test_fp8_ops_interleaved_on_four_streams():
    streams = [torch.cuda.Stream() for _ in range(4)]
    cases = []
    for i in range(16):
        m = 256 + 96 * i
        x = inputs.fp8_token_input(m, 2048, torch.bfloat16, seed=300 + i) * (1 + i % 5)
        cases.append(("tensor" if i % 2 == 0 else "token", x))
    xr, rr, wr = inputs.rmsnorm_inputs(512, 4096, torch.bfloat16, seed=401)
    g, u = inputs.swiglu_inputs(512, 14336, seed=402)
    dev_inputs = [(gran, x.cuda()) for gran, x in cases]
    rms_in = [t.cuda() for t in (xr, rr, wr)]
    sw_in = [t.cuda() for t in (g, u)]
    torch.cuda.synchronize()
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    outs, fused = [], []
    for i, (gran, xd) in enumerate(dev_inputs):
        with torch.cuda.stream(streams[i % 4]):
            outs.append(fp8_quant(xd, "e4m3", gran))
            if i % 4 == 1:
                fused.append(("rms", rmsnorm_residual_fp8(*rms_in, 1e-5)))
            if i % 4 == 3:
                fused.append(("swiglu", swiglu_fp8(*sw_in)))
    for s in streams:
        torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    for (gran, x), (q, s) in zip(cases, outs):
        ref = ofp8.quant_tensor if gran == "tensor" else ofp8.quant_token
        codes, s_ref = ref(x.float().numpy(), "e4m3")
        assert np.array_equal(q.view(torch.uint8).cpu().numpy(), codes), gran
        assert np.array_equal(s.cpu().numpy().view(np.uint32).ravel(), s_ref.view(np.uint32).ravel()), gran
    q_rms_ref, s_rms_ref, ro_ref, _ = eager.rmsnorm_residual_fp8(xr, rr, wr, 1e-5, "e4m3")
    q_sw_ref, s_sw_ref, _ = eager.swiglu_fp8(g, u, "e4m3")
    for kind, out in fused:
        if kind == "rms":
            q, s, ro = out
            assert torch.equal(ro.cpu(), ro_ref)
            assert np.array_equal(q.view(torch.uint8).cpu().numpy(), q_rms_ref)
            assert np.array_equal(s.cpu().numpy().view(np.uint32), s_rms_ref.view(np.uint32))
        else:
            q, s = out
            assert np.array_equal(q.view(torch.uint8).cpu().numpy(), q_sw_ref)
            assert np.array_equal(s.cpu().numpy().view(np.uint32), s_sw_ref.view(np.uint32))


def test_one_pass_tensor_calls_overlapping_on_two_streams():
    """Per-tensor FP8 at one-pass sizes, queued alternately on two streams
    without synchronising: the reference ABI with its int32, the Python API
    without one, and the no-allocation entry point. A one-pass call keeps its
    exchange in its own codes and scale buffers, so overlapping calls cannot
    mix; grids that together exceed what the GPU holds at once only make
    waiting workgroups fall back to reading x themselves. Every result equals
    the oracle's, and so does a call made alone afterwards."""
    from tests import _cck

    lib = _cck.load()
    streams = [torch.cuda.Stream() for _ in range(2)]
    shapes = [(2048, 4096), (4096, 4096), (8192, 4096), (2048, 4096), (4096, 4096), (8192, 4096)]
    xs = [inputs.randn(s, torch.bfloat16, seed=500 + i) * (1 + i) for i, s in enumerate(shapes)]
    for i, x in enumerate(xs):
        x.view(-1)[(i * 104729) % x.numel()] = -(100.0 + 7 * i)
    devs = [x.cuda() for x in xs]
    torch.cuda.synchronize()
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    outs = []
    for i, xd in enumerate(devs):
        m, n = xd.shape
        with torch.cuda.stream(streams[i % 2]):
            st = torch.cuda.current_stream().cuda_stream
            kind = ("abi", "api", "noalloc")[i % 3]
            q = torch.empty(m, n, dtype=torch.uint8, device="cuda")
            sc = torch.empty(1, dtype=torch.float32, device="cuda")
            word = torch.zeros(1, dtype=torch.int32, device="cuda") if kind == "abi" else None
            if kind == "noalloc":
                rc = lib.launch_fp8_quant_tensor_noalloc_fwd(xd.data_ptr(), q.data_ptr(), sc.data_ptr(), m, n, 2, 3, st)
            else:
                rc = lib.launch_fp8_quant_tensor_fwd(xd.data_ptr(), q.data_ptr(), sc.data_ptr(),
                                                     None if word is None else word.data_ptr(), m, n, 2, 3, st)
            assert rc == 0
            outs.append((q, sc, word))
    for s in streams:
        torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    for x, (q, sc, word) in zip(xs, outs):
        codes, s_ref = ofp8.quant_tensor(x.float().numpy(), "e4m3")
        assert np.array_equal(q.cpu().numpy(), codes)
        assert np.array_equal(sc.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
        if word is not None:
            amax = np.float32(np.abs(x.float().numpy()).max())
            assert int(word.item()) == int(np.array([amax], dtype=np.float32).view(np.int32)[0])
    x = inputs.randn((4096, 4096), torch.bfloat16, seed=599)
    q, s = fp8_quant(x.cuda(), "e4m3", "tensor")
    torch.cuda.synchronize()
    codes, s_ref = ofp8.quant_tensor(x.float().numpy(), "e4m3")
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), codes)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
