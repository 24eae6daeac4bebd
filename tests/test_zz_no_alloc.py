"""launch_fp8_quant_tensor_noalloc_fwd (no caller scratch; a library-owned
device array for its two-pass form) against the reference-ABI
launch_fp8_quant_tensor_fwd and the oracle (baselines/fp8_quant.py:162-178
with one scale for the tensor), bit for bit: codes and scale. Two calls in a
row, the second on a smaller input, so the second call starts from the array
as the first left it; plus the scalar (unaligned) path, both formats and
every input dtype.

Inputs of at most one workgroup's worth, and inputs from 2^20 vectors up that
fit in the registers of a resident grid, take the one-pass kernel (workgroup
maxima exchanged through slots in the call's own codes buffer and the scale
published in its scale word); the rest take the two-pass form, with its
partial maxima in the library's array. Both are covered, with calls of either
kind queued back to back, and the one-pass kernel's fallback (a workgroup
whose wait runs out reads all of x itself) is forced from the host with a
poll limit of zero.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import fp8 as ofp8
from oracle import inputs
from tests._parity import assert_codes_equal, assert_f32_bits_equal

pytestmark = pytest.mark.gpu

DTAG = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}
FTAG = {"e4m3": 3, "e5m2": 4}


def _lib():
    from tests import _cck

    return _cck.load()


def _noalloc(x_dev: torch.Tensor, q: torch.Tensor, fmt: str) -> torch.Tensor:
    scale = torch.full((1,), float("nan"), dtype=torch.float32, device="cuda")
    m, n = x_dev.shape
    rc = _lib().launch_fp8_quant_tensor_noalloc_fwd(x_dev.data_ptr(), q.data_ptr(), scale.data_ptr(), m, n,
                                                     DTAG[x_dev.dtype], FTAG[fmt],
                                                     torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    return scale


def _reference_abi(x_dev: torch.Tensor, fmt: str):
    q = torch.empty(x_dev.shape, dtype=torch.uint8, device="cuda")
    scale = torch.empty(1, dtype=torch.float32, device="cuda")
    amax = torch.zeros(1, dtype=torch.int32, device="cuda")
    m, n = x_dev.shape
    rc = _lib().launch_fp8_quant_tensor_fwd(x_dev.data_ptr(), q.data_ptr(), scale.data_ptr(), amax.data_ptr(), m, n,
                                            DTAG[x_dev.dtype], FTAG[fmt], torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    return q, scale


def _check_pair(x: torch.Tensor, fmt: str, q: torch.Tensor | None = None) -> None:
    x_dev = x.cuda()
    if q is None:
        q = torch.full(x.shape, 0x55, dtype=torch.uint8, device="cuda")
    scale = _noalloc(x_dev, q, fmt)
    q_ref, s_ref = _reference_abi(x_dev, fmt)
    torch.cuda.synchronize()
    assert torch.equal(q.cpu(), q_ref.cpu()), "codes differ from launch_fp8_quant_tensor_fwd"
    assert_f32_bits_equal(scale, s_ref.cpu().numpy())
    codes, s_oracle = ofp8.quant_tensor(x.float().numpy(), fmt)
    assert_codes_equal(q, codes)
    assert_f32_bits_equal(scale, s_oracle)


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16], ids=lambda d: str(d).split(".")[-1])
def test_two_calls_second_smaller(dtype, fmt):
    big = inputs.fp8_token_input(2048, 4096, dtype, seed=3)
    small = inputs.randn((300, 520), dtype, seed=4) * 0.01  # a much smaller amax than the first call's
    _check_pair(big, fmt)
    _check_pair(small, fmt)


def test_config1_shape_then_tiny():
    _check_pair(inputs.fp8_token_input(*inputs.CONFIG_SHAPES["fp8_token"], torch.bfloat16, seed=0), "e4m3")
    _check_pair(inputs.randn((2, 3), torch.bfloat16, seed=5), "e4m3")


@pytest.mark.parametrize("shape", [(1, 7), (33, 1001), (4096, 4100), (8192, 8192)], ids=lambda s: f"{s[0]}x{s[1]}")
def test_shapes_and_partial_grids(shape):
    """Sizes from below one workgroup to a grid-stride partial pass (more
    vectors than 512 workgroups take in one round)."""
    x = inputs.randn(shape, torch.bfloat16, seed=shape[1])
    x.view(-1)[x.numel() // 3] = -700.0
    _check_pair(x, "e4m3")


def test_unaligned_buffers_take_the_scalar_path():
    m, n = 513, 777
    x = inputs.randn((m, n), torch.bfloat16, seed=9)
    xb = torch.cat([torch.zeros(1, dtype=torch.bfloat16), x.reshape(-1)]).cuda()
    x_dev = xb[1:].view(m, n)
    assert x_dev.data_ptr() % 16 != 0
    buf = torch.full((m * n + 8,), 0x55, dtype=torch.uint8, device="cuda")
    q = buf[3:3 + m * n].view(m, n)
    scale = _noalloc(x_dev, q, "e4m3")
    torch.cuda.synchronize()
    codes, s_oracle = ofp8.quant_tensor(x.float().numpy(), "e4m3")
    assert_codes_equal(q, codes)
    assert_f32_bits_equal(scale, s_oracle)
    b = buf.cpu().numpy()
    assert (b[:3] == 0x55).all() and (b[3 + m * n:] == 0x55).all(), "wrote outside the codes buffer"


def test_back_to_back_without_synchronising():
    """Several calls queued on one stream without host synchronisation, each
    checked afterwards against the oracle."""
    xs = [inputs.randn((64 * (i + 1), 4096), torch.bfloat16, seed=20 + i) * (i + 1) for i in range(5)]
    outs = []
    for x in xs:
        q = torch.empty(x.shape, dtype=torch.uint8, device="cuda")
        outs.append((q, _noalloc(x.cuda(), q, "e4m3")))
    torch.cuda.synchronize()
    for x, (q, s) in zip(xs, outs):
        codes, s_oracle = ofp8.quant_tensor(x.float().numpy(), "e4m3")
        assert_codes_equal(q, codes)
        assert_f32_bits_equal(s, s_oracle)


@pytest.mark.parametrize("shape", [(4096, 8192), (4097, 8192)], ids=lambda s: f"{s[0]}x{s[1]}")
def test_register_capacity_boundary(shape):
    """[4096, 8192] bf16 is 16 vectors per thread over 256 workgroups of 1024
    threads (one pass when the GPU holds 256 at once); one more row streams
    what does not fit in registers."""
    x = inputs.randn(shape, torch.bfloat16, seed=shape[0])
    x.view(-1)[-5] = 900.0
    _check_pair(x, "e4m3")


def test_mixed_sequence_queued_without_synchronising():
    """One-pass grids of one workgroup (no exchange) and of 256 and 512
    workgroups, two-pass inputs between them (small ones, which take the
    library's array, and one beyond the one-pass capacity) and an unaligned
    one, all queued on one stream before any result is read."""
    shapes = [(1, 8), (2, 1024 * 8), (7, 1024 * 8), (64, 1024 * 8), (2048, 4096), (8193, 8192), (4096, 8192),
              (3, 1030), (2048, 4096), (1, 8), (100, 4096), (4096, 4096)]
    xs = [inputs.randn(s, torch.bfloat16, seed=40 + i) * (0.5 + i) for i, s in enumerate(shapes)]
    for i, x in enumerate(xs):
        x.view(-1)[(i * 7919) % x.numel()] = -(3.0 + 50 * i)
    outs = []
    for x in xs:
        q = torch.empty(x.shape, dtype=torch.uint8, device="cuda")
        outs.append((q, _noalloc(x.cuda(), q, "e4m3")))
    torch.cuda.synchronize()
    for x, (q, s) in zip(xs, outs):
        codes, s_oracle = ofp8.quant_tensor(x.float().numpy(), "e4m3")
        assert_codes_equal(q, codes)
        assert_f32_bits_equal(s, s_oracle)


def test_special_values_take_the_exact_path():
    """inf and NaN in a one-pass input: the scale is non-finite, every code
    comes from the exact encoder, as in the reference-ABI launcher."""
    for val in (float("inf"), float("nan")):
        x = inputs.randn((2048, 4096), torch.bfloat16, seed=61)
        x.view(-1)[12345] = val
        x_dev = x.cuda()
        q = torch.empty(x.shape, dtype=torch.uint8, device="cuda")
        scale = _noalloc(x_dev, q, "e4m3")
        q_ref, s_ref = _reference_abi(x_dev, "e4m3")
        torch.cuda.synchronize()
        assert torch.equal(q.cpu(), q_ref.cpu())
        assert_f32_bits_equal(scale, s_ref.cpu().numpy())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=lambda d: str(d).split(".")[-1])
def test_wait_fallback_reads_x_itself(dtype):
    """Poll limit 0: every workgroup but workgroup 0 (the reducer) stops
    waiting at once and takes the maximum over all of x itself; the results
    are the same bits, and the calls after it are unaffected."""
    lib = _lib()
    prev = lib.cck_fp8_tensor_noalloc_poll_limit(0)
    try:
        assert lib.cck_fp8_tensor_noalloc_poll_limit(-1) == 0
        _check_pair(inputs.randn((2048, 4096), dtype, seed=71) * 3, "e4m3")
        _check_pair(inputs.randn((24, 4096), dtype, seed=72), "e5m2")
        _check_pair(inputs.randn((4097, 8192), dtype, seed=74), "e4m3")  # beyond the register capacity
    finally:
        assert lib.cck_fp8_tensor_noalloc_poll_limit(prev) == 0
    assert lib.cck_fp8_tensor_noalloc_poll_limit(-1) == prev
    _check_pair(inputs.randn((2048, 4096), dtype, seed=73), "e4m3")


def test_graph_replays_with_eager_calls_between():
    """The entry point captured in a HIP graph (two calls: a one-pass size and
    a two-pass size), replayed with new inputs copied into the captured
    buffers and poisoned outputs; eager calls of other sizes run between the
    replays and move the array's state on. Every replay equals the reference
    ABI on the same inputs, bit for bit."""
    shapes = [(2048, 4096), (8193, 8192)]
    dev_in = [torch.empty(s, dtype=torch.bfloat16, device="cuda") for s in shapes]
    dev_q = [torch.empty(s, dtype=torch.uint8, device="cuda") for s in shapes]
    dev_s = [torch.empty(1, dtype=torch.float32, device="cuda") for _ in shapes]
    stream_of = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731

    def launch():
        for x, q, sc in zip(dev_in, dev_q, dev_s):
            m, n = x.shape
            assert _lib().launch_fp8_quant_tensor_noalloc_fwd(x.data_ptr(), q.data_ptr(), sc.data_ptr(), m, n, 2, 3,
                                                               stream_of()) == 0

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        launch()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        launch()
    torch.cuda.synchronize()
    for rep in range(4):
        xs = [inputs.randn(s, torch.bfloat16, seed=90 + 3 * rep + i) * (1 + rep) for i, s in enumerate(shapes)]
        for d, x in zip(dev_in, xs):
            d.copy_(x)
        for q, sc in zip(dev_q, dev_s):
            q.fill_(0x5A)
            sc.fill_(float("nan"))
        # eager calls of other sizes between the replays
        _check_pair(inputs.randn((64 * (rep + 1), 4096), torch.bfloat16, seed=80 + rep), "e4m3")
        graph.replay()
        torch.cuda.synchronize()
        for d, q, sc in zip(dev_in, dev_q, dev_s):
            q_ref, s_ref = _reference_abi(d, "e4m3")
            torch.cuda.synchronize()
            assert torch.equal(q.cpu(), q_ref.cpu()), f"replay {rep}: codes differ for {tuple(d.shape)}"
            assert_f32_bits_equal(sc, s_ref.cpu().numpy())


def test_rejects_size_beyond_int64_before_device_calls():
    lib = _lib()
    assert lib.launch_fp8_quant_tensor_noalloc_fwd(None, None, None, 1 << 40, 1 << 40, 2, 3, None) == 1
    assert lib.launch_fp8_quant_tensor_noalloc_fwd(None, None, None, 0, 8, 2, 3, None) == 0
    assert lib.launch_fp8_quant_tensor_noalloc_fwd(None, None, None, 4, 8, 9, 3, None) == 1
    assert lib.launch_fp8_quant_tensor_noalloc_fwd(None, None, None, 4, 8, 2, 7, None) == 1


def test_one_pass_calls_overlapping_on_two_streams_then_alone():
    """One-pass calls queued alternately on two streams without
    synchronising (their exchanges live in their own outputs, so overlapping
    calls cannot mix), then a call alone: all bit for bit."""
    streams = [torch.cuda.Stream() for _ in range(2)]
    shapes = [(4096, 4096), (2048, 4096), (4096, 8192), (2048, 4096)]
    xs = [inputs.randn(s, torch.bfloat16, seed=120 + i) * (2 + i) for i, s in enumerate(shapes)]
    devs = [x.cuda() for x in xs]
    torch.cuda.synchronize()
    for st in streams:
        st.wait_stream(torch.cuda.current_stream())
    outs = []
    for i, xd in enumerate(devs):
        with torch.cuda.stream(streams[i % 2]):
            q = torch.empty(xd.shape, dtype=torch.uint8, device="cuda")
            outs.append((q, _noalloc(xd, q, "e4m3")))
    for st in streams:
        torch.cuda.current_stream().wait_stream(st)
    torch.cuda.synchronize()
    for x, (q, sc) in zip(xs, outs):
        codes, s_oracle = ofp8.quant_tensor(x.float().numpy(), "e4m3")
        assert_codes_equal(q, codes)
        assert_f32_bits_equal(sc, s_oracle)
    _check_pair(inputs.randn((4096, 4096), torch.bfloat16, seed=129), "e4m3")
