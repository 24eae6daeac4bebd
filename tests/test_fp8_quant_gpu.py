"""FP8 quantisation kernels vs the CPU oracle: codes and scales bit-exact.

Case matrix follows the reference's (baselines/fp8_quant.py:84-114: standard
and edge shapes x {f32, f16, bf16} x {e4m3, e5m2}), for the reference's two
granularities and the build's per-token and static modes, plus the
BASELINE config-1 workload at full size and the edge inputs the reference
tests (all-zero input, tests/test_fp8_quant_kernel.py:84-89) and those the
domain adds (signed zeros, NaN / inf rows, static-scale overflow, unaligned
pointers, long rows).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from custom_cuda_kernals_amd.kernels import fp8_quant
from oracle import fp8 as ofp8
from oracle import inputs
from tests._parity import assert_codes_equal, assert_f32_bits_equal

pytestmark = pytest.mark.gpu

SHAPES = [(256, 256), (1024, 1024), (4096, 4096), (257, 513), (64, 64), (1, 256), (256, 1), (2048, 128)]
DTYPES = [torch.float32, torch.float16, torch.bfloat16]
FORMATS = ["e4m3", "e5m2"]


def _oracle(x: torch.Tensor, fmt: str, gran: str, scale=None):
    x32 = x.float().numpy()
    if scale is not None:
        return ofp8.quant_static(x32, scale, fmt), np.array([scale], dtype=np.float32)
    return {"token": ofp8.quant_token, "tensor": ofp8.quant_tensor, "block": ofp8.quant_block}[gran](x32, fmt)


def _check(x_cpu: torch.Tensor, fmt: str, gran: str, scale=None, x_dev=None):
    x_dev = x_cpu.cuda() if x_dev is None else x_dev
    q, s = fp8_quant(x_dev, fmt, gran, scale=scale)
    torch.cuda.synchronize()
    codes, s_ref = _oracle(x_cpu, fmt, gran, scale)
    assert q.dtype == ofp8_dtype(fmt) and tuple(q.shape) == tuple(x_cpu.shape)
    assert_codes_equal(q, codes)
    assert_f32_bits_equal(s, s_ref)


def ofp8_dtype(fmt):
    return torch.float8_e4m3fn if fmt == "e4m3" else torch.float8_e5m2


@pytest.mark.parametrize("gran", ["token", "block", "tensor"])
@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: f"{s[0]}x{s[1]}")
def test_dynamic_matches_oracle(shape, dtype, fmt, gran):
    x = inputs.randn(shape, dtype, seed=7 * shape[0] + shape[1] + DTYPES.index(dtype))
    _check(x, fmt, gran)


@pytest.mark.parametrize("scale", [0.05, 0.003, 1e-5])
@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
def test_static_matches_oracle_including_overflow(dtype, fmt, scale):
    x = inputs.randn((257, 1030), dtype, seed=3) * 4
    _check(x.to(dtype), fmt, "tensor", scale=scale)


@pytest.mark.parametrize("fmt", FORMATS)
def test_config1_per_token_full_size(fmt):
    m, n = inputs.CONFIG_SHAPES["fp8_token"]
    x = inputs.fp8_token_input(m, n, seed=0)
    _check(x, fmt, "token")


@pytest.mark.parametrize("gran", ["token", "block", "tensor"])
def test_all_zero_gives_zero_codes_and_min_scale(gran):
    x = torch.zeros(256, 256, dtype=torch.float32)
    q, s = fp8_quant(x.cuda(), "e4m3", gran)
    assert torch.all(q.float() == 0)
    assert torch.all(s == torch.tensor(1e-12, dtype=torch.float32).cuda())
    _check(x, "e4m3", gran)


@pytest.mark.parametrize("gran", ["token", "block", "tensor"])
@pytest.mark.parametrize("fmt", FORMATS)
def test_signed_zeros_nan_inf(gran, fmt):
    x = inputs.randn((130, 264), torch.bfloat16, seed=5)
    x[0, :] = -0.0
    x[1, 3] = float("nan")
    x[2, 7] = float("inf")
    x[3, 9] = float("-inf")
    x[4, 1] = -float("nan")
    x[5, 5:9] = 0.0
    x[5, 6] = -0.0
    x[6, :] = 1e-40  # bf16 subnormals
    if gran == "tensor":
        x[1, 3] = 1.0  # a NaN would make every code NaN; keep the tensor case finite + inf
    _check(x, fmt, gran)


@pytest.mark.parametrize("fmt", FORMATS)
def test_static_nan_inf_and_huge(fmt):
    x = inputs.randn((64, 256), torch.float32, seed=7)
    x[0, 0] = float("nan")
    x[1, 1] = float("inf")
    x[2, 2] = -3.0e38
    x[3, :] = 1e30
    _check(x, fmt, "tensor", scale=0.05)


@pytest.mark.parametrize("gran", ["token", "block", "tensor"])
@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
def test_unaligned_input_pointer(gran, dtype):
    m, n = 33, 264
    base = inputs.randn((m * n + 1,), dtype, seed=9)
    x_cpu = base[1:].view(m, n).clone()
    x_dev = base.cuda()[1:].view(m, n)
    assert x_dev.data_ptr() % 16 != 0
    _check(x_cpu, "e4m3", gran, x_dev=x_dev)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16], ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("cols", [64, 512, 1024, 2048, 2560, 3072, 4096, 5120, 6144, 8192, 10240, 12288, 16384, 20480,
                                  24576, 32768, 40960, 49152, 65536])
def test_every_row_shape_bucket(cols, dtype):
    _check(inputs.randn((3, cols), dtype, seed=cols), "e4m3", "token")


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
def test_long_rows_use_looping_path(dtype):
    x = inputs.randn((5, 40000), dtype, seed=11)
    _check(x, "e4m3", "token")


def test_rejects_bad_format_and_granularity():
    x = torch.randn(4, 8, device="cuda")
    with pytest.raises(ValueError):
        fp8_quant(x, "e4m4", "block")
    with pytest.raises(ValueError):
        fp8_quant(x, "e4m3", "row")
    with pytest.raises(ValueError):
        fp8_quant(x, "e4m3", "block", scale=0.1)


# ---- Tensor granularity: the one-pass exchange (workgroup maxima in slots in
# workgroup 0's share of the codes, the scale published in the scale word) and
# the two-pass forms (partial maxima in the codes buffer, a finishing
# atomicMax into the caller's int32 or slot arrays in the cast chunks, then
# the cast), exercised through the C ABI where the Python API cannot reach.

@pytest.mark.parametrize("where", ["first", "middle", "last"])
@pytest.mark.parametrize("shape", [(1, 1), (1, 3), (2, 3), (3, 1001), (4099, 4097), (2048, 4096), (8192, 4096)],
                         ids=lambda s: f"{s[0]}x{s[1]}")
def test_tensor_amax_found_anywhere(shape, where):
    """The largest |x| at the first, middle or last element: sizes below the
    partial-slot minimum, a scalar tail after the 16-byte vectors, a grid of
    512 partial workgroups that each stride over several vectors, and one-pass
    grids (the maximum in workgroup 0's own share, in the middle workgroup's,
    in the last one's)."""
    x = inputs.randn(shape, torch.bfloat16, seed=shape[0] * 31 + shape[1])
    flat = x.view(-1)
    idx = {"first": 0, "middle": flat.numel() // 2, "last": flat.numel() - 1}[where]
    flat[idx] = -1000.0
    _check(x, "e4m3", "tensor")


@pytest.mark.parametrize("via", ["api", "abi"])
@pytest.mark.parametrize("where", ["workgroup0", "last"])
@pytest.mark.parametrize("bits", [0x7F800001, 0xFF800001, 0x7FFFFFFF], ids=["snan1", "neg-snan1", "nan-max"])
def test_tensor_one_pass_nan_patterns_of_the_exchange(bits, where, via):
    """fp32 NaNs on the one-pass path ([2048, 4096]: 512 workgroups) whose
    |x| bits equal the scale word's empty pattern (0x7f800001) or are the
    largest NaN (0x7fffffff, next to the slots' empty pattern 0xffffffff), in
    workgroup 0's share or the last workgroup's: the exchange ends, the scale
    is NaN and every code equals the oracle's; through the reference ABI the
    int32 ends up holding a NaN's bits."""
    x = inputs.randn((2048, 4096), torch.float32, seed=91)
    idx = 5 if where == "workgroup0" else x.numel() - 5
    x.view(-1).view(torch.int32)[idx] = int(np.array([bits], dtype=np.uint32).view(np.int32)[0])
    if via == "api":
        _check(x, "e4m3", "tensor")
        return
    q = torch.empty(x.shape, dtype=torch.uint8, device="cuda")
    word = torch.zeros(1, dtype=torch.int32, device="cuda")
    scale = _tensor_abi(x.cuda(), q, word)
    codes, s_ref = ofp8.quant_tensor(x.numpy(), "e4m3")
    assert_codes_equal(q, codes)
    assert_f32_bits_equal(scale, s_ref)
    assert np.isnan(s_ref).all() and (int(word.item()) & 0x7FFFFFFF) > 0x7F800000


def _tensor_abi(x_dev: torch.Tensor, q: torch.Tensor, scratch: torch.Tensor | None, fmt_tag: int = 3):
    from tests import _cck

    lib = _cck.load()
    scale = torch.empty(1, dtype=torch.float32, device="cuda")
    m, n = x_dev.shape
    dtag = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}[x_dev.dtype]
    rc = lib.launch_fp8_quant_tensor_fwd(x_dev.data_ptr(), q.data_ptr(), scale.data_ptr(),
                                         None if scratch is None else scratch.data_ptr(), m, n,
                                         dtag, fmt_tag, torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    return scale


# (shape, what it reaches for bf16 / fp16; fp32 alike unless noted). The
# one-pass form takes inputs of at most 2048 vectors (one workgroup) and of at
# least 2^20 vectors; beyond what a resident grid holds in registers it
# streams the rest of each workgroup's chunk.
TENSOR_PATHS = [
    ((1024, 4096), "bf16/fp16: slot arrays in every cast chunk, XCD-aligned cast order; fp32: the finishing launch"),
    ((300, 4096), "slot arrays written by 75 partial workgroups (not a multiple of 8), chunks walked last-first"),
    ((2048, 4096), "one pass (config 1): 2 vectors per thread over 512 workgroups (fp32: 4)"),
    ((4096, 4096), "one pass: 4 vectors per thread over 512 workgroups (fp32: 16 over 256)"),
    ((8192, 4096), "one pass: 16 vectors per thread over 256 workgroups, the register capacity (fp32: beyond it)"),
    ((4097, 8200), "beyond the register capacity: each resident workgroup holds 16 vectors per thread of its chunk "
                   "and streams the rest twice; the last chunk partial"),
    ((4099, 4097), "two passes: the finishing launch, a scalar tail after the vectors"),
    ((4, 20482), "last cast chunk too short for a slot array: the finishing launch"),
    ((5, 2056), "one pass in one workgroup, no exchange (fp32: two passes, slot arrays)"),
    ((2, 3), "bf16/fp16: no whole vector, the finishing launch over scalars; fp32: a one-word slot array, a tail"),
    ((1, 8), "one vector: one pass in one workgroup"),
    ((1, 3), "too small for one slot: the one-workgroup amax"),
]


@pytest.mark.parametrize("scratch", ["zeroed", "preset", "none"])
@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("shape", [s for s, _ in TENSOR_PATHS], ids=lambda s: f"{s[0]}x{s[1]}")
def test_tensor_paths_through_the_abi(shape, dtype, scratch):
    """Each of the launcher's paths, with the caller's int32 zeroed (the
    reference's contract), preset above the tensor's amax (which then sets the
    scale) and absent (NULL): codes and scale bit-exact, the int32 left at
    max(initial, amax bits), and nothing written outside the codes buffer."""
    x = inputs.randn(shape, dtype, seed=shape[0] * 7 + shape[1])
    x.view(-1)[x.numel() // 3] = 30.0
    x32 = x.float().numpy()
    amax = np.float32(np.abs(x32).max())
    m, n = shape
    buf = torch.full((m * n + 512,), 0x55, dtype=torch.uint8, device="cuda")
    q = buf[256:256 + m * n].view(m, n)
    init = {"zeroed": 0, "preset": int(np.array([1000.0], dtype=np.float32).view(np.int32)[0]), "none": None}[scratch]
    word = None if init is None else torch.tensor([init], dtype=torch.int32, device="cuda")
    scale = _tensor_abi(x.cuda(), q, word)
    if scratch == "preset":
        s_ref = np.float32(np.float32(1000.0) / np.float32(448.0))
        assert_f32_bits_equal(scale, np.array([s_ref], dtype=np.float32))
        assert_codes_equal(q, ofp8.quant_static(x32, float(s_ref), "e4m3"))
    else:
        codes, s_ref = ofp8.quant_tensor(x32, "e4m3")
        assert_codes_equal(q, codes)
        assert_f32_bits_equal(scale, s_ref)
    if word is not None:
        want = max(init, int(np.array([amax], dtype=np.float32).view(np.int32)[0]))
        assert int(word.item()) == want
    b = buf.cpu().numpy()
    assert (b[:256] == 0x55).all() and (b[256 + m * n:] == 0x55).all(), "wrote outside the codes buffer"


@pytest.mark.parametrize("offset", [1, 2, 3])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=lambda d: str(d).split(".")[-1])
def test_tensor_codes_buffer_unaligned(offset, dtype):
    """A codes buffer that is not 4-byte aligned: the partial slots are placed
    at the first aligned word inside it, and every code is still written."""
    m, n = 700, 1003
    x = inputs.randn((m, n), dtype, seed=offset)
    buf = torch.full((m * n + 8,), 0x55, dtype=torch.uint8, device="cuda")
    q = buf[offset:offset + m * n]
    assert q.data_ptr() % 4 != 0
    scratch = torch.zeros(1, dtype=torch.int32, device="cuda")
    scale = _tensor_abi(x.cuda(), q, scratch)
    codes, s_ref = ofp8.quant_tensor(x.float().numpy(), "e4m3")
    assert_codes_equal(q, codes.reshape(-1))
    assert_f32_bits_equal(scale, s_ref)
    b = buf.cpu().numpy()
    assert (b[:offset] == 0x55).all() and (b[offset + m * n:] == 0x55).all(), "wrote outside the codes buffer"


@pytest.mark.parametrize("shape", [(2, 3), (4096, 4096)], ids=lambda s: f"{s[0]}x{s[1]}")
def test_tensor_scratch_holds_atomic_max(shape):
    """The reference atomicMax-es the tensor's max |x| bits into the caller's
    int32 (fp8_quant.cu:159-234): afterwards it holds those bits when it was
    zeroed, and max(initial, amax) bits otherwise, which then sets the scale."""
    x = inputs.randn(shape, torch.bfloat16, seed=11)
    x32 = x.float().numpy()
    amax = np.float32(np.abs(x32).max())
    q = torch.empty(shape, dtype=torch.uint8, device="cuda")
    scratch = torch.zeros(1, dtype=torch.int32, device="cuda")
    _tensor_abi(x.cuda(), q, scratch)
    assert int(scratch.item()) == int(np.array([amax], dtype=np.float32).view(np.int32)[0])
    preset = np.float32(1000.0)
    scratch = torch.tensor(np.array([preset], dtype=np.float32).view(np.int32), device="cuda")
    scale = _tensor_abi(x.cuda(), q, scratch)
    s_ref = np.float32(preset / np.float32(448.0))
    assert_f32_bits_equal(scale, np.array([s_ref], dtype=np.float32))
    assert_codes_equal(q, ofp8.quant_static(x32, float(s_ref), "e4m3"))


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("shape", [(200, 264), (129, 136), (1, 8), (300, 1024)], ids=lambda s: f"{s[0]}x{s[1]}")
def test_block_ragged_tiles_vector_path(shape, dtype):
    """Row and column counts that are not multiples of the 128x128 tile but
    keep 16-byte rows (the register-resident block kernel, not the scalar one)."""
    _check(inputs.randn(shape, dtype, seed=shape[0] + shape[1]), "e4m3", "block")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=lambda d: str(d).split(".")[-1])
def test_block_rows_beyond_32bit_tile_offsets(dtype):
    """Rows so long that 128 of them exceed 2 GiB: the block kernel addresses
    them with 64-bit pointers instead of 32-bit buffer offsets."""
    n = (1 << 31) // (128 * (4 if dtype == torch.float32 else 2)) + 128
    _check(inputs.randn((2, n), dtype, seed=3), "e4m3", "block")


def test_block_scales_keep_a_small_tile_resolved_next_to_an_outlier_tile():
    """The kernels' block and tensor outputs, dequantised with the library's
    own fp8_format.dequantize: the small tile next to an outlier tile keeps a
    smaller error under 128x128 scales (as the oracle test of the same name)."""
    from custom_cuda_kernals_amd.fp8_format import dequantize

    g = torch.Generator().manual_seed(11)
    x = torch.zeros(256, 256)
    x[:128, :128] = torch.randn(128, 128, generator=g) * 0.01
    x[128:, 128:] = torch.randn(128, 128, generator=g) * 100.0
    xd = x.cuda()
    errs = {}
    for gran in ("tensor", "block"):
        q, s = fp8_quant(xd, "e4m3", gran)
        deq = dequantize(q, s, gran).cpu()
        errs[gran] = float((deq[:128, :128] - x[:128, :128]).abs().mean())
    assert errs["block"] * 2 < errs["tensor"], errs


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
def test_block_two_tile_workgroups_on_large_ragged_input(dtype):
    """At >= 16384 tiles the block kernel runs two tiles side by side per
    workgroup. 131 x 131 tiles with a ragged last row and column of tiles
    (the last workgroup of each tile row has one tile past the edge): a tile's
    codes and scale depend only on that tile, so sampled tiles (corners, edges,
    random) are checked against the oracle, and every scale is checked for
    finiteness and position."""
    m, n = 128 * 130 + 17, 128 * 130 + 8
    g = torch.Generator(device="cuda").manual_seed(5)
    x = torch.randn(m, n, device="cuda", dtype=torch.float32, generator=g).to(dtype)
    q, s = fp8_quant(x, "e4m3", "block")
    torch.cuda.synchronize()
    assert tuple(s.shape) == (131, 131) and bool(torch.isfinite(s).all()) and bool((s > 0).all())
    rng = np.random.default_rng(3)
    tiles = {(0, 0), (0, 130), (130, 0), (130, 130), (65, 129), (129, 65), (130, 1), (1, 130)}
    tiles |= {(int(a), int(b)) for a, b in rng.integers(0, 131, size=(24, 2))}
    for ti, tj in sorted(tiles):
        r0, c0 = ti * 128, tj * 128
        xt = x[r0:r0 + 128, c0:c0 + 128].float().cpu().numpy()
        codes, s_ref = ofp8.quant_tensor(xt, "e4m3")
        assert_codes_equal(q[r0:r0 + 128, c0:c0 + 128].contiguous(), codes, f"tile {ti},{tj}")
        assert_f32_bits_equal(s[ti, tj].reshape(1), s_ref, f"scale {ti},{tj}")
