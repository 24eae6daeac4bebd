"""Benchmark of the MI355X activation path (one GPU).

Metric: achieved HBM TB/s and fraction of the 8 TB/s peak per
op. A "step" is one launch of an op over one batch of synthetic input that is
already resident in HBM. Each op is timed over exactly --steps launches
captured in one HIP graph (so host-side validation and launch latency are not
in the window), bracketed by torch.cuda.synchronize() and HIP events on the
stream the kernels run on, after the --warmup eager launches and untimed
replays of the graph for 0.15 s (GPU clocks ramp up under sustained load).
Every launch of a timed run uses a different set of input/output buffers,
rotating over enough sets that the working set is >= 2 GiB, so no step can be
served from the 256 MB Infinity Cache left warm by the previous one. Where
that takes more sets than --steps (ops whose set is under 2 GiB / steps), the
graph launches the op once per set, up to 16384 sets, and the op's time is
the replay's over that many launches, so the replays before the timed one
leave none of its buffers on chip. The headline op and every BASELINE config
op take exactly --steps launches (their sets are over 21 MB); only the small
MoE ops take more.

Each op also reports "per_call": the reference's own methodology (a cache
flush before every call, HIP events around one call through the binding, so
validation and launch latency are inside the window), as median and IQR.

The headline `value` is the BASELINE config-2 workload (fused RMSNorm +
residual, bf16 [8192, 4096]); every other config's op is reported under "ops".
Achieved bandwidth = algorithmic bytes per launch / average launch duration.

"ceilings" holds the practical ceiling of six config ops' traffic on this
GPU: pure streams with the same bytes per element and row structure and no
arithmetic (cck_hbm_stream), timed the same way, with each op's fraction of
its stream.

The CPU baseline (rank 0, N=1) times the CPU oracle - the torch-CPU
restatement of the reference's eager op (baselines/rmsnorm_residual.py) - on a
bounded sample of the same workload on this host's cores.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_GBPS = 8000.0
ROTATE_BYTES = 2 << 30
MAX_SETS = 16384  # >= 512 MB of rotation down to 32 KB sets, twice the Infinity Cache
WARM_S = 0.15


def _parse():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=100)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--ops", default="all", help="comma-separated op names, or 'all'")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=15.0, help="CPU-baseline time budget")
    p.add_argument("--no-graph", action="store_true",
                   help="launch the timed steps eagerly instead of replaying a captured HIP graph "
                        "(for counter-collection runs; includes host launch overhead)")
    p.add_argument("--block", action="store_true",
                   help="also time the Llama-3-8B decoder block (eager / fused / fp8) at S=4096")
    p.add_argument("--block-model", default="llama3-8b", choices=["llama3-8b", "llama3-70b"],
                   help="layer shapes of the --block decoder block (llama3-70b: hidden 8192, FFN 28672)")
    p.add_argument("--no-ceilings", action="store_true",
                   help="skip the practical-ceiling streams (pure traffic with six config ops' byte patterns)")
    p.add_argument("--markers", action="store_true",
                   help="wrap each op's timed graph replay in a ROCTx range named 'timed:<op>', so a "
                        "rocprofv3 --marker-trace --kernel-trace run can select exactly the timed dispatches")
    p.add_argument("--suite", choices=["configs", "reference"], default="configs",
                   help="reference: instead of the BASELINE configs, every case of the reference's own benchmark "
                        "lists (benchmarks/*_bench.py) in its three dtypes; --ops then names families "
                        "(rmsnorm_residual, swiglu, rope, fp8_quant, moe_router, token_gather, token_combine)")
    p.add_argument("--copy-calibration", action="store_true",
                   help="also run a 256 MiB device-to-device torch copy, the reference kernel "
                        "for scaling FETCH_SIZE / WRITE_SIZE counters")
    return p.parse_args()


def _c_lib():
    """The library's C ABI through ctypes (for entry points the Python binding
    does not wrap: the no-allocation FP8 launcher and the HBM streams)."""
    import ctypes

    lib = ctypes.CDLL(os.path.join(ROOT, "custom_cuda_kernals_amd", "libcustom_kernels_amd.so"))
    fn = lib.launch_fp8_quant_tensor_noalloc_fwd
    fn.restype = ctypes.c_int32
    fn.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int64] * 2 + [ctypes.c_int32] * 2 + [ctypes.c_void_p]
    fn = lib.cck_hbm_stream
    fn.restype = ctypes.c_int32
    fn.argtypes = [ctypes.c_int32] + [ctypes.c_void_p] * 4 + [ctypes.c_int64, ctypes.c_void_p]
    return lib


class _Markers:
    """ROCTx ranges (rocprofiler-sdk's roctx library) around the timed regions;
    a no-op when not requested."""

    def __init__(self, enabled):
        self.lib = None
        if enabled:
            import ctypes

            for name in ("librocprofiler-sdk-roctx.so.1", "libroctx64.so.4"):
                try:
                    self.lib = ctypes.CDLL(os.path.join("/opt/rocm/lib", name))
                    break
                except OSError:
                    continue
            if self.lib is None:
                raise RuntimeError("--markers: no ROCTx library under /opt/rocm/lib")
            self.lib.roctxRangePushA.argtypes = [ctypes.c_char_p]
            self.lib.roctxRangePushA.restype = ctypes.c_int
            self.lib.roctxRangePop.restype = ctypes.c_int

    def push(self, name):
        if self.lib is not None:
            self.lib.roctxRangePushA(name.encode())

    def pop(self):
        if self.lib is not None:
            self.lib.roctxRangePop()


MARKERS = _Markers(False)


def _ensure_built():
    from custom_cuda_kernals_amd import build

    if not build.is_built():
        build.build_all()


class Op:
    """One benchmarked op: a buffer-set factory, a launch on set i, algorithmic bytes."""

    def __init__(self, name, workload, nbytes, make_set, launch, set_bytes, shape=None):
        self.name, self.workload, self.nbytes = name, workload, nbytes
        self.make_set, self.launch, self.set_bytes = make_set, launch, set_bytes
        self.shape = shape


def _ops(torch, native):
    dev = "cuda"
    bf16 = torch.bfloat16
    f8 = torch.float8_e4m3fn
    g = torch.Generator(device=dev).manual_seed(0)

    def rn(*shape, dtype=bf16):
        return torch.randn(shape, device=dev, dtype=torch.float32, generator=g).to(dtype)

    ops = []

    # 1: per-token FP8, X [2048, 4096] bf16 with 0.1 % outliers x50
    m1, n1 = 2048, 4096

    def mk1():
        x = rn(m1, n1)
        idx = torch.randperm(m1 * n1, device=dev, generator=g)[: round(0.001 * m1 * n1)]
        x.view(-1)[idx] *= 50
        return dict(x=x, q=torch.empty(m1, n1, dtype=f8, device=dev), s=torch.empty(m1, device=dev))

    ops.append(Op("fp8_quant_token", "fp8_token_bf16_2048x4096", m1 * n1 * 3 + m1 * 4, mk1,
                  lambda b: native.fp8_quant_token_fwd(b["x"], b["q"], b["s"], "e4m3"), m1 * n1 * 3, [m1, n1]))

    # The reference's own two granularities on the config-1 input (drop-ins, not BASELINE
    # configs): 128x128 tiles, and one dynamic scale for the tensor, whose caller-zeroed
    # int32 amax scratch is cleared inside the timed op as the reference's wrapper does
    # (custom_cuda/kernels/fp8_quant.py:51-62).
    tiles = (math.ceil(m1 / 128), math.ceil(n1 / 128))

    def mk1g():
        d = mk1()
        d.update(sb=torch.empty(tiles, device=dev), st=torch.empty(1, device=dev),
                 amax=torch.zeros(1, dtype=torch.int32, device=dev))
        return d

    def tensor_fp8(b):
        b["amax"].zero_()
        native.fp8_quant_tensor_fwd(b["x"], b["q"], b["st"], b["amax"], "e4m3")

    ops.append(Op("fp8_quant_block", "fp8_block128_bf16_2048x4096", m1 * n1 * 3 + tiles[0] * tiles[1] * 4, mk1g,
                  lambda b: native.fp8_quant_block_fwd(b["x"], b["q"], b["sb"], "e4m3"), m1 * n1 * 3, [m1, n1]))
    ops.append(Op("fp8_quant_tensor", "fp8_tensor_bf16_2048x4096", m1 * n1 * 3 + 8, mk1g, tensor_fp8, m1 * n1 * 3,
                  [m1, n1]))

    # The same op as the Python API runs it (fp8_quant(x, "e4m3", "tensor")): no
    # amax word, so no zero-fill.
    ops.append(Op("fp8_quant_tensor_api", "fp8_tensor_api_bf16_2048x4096", m1 * n1 * 3 + 4, mk1g,
                  lambda b: native.fp8_quant_tensor_fwd(b["x"], b["q"], b["st"], None, "e4m3"), m1 * n1 * 3,
                  [m1, n1]))

    # The same tensor granularity through the no-allocation C entry point
    # (no amax scratch, no zero-fill; library-owned partial slots).
    lib = _c_lib()

    def tensor_noalloc(b):
        rc = lib.launch_fp8_quant_tensor_noalloc_fwd(b["x"].data_ptr(), b["q"].data_ptr(), b["st"].data_ptr(), m1, n1,
                                                      2, 3, torch.cuda.current_stream().cuda_stream)
        if rc != 0:
            raise RuntimeError(f"launch_fp8_quant_tensor_noalloc_fwd failed, hipError_t = {rc}")

    ops.append(Op("fp8_quant_tensor_noalloc", "fp8_tensor_noalloc_bf16_2048x4096", m1 * n1 * 3 + 4, mk1g,
                  tensor_noalloc, m1 * n1 * 3, [m1, n1]))

    # One dynamic scale through the reference ABI at [8192, 4096] bf16 (not a
    # BASELINE config): the input the one-pass form holds at its register
    # capacity (16 vectors per thread over 256 workgroups on MI355X).
    m1t, n1t = 8192, 4096

    def mk1t():
        return dict(x=rn(m1t, n1t), q=torch.empty(m1t, n1t, dtype=f8, device=dev), st=torch.empty(1, device=dev),
                    amax=torch.zeros(1, dtype=torch.int32, device=dev))

    ops.append(Op("fp8_quant_tensor_8192x4096", "fp8_tensor_bf16_8192x4096", m1t * n1t * 3 + 8, mk1t, tensor_fp8,
                  m1t * n1t * 3, [m1t, n1t]))

    # Static scale 0.05 on its own (config 5's static mode fuses it into the producers).
    m1s, n1s = 16384, 4096

    def mk1s():
        return dict(x=rn(m1s, n1s), q=torch.empty(m1s, n1s, dtype=f8, device=dev))

    ops.append(Op("fp8_quant_static", "fp8_static0.05_bf16_16384x4096", m1s * n1s * 3, mk1s,
                  lambda b: native.fp8_quant_static_fwd(b["x"], b["q"], 0.05, "e4m3"), m1s * n1s * 3, [m1s, n1s]))

    # 2: RMSNorm + residual, [8192, 4096] bf16, eps 1e-5
    m2, n2 = 8192, 4096
    w2 = (1.0 + 0.1 * torch.randn(n2, device=dev, generator=g)).to(bf16)

    def mk2():
        return dict(x=rn(m2, n2), r=rn(m2, n2), y=torch.empty(m2, n2, dtype=bf16, device=dev),
                    ro=torch.empty(m2, n2, dtype=bf16, device=dev))

    ops.append(Op("rmsnorm_residual", "rmsnorm_residual_bf16_8192x4096", m2 * n2 * 8 + n2 * 2, mk2,
                  lambda b: native.rmsnorm_residual_fwd(b["x"], b["r"], w2, b["y"], b["ro"], 1e-5), m2 * n2 * 8,
                  [m2, n2]))

    # 3 / 3v: SwiGLU [8192, 14336] bf16, and SwiGLU + per-token FP8
    m3, n3 = 8192, 14336

    def mk3():
        return dict(g=rn(m3, n3), u=rn(m3, n3), y=torch.empty(m3, n3, dtype=bf16, device=dev),
                    q=torch.empty(m3, n3, dtype=f8, device=dev), s=torch.empty(m3, device=dev))

    ops.append(Op("swiglu", "swiglu_bf16_8192x14336", m3 * n3 * 6, mk3,
                  lambda b: native.swiglu_fwd(b["g"], b["u"], b["y"]), m3 * n3 * 6, [m3, n3]))
    ops.append(Op("swiglu_fp8_token", "swiglu_fp8_token_bf16_8192x14336", m3 * n3 * 5 + m3 * 4, mk3,
                  lambda b: native.swiglu_fp8_fwd(b["g"], b["u"], b["q"], b["s"], "e4m3", None), m3 * n3 * 5,
                  [m3, n3]))

    # 4: RoPE in place, q [8,4096,32,128], k [8,4096,8,128] bf16, theta 5e5
    B, S, HQ, HKV, D = 8, 4096, 32, 8, 128
    inv = 1.0 / (500000.0 ** (torch.arange(0, D, 2, dtype=torch.float32, device=dev) / D))
    ang = torch.outer(torch.arange(S, dtype=torch.float32, device=dev), inv)
    cos4, sin4 = ang.cos().contiguous(), ang.sin().contiguous()
    rope_elems = B * S * (HQ + HKV) * D

    def mk4():
        return dict(q=rn(B, S, HQ, D), k=rn(B, S, HKV, D))

    ops.append(Op("rope_inplace", "rope_bf16_q8x4096x32x128_k8x4096x8x128", rope_elems * 4 + 2 * S * (D // 2) * 4, mk4,
                  lambda b: native.rope_fwd(b["q"], b["k"], cos4, sin4, b["q"], b["k"]), rope_elems * 4,
                  [B, S, HQ, HKV, D]))

    # 5a / 5b: T = 16384 chain, per-token and static 0.05
    m5, n5a, n5b = 16384, 4096, 14336
    w5 = (1.0 + 0.1 * torch.randn(n5a, device=dev, generator=g)).to(bf16)

    def mk5a():
        return dict(x=rn(m5, n5a), r=rn(m5, n5a), q=torch.empty(m5, n5a, dtype=f8, device=dev),
                    ro=torch.empty(m5, n5a, dtype=bf16, device=dev), s=torch.empty(m5, device=dev))

    def mk5b():
        return dict(g=rn(m5, n5b), u=rn(m5, n5b), q=torch.empty(m5, n5b, dtype=f8, device=dev),
                    s=torch.empty(m5, device=dev))

    e5a, e5b = m5 * n5a, m5 * n5b
    ops.append(Op("rmsnorm_residual_fp8_token", "chain_rmsnorm_fp8_token_bf16_16384x4096",
                  e5a * 7 + m5 * 4 + n5a * 2, mk5a,
                  lambda b: native.rmsnorm_residual_fp8_fwd(b["x"], b["r"], w5, b["q"], b["s"], b["ro"], 1e-5, "e4m3", None),
                  e5a * 7, [m5, n5a]))
    ops.append(Op("swiglu_fp8_token_T16384", "chain_swiglu_fp8_token_bf16_16384x14336", e5b * 5 + m5 * 4, mk5b,
                  lambda b: native.swiglu_fp8_fwd(b["g"], b["u"], b["q"], b["s"], "e4m3", None), e5b * 5, [m5, n5b]))
    ops.append(Op("rmsnorm_residual_fp8_static", "chain_rmsnorm_fp8_static0.05_bf16_16384x4096",
                  e5a * 7 + n5a * 2, mk5a,
                  lambda b: native.rmsnorm_residual_fp8_fwd(b["x"], b["r"], w5, b["q"], None, b["ro"], 1e-5, "e4m3", 0.05),
                  e5a * 7, [m5, n5a]))
    ops.append(Op("swiglu_fp8_static_T16384", "chain_swiglu_fp8_static0.05_bf16_16384x14336", e5b * 5, mk5b,
                  lambda b: native.swiglu_fp8_fwd(b["g"], b["u"], b["q"], None, "e4m3", 0.05), e5b * 5, [m5, n5b]))

    # MoE dispatch (the reference's standard cases, baselines/token_permute.py:128-146 and
    # baselines/moe_router.py:72-79): not BASELINE configs; reported beside them.
    gs, gd, gh = 2048, 4096, 4096

    def mkg():
        return dict(src=rn(gs, gh), idx=torch.randint(0, gs, (gd,), device=dev, generator=g),
                    dst=torch.empty(gd, gh, dtype=bf16, device=dev))

    ops.append(Op("token_gather", "moe_gather_bf16_2048to4096x4096", gd * gh * 4 + gd * 8, mkg,
                  lambda b: native.token_gather_fwd(b["src"], b["idx"], b["dst"]), gs * gh * 2 + gd * gh * 2,
                  [gs, gd, gh]))
    for ck in (2, 6):
        ct, ch = 2048, 4096

        def mkc(ck=ck, ct=ct, ch=ch):
            return dict(eo=rn(ct * ck, ch), ui=torch.randperm(ct * ck, device=dev, generator=g).view(ct, ck),
                        w=torch.rand(ct, ck, device=dev, generator=g), out=torch.empty(ct, ch, dtype=bf16, device=dev))

        ops.append(Op(f"token_combine_k{ck}", f"moe_combine_bf16_T{ct}_k{ck}x{ch}", ct * ck * ch * 2 + ct * ch * 2 + ct * ck * 12,
                      mkc, lambda b: native.token_combine_fwd(b["eo"], b["ui"], b["w"], b["out"]),
                      ct * ck * ch * 2 + ct * ch * 2, [ct, ck, ch]))
    rt, re_, rk = 2048, 160, 6

    def mkr():
        return dict(lg=rn(rt, re_, dtype=torch.float32), w=torch.empty(rt, rk, device=dev),
                    i=torch.empty(rt, rk, dtype=torch.int64, device=dev))

    ops.append(Op("moe_router", "moe_router_f32_2048x160_top6", rt * re_ * 4 + rt * rk * 12, mkr,
                  lambda b: native.moe_router_fwd(b["lg"], b["w"], b["i"], True), rt * re_ * 4, [rt, re_, rk]))
    # The reference benchmark's Mixtral-shaped case (benchmarks/moe_router_bench.py:40): one lane per token.
    mt, me, mk = 4096, 8, 2

    def mkr8():
        return dict(lg=rn(mt, me, dtype=torch.float32), w=torch.empty(mt, mk, device=dev),
                    i=torch.empty(mt, mk, dtype=torch.int64, device=dev))

    ops.append(Op("moe_router_e8", "moe_router_f32_4096x8_top2", mt * me * 4 + mt * mk * 12, mkr8,
                  lambda b: native.moe_router_fwd(b["lg"], b["w"], b["i"], True), mt * me * 4, [mt, me, mk]))

    # The index bookkeeping between them (compute_permutation with num_experts):
    # the router's [2048, 6] expert ids in, permute / unpermute int64 out.
    def mkp():
        return dict(ids=torch.randint(0, re_, (rt, rk), device=dev, generator=g),
                    p=torch.empty(rt * rk, dtype=torch.int64, device=dev),
                    u=torch.empty(rt, rk, dtype=torch.int64, device=dev))

    ops.append(Op("moe_permutation", "moe_permutation_2048x6_of_160", rt * rk * 24, mkp,
                  lambda b: native.moe_permutation_fwd(b["ids"], b["p"], b["u"], re_), rt * rk * 24, [rt, rk, re_]))
    return ops


def _time_op(torch, op, steps, warmup, use_graph=True, per_call=True):
    nsets = min(MAX_SETS, max(2, math.ceil(ROTATE_BYTES / op.set_bytes)))
    sets = [op.make_set() for _ in range(nsets)]
    launches = max(steps, nsets)
    torch.cuda.synchronize()
    for i in range(warmup):
        op.launch(sets[i % nsets])
    torch.cuda.synchronize()
    if not use_graph:
        stream = torch.cuda.current_stream()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for i in range(steps):
            op.launch(sets[i % nsets])
        end.record(stream)
        torch.cuda.synchronize()
        ms = start.elapsed_time(end)
        us = ms * 1000.0 / steps
        del sets
        torch.cuda.empty_cache()
        return {"workload": op.workload, "shape": op.shape, "us": round(us, 3),
                "GB_per_s": round(op.nbytes / (us * 1e-6) / 1e9, 1), "steps": steps, "graph": False}
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            for i in range(launches):
                op.launch(sets[i % nsets])
    torch.cuda.current_stream().wait_stream(side)
    graph.replay()  # untimed replay: first replay uploads the graph
    torch.cuda.synchronize()
    # Untimed replays until the GPU has been busy for WARM_S: the clocks ramp
    # up under sustained load, and the first replays after a capture measured
    # up to 10 % slower than the settled ones (48.2, 45.1, 44.0, 43.6 us per
    # step for RMSNorm at config 2 on MI355X).
    t_end = time.perf_counter() + WARM_S
    for _ in range(1000):
        if time.perf_counter() >= t_end:
            break
        graph.replay()
        torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    MARKERS.push(f"timed:{op.name}")
    start.record(stream)
    graph.replay()
    end.record(stream)
    torch.cuda.synchronize()
    MARKERS.pop()
    ms = start.elapsed_time(end)
    us = ms * 1000.0 / launches
    gbps = op.nbytes / (us * 1e-6) / 1e9
    del graph
    per_call = _per_call_us(torch, op, sets) if per_call else None
    del sets
    torch.cuda.empty_cache()
    return {"workload": op.workload, "shape": op.shape, "us": round(us, 3), "GB_per_s": round(gbps, 1),
            "frac_of_8TBps": round(gbps / PEAK_GBPS, 4), "algorithmic_bytes": op.nbytes,
            "steps": launches, "buffer_sets": nsets, "total_ms": round(ms, 4), "per_call": per_call}


def _ceilings(torch, steps, warmup):
    """Practical HBM ceilings on this GPU: pure traffic streams with the byte
    pattern of six config ops (cck_hbm_stream, csrc/calibrate.hip: 16-byte
    nontemporal vectors, no arithmetic), timed exactly like the ops. An op's
    fraction of the 8 TB/s peak reads against its pattern's fraction here."""
    fn = _c_lib().cck_hbm_stream
    u8 = torch.uint8
    # (name, pattern, op it bounds, vectors per input stream, input streams, output bytes per vector)
    cases = [
        ("copy_1r1w", 0, "rope_inplace", 8 * 4096 * 40 * 128 * 2 // 16, 1, 16),
        ("stream_2r1w", 1, "swiglu", 8192 * 14336 * 2 // 16, 2, 16),
        ("rows_2r2w_barrier", 2, "rmsnorm_residual", 8192 * 4096 * 2 // 16, 2, 32),
        ("stream_r16w8", 3, "fp8_quant_token", 2048 * 4096 * 2 // 16, 1, 8),
        ("rows_2r_w8", 4, "swiglu_fp8_token", 8192 * 14336 * 2 // 16, 2, 8),
        ("rows_2r_w16_w8", 5, "rmsnorm_residual_fp8_token", 16384 * 4096 * 2 // 16, 2, 24),
    ]
    out = {}
    for name, pattern, bounds, nv, reads, wbytes in cases:
        def make_set(nv=nv, reads=reads, wbytes=wbytes):
            s = {"a": torch.empty(nv * 16, dtype=u8, device="cuda"),
                 "c": torch.empty(nv * min(wbytes, 16), dtype=u8, device="cuda")}
            if reads == 2:
                s["b"] = torch.empty(nv * 16, dtype=u8, device="cuda")
            if wbytes > 16:
                s["d"] = torch.empty(nv * (wbytes - 16), dtype=u8, device="cuda")
            return s

        def launch(s, pattern=pattern, nv=nv):
            ptr = lambda k: s[k].data_ptr() if k in s else None
            rc = fn(pattern, ptr("a"), ptr("b"), ptr("c"), ptr("d"), nv, torch.cuda.current_stream().cuda_stream)
            if rc != 0:
                raise RuntimeError(f"cck_hbm_stream failed, hipError_t = {rc}")

        nbytes = nv * (16 * reads + wbytes)
        op = Op(name, f"hbm_{name}", nbytes, make_set, launch, nbytes, None)
        r = _time_op(torch, op, steps, warmup, per_call=False)
        out[name] = {"bounds": bounds, "us": r["us"], "GB_per_s": r["GB_per_s"], "frac_of_8TBps": r["frac_of_8TBps"],
                     "bytes": nbytes}
    return out


def _anchors(torch, steps, warmup):
    """Vendor kernels with config 1's traffic, timed exactly like the ops: the
    floor of a cold 24 MiB launch is set by launch ramp and DRAM latency, not
    by bandwidth, so it is anchored on PyTorch's own kernels on the same GPU.
    torch_bf16_to_fp8: `q.copy_(x)`, the elementwise bf16 -> float8_e4m3fn
    conversion (reads 16 MiB, writes 8 MiB, exactly config 1's bytes);
    torch_copy_16MiB: a same-dtype 16 MiB device copy (reads and writes 16 MiB)."""
    m, n = 2048, 4096

    def make_set():
        return {"x": torch.randn(m, n, device="cuda").to(torch.bfloat16),
                "q": torch.empty(m, n, dtype=torch.float8_e4m3fn, device="cuda"),
                "y": torch.empty(m, n, dtype=torch.bfloat16, device="cuda")}

    cases = [("torch_bf16_to_fp8", lambda b: b["q"].copy_(b["x"]), m * n * 3),
             ("torch_copy_16MiB", lambda b: b["y"].copy_(b["x"]), m * n * 4)]
    out = {}
    for name, launch, nbytes in cases:
        op = Op(name, f"{name}_2048x4096", nbytes, make_set, launch, m * n * 5, [m, n])
        r = _time_op(torch, op, steps, warmup, per_call=False)
        out[name] = {"bounds": "fp8_quant_token", "us": r["us"], "GB_per_s": r["GB_per_s"],
                     "frac_of_8TBps": r["frac_of_8TBps"], "bytes": nbytes}

    # The reference's own bookkeeping (baselines/token_permute.py:55-70: a
    # stable torch.argsort and its inverse) on the same [2048, 6] ids.
    from custom_cuda_kernals_amd.kernels import compute_permutation

    t, k, e = 2048, 6, 160

    def make_ids():
        return {"ids": torch.randint(0, e, (t, k), device="cuda")}

    op = Op("torch_compute_permutation", "moe_permutation_2048x6_of_160", t * k * 24, make_ids,
            lambda b: compute_permutation(b["ids"]), t * k * 24, [t, k, e])
    r = _time_op(torch, op, steps, warmup, per_call=False)
    out["torch_compute_permutation"] = {"bounds": "moe_permutation", "us": r["us"], "GB_per_s": r["GB_per_s"],
                                        "frac_of_8TBps": r["frac_of_8TBps"], "bytes": t * k * 24}
    return out


# Fractions of peak the reference publishes for a named case of its own
# benchmarks (RTX 4070 Laptop GPU, 256 GB/s; project_plan.md:701-702, 726-733).
REFERENCE_PUBLISHED = {("swiglu", "bs2_seq2048_d11008", "float16"): 0.855,
                       ("rope", "batchsweep_16", "float16"): 0.831}


def _reference_suite(torch, native):
    """The reference's own benchmark case lists (benchmarks/{rmsnorm_residual,
    swiglu,rope,fp8_quant,moe_router,token_permute}_bench.py), every case in
    the three dtypes they run, through this library's launchers, with the
    reference's bytes (`_ideal_bytes_moved`: weight and cos/sin tables left
    out, FP8 scales left out, router outputs counted). Yields (family, case,
    dtype name, Op)."""
    dev = "cuda"
    g = torch.Generator(device=dev).manual_seed(0)
    dts = (("float32", torch.float32), ("float16", torch.float16), ("bfloat16", torch.bfloat16))

    def rn(shape, dt):
        return torch.randn(shape, device=dev, dtype=torch.float32, generator=g).to(dt)

    def op(name, nbytes, make, launch, set_bytes, shape):
        return Op(name, name, nbytes, make, launch, set_bytes, shape)

    sweep = [("seqsweep_128", 1, 128), ("seqsweep_512", 1, 512), ("seqsweep_2048", 1, 2048),
             ("seqsweep_8192", 1, 8192), ("batchsweep_1", 1, 1024), ("batchsweep_4", 4, 1024),
             ("batchsweep_16", 16, 1024)]
    # rmsnorm_residual_bench.py:66-79
    for case, b, s, h in [("bs4_seq128_h768", 4, 128, 768), ("bs2_seq2048_h4096", 2, 2048, 4096),
                          ("bs1_seq4096_h4096", 1, 4096, 4096)] + [(c, b, s, 4096) for c, b, s in sweep]:
        for dn, dt in dts:
            es, rows = torch.tensor([], dtype=dt).element_size(), b * s
            w = (1.0 + 0.1 * torch.randn(h, device=dev, generator=g)).to(dt)
            yield "rmsnorm_residual", case, dn, op(
                f"rmsnorm_residual/{case}/{dn}", rows * h * es * 4,
                lambda rows=rows, h=h, dt=dt: dict(x=rn((rows, h), dt), r=rn((rows, h), dt),
                                                   y=torch.empty(rows, h, dtype=dt, device=dev),
                                                   ro=torch.empty(rows, h, dtype=dt, device=dev)),
                lambda d, w=w: native.rmsnorm_residual_fwd(d["x"], d["r"], w, d["y"], d["ro"], 1e-5),
                rows * h * es * 4, [rows, h])
    # swiglu_bench.py:39-50
    for case, b, s, d_ff in [("bs4_seq128_d3072", 4, 128, 3072), ("bs2_seq2048_d11008", 2, 2048, 11008),
                             ("bs1_seq4096_d11008", 1, 4096, 11008)] + [(c, b, s, 11008) for c, b, s in sweep]:
        for dn, dt in dts:
            es, rows = torch.tensor([], dtype=dt).element_size(), b * s
            yield "swiglu", case, dn, op(
                f"swiglu/{case}/{dn}", rows * d_ff * es * 3,
                lambda rows=rows, d_ff=d_ff, dt=dt: dict(g=rn((rows, d_ff), dt), u=rn((rows, d_ff), dt),
                                                         y=torch.empty(rows, d_ff, dtype=dt, device=dev)),
                lambda d: native.swiglu_fwd(d["g"], d["u"], d["y"]), rows * d_ff * es * 3, [rows, d_ff])
    # rope_bench.py:39-50 (out of place, as the reference's rope(q, k, cos, sin) returns new tensors)
    for case, b, s, hq, hkv, hd in [("bs4_seq128_mha", 4, 128, 12, 12, 64), ("bs2_seq2048_gqa", 2, 2048, 32, 8, 128),
                                    ("bs1_seq4096_gqa", 1, 4096, 32, 8, 128)] + [(c, b, s, 32, 8, 128)
                                                                                 for c, b, s in sweep]:
        inv = 1.0 / (10000.0 ** (torch.arange(0, hd, 2, dtype=torch.float32, device=dev) / hd))
        ang = torch.outer(torch.arange(s, dtype=torch.float32, device=dev), inv)
        cos, sin = ang.cos().contiguous(), ang.sin().contiguous()
        for dn, dt in dts:
            es, elems = torch.tensor([], dtype=dt).element_size(), b * s * (hq + hkv) * hd
            yield "rope", case, dn, op(
                f"rope/{case}/{dn}", elems * es * 2,
                lambda b=b, s=s, hq=hq, hkv=hkv, hd=hd, dt=dt: dict(
                    q=rn((b, s, hq, hd), dt), k=rn((b, s, hkv, hd), dt),
                    qo=torch.empty(b, s, hq, hd, dtype=dt, device=dev), ko=torch.empty(b, s, hkv, hd, dtype=dt, device=dev)),
                lambda d, cos=cos, sin=sin: native.rope_fwd(d["q"], d["k"], cos, sin, d["qo"], d["ko"]),
                elems * es * 2, [b, s, hq, hkv, hd])
    # fp8_quant_bench.py:40-59: tensor (with the reference wrapper's zeroed int32) and 128 x 128 blocks
    for case, m, n in [("small", 256, 256), ("medium", 1024, 1024), ("large", 4096, 4096), ("xlarge", 8192, 8192)]:
        for dn, dt in dts:
            es = torch.tensor([], dtype=dt).element_size()
            for fmt in ("e4m3", "e5m2"):
                f8 = torch.float8_e4m3fn if fmt == "e4m3" else torch.float8_e5m2

                def mk(m=m, n=n, dt=dt, f8=f8):
                    return dict(x=rn((m, n), dt), q=torch.empty(m, n, dtype=f8, device=dev),
                                st=torch.empty(1, device=dev), amax=torch.zeros(1, dtype=torch.int32, device=dev),
                                sb=torch.empty((m + 127) // 128, (n + 127) // 128, device=dev))

                def tensor(d, fmt=fmt):
                    d["amax"].zero_()
                    native.fp8_quant_tensor_fwd(d["x"], d["q"], d["st"], d["amax"], fmt)

                yield "fp8_quant", f"{case}_{fmt}_tensor", dn, op(f"fp8_quant/{case}_{fmt}_tensor/{dn}",
                                                                 m * n * (es + 1), mk, tensor, m * n * (es + 1), [m, n])
                yield "fp8_quant", f"{case}_{fmt}_block", dn, op(
                    f"fp8_quant/{case}_{fmt}_block/{dn}", m * n * (es + 1), mk,
                    lambda d, fmt=fmt: native.fp8_quant_block_fwd(d["x"], d["q"], d["sb"], fmt), m * n * (es + 1),
                    [m, n])
    # moe_router_bench.py:39-51
    for case, t, e, k in [("mixtral_like", 4096, 8, 2), ("deepseek_like", 4096, 160, 6), ("ksweep_k1", 4096, 32, 1),
                          ("ksweep_k2", 4096, 32, 2), ("ksweep_k4", 4096, 32, 4), ("ksweep_k8", 4096, 32, 8),
                          ("tsweep_512", 512, 8, 2), ("tsweep_2048", 2048, 8, 2), ("tsweep_8192", 8192, 8, 2),
                          ("tsweep_32768", 32768, 8, 2)]:
        for dn, dt in dts:
            es = torch.tensor([], dtype=dt).element_size()
            yield "moe_router", case, dn, op(
                f"moe_router/{case}/{dn}", t * e * es + t * k * 12,
                lambda t=t, e=e, k=k, dt=dt: dict(lg=rn((t, e), dt), w=torch.empty(t, k, device=dev),
                                                  i=torch.empty(t, k, dtype=torch.int64, device=dev)),
                lambda d: native.moe_router_fwd(d["lg"], d["w"], d["i"], True), t * e * es + t * k * 12, [t, e, k])
    # token_permute_bench.py:56-73
    for case, ns, nd, h in [("mixtral_like", 2048, 4096, 4096), ("large_hidden", 2048, 4096, 11008),
                            ("nsweep_1024", 1024, 1024, 4096), ("nsweep_4096", 4096, 4096, 4096),
                            ("nsweep_16384", 16384, 16384, 4096), ("nsweep_65536", 65536, 65536, 4096)]:
        for dn, dt in dts:
            es = torch.tensor([], dtype=dt).element_size()
            yield "token_gather", case, dn, op(
                f"token_gather/{case}/{dn}", 2 * nd * h * es,
                lambda ns=ns, nd=nd, h=h, dt=dt: dict(src=rn((ns, h), dt),
                                                      idx=torch.randint(0, ns, (nd,), device=dev, generator=g),
                                                      dst=torch.empty(nd, h, dtype=dt, device=dev)),
                lambda d: native.token_gather_fwd(d["src"], d["idx"], d["dst"]), (ns + nd) * h * es, [ns, nd, h])
    for case, t, k, h in [("mixtral_like", 2048, 2, 4096), ("deepseek_like", 2048, 6, 4096), ("tsweep_512", 512, 2, 4096),
                          ("tsweep_2048", 2048, 2, 4096), ("tsweep_8192", 8192, 2, 4096),
                          ("tsweep_32768", 32768, 2, 4096)]:
        for dn, dt in dts:
            es = torch.tensor([], dtype=dt).element_size()
            yield "token_combine", case, dn, op(
                f"token_combine/{case}/{dn}", (k + 1) * t * h * es,
                lambda t=t, k=k, h=h, dt=dt: dict(
                    eo=rn((t * k, h), dt), ui=torch.randperm(t * k, device=dev, generator=g).view(t, k),
                    w=torch.rand(t, k, device=dev, generator=g), out=torch.empty(t, h, dtype=dt, device=dev)),
                lambda d: native.token_combine_fwd(d["eo"], d["ui"], d["w"], d["out"]), (k + 1) * t * h * es,
                [t, k, h])


def _run_reference_suite(torch, native, args):
    """Times every case of _reference_suite like the config ops (graph-replayed
    kernel time over a >= 2 GiB rotation, plus the per-call time under the
    reference's own method) and prints one table row per case to stderr and
    one JSON line with all of them."""
    wanted = None if args.ops == "all" else set(args.ops.split(","))
    cases = []
    print("# family | case | dtype | kernel us | of 8 TB/s | per-call us | reference published",
          file=sys.stderr, flush=True)
    for fam, case, dn, op in _reference_suite(torch, native):
        if wanted and fam not in wanted:
            continue
        r = _time_op(torch, op, args.steps, args.warmup)
        pub = REFERENCE_PUBLISHED.get((fam, case, dn))
        row = {"family": fam, "case": case, "dtype": dn, "shape": op.shape, "bytes": op.nbytes, "us": r["us"],
               "frac_of_8TBps": r["frac_of_8TBps"], "per_call_median_us": r["per_call"]["median_us"],
               "reference_published_frac": pub}
        cases.append(row)
        print(f"# {fam} | {case} | {dn} | {r['us']:.2f} | {100 * r['frac_of_8TBps']:.1f} % | "
              f"{r['per_call']['median_us']:.2f} | {'' if pub is None else f'{100 * pub:.1f} % of 256 GB/s'}",
              file=sys.stderr, flush=True)
    print(json.dumps({"suite": "reference", "metric": "achieved HBM bandwidth per case, reference bytes",
                      "peak_GB_per_s": PEAK_GBPS, "steps": args.steps, "cases": cases}), flush=True)


def _per_call_us(torch, op, sets, calls=30):
    """The reference's methodology (benchmarks/*_bench.py, examples/llama_block.py:220-250):
    a 512 MiB write between calls so nothing is cache-resident, then HIP events
    around one call through the binding (validation and launch included);
    median and inter-quartile range in microseconds."""
    flush = torch.empty(512 << 20, dtype=torch.uint8, device="cuda")
    times = []
    for i in range(calls):
        flush.fill_(i & 0xFF)
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        op.launch(sets[i % len(sets)])
        end.record()
        torch.cuda.synchronize()
        times.append(start.elapsed_time(end) * 1000.0)
    del flush
    times.sort()
    q = lambda f: times[min(len(times) - 1, int(f * len(times)))]
    return {"median_us": round(q(0.5), 3), "iqr_us": round(q(0.75) - q(0.25), 3), "calls": calls}


def _cpu_time(fn, sets, budget_s: float):
    """Median wall time (s) of fn(*set) over rotating input sets, ~budget_s."""
    for i in range(min(2, len(sets))):
        fn(*sets[i])
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 5:
        t0 = time.perf_counter_ns()
        fn(*sets[len(times) % len(sets)])
        times.append(time.perf_counter_ns() - t0)
    times.sort()
    return times[len(times) // 2] * 1e-9, len(times)


def _host_cpu(load_before: float) -> dict:
    """The host the CPU baseline ran on: its CPU model, torch's vector
    capability and the 1-minute load average before the timing (other
    tenants of the host slow the baseline down)."""
    import torch

    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            model = next((ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name")), model)
    except OSError:
        pass
    quota = None  # CPUs the cgroup may use (cgroup v2 cpu.max, else v1 cfs quota / period)
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            q, period = f.read().split()
        quota = None if q == "max" else round(int(q) / int(period), 2)
    except (OSError, ValueError):
        try:
            with open("/sys/fs/cgroup/cpu/cpu.cfs_quota_us") as f, open("/sys/fs/cgroup/cpu/cpu.cfs_period_us") as g:
                q, period = int(f.read()), int(g.read())
            quota = None if q < 0 else round(q / period, 2)
        except (OSError, ValueError):
            pass
    return {"cpu": model, "capability": torch.backends.cpu.get_cpu_capability(), "cgroup_cpu_quota": quota,
            "loadavg_1m_before": round(load_before, 2), "loadavg_1m_after": round(os.getloadavg()[0], 2)}


def _cpu_baseline(budget_s: float):
    """The CPU oracle (torch-CPU / numpy restatements of the reference's eager
    baselines) timed on this host's cores, each op on a bounded row sample of
    its config's workload, rotating over distinct inputs larger than any
    host's last-level cache so that (like the GPU timing) no run is served
    from cache. The headline is RMSNorm + residual (config 2); `per_op` holds
    every config op."""
    import torch

    from oracle import eager, inputs

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    bf16 = torch.bfloat16
    load_before = os.getloadavg()[0]

    def rot_sets(make, set_bytes, total=256 << 20, cap=64):
        return [make(i) for i in range(max(2, min(cap, total // set_bytes)))]

    per_op = {}

    def record(name, fn, sets, nbytes, sample, share):
        med, runs = _cpu_time(fn, sets, budget_s * share)
        per_op[name] = {"ms_per_run": round(med * 1e3, 3), "TB_per_s": round(nbytes / med / 1e12, 6),
                        "frac_of_8TBps": round(nbytes / med / 8e12, 6), "runs": runs, "sets": len(sets),
                        "sample": sample}

    # 2: RMSNorm + residual, [1024, 4096] rows of config 2 (1 GiB rotation, the headline)
    rows, cols = 1024, 4096
    x0, r0, w = inputs.rmsnorm_inputs(rows, cols, bf16, seed=0)
    sets = [(x0.roll(i, 0), r0.roll(-i, 0), w, 1e-5) for i in range((1 << 30) // (rows * cols * 4))]
    record("rmsnorm_residual", eager.rmsnorm_residual, sets, rows * cols * 8 + cols * 2,
           f"eager rmsnorm_residual, bf16 [{rows},{cols}]", 0.45)
    del sets
    # 1: per-token FP8 with torch's CPU cast, [512, 4096] rows of the config-1 input
    xt = inputs.fp8_token_input(2048, 4096, bf16, seed=0)
    sets = rot_sets(lambda i: (xt[(i % 4) * 512:(i % 4 + 1) * 512].roll(i, 1).contiguous(), "e4m3"),
                    512 * 4096 * 2)
    record("fp8_quant_token", eager.fp8_quant_token_torch, sets, 512 * 4096 * 3 + 512 * 4,
           "eager per-row fp8 quant (torch cast), bf16 [512,4096] rows of the config-1 input", 0.1)
    del sets, xt
    # 3: SwiGLU, [256, 14336] rows of config 3
    sets = rot_sets(lambda i: inputs.swiglu_inputs(256, 14336, bf16, seed=i), 256 * 14336 * 4, cap=16)
    record("swiglu", eager.swiglu, sets, 256 * 14336 * 6, "eager swiglu, bf16 [256,14336]", 0.1)
    # 3v: SwiGLU + per-token FP8 (composition), same rows
    record("swiglu_fp8_token", lambda g, u: eager.fp8_quant_token_torch(eager.swiglu(g, u)), sets,
           256 * 14336 * 5 + 256 * 4, "eager swiglu then per-row fp8 quant (torch cast), bf16 [256,14336]", 0.1)
    del sets
    # 4: RoPE, q [1,512,32,128] + k [1,512,8,128] of config 4 (theta 5e5)
    cos, sin = eager.compute_cos_sin(512, 128, inputs.ROPE_THETA)
    sets = rot_sets(lambda i: inputs.rope_inputs(1, 512, 32, 8, 128, bf16, seed=i)[:2] + (cos, sin),
                    512 * 40 * 128 * 2, cap=16)
    record("rope", eager.rope, sets, 512 * 40 * 128 * 4, "eager rope, q [1,512,32,128] + k [1,512,8,128] bf16", 0.1)
    del sets
    # 5a: RMSNorm + residual + per-token FP8 (composition), [512, 4096] rows of config 5
    x5, r5, w5 = inputs.rmsnorm_inputs(512, 4096, bf16, seed=1)
    sets = [(x5.roll(i, 0), r5.roll(-i, 0), w5, 1e-5) for i in range(16)]
    record("rmsnorm_residual_fp8_token",
           lambda x, r, w, eps: eager.fp8_quant_token_torch(eager.rmsnorm_residual(x, r, w, eps)[0]),
           sets, 512 * 4096 * 7 + 512 * 4 + 4096 * 2,
           "eager rmsnorm_residual then per-row fp8 quant (torch cast), bf16 [512,4096]", 0.15)
    del sets

    head = per_op["rmsnorm_residual"]
    return {"value": head["TB_per_s"], "unit": "TB/s", "cores": torch.get_num_threads(), "kind": "port",
            "host": _host_cpu(load_before),
            "sample": f"oracle eager rmsnorm_residual on bf16 [{rows},{cols}] rows of the config-2 workload, "
                      f"rotating over 1 GiB of distinct inputs, median of {head['runs']} runs, "
                      f"{head['ms_per_run']:.3f} ms/run; per_op: every config op's oracle on a row sample",
            "per_op": per_op}


def _block_latency(torch, model="llama3-8b"):
    """Llama-3 decoder block (the reference's Llama-3-8B, or Llama-3-70B's
    layer shapes), B=1 S=4096 bf16, in the three variants of
    custom_cuda_kernals_amd.llama_block (the reference's integration proof,
    examples/llama_block.py, with an FP8 variant added)."""
    from custom_cuda_kernals_amd.llama_block import CONFIGS, LlamaBlock, block_latency_ms

    torch.manual_seed(0)
    seq, cfg = 4096, CONFIGS[model]
    ref = LlamaBlock(seq, cfg, mode="eager").eval()
    g = torch.Generator(device="cuda").manual_seed(0)
    x = torch.randn(1, seq, cfg.hidden_size, dtype=torch.bfloat16, device="cuda", generator=g) * 0.02
    out = {"model": model}
    for mode in ("eager", "fused", "fp8"):
        blk = ref if mode == "eager" else LlamaBlock(seq, cfg, mode=mode).eval()
        if blk is not ref:
            blk.load_state_dict(ref.state_dict())
        out[mode] = block_latency_ms(blk, x)
        print(f"# block {mode}: {out[mode]}", file=sys.stderr, flush=True)
        if blk is not ref:
            del blk
    out["speedup_fused_vs_eager"] = round(out["eager"]["median_ms"] / out["fused"]["median_ms"], 3)
    out["speedup_fp8_vs_eager"] = round(out["eager"]["median_ms"] / out["fp8"]["median_ms"], 3)
    return out


def _traffic(op_name):
    """Measured HBM bytes per launch of `op_name` from the committed counter
    summary (profiles/pmc_traffic.json, written from two rocprofv3 --pmc runs,
    FETCH_SIZE and WRITE_SIZE, scaled by the same counters on a plain copy);
    None when no summary covers the op."""
    path = os.path.join(ROOT, "profiles", "pmc_traffic.json")
    try:
        with open(path) as f:
            data = json.load(f)
        return data["ops"][op_name]["hbm_bytes_per_launch"]
    except (OSError, KeyError, ValueError):
        return None


def main():
    args = _parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus must be 1 "
                          "(the per-GPU kernels shard by token rows with no communication; only one GPU is measured)"}))
        sys.exit(2)

    import torch

    global MARKERS
    MARKERS = _Markers(args.markers)
    _ensure_built()
    from custom_cuda_kernals_amd._lib import native

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        sys.exit(1)

    if args.suite == "reference":
        _run_reference_suite(torch, native, args)
        return
    ops = _ops(torch, native)
    wanted = None if args.ops == "all" else set(args.ops.split(","))
    results = {}
    for op in ops:
        if wanted and op.name not in wanted:
            continue
        results[op.name] = _time_op(torch, op, args.steps, args.warmup, use_graph=not args.no_graph)
        print(f"# {op.name}: {results[op.name]}", file=sys.stderr, flush=True)
    ceilings = None
    if not args.no_ceilings and not args.no_graph:
        ceilings = _ceilings(torch, args.steps, args.warmup)
        for name, c in ceilings.items():
            done = results.get(c["bounds"])
            if done:
                c["op_frac_of_ceiling"] = round(done["GB_per_s"] / c["GB_per_s"], 4)
            print(f"# ceiling {name}: {c}", file=sys.stderr, flush=True)
    anchors = None
    if not args.no_ceilings and not args.no_graph:
        anchors = _anchors(torch, args.steps, args.warmup)
        for name, a in anchors.items():
            done = results.get(a["bounds"])
            if done:
                a["op_frac_of_anchor_bandwidth"] = round(done["GB_per_s"] / a["GB_per_s"], 4)
                a["op_speedup_over_anchor"] = round(a["us"] / done["us"], 4)
            print(f"# anchor {name}: {a}", file=sys.stderr, flush=True)
    if args.copy_calibration:
        src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print("# copy calibration: 3 x torch copy_ of 268435456 bytes", file=sys.stderr, flush=True)

    head = results.get("rmsnorm_residual") or next(iter(results.values()))
    head_name = "rmsnorm_residual" if "rmsnorm_residual" in results else next(iter(results))
    achieved = head["GB_per_s"]
    line = {
        "metric": "achieved HBM TB/s & % of 8 TB/s peak per op (FP8 quant, RMSNorm, SwiGLU, RoPE)",
        "value": round(achieved / 1000.0, 4),
        "unit": "TB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["us"] / 1000.0, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) inputs generated on the GPU, resident in HBM)",
        "config": {"workload": head["workload"], "op": head_name, "shape": head.get("shape"),
                   "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_GBPS, 4), "traffic": _traffic(head_name)},
        "ops": results,
    }
    if ceilings:
        line["ceilings"] = ceilings
    if anchors:
        line["anchors"] = anchors
    if args.block:
        line["block"] = _block_latency(torch, args.block_model)
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = _cpu_baseline(args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
