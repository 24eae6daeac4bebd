"""Every op captured in a HIP graph (torch.cuda.CUDAGraph) through the
binding, with preallocated buffers, then replayed: before each replay new
inputs are copied into the captured input buffers and the outputs are
overwritten with garbage by eager work, and every replay must reproduce the
eager launch on the same inputs bit for bit. The per-tensor FP8 op clears
its amax scratch with torch's zero_() inside the graph (a fill kernel; the
library itself issues no memset). Three input sets, two rounds of replays.
"""

from __future__ import annotations

import pytest
import torch

from custom_cuda_kernals_amd import _native as native
from oracle import inputs

pytestmark = pytest.mark.gpu

BF16, F8 = torch.bfloat16, torch.float8_e4m3fn


def _bits(t: torch.Tensor) -> torch.Tensor:
    t = t.detach()
    return t.view(torch.uint8) if t.element_size() == 1 else t.view(torch.int16) if t.element_size() == 2 else t.view(
        torch.int32) if t.element_size() == 4 else t.view(torch.int64)


def _poison(t: torch.Tensor) -> None:
    _bits(t).fill_(0x5A)


def _replay_matches_eager(ins, outs, launch, input_sets):
    """ins / outs: device tensors the launch reads / writes; input_sets: lists
    of CPU tensors matching ins."""
    refs = []
    for cpu_in in input_sets:
        for d, c in zip(ins, cpu_in):
            d.copy_(c)
        for o in outs:
            _poison(o)
        launch()
        torch.cuda.synchronize()
        refs.append([_bits(o).clone() for o in outs])
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
    for _ in range(2):
        for cpu_in, ref in zip(input_sets, refs):
            for d, c in zip(ins, cpu_in):
                d.copy_(c)
            for o in outs:
                _poison(o)
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            for o, r in zip(outs, ref):
                assert torch.equal(_bits(o), r), "graph replay differs from the eager launch"


def test_rmsnorm_residual_graph():
    m, n = 64, 4096
    sets = [list(inputs.rmsnorm_inputs(m, n, BF16, seed=s)) for s in range(3)]
    x, r, w = [t.cuda() for t in sets[0]]
    y, ro = torch.empty_like(x), torch.empty_like(x)
    _replay_matches_eager([x, r, w], [y, ro], lambda: native.rmsnorm_residual_fwd(x, r, w, y, ro, 1e-5), sets)


@pytest.mark.parametrize("static", [None, 0.05])
def test_rmsnorm_residual_fp8_graph(static):
    m, n = 64, 4096
    sets = [list(inputs.rmsnorm_inputs(m, n, BF16, seed=s)) for s in range(3)]
    x, r, w = [t.cuda() for t in sets[0]]
    q, ro = torch.empty(m, n, dtype=F8, device="cuda"), torch.empty_like(x)
    s = torch.empty(m, device="cuda")
    outs = [q, ro] + ([s] if static is None else [])
    _replay_matches_eager([x, r, w], outs, lambda: native.rmsnorm_residual_fp8_fwd(
        x, r, w, q, s if static is None else None, ro, 1e-5, "e4m3", static), sets)


def test_swiglu_graph():
    sets = [list(inputs.swiglu_inputs(32, 14336, BF16, seed=s)) for s in range(3)]
    g, u = [t.cuda() for t in sets[0]]
    y = torch.empty_like(g)
    _replay_matches_eager([g, u], [y], lambda: native.swiglu_fwd(g, u, y), sets)


@pytest.mark.parametrize("static", [None, 0.05])
def test_swiglu_fp8_graph(static):
    m, n = 32, 14336
    sets = [list(inputs.swiglu_inputs(m, n, BF16, seed=s)) for s in range(3)]
    g, u = [t.cuda() for t in sets[0]]
    q, s = torch.empty(m, n, dtype=F8, device="cuda"), torch.empty(m, device="cuda")
    outs = [q] + ([s] if static is None else [])
    _replay_matches_eager([g, u], outs, lambda: native.swiglu_fp8_fwd(g, u, q, s if static is None else None, "e4m3",
                                                                      static), sets)


def test_rope_in_place_graph():
    sets = []
    for s in range(3):
        q, k, cos, sin = inputs.rope_inputs(2, 64, 32, 8, 128, dtype=BF16, seed=s, theta=500000.0)
        sets.append([q, k, cos, sin])
    q, k, cos, sin = [t.cuda() for t in sets[0]]
    _replay_matches_eager([q, k, cos, sin], [q, k], lambda: native.rope_fwd(q, k, cos, sin, q, k), sets)


@pytest.mark.parametrize("gran", ["token", "block", "tensor", "tensor_api", "tensor_api_finish", "tensor_api_onepass",
                                  "tensor_onepass", "static"])
def test_fp8_quant_graph(gran):
    """tensor: the reference ABI (its int32 cleared inside the graph); tensor_api:
    no amax word, as the Python API calls it (slot arrays in the cast chunks at
    this size); tensor_api_finish: the same with one slot array and the
    finishing launch; tensor_api_onepass / tensor_onepass: the one-pass form
    (its init launch and the exchange in the codes and scale buffers), without
    and with the amax word."""
    m, n = {"tensor_api_finish": (4099, 4097), "tensor_api_onepass": (2048, 4096),
            "tensor_onepass": (4096, 4096)}.get(gran, (256, 4096))
    sets = [[inputs.fp8_token_input(m, n, BF16, seed=s)] for s in range(3)]
    x = sets[0][0].cuda()
    q = torch.empty(m, n, dtype=F8, device="cuda")
    if gran == "token":
        s = torch.empty(m, device="cuda")
        launch, outs = (lambda: native.fp8_quant_token_fwd(x, q, s, "e4m3")), [q, s]
    elif gran == "block":
        s = torch.empty(m // 128, n // 128, device="cuda")
        launch, outs = (lambda: native.fp8_quant_block_fwd(x, q, s, "e4m3")), [q, s]
    elif gran in ("tensor", "tensor_onepass"):
        s = torch.empty(1, device="cuda")
        amax = torch.zeros(1, dtype=torch.int32, device="cuda")

        def launch():
            amax.zero_()
            native.fp8_quant_tensor_fwd(x, q, s, amax, "e4m3")

        outs = [q, s, amax]
    elif gran.startswith("tensor_api"):
        s = torch.empty(1, device="cuda")
        launch, outs = (lambda: native.fp8_quant_tensor_fwd(x, q, s, None, "e4m3")), [q, s]
    else:
        launch, outs = (lambda: native.fp8_quant_static_fwd(x, q, 0.05, "e4m3")), [q]
    _replay_matches_eager([x], outs, launch, sets)


def test_moe_ops_graph():
    sets_g = [list(inputs.gather_inputs(512, 1024, 4096, BF16, seed=s)) for s in range(3)]
    src, idx = [t.cuda() for t in sets_g[0]]
    dst = torch.empty(1024, 4096, dtype=BF16, device="cuda")
    _replay_matches_eager([src, idx], [dst], lambda: native.token_gather_fwd(src, idx, dst), sets_g)
    # 8192 rows of 4096: 2^22 destination vectors, the flat gather form
    sets_f = [list(inputs.gather_inputs(1024, 8192, 4096, BF16, seed=s)) for s in range(3)]
    src_f, idx_f = [t.cuda() for t in sets_f[0]]
    dst_f = torch.empty(8192, 4096, dtype=BF16, device="cuda")
    _replay_matches_eager([src_f, idx_f], [dst_f], lambda: native.token_gather_fwd(src_f, idx_f, dst_f), sets_f)
    sets_c = [list(inputs.combine_inputs(256, 6, 4096, BF16, seed=s)) for s in range(3)]
    eo, ui, w = [t.cuda() for t in sets_c[0]]
    out = torch.empty(256, 4096, dtype=BF16, device="cuda")
    _replay_matches_eager([eo, ui, w], [out], lambda: native.token_combine_fwd(eo, ui, w, out), sets_c)
    # hidden 4104 (4096 vector columns + 8 scalar ones) and k = 20 (the block cascade): two launches
    sets_c2 = [list(inputs.combine_inputs(64, 20, 4104, BF16, seed=s)) for s in range(3)]
    eo2, ui2, w2 = [t.cuda() for t in sets_c2[0]]
    out2 = torch.empty(64, 4104, dtype=BF16, device="cuda")
    _replay_matches_eager([eo2, ui2, w2], [out2], lambda: native.token_combine_fwd(eo2, ui2, w2, out2), sets_c2)
    # the router's forms: a wave per token (160 experts), eight lanes (160 at 12288 tokens), four lanes (32),
    # one lane (8)
    for t, e, k in ((512, 160, 6), (12288, 160, 6), (512, 32, 8), (4096, 8, 2)):
        sets_r = [[inputs.router_inputs(t, e, torch.bfloat16, seed=s)] for s in range(3)]
        lg = sets_r[0][0].cuda()
        tw, ti = torch.empty(t, k, device="cuda"), torch.empty(t, k, dtype=torch.int64, device="cuda")
        _replay_matches_eager([lg], [tw, ti], lambda: native.moe_router_fwd(lg, tw, ti, True), sets_r)
    g = torch.Generator().manual_seed(7)
    sets_p = [[torch.randint(0, 160, (2048, 6), generator=g)] for _ in range(3)]
    ids = sets_p[0][0].cuda()
    perm, unperm = torch.empty(2048 * 6, dtype=torch.int64, device="cuda"), torch.empty(2048, 6, dtype=torch.int64,
                                                                                          device="cuda")
    _replay_matches_eager([ids], [perm, unperm], lambda: native.moe_permutation_fwd(ids, perm, unperm, 160), sets_p)
    # 16384 x 8 entries: the three-launch permutation (counts kept in permute_index between launches)
    sets_q = [[torch.randint(0, 256, (16384, 8), generator=g)] for _ in range(3)]
    ids_q = sets_q[0][0].cuda()
    perm_q = torch.empty(16384 * 8, dtype=torch.int64, device="cuda")
    unperm_q = torch.empty(16384, 8, dtype=torch.int64, device="cuda")
    _replay_matches_eager([ids_q], [perm_q, unperm_q],
                          lambda: native.moe_permutation_fwd(ids_q, perm_q, unperm_q, 256), sets_q)
