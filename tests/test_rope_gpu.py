"""RoPE kernel vs the CPU oracle (torch-CPU restatement of
baselines/rope.py:129-145): bit-exact (products and differences rounded
separately in fp32, one rounding to the storage type), out-of-place and in
place. Shapes: the reference's case table (baselines/rope.py:72-100), its
scalar-fallback head dims (tests/test_rope_kernel.py:59-84) and BASELINE
config 4 at full size, in place, plus head dims 256 and 512 so that every
launch shape of the vector kernel (1 to 32 chunk lanes per token) runs.
"""

from __future__ import annotations

import pytest
import torch

from custom_cuda_kernals_amd.kernels import rope
from oracle import eager, inputs
from tests._parity import bits_equal

pytestmark = pytest.mark.gpu

CASES = [(4, 128, 12, 12, 64), (2, 2048, 32, 8, 128), (1, 4096, 32, 8, 128), (3, 17, 8, 2, 64),
         (8, 1, 8, 8, 64), (1, 8192, 8, 8, 64), (0, 128, 8, 8, 64), (1, 1, 1, 1, 64), (2, 32, 4, 1, 16),
         # head_dim 256 / 512: 32 and 16 chunk lanes (one and two tokens per workgroup)
         (2, 16, 4, 2, 256), (1, 8, 3, 1, 512),
         # a thread per (head, chunk) in workgroups of 5-16 waves: 72, 64, 33 and 128 heads of 128 (8 chunk
         # lanes; fp32 16: 1152 threads fall back to rounds), 48 and 129 heads of 64 (fp32: 8 chunk lanes)
         (1, 64, 64, 8, 128), (2, 33, 32, 32, 128), (1, 50, 29, 4, 128), (1, 20, 120, 8, 128), (3, 7, 40, 8, 64),
         (1, 9, 100, 29, 64),
         # up to one round of resident workgroups the tables are staged in LDS (1024 tokens), beyond it not
         (1, 1024, 32, 8, 128)]
DTYPES = [torch.float32, torch.float16, torch.bfloat16]


def _run(case, dtype, theta, inplace=False, seed=0):
    q, k, cos, sin = inputs.rope_inputs(*case, dtype=dtype, seed=seed, theta=theta)
    qd, kd = q.cuda(), k.cuda()
    qo, ko = rope(qd, kd, cos.cuda(), sin.cuda(), inplace=inplace)
    if inplace:
        assert qo.data_ptr() == qd.data_ptr() and ko.data_ptr() == kd.data_ptr()
    q_ref, k_ref = eager.rope(q, k, cos, sin)
    assert bits_equal(qo, q_ref).all(), "q differs from the oracle"
    assert bits_equal(ko, k_ref).all(), "k differs from the oracle"


@pytest.mark.parametrize("inplace", [False, True])
@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c)))
def test_matches_oracle(case, dtype, inplace):
    _run(case, dtype, 10000.0, inplace, seed=sum(case))


@pytest.mark.parametrize("head_dim", [6, 10, 14, 2])
@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
def test_odd_half_dims_scalar_path(head_dim, dtype):
    _run((2, 9, 3, 1, head_dim), dtype, 10000.0)


def test_config4_full_size_in_place():
    _run(inputs.CONFIG_SHAPES["rope"], torch.bfloat16, inputs.ROPE_THETA, inplace=True)


def test_rejections():
    q = torch.randn(1, 4, 2, 8, device="cuda")
    k = torch.randn(1, 4, 1, 8, device="cuda")
    cos = torch.randn(4, 4, device="cuda")
    with pytest.raises(ValueError):
        rope(q, k, cos.half(), cos)
    with pytest.raises(ValueError):
        rope(q, k, torch.randn(4, 3, device="cuda"), torch.randn(4, 3, device="cuda"))
    with pytest.raises(ValueError):
        rope(q, torch.randn(1, 4, 1, 8, device="cuda", dtype=torch.float16), cos, cos)
