"""Resource use of every gfx950 kernel in the in-tree library, read on the CPU
from the code objects' AMDGPU metadata (tests/_code_object.py).

A kernel with a private segment (register spills to scratch memory) makes
the HIP runtime allocate queue scratch the first time such a dispatch needs
it: a device allocation hidden inside a launch, which
launch_fp8_quant_tensor_noalloc_fwd promises never to make, and a slowdown
anywhere else. So no kernel of the library may have one, and none may use a
dynamic stack.
"""

from __future__ import annotations

import re

import pytest

from tests import _cck
from tests._code_object import gfx950_kernels


@pytest.fixture(scope="module")
def kernels():
    ks = gfx950_kernels(_cck.LIB_PATH)
    assert len(ks) > 100, "the library's gfx950 kernels were not found"
    return ks


def test_no_kernel_has_a_private_segment(kernels):
    spilled = [(k[".name"], k[".private_segment_fixed_size"], k[".vgpr_spill_count"]) for k in kernels
               if k[".private_segment_fixed_size"] or k[".vgpr_spill_count"] or k[".uses_dynamic_stack"]]
    assert not spilled, f"kernels with scratch (name, private bytes per lane, VGPR spills): {spilled}"


def test_no_alloc_path_kernels_are_present_and_scratch_free(kernels):
    """The kernels behind launch_fp8_quant_tensor_noalloc_fwd: the one-pass
    kernel at every vectors-per-thread shape, its init launch, and the
    two-pass form's partial and cast kernels."""
    names = [k[".name"] for k in kernels]
    for pattern in (r"fp8_onepass_init", r"fp8_tensor_onepass.*ELi1ELi8ELb0E", r"fp8_tensor_onepass.*ELi2ELi8ELb0E",
                    r"fp8_tensor_onepass.*ELi4ELi8ELb0E", r"fp8_tensor_onepass.*ELi16ELi4ELb0E",
                    r"fp8_tensor_onepass.*ELi16ELi4ELb1E", r"fp8_tensor_partial", r"fp8_tensor_cast"):
        hits = [k for k in kernels if re.search(pattern, k[".name"])]
        assert hits, f"no kernel matches {pattern} among {len(names)}"
        assert all(k[".private_segment_fixed_size"] == 0 for k in hits), pattern


def test_one_pass_shapes_fit_their_register_budget(kernels):
    """Two 1024-thread workgroups per CU (64 VGPRs) at 1, 2 and 4 vectors per
    thread; one (128 VGPRs) at 16, holding all of x or streaming the rest
    (SPILL): the occupancy the launcher sizes grids by."""
    seen = 0
    for k in kernels:
        m = re.search(r"fp8_tensor_onepass.*ELi(\d+)ELi(\d+)ELb([01])EEEv", k[".name"])
        if m:
            seen += 1
            wpe = int(m.group(2))
            assert k[".vgpr_count"] <= 512 // wpe, (k[".name"], k[".vgpr_count"])
    assert seen == 3 * 2 * 5, seen  # 3 dtypes x 2 formats x (4 held shapes + SPILL)


def test_block_tiles_fit_two_workgroups_per_cu(kernels):
    """Every 128 x 128-block FP8 instance leaves room for two 512-thread
    workgroups per CU (at most 128 VGPRs). Loading the tile under per-vector
    branches once took the fp32 tile to 232 VGPRs (one workgroup per CU, half
    the speed)."""
    hits = [k for k in kernels if "fp8_block_resident" in k[".name"]]
    assert len(hits) >= 3 * 2 * 3, len(hits)
    for k in hits:
        assert k[".vgpr_count"] <= 128, (k[".name"], k[".vgpr_count"])
