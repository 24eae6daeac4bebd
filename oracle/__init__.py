"""CPU oracle for the activation path - TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import this package, and only as the checker (or, in the bench, as the
timed CPU baseline). The product path (``custom_cuda_kernals_amd``) never
imports it and has no CPU fallback.

Contents
* ``fp8``    - numpy restatement of the reference's FP8 quantisation
               (baselines/fp8_quant.py:126-189) with an exact float64-based
               e4m3fn / e5m2 encoder, plus the per-token / static modes the
               build adds by applying the same formula per row / with a given
               scale.
* ``eager``  - torch-CPU restatements of the eager baselines in the same op
               order (baselines/rmsnorm_residual.py:123-136,
               baselines/swiglu.py:107-112, baselines/rope.py:103-145) and the
               fused compositions.
* ``inputs`` - seeded CPU input generators for BASELINE.json configs 1-5 and
               small parity cases.

How each function is pinned is listed in the module docstrings and tested in
``tests/test_oracle_*.py``.
"""
