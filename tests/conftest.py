"""Test configuration.

* Marker ``gpu``: needs an MI355X (HIP device); everything else runs on CPU.
* The in-tree native artefacts are built on first use if absent
  (``custom_cuda_kernals_amd.build``); an existing build is used as is.
"""

from __future__ import annotations

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (MI355X)")
    config.addinivalue_line("markers", "slow: long-running CPU check")
    from custom_cuda_kernals_amd import build

    if not build.is_built():
        build.build_all()


def pytest_collection_modifyitems(config, items):
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this container")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
