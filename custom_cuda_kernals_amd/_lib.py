"""Loads the native binding. There is no fallback: without the built HIP
library every op raises at import time.

``torch`` is imported first so that its HIP runtime (soname
``libamdhip64.so.7``) is the one the kernel library binds to; loading the
kernel library first would pull in a second copy of the runtime.
"""

from __future__ import annotations

import torch  # noqa: F401  (must precede the native import, see above)

try:
    from custom_cuda_kernals_amd import _native as native
except ImportError as exc:  # pragma: no cover - exercised only on unbuilt trees
    raise ImportError(
        "custom_cuda_kernals_amd._native is not built; run "
        "`python -m custom_cuda_kernals_amd.build` (hipcc, gfx950) first"
    ) from exc

__all__ = ["native"]
