"""The namespace call sites use for the quantized matmuls, in the role of
``mlx.core`` for the reference (``mx.gather_qmm``, ``mx.quantized_matmul``).

Until an overlay patch is installed these are the stock torch
implementations of :mod:`titan_amd.stock`.  :mod:`titan_amd.patches` reroutes
them to the HIP kernels by replacing the attributes, capturing what was there
as the fallback, exactly as the reference's overlays replace
``mx.gather_qmm`` (engine/patches/moe-int8/patch.py:140-156).  Call sites
must therefore look the functions up here at call time
(``core.gather_qmm(...)``), not import them by name.
"""

from __future__ import annotations

from .stock import gather_qmm, quantized_matmul

__all__ = ["gather_qmm", "quantized_matmul"]
