"""Overlay: route sorted routed-expert prefill gathers through the
int8-activation x int4-weight grouped GEMM (engine/patches/moe-int8/patch.py).

Routed only when ALL of: ``sorted_indices=True``, ``rhs_indices`` present and
``lhs_indices`` absent, ``transpose=True``, affine 4-bit ``group_size=64``,
bf16 rows ``[R, 1, K]`` on the GPU, ``K % 512 == 0`` and ``K <= 4096`` (the
gate_up and the down projection), ``N % 256 == 0`` and the token floor.
Everything else falls through to what was installed before.

    TITAN_AMD_MOE_INT8_PREFILL=1        enable (default off: it changes the numbers)
    TITAN_AMD_MOE_INT8_MIN_TOKENS=512   token floor of the SwitchGLU call
    TITAN_AMD_MOE_INT8_MIN_ROWS=4096    routed-row floor when the token count is unknown
    TITAN_AMD_MOE_INT8_SKIP_DOWN=1      leave projections with K <= 1024 (the down
                                        projection) to the layers below

Memory: none unless ``warmup(model)`` builds each routed weight tensor's
tile-layout repack (:class:`Int8Tables`, as large as the tensor and shared
with the bf16 overlay) ahead of the first prefill; without it the MLX-layout
int8 kernel reads the tensors as they are.  A call builds nothing.
``TITAN_AMD_TILE_CACHE=0``: warmup prepares nothing.
"""

from __future__ import annotations

import os

from ..kernels import moe_gather_int8 as _k
from ..kernels import prepared
from ._overlay import Overlay, arg, switch_linears

MARKER = "_titan_amd_moe_int8"


def _key_args(x, w, args, kwargs):
    return (x, w, arg(args, kwargs, 0, "scales"), arg(args, kwargs, 1, "biases"),
            arg(args, kwargs, 3, "rhs_indices"))


def _should_route(ov, x, w, args, kwargs) -> bool:
    if not ov.enabled() or not kwargs.get("sorted_indices"):
        return False
    if arg(args, kwargs, 2, "lhs_indices") is not None or arg(args, kwargs, 7, "mode", "affine") != "affine":
        return False
    if not arg(args, kwargs, 4, "transpose", True):
        return False
    if x.dim() < 1 or ov.below_floor(int(x.shape[0])):
        return False
    if _skip_down() and x.shape[-1] <= 1024:
        return False
    return supported(x, w, *[arg(args, kwargs, i, n) for i, n in ((0, "scales"), (1, "biases"))],
                     arg(args, kwargs, 3, "rhs_indices"), True, arg(args, kwargs, 5, "group_size", 64),
                     arg(args, kwargs, 6, "bits", 4))


def _skip_down() -> bool:
    return os.environ.get("TITAN_AMD_MOE_INT8_SKIP_DOWN", "0") == "1"


def supported(x, w, scales, biases, rhs, transpose, group_size, bits) -> bool:
    """Would the int8 kernel take this call (shapes only)?"""
    if rhs is None or scales is None or biases is None or not transpose:
        return False
    return _k.supports(_k.key(x, w, scales, biases, rhs, True, group_size=group_size, bits=bits))


def _route(x, w, args, kwargs):
    return _k.hip(x, w, arg(args, kwargs, 0, "scales"), arg(args, kwargs, 1, "biases"),
                  arg(args, kwargs, 3, "rhs_indices"), group_size=arg(args, kwargs, 5, "group_size", 64),
                  bits=arg(args, kwargs, 6, "bits", 4))


_OV = Overlay("moe int8 prefill", MARKER, "TITAN_AMD_MOE_INT8_PREFILL", False,
              {"gather_qmm": (_should_route, _route)}, "TITAN_AMD_MOE_INT8_MIN_TOKENS", 512,
              "TITAN_AMD_MOE_INT8_MIN_ROWS", 4096)


def enabled() -> bool:
    return _OV.enabled()


def install(namespace=None) -> bool:
    """Idempotent.  Returns True when this call installed the hooks."""
    return _OV.install(namespace)


def uninstall() -> None:
    _OV.uninstall()


def stats() -> dict:
    return _OV.stats()


def clear_cache() -> None:
    """Drop the prepared tables (the tile-layout repacks)."""
    prepared.clear_cache()


def warmup(model=None) -> int:
    """Build the tables of every routed weight tensor the kernel would take,
    ahead of the first prefill chunk (engine/patches/moe-int8/patch.py:179-198).
    Returns how many tensors were prepared (0 with the tile cache off)."""
    if not prepared.enabled():
        return 0
    n = 0
    for m in switch_linears(model):
        if (m.bits, m.group_size, m.mode) != (_k.BITS, _k.GROUP, "affine") or m.bias is not None:
            continue
        K = m.input_dims
        if _k.pick_cfg(m.output_dims) is None or K % 512 or K > 4096 or (_skip_down() and K <= 1024):
            continue
        if not m.weight.is_cuda:
            continue
        _k.build_tables(m.weight, m.scales, m.biases)
        n += 1
    return n
