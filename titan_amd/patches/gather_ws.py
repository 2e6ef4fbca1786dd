"""Overlay: route sorted routed-expert prefill gathers through the bf16
grouped GEMM (engine/patches/round3/gather-ws/patch.py).

Routed only when ALL of: ``sorted_indices=True``, ``rhs_indices`` present and
``lhs_indices`` absent, ``transpose=True``, affine 4-bit ``group_size=64``,
bf16 rows ``[R, 1, K]`` on the GPU with ``R >= 64``, ``K % 128 == 0``,
``N % 256 == 0`` and the token floor.  Everything else falls through.

Precedence against the int8 overlay (gather-ws/patch.py:93-151): when the int8
overlay is installed below this one and enabled, calls it would take are handed
down to it (counted as ``to_int8``); installed the other way round, int8 sits
on top and takes what it wants first.

    TITAN_AMD_MOE_GATHER_WS=1            enable (default on)
    TITAN_AMD_MOE_GATHER_WS_MIN_TOKENS=7 token floor (7 tokens x top-10 = the 64-row sort threshold)
    TITAN_AMD_MOE_GATHER_WS_MIN_ROWS=64  routed-row floor when the token count is unknown

Memory: none by default, as the reference's overlay: a call reads the
tensors as they are (the MLX-layout kernel) unless ``warmup(model)`` has
repacked them into the tile layout (one copy per routed weight tensor, as
large as the tensor, shared with the int8 overlay; ~20% faster).  A call
never builds a repack, so it allocates nothing beyond its output and tile
table and can be captured in a graph.  ``TITAN_AMD_TILE_CACHE=0``: warmup
prepares nothing.  The tile table is built per call or passed by the caller.
"""

from __future__ import annotations


from ..kernels import moe_gather_ws as _k
from ..kernels import prepared
from . import moe_int8
from ._overlay import Overlay, arg, switch_linears

MARKER = "_titan_amd_moe_gather_ws"


def supported(x, w, scales, biases, rhs, transpose, group_size, bits) -> bool:
    if rhs is None or scales is None or biases is None or not transpose:
        return False
    return _k.supports(_k.key(x, w, scales, biases, rhs, group_size=group_size, bits=bits))


def _int8_active(ov) -> bool:
    below = ov.fallback_of("gather_qmm")
    return moe_int8.enabled() and getattr(below, moe_int8.MARKER, False)


def _should_route(ov, x, w, args, kwargs) -> bool:
    if not ov.enabled() or not kwargs.get("sorted_indices"):
        return False
    if arg(args, kwargs, 2, "lhs_indices") is not None or arg(args, kwargs, 7, "mode", "affine") != "affine":
        return False
    transpose = arg(args, kwargs, 4, "transpose", True)
    if not transpose or x.dim() < 1 or ov.below_floor(int(x.shape[0])):
        return False
    s, b, rhs = arg(args, kwargs, 0, "scales"), arg(args, kwargs, 1, "biases"), arg(args, kwargs, 3, "rhs_indices")
    gs, bits = arg(args, kwargs, 5, "group_size", 64), arg(args, kwargs, 6, "bits", 4)
    if not supported(x, w, s, b, rhs, transpose, gs, bits):
        return False
    if _int8_active(ov) and moe_int8.supported(x, w, s, b, rhs, transpose, gs, bits):
        ov.count("to_int8")
        return False
    return True


def _route(x, w, args, kwargs):
    return _k.hip(x, w, arg(args, kwargs, 0, "scales"), arg(args, kwargs, 1, "biases"),
                  arg(args, kwargs, 3, "rhs_indices"), group_size=arg(args, kwargs, 5, "group_size", 64),
                  bits=arg(args, kwargs, 6, "bits", 4))


def _self_check(found) -> bool:
    """A small sorted gather through the kernel against the implementation
    being replaced; skipped without a GPU (nothing can be routed there)."""
    import torch

    if not torch.cuda.is_available():
        return True
    from ._selfcheck import sorted_gather_matches

    return sorted_gather_matches(found["gather_qmm"], _k.hip)


_OV = Overlay("moe gather-ws prefill", MARKER, "TITAN_AMD_MOE_GATHER_WS", True,
              {"gather_qmm": (_should_route, _route)}, "TITAN_AMD_MOE_GATHER_WS_MIN_TOKENS", 7,
              "TITAN_AMD_MOE_GATHER_WS_MIN_ROWS", 64, self_check=_self_check, extra_stats=("to_int8",))


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
    """Drop the prepared tile-layout repacks."""
    prepared.clear_cache()


def warmup(model=None) -> int:
    """Repack every routed weight tensor the grouped GEMM would take into the
    tile layout, ahead of the first prefill chunk.  Returns how many tensors
    were prepared (0 with the tile cache off)."""
    if not prepared.enabled():
        return 0
    n = 0
    for m in switch_linears(model):
        if (m.bits, m.group_size, m.mode) != (_k.BITS, _k.GROUP, "affine") or m.bias is not None:
            continue
        if _k.pick_cfg(m.output_dims) is None or m.input_dims % 128 or not m.weight.is_cuda:
            continue
        prepared.tile_weights(m.weight, m.scales, m.biases)
        n += 1
    return n
