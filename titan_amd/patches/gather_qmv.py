"""Overlay: route unsorted (decode-width) ``gather_qmm`` calls and
``quantized_matmul`` through the gather-GEMV kernels.

The reference leaves these shapes on MLX's own gather_qmv
(titan/adapters/mlx/compiled.py:490-518, 209-218); this overlay is their
drop-in.  Routed when: ``sorted_indices`` false, affine ``transpose=True``
weights with biases, bf16 activations on the GPU.  Shapes the kernels do not
take (bits other than 4 and 8, group sizes other than 32/64/128, K outside the
kernels' range: 8-bit codes up to K = 4096) raise
:class:`~titan_amd._lib.QmoeUnsupported` inside the route and are handed down.

    TITAN_AMD_MOE_DECODE=1   enable (default on)
"""

from __future__ import annotations

import torch

from .. import ops
from ._overlay import Overlay, arg

MARKER = "_titan_amd_gather_qmv"


def _gpu_bf16(x) -> bool:
    return isinstance(x, torch.Tensor) and x.is_cuda and x.dtype == torch.bfloat16


def _route_gather_ok(ov, x, w, args, kwargs) -> bool:
    if not ov.enabled() or kwargs.get("sorted_indices") or not _gpu_bf16(x):
        return False
    return (arg(args, kwargs, 7, "mode", "affine") == "affine" and bool(arg(args, kwargs, 4, "transpose", True))
            and arg(args, kwargs, 1, "biases") is not None)


def _route_gather(x, w, args, kwargs):
    return ops.gather_qmm(x, w, arg(args, kwargs, 0, "scales"), arg(args, kwargs, 1, "biases"),
                          lhs_indices=arg(args, kwargs, 2, "lhs_indices"),
                          rhs_indices=arg(args, kwargs, 3, "rhs_indices"), transpose=True,
                          group_size=arg(args, kwargs, 5, "group_size", 64), bits=arg(args, kwargs, 6, "bits", 4))


def _route_qmm_ok(ov, x, w, args, kwargs) -> bool:
    if not ov.enabled() or not _gpu_bf16(x):
        return False
    return (arg(args, kwargs, 5, "mode", "affine") == "affine" and bool(arg(args, kwargs, 2, "transpose", True))
            and arg(args, kwargs, 1, "biases") is not None)


def _route_qmm(x, w, args, kwargs):
    return ops.quantized_matmul(x, w, arg(args, kwargs, 0, "scales"), arg(args, kwargs, 1, "biases"),
                                group_size=arg(args, kwargs, 3, "group_size", 64), bits=arg(args, kwargs, 4, "bits", 4))


def _self_check(found) -> bool:
    if not torch.cuda.is_available():
        return True
    from ._selfcheck import decode_gather_matches

    return decode_gather_matches(found["gather_qmm"], ops.gather_qmm)


_OV = Overlay("moe decode gather-qmv", MARKER, "TITAN_AMD_MOE_DECODE", True,
              {"gather_qmm": (_route_gather_ok, _route_gather), "quantized_matmul": (_route_qmm_ok, _route_qmm)},
              self_check=_self_check)


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
    """Nothing is cached."""


def warmup(model=None) -> int:
    return 0
