"""MoE un-permute + routed weighted sum in one launch
(titan/kernels/moe_weighted_sum.py).

``out[t, :] = sum_j score[t, j] * y[inv(t * k + j), :]`` over the expert
outputs, reading the sorted rows through ``inv_order`` (or token-major rows
when it is None) and writing [rows, D] once.  Modes (moe_weighted_sum.py:44-49):

``clone`` bf16 products, eight bf16 partial accumulators (slot ``j % 8``)
          combined in order, the arithmetic of MLX's bf16 axis reduce;
``ops``   bf16-rounded products, fp32 accumulation;
``fast``  fp32 scores and products throughout.
"""

from __future__ import annotations

import math

import torch

from .. import _lib, ops
from .registry import KernelOp, ShapeClass, shape_class

__all__ = ["DEFAULT_MODE", "MODES", "OP", "hip", "key", "reference", "supports"]

# mode -> (partial accumulators, round products to bf16, accumulate in bf16, scores in input dtype)
MODES = {
    "fast": (8, 0, 0, False),
    "ops": (8, 1, 0, True),
    "clone": (8, 1, 1, True),
}
DEFAULT_MODE = "clone"


def reference(xs, inv_order, scores, out_shape, mode=DEFAULT_MODE):
    """The stock three-pass tail in torch ops (moe_weighted_sum.py:142-160):
    gather by ``inv_order``, scale by the scores, sum over k."""
    dim = int(out_shape[-1])
    rows = math.prod(int(d) for d in out_shape[:-1])
    k = scores.shape[-1]
    flat = xs.reshape(rows * k, dim)
    if inv_order is not None:
        flat = flat[inv_order.reshape(rows * k).long()]
    y = flat.reshape(*out_shape[:-1], k, dim)
    return (y * scores.reshape(*out_shape[:-1], k, 1).to(y.dtype)).sum(dim=-2)


def hip(xs, inv_order, scores, out_shape, mode=DEFAULT_MODE):
    """The fused kernel; same signature as :func:`reference`."""
    return ops.moe_weighted_sum(xs, inv_order, scores, out_shape, mode)


def key(xs, inv_order, scores, out_shape, mode=DEFAULT_MODE) -> ShapeClass:
    return shape_class(xs, inv_order, scores, extra=(tuple(out_shape), mode, inv_order is None))


def supports(k: ShapeClass) -> bool:
    """moe_weighted_sum.py:169-180 with this kernel's limits: bf16 rows, D a
    multiple of 8, at most 65535 output rows."""
    if k.device != "gpu" or not k.extra:
        return False
    out_shape, mode = k.extra[0], k.extra[1]
    if mode not in MODES or mode not in _lib.WSUM_MODES:
        return False
    if k.dtypes[0] != torch.bfloat16:
        return False
    if len(out_shape) < 2 or out_shape[-1] % 8:
        return False
    return math.prod(out_shape[:-1]) <= 65535


OP = KernelOp(
    name="moe_weighted_sum",
    reference_fn=reference,
    fast_fn=hip,
    key=key,
    supports_key=supports,
    tolerance=0.0,
    shapes=(
        {"T": 9, "K": 10, "D": 256},
        {"T": 13, "K": 10, "D": 2560},
        {"T": 1, "K": 10, "D": 2048},
        {"T": 2048, "K": 10, "D": 2048},
    ),
    exactness="bit-identical to the oracle's restatement of each mode",
    source="titan/kernels/moe_weighted_sum.py",
)
