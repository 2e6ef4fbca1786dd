"""Sorted-gather MoE matmul on bf16 MFMA (titan/kernels/moe_gather_ws.py).

Replaces ``gather_qmm(..., sorted_indices=True)`` on the routed-expert prefill
GEMMs: int4 affine weights, bf16 activations, fp32 accumulation, bf16 output.
The weights of a (tile, column block) are dequantised in registers as
``bf16_rne(fmaf(q, s, b))`` (moe_gather_ws.py:343-344) and fed to
``v_mfma_f32_32x32x16_bf16``; rows are tiled raggedly per expert through the
caller-owned :class:`TileTable` (moe_gather_ws.py:159-202).  The weight tensor
is read in the tile layout when a repack of it was prepared ahead of time
(:mod:`.prepared`, filled by the patches' ``warmup``); otherwise -- no
warmup, or ``TITAN_AMD_TILE_CACHE=0`` -- the MLX-layout kernel reads the
tensors as they are (the same bits, ~20% slower).  A call builds nothing.

Exactness: the reference holds its Metal kernel bit-identical to MLX's own
sorted gather.  Here the bar is at most one bf16 ULP on live elements against
an fp64 sum over the bf16-dequantised weights, because the MFMA's internal
summation order is not MLX's.
"""

from __future__ import annotations

import torch

from .. import ops, stock
from ..ops import TileTable, max_tiles
from . import prepared
from .registry import KernelOp, ShapeClass, shape_class

__all__ = ["GROUP", "BITS", "OP", "TileTable", "build_tiles", "key", "max_tiles", "hip", "pick_cfg",
           "reference", "supports"]

GROUP = 64
BITS = 4


def pick_cfg(N: int):
    """(tile rows, waves per block) of the column block that divides N, or
    None (moe_gather_ws.py:394-400).  Four waves cover a 256-column block."""
    if N % 256 == 0:
        return (ops.tile_rows(), 4)
    return None


def build_tiles(rhs_indices: torch.Tensor, num_experts: int, tile_rows: int | None = None) -> TileTable:
    """Segment the sorted expert ids into a :class:`TileTable` on the device
    (moe_gather_ws.py:181-202).  The caller owns it and shares it between the
    two projections of one SwitchGLU."""
    return ops.build_tiles(rhs_indices, num_experts, tile_rows)


def reference(x, wq, scales, biases, rhs_indices, tiles=None, *, group_size=GROUP, bits=BITS):
    """``y[r] = x[r] @ dequant(w[expert(r)]).T`` through the stock gather
    (moe_gather_ws.py:403-414); ``tiles`` is ignored."""
    return stock.gather_qmm(x, wq, scales, biases, rhs_indices=rhs_indices, transpose=True,
                            group_size=group_size, bits=bits, sorted_indices=True)


def hip(x, wq, scales, biases, rhs_indices, tiles=None, *, group_size=GROUP, bits=BITS):
    """The grouped GEMM; same signature as :func:`reference`.  ``x`` is
    [R, 1, K] sorted by expert and ``rhs_indices`` the matching ids."""
    E, N = int(wq.shape[0]), int(scales.shape[1])
    if pick_cfg(N) is None:
        raise ops.QmoeUnsupported(ops._lib.ERR_UNSUPPORTED, f"no column block for N = {N}")
    R, K = int(x.shape[0]), int(x.shape[-1])
    if tiles is None:
        tiles = build_tiles(rhs_indices, E)
    if tiles.tile_rows != ops.tile_rows() or tiles.num_experts != E or tiles.rows != R:
        raise ValueError("tile table does not match this call")
    tw = prepared.lookup(wq, scales, biases) if prepared.enabled() else None
    if tw is not None:
        y = ops.gather_qmm_sorted_tiles(x.reshape(R, K), tw, tiles)
    else:
        y = ops.gather_qmm_sorted(x.reshape(R, K), wq, scales, biases, tiles, None, group_size, bits)
    return y.reshape(R, 1, N)


def key(x, wq, scales, biases, rhs_indices, tiles=None, *, group_size=GROUP, bits=BITS) -> ShapeClass:
    return shape_class(x, wq, scales, biases, rhs_indices, extra=(group_size, bits))


def supports(k: ShapeClass) -> bool:
    """moe_gather_ws.py:448-463, with this kernel's limits: K a multiple of
    128, N of 256, at least 64 rows (the sort threshold of SwitchGLU)."""
    if k.device != "gpu" or len(k.shapes) != 5 or k.extra != (GROUP, BITS):
        return False
    xs, ws, ss, bs, idx = k.shapes
    xd, wd, sd, bd, _ = k.dtypes
    if len(ws) != 3 or len(ss) != 3 or len(bs) != 3 or len(idx) != 1:
        return False
    if xd != torch.bfloat16 or sd != torch.bfloat16 or bd != torch.bfloat16:
        return False
    if wd not in (torch.int32, torch.uint32):
        return False
    if len(xs) != 3 or xs[1] != 1 or xs[0] != idx[0] or xs[0] < ops.SORTED_MIN_ROWS:
        return False
    if xs[-1] % 128 or ws[-1] * 8 != xs[-1] or ss[-1] * GROUP != xs[-1]:
        return False
    return pick_cfg(ss[1]) is not None


OP = KernelOp(
    name="moe_gather_ws",
    reference_fn=reference,
    fast_fn=hip,
    key=key,
    supports_key=supports,
    tolerance=1.0,  # bf16 ULPs on live elements, against the fp64 golden
    shapes=(
        {"R": 64, "K": 256, "N": 256, "E": 8, "bits": 4},
        {"R": 512, "K": 2048, "N": 1024, "E": 32, "bits": 4},
        {"R": 40960, "K": 2048, "N": 1024, "E": 256, "bits": 4},
    ),
    exactness="<= 1 bf16 ULP on live elements vs the fp64 sum over bf16-dequantised weights",
    source="titan/kernels/moe_gather_ws.py",
)
