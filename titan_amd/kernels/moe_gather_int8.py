"""int8-activation x int4-weight sorted-gather MoE matmul on int8 MFMA
(titan/kernels/moe_gather_int8.py).

Activations are quantised per token, symmetrically: ``sx = max|x| / 127``
(fp32), ``xi = clamp(rint(x / sx), -127, 127)``.  Per 64-wide group the kernel
forms ``D = sum xi * q`` with one ``v_mfma_i32_16x16x64_i8`` per 16 x 16 tile
(codes 0..15 are valid int8 operands as they are, so no re-centring and no
nibble-sum table) and ``R = sum xi`` exactly, then
``y = sx * sum_g (s * D + b * R)`` in fp32.  The weights are read in the tile
layout, repacked once per tensor: :class:`Int8Tables` holds that copy.

Not exact against the unquantised product, by design: this is the one op whose
fast path changes the numbers, so, as in the reference
(moe_gather_int8.py:431-442), it is selected only when the caller passes
prepared :class:`Int8Tables`, and its test bounds the relative RMS error
against the fake-quant product ``(sx * xi) @ deq(W)^T``.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from .. import ops, stock
from . import prepared
from .moe_gather_ws import build_tiles
from .registry import KernelOp, ShapeClass, shape_class

__all__ = ["BITS", "GROUP", "Int8Tables", "OP", "build_tables", "hip", "key", "pick_cfg",
           "quantize_activations", "reference", "supports"]

GROUP = 64
BITS = 4


@dataclass(frozen=True)
class Int8Tables:
    """Caller-owned prepared state for one weight tensor
    (moe_gather_int8.py:189-248): its tile-layout repack, per (expert,
    64-column block, group) a 2 KiB code chunk and a 256-byte chunk of
    scale|bias words -- the operands the int8 kernel copies contiguously.  The
    reference's tables add 18.8% of the weights (transposed scales, folded
    bias, nibble sums); these are a permuted copy of the weights themselves,
    shared with the bf16 path through the prepared cache.  Passing them is the
    caller's opt-in to the approximate path.  ``tw`` None (the tile cache off,
    ``TITAN_AMD_TILE_CACHE=0``): the MLX-layout int8 kernel reads the tensors
    as they are."""

    tw: ops.TileWeights | None

    @property
    def nbytes(self) -> int:
        return 0 if self.tw is None else self.tw.nbytes


def build_tables(wq, scales, biases) -> Int8Tables:
    """One weight tensor's tables: its tile-layout repack, built once per tensor
    (cached by the tensors' identity, :mod:`.prepared`); none with the tile
    cache off."""
    if wq.dim() != 3 or scales.shape != biases.shape or scales.dim() != 3:
        raise ValueError("expected w [E, N, K/8] and scales/biases [E, N, K/64]")
    if wq.shape[-1] * 8 != scales.shape[-1] * GROUP:
        raise ValueError("w and scales disagree on K")
    return Int8Tables(prepared.tile_weights(wq, scales, biases) if prepared.enabled() else None)


def pick_cfg(N: int):
    return (ops.tile_rows(), 4) if N % 256 == 0 else None


def quantize_activations(x: torch.Tensor):
    """Per-token symmetric int8 of bf16 rows: (xi int8 [R, K], sx fp32 [R])."""
    return ops.quantize_act_int8(x)


def reference(x, wq, scales, biases, rhs_indices, tables=None, tiles=None, *, group_size=GROUP, bits=BITS):
    """The stock (unquantised) gather (moe_gather_int8.py:377-390)."""
    return stock.gather_qmm(x, wq, scales, biases, rhs_indices=rhs_indices, transpose=True,
                            group_size=group_size, bits=bits, sorted_indices=True)


def hip(x, wq, scales, biases, rhs_indices, tables=None, tiles=None, *, group_size=GROUP, bits=BITS):
    """Quantise the rows, then the int8 grouped GEMM.  Same signature as
    :func:`reference`; ``tables`` None takes the tensor's prepared copy when
    one was built (``warmup``), else the MLX-layout kernel (nothing is built
    here)."""
    E, N = int(wq.shape[0]), int(scales.shape[1])
    if pick_cfg(N) is None:
        raise ops.QmoeUnsupported(ops._lib.ERR_UNSUPPORTED, f"no int8 tiling for N = {N}")
    if tables is None:
        tables = Int8Tables(prepared.lookup(wq, scales, biases) if prepared.enabled() else None)
    R, K = int(x.shape[0]), int(x.shape[-1])
    if tiles is None:
        tiles = build_tiles(rhs_indices, E)
    if tiles.tile_rows != ops.tile_rows() or tiles.num_experts != E or tiles.rows != R:
        raise ValueError("tile table does not match this call")
    xi, sx = quantize_activations(x.reshape(R, K))
    if tables.tw is not None:
        y = ops.gather_qmm_int8_sorted_tiles(xi, sx, tables.tw, tiles)
    else:
        y = ops.gather_qmm_int8_sorted(xi, sx, wq, scales, biases, tiles, None, group_size, bits)
    return y.reshape(R, 1, N)


def key(x, wq, scales, biases, rhs_indices, tables=None, tiles=None, *, group_size=GROUP,
        bits=BITS) -> ShapeClass:
    return shape_class(x, wq, scales, biases, rhs_indices, extra=(group_size, bits, tables is not None))


def supports(k: ShapeClass) -> bool:
    """Opt-in (tables passed), 4-bit group 64, [R, 1, K] bf16 rows, K a
    multiple of 512 up to 4096 (the gate_up and the down projection; the
    quantiser reads 16-byte runs of K/64 elements per lane), N of 256
    (moe_gather_int8.py:435-450)."""
    if k.device != "gpu" or len(k.shapes) != 5 or len(k.extra) != 3:
        return False
    group_size, bits, has_tables = k.extra
    if not has_tables or (group_size, bits) != (GROUP, BITS):
        return False
    xs, ws, ss, _bs, idx = k.shapes
    if len(ws) != 3 or len(ss) != 3 or len(idx) != 1 or k.dtypes[0] != torch.bfloat16:
        return False
    if len(xs) != 3 or xs[1] != 1 or xs[0] != idx[0] or xs[-1] % 512 or xs[-1] > 4096 \
            or xs[0] < ops.SORTED_MIN_ROWS:
        return False
    return pick_cfg(ss[1]) is not None


OP = KernelOp(
    name="moe_gather_int8",
    default_off=True,
    default_off_reason="changes the numbers (per-token int8 activations); opt in by naming it",
    aliases=("moe_gather_gate_up",),
    reference_fn=reference,
    fast_fn=hip,
    key=key,
    supports_key=supports,
    tolerance=0.01,  # relative RMS against the unquantised product
    shapes=(
        {"R": 300, "K": 1024, "N": 256, "E": 8, "bits": 4},
        {"R": 640, "K": 2048, "N": 512, "E": 16, "bits": 4},
        {"R": 40960, "K": 2048, "N": 1024, "E": 256, "bits": 4},
        {"R": 40960, "K": 512, "N": 2048, "E": 256, "bits": 4},
    ),
    exactness="not exact: per-token int8 activations; integer parts exact, fp32 rescale",
    source="titan/kernels/moe_gather_int8.py",
)
