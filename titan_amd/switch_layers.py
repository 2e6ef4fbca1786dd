"""Routed-expert layers over quantized weights
(titan/adapters/mlx/vendor/mlx_lm/models/switch_layers.py).

:class:`QuantizedSwitchLinear` is the gather site: for sorted calls it asks
the registry for ``moe.gather_qmm_int8`` and then ``moe.gather_qmm_ws``
(switch_layers.py:100-123) and otherwise calls the namespace's
``gather_qmm`` (:mod:`titan_amd.core`, which an installed overlay patch may
have rerouted).  :class:`SwitchGLU` sorts the (token, slot) pairs by expert
when there are at least 64 of them (switch_layers.py:213-245), runs the fused
gate_up projection (gate rows first, loader.py:19-27), SwiGLU, the down
projection, and un-sorts.

Tensors stay on their device.  For ROCm tensors the sort is the HIP counting
sort, which also yields the tile table both projections share; CPU tensors use
torch's stable argsort and the stock gather.
"""

from __future__ import annotations

import torch

from . import core, kernels, ops
from ._lib import QmoeLibraryMissing

__all__ = ["QuantizedSwitchLinear", "SwitchGLU", "SwiGLU", "swiglu"]


def swiglu(gate: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """``silu(gate) * x`` (activations.py:9-11), in fp32, one bf16 rounding."""
    g = gate.to(torch.float32)
    return (g * torch.sigmoid(g) * x.to(torch.float32)).to(x.dtype)


class SwiGLU:
    """The default activation module: called as ``activation(x, gate)`` with
    the up projection first (switch_layers.py:189-194), ``silu(gate) * x``."""

    def __call__(self, x: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
        return swiglu(gate, x)


def _gather_sort(x: torch.Tensor, indices: torch.Tensor, num_experts: int):
    """Stable sort of the flattened pairs by expert (switch_layers.py:13-18):
    rows of x in sorted order, sorted ids, inverse permutation, tile table
    (None off the GPU)."""
    M = indices.shape[-1]
    flat = indices.reshape(-1)
    if flat.is_cuda:
        r = ops.route(flat, num_experts)
        order, inv, ids, tiles = r.order.long(), r.inv_order.long(), r.sorted_ids, r.tiles
    else:
        order = torch.argsort(flat, stable=True)
        inv = torch.argsort(order)
        ids, tiles = flat[order], None
    return x.flatten(0, -3)[order // M], ids, inv, tiles


def _scatter_unsort(x: torch.Tensor, inv_order: torch.Tensor, shape=None) -> torch.Tensor:
    """switch_layers.py:21-25."""
    x = x[inv_order]
    if shape is not None:
        x = x.unflatten(0, tuple(shape))
    return x


class QuantizedSwitchLinear:
    """Per-expert quantized linear layer: weight [E, N, K*bits/32] packed
    words, scales/biases [E, N, K/group_size] bf16, optional bias [E, N]."""

    def __init__(self, weight, scales, biases, group_size: int = 64, bits: int = 4, mode: str = "affine",
                 bias: torch.Tensor | None = None):
        self.weight, self.scales, self.biases = weight, scales, biases
        self.group_size, self.bits, self.mode = group_size, bits, mode
        self.bias = bias

    @property
    def input_dims(self) -> int:
        return self.scales.shape[2] * self.group_size

    @property
    def output_dims(self) -> int:
        return self.weight.shape[1]

    @property
    def num_experts(self) -> int:
        return self.weight.shape[0]

    def __call__(self, x, indices, sorted_indices: bool = False, tiles=None):
        """switch_layers.py:76-127: registry ops first for sorted calls, the
        namespace's gather otherwise or when both decline."""
        gathered = None
        if sorted_indices and self.mode == "affine" and self.bias is None:
            for name in ("moe.gather_qmm_int8", "moe.gather_qmm_ws"):
                op = kernels.get(name)
                if op is None:
                    continue
                try:
                    gathered = op(x, self.weight, self.scales, self.biases, indices, tiles=tiles,
                                  group_size=self.group_size, bits=self.bits)
                except QmoeLibraryMissing:
                    raise
                except Exception:  # noqa: BLE001 - fail closed to the namespace's gather
                    gathered = None
                if gathered is not None:
                    break
        if gathered is None:
            gathered = core.gather_qmm(x, self.weight, self.scales, self.biases, rhs_indices=indices,
                                       transpose=True, group_size=self.group_size, bits=self.bits,
                                       mode=self.mode, sorted_indices=sorted_indices)
        if self.bias is not None:
            gathered = gathered + self.bias[indices].unsqueeze(-2).to(gathered.dtype)
        return gathered


class SwitchGLU:
    """Routed SwiGLU MLP.  Either ``gate_up_proj`` (fused [E, 2I, K], gate rows
    first) or ``gate_proj`` and ``up_proj``; then ``down_proj``."""

    def __init__(self, down_proj: QuantizedSwitchLinear, gate_up_proj: QuantizedSwitchLinear | None = None,
                 gate_proj: QuantizedSwitchLinear | None = None, up_proj: QuantizedSwitchLinear | None = None,
                 activation=None):
        if gate_up_proj is None and (gate_proj is None or up_proj is None):
            raise ValueError("need gate_up_proj, or both gate_proj and up_proj")
        self.gate_up_proj, self.gate_proj, self.up_proj = gate_up_proj, gate_proj, up_proj
        self.down_proj = down_proj
        # called as activation(x_up, x_gate), the reference's operand order
        # (that of the SwiGLU module).  The bare swiglu function takes
        # (gate, x) instead (activations.py:9-11), so passed here it is
        # wrapped in the module, which gives it the right halves; the
        # reference would compute silu(up) * gate with it.
        if activation is None or activation is swiglu:
            activation = SwiGLU()
        self.activation = activation

    @property
    def num_experts(self) -> int:
        return self.down_proj.num_experts

    def __call__(self, x: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
        """x [..., D], indices [..., k] -> [..., k, D] (switch_layers.py:213-245)."""
        x = x.unsqueeze(-2).unsqueeze(-2)
        do_sort = indices.numel() >= 64
        idx, inv_order, tiles = indices, None, None
        if do_sort:
            x, idx, inv_order, tiles = _gather_sort(x, indices, self.num_experts)
        if self.gate_up_proj is not None:
            gu = self.gate_up_proj(x, idx, sorted_indices=do_sort, tiles=tiles)
            x_gate, x_up = gu.chunk(2, dim=-1)
        else:
            x_up = self.up_proj(x, idx, sorted_indices=do_sort, tiles=tiles)
            x_gate = self.gate_proj(x, idx, sorted_indices=do_sort, tiles=tiles)
        x = self.down_proj(self.activation(x_up, x_gate), idx, sorted_indices=do_sort, tiles=tiles)
        if do_sort:
            x = _scatter_unsort(x, inv_order, indices.shape)
        return x.squeeze(-2)
