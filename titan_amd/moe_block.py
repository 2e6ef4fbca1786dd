"""The routed mixture-of-experts block as one call
(titan/adapters/mlx/vendor/mlx_vlm/models/qwen3_5_moe/language.py:45-91,
Qwen3_5MoeSparseMoeBlock.__call__, with the fused router of
engine/patches/decode-fusion/fused_kernels.py:232-371).

    logits  = x @ W_router^T, fp32                   qmoe_router_logits (quantized router,
                                                     T <= 16), else qmoe_router_logits_dense
    idx, sc = top-k of logits, softmax over the k    qmoe_router_topk
    decode  (T * k < 64, switch_layers.py:218):
        h   = silu(x W_gate^T) * (x W_up^T)          qmoe_moe_gate_up_swiglu_tiles[_topk]
        y   = sum_j sc_j * W_down[idx_j] h_j          qmoe_moe_down_wsum_tiles
        (the _topk form selects idx and sc from the logits in-kernel, by the
        top-k's own code, and writes them for the down kernel, so the decode
        block is three launches)
    prefill:
        order, tiles = stable sort of the pairs       qmoe_route
        h   = SwiGLU gate_up grouped GEMM             qmoe_gather_qmm_swiglu_sorted_tiles
        yd  = down grouped GEMM over h                qmoe_gather_qmm_sorted_tiles
        y   = un-permute + weighted sum               qmoe_weighted_sum

Expert selection follows the fused router, not stock MLX: top-k on fp32
logits with ties to the lower expert index, scores in fp32.  Stock rounds the
softmax to bf16 first and breaks bf16 ties arbitrarily
(decode-fusion/REPORT.md:65-78), so the two can pick different experts on
near-ties; everything after the selection has the same semantics.

The optional shared expert (language.py:81-89: a dense SwiGLU MLP gated by
sigmoid(x w_gate)) runs through the same kernels as a one-expert table.

Resident weights (``resident``): by default one copy, in the tile layout --
the block repacks gate_up (in the gate/up-paired row order) and down at
construction and keeps only those, since every path it runs, decode GEMVs and
prefill grouped GEMMs, has a tile-layout kernel.  The tile layout is made for
the GEMMs (one contiguous 2 KiB chunk per 64 columns and group); the decode
GEMVs read it slower than the MLX layout (at one token x top-10 of 256
experts, hidden 2048: gate_up 5.7 against 5.0 us, down at 8 tokens 14.4
against 11.1 us), so ``resident="both"`` keeps the MLX tensors too and
decodes from them, at twice the memory.  Shapes outside the tile-layout
decode kernels' envelope (hidden a multiple of 2048 up to 8192, intermediate
512, top-k up to 16) keep the MLX tensors for decode either way.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import ops

__all__ = ["SparseMoeBlock", "SharedExpert", "DECODE_MAX_PAIRS", "ROUTER_GEMV_MAX_T", "TILE_DECODE_MAX_K",
           "tile_decode_supported"]

# switch_layers.py:218: SwitchGLU sorts when indices.size >= 64
DECODE_MAX_PAIRS = 64
# a quantized router's logits come from its codes up to this many tokens, and
# from its dequantised bf16 copy above (qmoe_router_logits_dense, a tiled MFMA
# GEMM from 48 tokens on)
ROUTER_GEMV_MAX_T = 16


# qmoe_moe_down_wsum_tiles takes at most this many experts per token (the
# MLX-layout qmoe_moe_down_wsum takes up to 64)
TILE_DECODE_MAX_K = 16


def tile_decode_supported(hidden: int, inter: int, group_size: int = ops.GROUP, bits: int = ops.BITS,
                          top_k: int = 1) -> bool:
    """Do the tile-layout decode kernels (qmoe_moe_gate_up_swiglu_tiles,
    qmoe_moe_down_wsum_tiles) take a SwiGLU MLP of this shape and top-k?"""
    return ((group_size, bits) == (ops.GROUP, ops.BITS) and hidden % 2048 == 0 and hidden <= 8192
            and inter == 512 and 1 <= top_k <= TILE_DECODE_MAX_K)


@dataclass
class SharedExpert:
    """Dense quantized SwiGLU MLP and its scalar gate (language.py:51-53, 81-89):
    gate_up (w, s, b) [1, 2S, H*bits/32] gate rows first, down (w, s, b)
    [1, H, S*bits/32], gate weight bf16 [1, H]."""

    gate_up: tuple
    down: tuple
    gate_weight: torch.Tensor


class SparseMoeBlock:
    """Routed experts of one MoE layer over MLX-affine 4-bit weights.

    ``router_weight`` bf16 [E, H], or an affine-quantized (w, scales, biases)
    triple with ``router_quant = (group_size, bits)`` whose decode logits come
    straight from the codes (the fused router, fused_kernels.py:232-260);
    ``gate_up`` = (w, scales, biases) of the
    fused [E, 2I, H] projection (gate rows first, loader.py:19-27); ``down`` =
    (w, scales, biases) of [E, H, I].  Both are repacked into the tile layout
    once, here (gate_up in the gate/up-paired row order of the SwiGLU kernels).
    ``resident``: "tiles" keeps only that copy when the tile-layout decode
    kernels take the shape (:func:`tile_decode_supported`); "both" also keeps
    the MLX tensors and decodes from them (faster GEMVs, twice the memory);
    ``prefill_tiles=False`` keeps only the MLX tensors and takes decode widths
    only.  ``nbytes`` reports what stays resident.

    ``sort_min_pairs`` is where the sorted path takes over (default 64, stock
    SwitchGLU's rule).  The two paths round differently -- the decode kernels
    use the exact affine weights, the grouped GEMMs bf16-materialised ones,
    as MLX's qmv and qmm do -- so the default keeps stock's numerics; a
    larger value trades that for speed at mid widths, where the decode
    kernels are faster on this part."""

    def __init__(self, router_weight: torch.Tensor, gate_up: tuple, down: tuple, top_k: int,
                 norm_topk_prob: bool = True, wsum_mode: str = "fast", group_size: int = ops.GROUP,
                 bits: int = ops.BITS, shared: SharedExpert | None = None, prefill_tiles: bool = True,
                 sort_min_pairs: int = DECODE_MAX_PAIRS, router_quant: tuple = (ops.GROUP, ops.BITS),
                 resident: str = "tiles"):
        self.router_weight = router_weight if isinstance(router_weight, torch.Tensor) else tuple(router_weight)
        self.router_quant = tuple(router_quant)
        if isinstance(self.router_weight, torch.Tensor):
            dense = self.router_weight.to(torch.bfloat16).contiguous()
        else:  # prefill logits: a GEMM over the weights dequantised once (bf16(fma(q, s, b)))
            dense = ops.dequantize(*self.router_weight, *self.router_quant)
        self._router_dense = dense  # [E, H]
        self.top_k = int(top_k)
        self.norm = bool(norm_topk_prob)
        self.wsum_mode = wsum_mode
        self.group_size, self.bits = group_size, bits
        self.num_experts = int(gate_up[0].shape[0])
        self.hidden = int(down[0].shape[1])
        self.intermediate = int(gate_up[0].shape[1]) // 2
        self.gu_tiles = self.down_tiles = None
        if prefill_tiles:
            self.gu_tiles = ops.repack_tiles(*gate_up, group_size, bits, swiglu_pairs=True)
            self.down_tiles = ops.repack_tiles(*down, group_size, bits)
        if resident not in ("tiles", "both"):
            raise ValueError(f"resident={resident!r}: 'tiles' or 'both'")
        self.resident = resident if prefill_tiles else "mlx"
        # decode from the same tile-layout copy when its kernels take the shape;
        # the MLX tensors stay resident only when something still reads them
        self.decode_tiles = self.resident == "tiles" and tile_decode_supported(self.hidden, self.intermediate,
                                                                               group_size, bits, self.top_k)
        self.gate_up = None if self.decode_tiles else tuple(gate_up)
        self.down = None if self.decode_tiles else tuple(down)
        # the sorted (grouped GEMM) path from this many (token, expert) pairs
        # on; below it the decode kernels (which take at most 16 tokens)
        self.sort_min_pairs = int(sort_min_pairs)
        self.shared = shared
        self._shared_tiles = None
        self._shared_decode_tiles = False
        if shared is not None and prefill_tiles:
            self._shared_tiles = (ops.repack_tiles(*shared.gate_up, group_size, bits, swiglu_pairs=True),
                                  ops.repack_tiles(*shared.down, group_size, bits))
            S = int(shared.gate_up[0].shape[1]) // 2
            if self.resident == "tiles" and tile_decode_supported(self.hidden, S, group_size, bits):
                self._shared_decode_tiles = True
                self.shared = SharedExpert(None, None, shared.gate_weight)

    @property
    def nbytes(self) -> int:
        """Device bytes of the resident expert weights (routed and shared)."""
        tensors = []
        for tw in (self.gu_tiles, self.down_tiles, *(self._shared_tiles or ())):
            if tw is not None:
                tensors += [tw.wp, tw.sb]
        for grp in (self.gate_up, self.down, *((self.shared.gate_up, self.shared.down) if self.shared else ())):
            if grp is not None:
                tensors += list(grp)
        return sum(t.numel() * t.element_size() for t in tensors)

    # ------------------------------------------------------------- router
    def route_logits(self, x2: torch.Tensor) -> torch.Tensor:
        """fp32 router logits [T, E] for tokens x2 [T, H]."""
        if x2.shape[0] <= ROUTER_GEMV_MAX_T:
            return ops.router_logits(x2, self.router_weight, *self.router_quant)
        return ops.router_logits(x2, self._router_dense)

    def route(self, x2: torch.Tensor):
        """(idx int32 [T, k], scores fp32 [T, k]) for tokens x2 [T, H]."""
        return ops.router_topk(self.route_logits(x2), self.top_k, self.norm)

    # ------------------------------------------------------------- experts
    def experts(self, x2: torch.Tensor, idx: torch.Tensor, scores: torch.Tensor) -> torch.Tensor:
        """sum_j scores[t, j] * expert_{idx[t, j]}(x2[t]) for x2 [T, H]."""
        T = x2.shape[0]
        k = idx.shape[-1]
        decode = T * k < self.sort_min_pairs and T <= 16
        if not decode and self.gu_tiles is None:
            if T > 16:
                raise ValueError("block built with prefill_tiles=False takes decode widths only (T <= 16)")
            decode = True
        if decode:
            if self.decode_tiles:
                h = ops.gate_up_silu_tiles(x2, self.gu_tiles, idx)
                return ops.down_wsum_tiles(h, self.down_tiles, idx, scores)
            h = ops.gate_up_silu(x2, *self.gate_up, idx, self.group_size, self.bits)
            return ops.down_wsum(h, *self.down, idx, scores, self.group_size, self.bits)
        r = ops.route(idx, self.num_experts)
        lhs = torch.div(r.order, k, rounding_mode="floor").to(torch.int32)
        h = ops.gather_qmm_swiglu_sorted_tiles(x2, self.gu_tiles, r.tiles, x_rows=lhs)
        yd = ops.gather_qmm_sorted_tiles(h, self.down_tiles, r.tiles)
        return ops.moe_weighted_sum(yd, r.inv_order, scores, (T, self.hidden), self.wsum_mode)

    def shared_expert(self, x2: torch.Tensor) -> torch.Tensor:
        """sigmoid(x w_gate) * SwiGLU-MLP(x) (language.py:81-89)."""
        sh = self.shared
        T = x2.shape[0]
        zeros = torch.zeros(T, 1, dtype=torch.int32, device=x2.device)
        ones = torch.ones(T, 1, dtype=torch.float32, device=x2.device)
        if T <= 16 and self._shared_decode_tiles:  # the fused down kernel takes up to 16 tokens
            gu_t, dn_t = self._shared_tiles
            h = ops.gate_up_silu_tiles(x2, gu_t, zeros)
            y = ops.down_wsum_tiles(h, dn_t, zeros, ones)
        elif T <= 16 or self._shared_tiles is None:
            h = ops.gate_up_silu(x2, *sh.gate_up, zeros, self.group_size, self.bits)
            y = ops.down_wsum(h, *sh.down, zeros, ones, self.group_size, self.bits)
        else:
            gu_t, dn_t = self._shared_tiles
            tiles = ops.build_tiles(zeros.reshape(-1), 1)
            h = ops.gather_qmm_swiglu_sorted_tiles(x2, gu_t, tiles)
            y = ops.gather_qmm_sorted_tiles(h, dn_t, tiles)
        z = ops.router_logits(x2, sh.gate_weight)
        return (torch.sigmoid(z) * y.float()).to(torch.bfloat16)

    def decodes_with_topk(self, T: int) -> bool:
        """Does a call with T tokens take the gate_up decode kernel that picks
        its experts from the router logits itself and hands the ids and scores
        to the down kernel (qmoe_moe_gate_up_swiglu_tiles_topk: one launch
        fewer than router_topk + the decode kernels, same results)?"""
        return (self.decode_tiles and T <= 16 and T * self.top_k < self.sort_min_pairs
                and self.num_experts <= 1024)

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        H = x.shape[-1]
        x2 = x.reshape(-1, H).to(torch.bfloat16).contiguous()
        if self.decodes_with_topk(x2.shape[0]):
            h, idx, scores = ops.gate_up_silu_tiles_topk(x2, self.gu_tiles, self.route_logits(x2), self.top_k,
                                                         self.norm)
            y = ops.down_wsum_tiles(h, self.down_tiles, idx, scores)
        else:
            idx, scores = self.route(x2)
            y = self.experts(x2, idx, scores)
        if self.shared is not None:
            y = (y.float() + self.shared_expert(x2).float()).to(torch.bfloat16)
        return y.reshape(x.shape)
