"""The stock semantics of the quantized matmuls, in plain torch ops.

This is what an un-patched caller gets (the role ``mx.gather_qmm`` and
``mx.quantized_matmul`` play for the reference, called at
titan/adapters/mlx/vendor/mlx_lm/models/switch_layers.py:87-98 and
titan/adapters/mlx/compiled.py:209-218) and what the registry answers with for
a shape class the HIP kernels do not take.  It runs on the device of its
inputs with torch's own kernels: dequantise to bf16, then multiply in fp32.
It is slow and general (bits 2, 4 and 8; any group size dividing K;
``transpose`` either way); the HIP path is fast and narrow.

Dequantisation is ``bf16(q * s + b)`` computed in fp32.  ``q * s`` is exact in
fp32 for codes of at most 8 bits and bf16 scales (at most 16 significant bits),
so this equals the single rounding ``bf16_rne(fmaf(q, s, b))`` of
titan/kernels/moe_gather_ws.py:343-344.
"""

from __future__ import annotations

import math

import torch

__all__ = ["unpack", "dequantize", "gather_qmm", "quantized_matmul"]

_BITS = (2, 4, 8)


def unpack(w: torch.Tensor, bits: int) -> torch.Tensor:
    """Packed 32-bit words [..., KW] -> codes uint8 [..., KW * 32 / bits]; the
    low bits of a word hold the earliest element
    (tests/kernels/test_moe_gather_int8.py:104-115)."""
    if bits not in _BITS:
        raise ValueError(f"bits={bits}: the stock path unpacks {_BITS}")
    per = 32 // bits
    v = w.to(torch.int64) & 0xFFFFFFFF
    shifts = torch.arange(per, device=w.device, dtype=torch.int64) * bits
    q = (v.unsqueeze(-1) >> shifts) & ((1 << bits) - 1)
    return q.reshape(*w.shape[:-1], w.shape[-1] * per).to(torch.uint8)


def dequantize(w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor | None, group_size: int,
               bits: int) -> torch.Tensor:
    """[..., N, KW] words + [..., N, G] scales/biases -> bf16 [..., N, K]."""
    q = unpack(w, bits).to(torch.float32)
    K = q.shape[-1]
    if K % group_size or scales.shape[-1] != K // group_size:
        raise ValueError(f"K={K}, group_size={group_size} and scales {tuple(scales.shape)} disagree")
    qg = q.reshape(*q.shape[:-1], K // group_size, group_size)
    y = qg * scales.to(torch.float32).unsqueeze(-1)
    if biases is not None:
        y = y + biases.to(torch.float32).unsqueeze(-1)
    return y.reshape(q.shape).to(torch.bfloat16)


def _matmul(x: torch.Tensor, wd: torch.Tensor, transpose: bool) -> torch.Tensor:
    """x [..., M, K] times bf16 weights (W^T when ``transpose``), fp32 products
    and sums, bf16 result."""
    w32 = wd.to(torch.float32)
    return (x.to(torch.float32) @ (w32.transpose(-1, -2) if transpose else w32)).to(torch.bfloat16)


def quantized_matmul(x, w, scales, biases=None, transpose=True, group_size=64, bits=4, mode="affine"):
    """``x @ deq(W)^T`` (transpose) or ``x @ deq(W)``."""
    if mode != "affine":
        raise ValueError(f"mode={mode!r}: the stock path dequantizes affine weights")
    return _matmul(x, dequantize(w, scales, biases, group_size, bits), transpose)


def gather_qmm(x, w, scales, biases=None, lhs_indices=None, rhs_indices=None, transpose=True, group_size=64,
               bits=4, mode="affine", sorted_indices=False):
    """``out[i] = x[lhs[i]] @ deq(W[rhs[i]])^T`` over the broadcast batch of
    ``lhs_indices`` (default: x's batch) and ``rhs_indices`` (default: every
    expert); result [*batch, M, N] in bf16.  Each distinct expert is
    dequantised once.  ``sorted_indices`` is a promise the stock path does not
    need."""
    if mode != "affine":
        raise ValueError(f"mode={mode!r}: the stock path dequantizes affine weights")
    dev = x.device
    M, K = x.shape[-2], x.shape[-1]
    xb = tuple(x.shape[:-2])
    E = w.shape[0]
    rhs = torch.arange(E, device=dev) if rhs_indices is None else rhs_indices.to(dev).long()
    if lhs_indices is None:
        batch = torch.broadcast_shapes(xb, tuple(rhs.shape))
        xi = torch.arange(math.prod(xb), device=dev).reshape(xb).expand(batch).reshape(-1)
    else:
        lhs = lhs_indices.to(dev).long()
        batch = torch.broadcast_shapes(tuple(lhs.shape), tuple(rhs.shape))
        xi = lhs.expand(batch).reshape(-1)
    e = rhs.expand(batch).reshape(-1)
    x2 = x.reshape(-1, M, K)
    N = scales.shape[-2] if transpose else w.shape[-1] * (32 // bits)
    out = torch.empty(e.numel(), M, N, dtype=torch.bfloat16, device=dev)
    for ex in torch.unique(e).tolist():
        sel = (e == ex).nonzero().flatten()
        wd = dequantize(w[ex], scales[ex], None if biases is None else biases[ex], group_size, bits)
        out[sel] = _matmul(x2[xi[sel]], wd, transpose)
    return out.reshape(*batch, M, N)
