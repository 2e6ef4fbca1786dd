"""Torch-facing wrappers of the libqmoe C ABI.

Tensors are ROCm torch tensors: bf16 activations, packed weights as ``int32``
or ``uint32`` (the bits are what matter), bf16 scales and biases.  Every
function enqueues on torch's current stream and never synchronises.  Each
raises :class:`~titan_amd._lib.QmoeUnsupported` for a configuration without a
kernel and :class:`~titan_amd._lib.QmoeLibraryMissing` when the library is not
built: there is no other implementation behind these names.

Call-surface parity with the reference (paths relative to its root):

* :func:`gather_qmm`            mx.gather_qmm as called at
  titan/adapters/mlx/vendor/mlx_lm/models/switch_layers.py:87-98
* :func:`quantized_matmul`      mx.quantized_matmul (titan/adapters/mlx/compiled.py:209-218)
* :func:`route` / :func:`build_tiles`   _gather_sort (switch_layers.py:13-18) and
  titan/kernels/moe_gather_ws.py:181-202
* :func:`moe_weighted_sum`      titan/kernels/moe_weighted_sum.py:142-195
* :func:`gate_up_silu` / :func:`down_wsum`
  engine/patches/decode-fusion/fused_kernels.py:194-231
* :func:`quantize_act_int8` / :func:`gather_qmm_int8`
  titan/kernels/moe_gather_int8.py:168-182, 393-425
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import _lib
from ._lib import QmoeError, QmoeUnsupported

GROUP = 64
BITS = 4
# SwitchGLU sorts when indices.size >= 64 (switch_layers.py:218); the grouped
# GEMM takes sorted calls from that size up.
SORTED_MIN_ROWS = 64


def tile_rows() -> int:
    """Rows per tile of the grouped GEMM (the tile table must use this)."""
    return int(_lib.load().qmoe_gemm_tile_rows())


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _dev(t: torch.Tensor, name: str) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.device.type != "cuda":
        raise QmoeUnsupported(_lib.ERR_UNSUPPORTED, f"{name} is on {t.device}; libqmoe runs on the GPU")


def _ready(t: torch.Tensor) -> torch.Tensor:
    """Contiguous and 16-byte aligned (a copy only when it is not)."""
    if not t.is_contiguous():
        t = t.contiguous()
    if t.data_ptr() % 16:
        t = t.clone()
    return t


def _bf16(t: torch.Tensor, name: str) -> torch.Tensor:
    _dev(t, name)
    if t.dtype != torch.bfloat16:
        raise QmoeUnsupported(_lib.ERR_UNSUPPORTED, f"{name} must be bfloat16, got {t.dtype}")
    return _ready(t)


def _words(t: torch.Tensor, name: str) -> torch.Tensor:
    _dev(t, name)
    if t.dtype not in (torch.int32, torch.uint32):
        raise QmoeUnsupported(_lib.ERR_UNSUPPORTED, f"{name} must hold packed uint32 words, got {t.dtype}")
    return _ready(t)


def _i32(t: torch.Tensor, name: str, device) -> torch.Tensor:
    if not isinstance(t, torch.Tensor):
        t = torch.as_tensor(t)
    if t.device != device:
        t = t.to(device)
    if t.dtype != torch.int32:
        t = t.to(torch.int32)
    return _ready(t)


def _f32(t: torch.Tensor, name: str, device) -> torch.Tensor:
    if t.device != device:
        t = t.to(device)
    if t.dtype != torch.float32:
        t = t.to(torch.float32)
    return _ready(t)


def _ptr(t):
    return None if t is None else t.data_ptr()


# ------------------------------------------------------------------ layout


def unpack(w: torch.Tensor, bits: int = BITS) -> torch.Tensor:
    """uint8 codes [..., words * 32/bits], low bits first."""
    w = _words(w, "w")
    per = 32 // bits
    out = torch.empty(*w.shape[:-1], w.shape[-1] * per, dtype=torch.uint8, device=w.device)
    _lib.call("qmoe_unpack", w.data_ptr(), w.numel(), bits, out.data_ptr(), _stream(w))
    return out


def dequantize(w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, group_size: int = GROUP,
               bits: int = BITS) -> torch.Tensor:
    """bf16_rne(fmaf(q, s, b)) for every element (mx.dequantize)."""
    w, scales, biases = _words(w, "w"), _bf16(scales, "scales"), _bf16(biases, "biases")
    K = w.shape[-1] * 32 // bits
    rows = w.numel() // w.shape[-1]
    out = torch.empty(*w.shape[:-1], K, dtype=torch.bfloat16, device=w.device)
    _lib.call("qmoe_dequantize", w.data_ptr(), scales.data_ptr(), biases.data_ptr(), rows, K,
              group_size, bits, out.data_ptr(), _stream(w))
    return out


# ------------------------------------------------------------------ routing


def max_tiles(rows: int, num_experts: int, tile_rows_: int) -> int:
    """Static bound on sum(ceil(rows_e / tile_rows)) (moe_gather_ws.py:176-178)."""
    return (rows + tile_rows_ - 1) // tile_rows_ + num_experts


@dataclass(frozen=True)
class TileTable:
    """Segment offsets plus the ragged (row_start, expert) tile list, built on
    the device and owned by the caller (moe_gather_ws.py:159-173)."""

    offsets: torch.Tensor   # [E + 1] int32
    tile_row: torch.Tensor  # [maxt] int32
    tile_exp: torch.Tensor  # [maxt] int32
    ntiles: torch.Tensor    # [1] int32
    maxt: int
    tile_rows: int
    num_experts: int
    rows: int


@dataclass(frozen=True)
class Routing:
    """Stable expert sort of flattened (token, slot) pairs plus its tile table."""

    order: torch.Tensor       # [n] pair index of sorted row i
    inv_order: torch.Tensor   # [n] argsort(order)
    sorted_ids: torch.Tensor  # [n] ids[order]
    tiles: TileTable
    bad_ids: torch.Tensor     # [1] int32 count of ids outside [0, E) (clamped)


def build_tiles(sorted_ids: torch.Tensor, num_experts: int, tile_rows_: int | None = None) -> TileTable:
    """Tile table over ids already sorted ascending."""
    _dev(sorted_ids, "sorted_ids")
    dev = sorted_ids.device
    ids = _i32(sorted_ids.reshape(-1), "sorted_ids", dev)
    tr = tile_rows() if tile_rows_ is None else int(tile_rows_)
    n = ids.numel()
    mt = max_tiles(n, num_experts, tr)
    offsets = torch.empty(num_experts + 1, dtype=torch.int32, device=dev)
    trow = torch.empty(mt, dtype=torch.int32, device=dev)
    texp = torch.empty(mt, dtype=torch.int32, device=dev)
    nt = torch.empty(1, dtype=torch.int32, device=dev)
    _lib.call("qmoe_build_tiles", ids.data_ptr(), n, num_experts, tr, offsets.data_ptr(),
              trow.data_ptr(), texp.data_ptr(), nt.data_ptr(), mt, _stream(ids))
    return TileTable(offsets, trow, texp, nt, mt, tr, num_experts, n)


def route(ids: torch.Tensor, num_experts: int, tile_rows_: int | None = None) -> Routing:
    """Stable argsort of expert ids with inverse and tile table, no host sync."""
    _dev(ids, "ids")
    dev = ids.device
    flat = _i32(ids.reshape(-1), "ids", dev)
    n = flat.numel()
    tr = tile_rows() if tile_rows_ is None else int(tile_rows_)
    mt = max_tiles(n, num_experts, tr)
    L = _lib.load()
    ws_bytes = int(L.qmoe_route_workspace_size(n, num_experts))
    ws = torch.empty(max(ws_bytes, 256) // 4, dtype=torch.int32, device=dev)
    order = torch.empty(n, dtype=torch.int32, device=dev)
    inv = torch.empty(n, dtype=torch.int32, device=dev)
    srt = torch.empty(n, dtype=torch.int32, device=dev)
    offsets = torch.empty(num_experts + 1, dtype=torch.int32, device=dev)
    trow = torch.empty(mt, dtype=torch.int32, device=dev)
    texp = torch.empty(mt, dtype=torch.int32, device=dev)
    nt = torch.empty(1, dtype=torch.int32, device=dev)
    _lib.call("qmoe_route", flat.data_ptr(), n, num_experts, tr, order.data_ptr(), inv.data_ptr(),
              srt.data_ptr(), offsets.data_ptr(), trow.data_ptr(), texp.data_ptr(), nt.data_ptr(), mt,
              ws.data_ptr(), ws.numel() * 4, _stream(flat))
    tiles = TileTable(offsets, trow, texp, nt, mt, tr, num_experts, n)
    return Routing(order, inv, srt, tiles, ws[:1])


# ------------------------------------------------------------- gather_qmm


def _check_quant(w, scales, group_size, bits, K):
    if bits not in (4, 8):
        raise QmoeUnsupported(_lib.ERR_UNSUPPORTED, f"bits={bits}")
    if w.shape[-1] * 32 // bits != K:
        raise ValueError(f"x has K={K} but w packs {w.shape[-1] * 32 // bits} elements per row")
    if scales.shape[-1] * group_size != K:
        raise ValueError(f"scales carry {scales.shape[-1]} groups of {group_size}, K={K}")


def gather_qmv(x: torch.Tensor, x_rows: torch.Tensor | None, experts: torch.Tensor, w: torch.Tensor,
               scales: torch.Tensor, biases: torch.Tensor, group_size: int = GROUP,
               bits: int = BITS) -> torch.Tensor:
    """Row form, matrix-vector kernel: out[r] = x[x_rows[r]] @ deq(W[experts[r]])^T."""
    x = _bf16(x, "x")
    K = x.shape[-1]
    x2 = x.reshape(-1, K)
    w, scales, biases = _words(w, "w"), _bf16(scales, "scales"), _bf16(biases, "biases")
    _check_quant(w, scales, group_size, bits, K)
    dev = x.device
    e = _i32(experts.reshape(-1), "experts", dev)
    xr = None if x_rows is None else _i32(x_rows.reshape(-1), "x_rows", dev)
    E, N = w.shape[0], w.shape[1]
    out = torch.empty(e.numel(), N, dtype=torch.bfloat16, device=dev)
    _lib.call("qmoe_gather_qmv", x2.data_ptr(), _ptr(xr), e.data_ptr(), e.numel(), K, w.data_ptr(),
              scales.data_ptr(), biases.data_ptr(), E, N, group_size, bits, out.data_ptr(), _stream(x))
    return out


def gather_qmm_sorted(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
                      tiles: TileTable, x_rows: torch.Tensor | None = None, group_size: int = GROUP,
                      bits: int = BITS) -> torch.Tensor:
    """Grouped GEMM over expert-sorted rows described by ``tiles``:
    out[r] = x[x_rows[r]] @ deq(W[e(r)])^T, rows [0, tiles.rows)."""
    x = _bf16(x, "x")
    K = x.shape[-1]
    x2 = x.reshape(-1, K)
    w, scales, biases = _words(w, "w"), _bf16(scales, "scales"), _bf16(biases, "biases")
    _check_quant(w, scales, group_size, bits, K)
    dev = x.device
    xr = None if x_rows is None else _i32(x_rows.reshape(-1), "x_rows", dev)
    R = tiles.rows
    E, N = w.shape[0], w.shape[1]
    if tiles.num_experts != E:
        raise ValueError("tile table was built for a different expert count")
    if tiles.tile_rows != tile_rows():
        raise ValueError(f"tile table uses {tiles.tile_rows} rows per tile, the GEMM needs {tile_rows()}")
    out = torch.empty(R, N, dtype=torch.bfloat16, device=dev)
    _lib.call("qmoe_gather_qmm_sorted", x2.data_ptr(), _ptr(xr), R, K, w.data_ptr(), scales.data_ptr(),
              biases.data_ptr(), E, N, group_size, bits, tiles.offsets.data_ptr(),
              tiles.tile_row.data_ptr(), tiles.tile_exp.data_ptr(), tiles.ntiles.data_ptr(), tiles.maxt,
              out.data_ptr(), _stream(x))
    return out


@dataclass(frozen=True)
class TileWeights:
    """Expert weights repacked into the tile layout (qmoe_repack_tiles): per
    (expert, 64-column block, group) a 2 KiB chunk of codes ``wp`` and a
    256-byte chunk of scale|bias words ``sb``.  Built once per weight tensor
    at load time and owned by the caller, in the role of the reference's
    prepared tables (titan/kernels/moe_gather_int8.py:189-248)."""

    wp: torch.Tensor  # int32 [E, N/64, G, 2, 2, 32, 4]
    sb: torch.Tensor  # int32 [E, N/64, G, 64]
    num_experts: int
    N: int
    K: int
    group_size: int = GROUP
    bits: int = BITS
    swiglu_pairs: bool = False  # rows in the gate/up-paired order of qmoe_gather_qmm_swiglu_sorted_tiles

    @property
    def nbytes(self) -> int:
        return self.wp.numel() * 4 + self.sb.numel() * 4


def swiglu_pair_order(N: int, device=None) -> torch.Tensor:
    """Row order of a fused [gate(I) | up(I)] weight in which every 64-row
    block holds 32 gate rows and the up rows of the same 32 indices: row
    64c + j is gate row 32c + j (j < 32) or up row I + 32c + j - 32."""
    if N % 64:
        raise QmoeUnsupported(_lib.ERR_UNSUPPORTED, f"N={N}: gate/up pairing needs N % 64 == 0")
    I = N // 2
    t = torch.arange(N, device=device)
    c, j = t // 64, t % 64
    return torch.where(j < 32, 32 * c + j, I + 32 * c + j - 32)


def repack_tiles(w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, group_size: int = GROUP,
                 bits: int = BITS, swiglu_pairs: bool = False) -> TileWeights:
    """MLX-layout expert weights [E, N, K/8] -> :class:`TileWeights`.  With
    ``swiglu_pairs`` a fused gate_up weight is first put in the gate/up-paired
    row order (:func:`swiglu_pair_order`) for the SwiGLU-epilogue GEMM."""
    w, scales, biases = _words(w, "w"), _bf16(scales, "scales"), _bf16(biases, "biases")
    if w.dim() != 3:
        raise QmoeUnsupported(_lib.ERR_UNSUPPORTED, f"w must be [E, N, K/8], got {tuple(w.shape)}")
    E, N, KW = w.shape
    K = KW * 32 // bits
    _check_quant(w, scales, group_size, bits, K)
    if swiglu_pairs:
        perm = swiglu_pair_order(N, w.device)
        w, scales, biases = (t.index_select(1, perm).contiguous() for t in (w, scales, biases))
    G = K // group_size
    wp = torch.empty(E, max(N // 64, 0), G, 2, 2, 32, 4, dtype=torch.int32, device=w.device)
    sb = torch.empty(E, max(N // 64, 0), G, 64, dtype=torch.int32, device=w.device)
    _lib.call("qmoe_repack_tiles", w.data_ptr(), scales.data_ptr(), biases.data_ptr(), E, N, K, group_size, bits,
              wp.data_ptr(), sb.data_ptr(), _stream(w))
    return TileWeights(wp, sb, E, N, K, group_size, bits, swiglu_pairs)


def gather_qmm_sorted_tiles(x: torch.Tensor, tw: TileWeights, tiles: TileTable,
                            x_rows: torch.Tensor | None = None) -> torch.Tensor:
    """:func:`gather_qmm_sorted` over tile-layout weights; bit-identical result."""
    x = _bf16(x, "x")
    K = x.shape[-1]
    if K != tw.K:
        raise ValueError(f"x has K={K}, the weights K={tw.K}")
    if tiles.num_experts != tw.num_experts or tiles.tile_rows != tile_rows():
        raise ValueError("tile table does not match this call")
    xr = None if x_rows is None else _i32(x_rows.reshape(-1), "x_rows", x.device)
    out = torch.empty(tiles.rows, tw.N, dtype=torch.bfloat16, device=x.device)
    _lib.call("qmoe_gather_qmm_sorted_tiles", x.data_ptr(), _ptr(xr), tiles.rows, K, tw.wp.data_ptr(),
              tw.sb.data_ptr(), tw.num_experts, tw.N, tiles.offsets.data_ptr(), tiles.tile_row.data_ptr(),
              tiles.tile_exp.data_ptr(), tiles.ntiles.data_ptr(), tiles.maxt, out.data_ptr(), _stream(x))
    return out


def gather_qmv_tiles(x: torch.Tensor, x_rows: torch.Tensor | None, experts: torch.Tensor,
                     tw: TileWeights) -> torch.Tensor:
    """:func:`gather_qmv` over tile-layout weights: out[r] = x[x_rows[r]] . W[experts[r]]^T."""
    x = _bf16(x, "x")
    K = x.shape[-1]
    if K != tw.K:
        raise ValueError(f"x has K={K}, the weights K={tw.K}")
    ex = _i32(experts.reshape(-1), "experts", x.device)
    xr = None if x_rows is None else _i32(x_rows.reshape(-1), "x_rows", x.device)
    n = ex.numel()
    out = torch.empty(n, tw.N, dtype=torch.bfloat16, device=x.device)
    _lib.call("qmoe_gather_qmv_tiles", x.data_ptr(), _ptr(xr), ex.data_ptr(), n, K, tw.wp.data_ptr(),
              tw.sb.data_ptr(), tw.num_experts, tw.N, out.data_ptr(), _stream(x))
    return out


def gate_up_silu_tiles(x: torch.Tensor, tw: TileWeights, idx: torch.Tensor) -> torch.Tensor:
    """:func:`gate_up_silu` over tile-layout fused gate_up weights [E, 2I, K] in
    the gate/up-paired row order (``repack_tiles(..., swiglu_pairs=True)``, the
    layout of :func:`gather_qmm_swiglu_sorted_tiles`)."""
    if not tw.swiglu_pairs:
        raise ValueError("the decode SwiGLU kernel needs weights repacked with swiglu_pairs=True")
    x = _bf16(x, "x")
    T, K = x.shape
    if K != tw.K:
        raise ValueError(f"x has K={K}, the weights K={tw.K}")
    idx = _i32(idx, "idx", x.device)
    k = idx.shape[-1]
    I = tw.N // 2
    h = torch.empty(T, k, I, dtype=torch.bfloat16, device=x.device)
    _lib.call("qmoe_moe_gate_up_swiglu_tiles", x.data_ptr(), idx.data_ptr(), T, k, K, tw.wp.data_ptr(),
              tw.sb.data_ptr(), tw.num_experts, I, h.data_ptr(), _stream(x))
    return h


def down_wsum_tiles(h: torch.Tensor, tw: TileWeights, idx: torch.Tensor, scores: torch.Tensor) -> torch.Tensor:
    """:func:`down_wsum` over tile-layout down weights [E, D, I]."""
    if tw.swiglu_pairs:
        raise ValueError("down weights are repacked in their own row order (swiglu_pairs=False)")
    h = _bf16(h, "h")
    T, k, I = h.shape
    if I != tw.K:
        raise ValueError(f"h has I={I}, the weights K={tw.K}")
    idx = _i32(idx, "idx", h.device)
    sc = _f32(scores, "scores", h.device)
    y = torch.empty(T, tw.N, dtype=torch.bfloat16, device=h.device)
    _lib.call("qmoe_moe_down_wsum_tiles", h.data_ptr(), idx.data_ptr(), sc.data_ptr(), T, k, I, tw.wp.data_ptr(),
              tw.sb.data_ptr(), tw.num_experts, tw.N, y.data_ptr(), _stream(h))
    return y


def _logits(logits: torch.Tensor, T: int, E: int, device) -> torch.Tensor:
    lg = _f32(logits, "logits", device)
    if tuple(lg.shape) != (T, E):
        raise ValueError(f"logits must be [T, E] = [{T}, {E}], got {tuple(lg.shape)}")
    return lg


def gate_up_silu_tiles_topk(x: torch.Tensor, tw: TileWeights, logits: torch.Tensor, top_k: int,
                            norm: bool = True):
    """:func:`gate_up_silu_tiles` with each token's experts chosen in the kernel
    from its fp32 router logits [T, E] by :func:`router_topk`'s selection.
    Returns (h [T, k, I], idx int32 [T, k], scores fp32 [T, k]), equal to
    ``idx, scores = router_topk(logits, top_k, norm)`` and
    ``h = gate_up_silu_tiles(x, tw, idx)``, with one launch fewer."""
    if not tw.swiglu_pairs:
        raise ValueError("the decode SwiGLU kernel needs weights repacked with swiglu_pairs=True")
    x = _bf16(x, "x")
    T, K = x.shape
    if K != tw.K:
        raise ValueError(f"x has K={K}, the weights K={tw.K}")
    lg = _logits(logits, T, tw.num_experts, x.device)
    I = tw.N // 2
    h = torch.empty(T, top_k, I, dtype=torch.bfloat16, device=x.device)
    idx = torch.empty(T, top_k, dtype=torch.int32, device=x.device)
    scores = torch.empty(T, top_k, dtype=torch.float32, device=x.device)
    _lib.call("qmoe_moe_gate_up_swiglu_tiles_topk", x.data_ptr(), lg.data_ptr(), int(bool(norm)), T, top_k, K,
              tw.wp.data_ptr(), tw.sb.data_ptr(), tw.num_experts, I, h.data_ptr(), idx.data_ptr(),
              scores.data_ptr(), _stream(x))
    return h, idx, scores


def gemm_supported(K: int, N: int, group_size: int, bits: int) -> bool:
    return bits == 4 and group_size == 64 and K % 128 == 0 and N % 256 == 0


def gather_qmm(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor | None = None,
               lhs_indices: torch.Tensor | None = None, rhs_indices: torch.Tensor | None = None,
               transpose: bool = True, group_size: int = GROUP, bits: int = BITS, mode: str = "affine",
               sorted_indices: bool = False, *, tiles: TileTable | None = None) -> torch.Tensor:
    """mx.gather_qmm for transpose=True affine weights.

    ``x`` is [..., M, K] and ``w`` [E, N, K*bits/32].  The batch is the
    broadcast of ``lhs_indices`` (default: x's own batch) with ``rhs_indices``
    (default: every expert), and the result is [*batch, M, N]:
    out[i, m] = x[lhs[i], m] @ deq(W[rhs[i]])^T.  ``sorted_indices`` promises
    ascending ``rhs_indices`` and selects the grouped GEMM for 64 rows or more.
    """
    if mode != "affine":
        raise QmoeUnsupported(_lib.ERR_UNSUPPORTED, f"mode={mode!r}: only affine quantization")
    if not transpose:
        raise QmoeUnsupported(_lib.ERR_UNSUPPORTED, "transpose=False")
    if biases is None:
        raise QmoeUnsupported(_lib.ERR_UNSUPPORTED, "affine weights need biases")
    if w.dim() != 3:
        raise QmoeUnsupported(_lib.ERR_UNSUPPORTED, f"w must be [E, N, K*bits/32], got {tuple(w.shape)}")
    x = _bf16(x, "x")
    dev = x.device
    if x.dim() < 2:
        raise ValueError("x must be at least 2-D ([..., M, K])")
    M, K = x.shape[-2], x.shape[-1]
    xb = tuple(x.shape[:-2])
    E = w.shape[0]
    rhs = torch.arange(E, device=dev, dtype=torch.int32) if rhs_indices is None else rhs_indices.to(dev)
    if lhs_indices is None:
        batch = torch.broadcast_shapes(xb, tuple(rhs.shape))
        nxb = math.prod(xb)
        xidx = torch.arange(nxb, device=dev, dtype=torch.int32).reshape(xb).expand(batch).reshape(-1)
        identity_x = xb == tuple(batch)
    else:
        lhs = lhs_indices.to(dev)
        batch = torch.broadcast_shapes(tuple(lhs.shape), tuple(rhs.shape))
        xidx = lhs.to(torch.int32).expand(batch).reshape(-1)
        identity_x = False
    e = rhs.to(torch.int32).expand(batch).reshape(-1)
    if M == 1:
        x_rows, experts = xidx, e
    else:
        ar = torch.arange(M, device=dev, dtype=torch.int32)
        x_rows = (xidx[:, None] * M + ar[None, :]).reshape(-1)
        experts = e.repeat_interleave(M)
    n_rows = experts.numel()
    N = w.shape[1]
    if n_rows == 0:
        return torch.empty(*batch, M, N, dtype=torch.bfloat16, device=dev)
    xr = None if identity_x else x_rows
    if sorted_indices and n_rows >= SORTED_MIN_ROWS and gemm_supported(K, N, group_size, bits):
        if tiles is None or tiles.rows != n_rows:
            tiles = build_tiles(experts, E)
        out = gather_qmm_sorted(x, w, scales, biases, tiles, xr, group_size, bits)
    else:
        out = gather_qmv(x, xr, experts, w, scales, biases, group_size, bits)
    return out.reshape(*batch, M, N)


def quantized_matmul(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
                     transpose: bool = True, group_size: int = GROUP, bits: int = BITS,
                     mode: str = "affine") -> torch.Tensor:
    """mx.quantized_matmul for transpose=True affine weights: x[..., K] @ deq(W)^T."""
    if mode != "affine":
        raise QmoeUnsupported(_lib.ERR_UNSUPPORTED, f"mode={mode!r}")
    if not transpose:
        raise QmoeUnsupported(_lib.ERR_UNSUPPORTED, "transpose=False")
    x = _bf16(x, "x")
    w, scales, biases = _words(w, "w"), _bf16(scales, "scales"), _bf16(biases, "biases")
    if w.dim() != 2:
        raise QmoeUnsupported(_lib.ERR_UNSUPPORTED, f"w must be [N, K*bits/32], got {tuple(w.shape)}")
    K = x.shape[-1]
    _check_quant(w, scales, group_size, bits, K)
    N = w.shape[0]
    M = x.numel() // K
    out = torch.empty(*x.shape[:-1], N, dtype=torch.bfloat16, device=x.device)
    _lib.call("qmoe_quantized_matmul", x.data_ptr(), M, K, w.data_ptr(), scales.data_ptr(),
              biases.data_ptr(), N, group_size, bits, out.data_ptr(), _stream(x))
    return out


# ------------------------------------------------------------ fused decode


def gate_up_silu(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
                 idx: torch.Tensor, group_size: int = GROUP, bits: int = BITS) -> torch.Tensor:
    """x [T, K], fused gate_up W [E, 2I, K*bits/32] (gate rows first), idx [T, k]
    -> h [T, k, I] = silu(gate) * up, fp32 until the bf16 store."""
    x = _bf16(x, "x")
    w, scales, biases = _words(w, "w"), _bf16(scales, "scales"), _bf16(biases, "biases")
    T, K = x.shape
    _check_quant(w, scales, group_size, bits, K)
    idx = _i32(idx, "idx", x.device)
    k = idx.shape[-1]
    E, two_i = w.shape[0], w.shape[1]
    I = two_i // 2
    h = torch.empty(T, k, I, dtype=torch.bfloat16, device=x.device)
    _lib.call("qmoe_moe_gate_up_swiglu", x.data_ptr(), idx.data_ptr(), T, k, K, w.data_ptr(),
              scales.data_ptr(), biases.data_ptr(), E, I, group_size, bits, h.data_ptr(), _stream(x))
    return h


def down_wsum(h: torch.Tensor, w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
              idx: torch.Tensor, scores: torch.Tensor, group_size: int = GROUP,
              bits: int = BITS) -> torch.Tensor:
    """h [T, k, I], down W [E, D, I*bits/32], idx [T, k], scores [T, k]
    -> y [T, D] = sum_j scores[t, j] * W[idx[t, j]] @ h[t, j]."""
    h = _bf16(h, "h")
    w, scales, biases = _words(w, "w"), _bf16(scales, "scales"), _bf16(biases, "biases")
    T, k, I = h.shape
    _check_quant(w, scales, group_size, bits, I)
    idx = _i32(idx, "idx", h.device)
    sc = _f32(scores, "scores", h.device)
    E, D = w.shape[0], w.shape[1]
    y = torch.empty(T, D, dtype=torch.bfloat16, device=h.device)
    _lib.call("qmoe_moe_down_wsum", h.data_ptr(), idx.data_ptr(), sc.data_ptr(), T, k, I, w.data_ptr(),
              scales.data_ptr(), biases.data_ptr(), E, D, group_size, bits, y.data_ptr(), _stream(h))
    return y


# ------------------------------------------------------------ weighted sum


def moe_weighted_sum(xs: torch.Tensor, inv_order: torch.Tensor | None, scores: torch.Tensor,
                     out_shape, mode: str = "clone") -> torch.Tensor:
    """Un-permute + router-weighted top-k sum (moe_weighted_sum.py:142-195).

    ``xs`` flattens to [R*k, D]; ``inv_order`` is the [R*k] permutation from
    the sort or None for token-major input; ``scores`` is [..., k]."""
    if mode not in _lib.WSUM_MODES:
        raise QmoeUnsupported(_lib.ERR_UNSUPPORTED, f"mode={mode!r}")
    xs = _bf16(xs, "xs")
    dim = int(out_shape[-1])
    rows = math.prod(int(d) for d in out_shape[:-1])
    k = scores.shape[-1]
    xs2 = xs.reshape(rows * k, dim)
    sc = _f32(scores.reshape(rows * k), "scores", xs.device)
    inv = None if inv_order is None else _i32(inv_order.reshape(-1), "inv_order", xs.device)
    out = torch.empty(*out_shape, dtype=torch.bfloat16, device=xs.device)
    _lib.call("qmoe_weighted_sum", xs2.data_ptr(), _ptr(inv), sc.data_ptr(), rows, k, dim,
              _lib.WSUM_MODES[mode], out.data_ptr(), _stream(xs))
    return out


# -------------------------------------------------------------------- int8


def quantize_act_int8(x: torch.Tensor):
    """Per-token symmetric int8: (xi int8 [R, K], sx float32 [R])."""
    x = _bf16(x, "x")
    K = x.shape[-1]
    x2 = x.reshape(-1, K)
    R = x2.shape[0]
    xi = torch.empty(R, K, dtype=torch.int8, device=x.device)
    sx = torch.empty(R, dtype=torch.float32, device=x.device)
    _lib.call("qmoe_quantize_act_int8", x2.data_ptr(), R, K, xi.data_ptr(), sx.data_ptr(), _stream(x))
    return xi, sx


def gather_qmm_int8_sorted(xi: torch.Tensor, sx: torch.Tensor, w: torch.Tensor, scales: torch.Tensor,
                           biases: torch.Tensor, tiles: TileTable, x_rows: torch.Tensor | None = None,
                           group_size: int = GROUP, bits: int = BITS) -> torch.Tensor:
    """int8-activation x int4-weight grouped GEMM over expert-sorted rows."""
    _dev(xi, "xi")
    if xi.dtype != torch.int8:
        raise QmoeUnsupported(_lib.ERR_UNSUPPORTED, f"xi must be int8, got {xi.dtype}")
    xi = _ready(xi)
    sx = _f32(sx, "sx", xi.device)
    K = xi.shape[-1]
    w, scales, biases = _words(w, "w"), _bf16(scales, "scales"), _bf16(biases, "biases")
    _check_quant(w, scales, group_size, bits, K)
    xr = None if x_rows is None else _i32(x_rows.reshape(-1), "x_rows", xi.device)
    E, N = w.shape[0], w.shape[1]
    if tiles.num_experts != E or tiles.tile_rows != tile_rows():
        raise ValueError("tile table does not match this call")
    out = torch.empty(tiles.rows, N, dtype=torch.bfloat16, device=xi.device)
    _lib.call("qmoe_gather_qmm_int8_sorted", xi.data_ptr(), sx.data_ptr(), _ptr(xr), tiles.rows, K,
              w.data_ptr(), scales.data_ptr(), biases.data_ptr(), E, N, group_size, bits,
              tiles.offsets.data_ptr(), tiles.tile_row.data_ptr(), tiles.tile_exp.data_ptr(),
              tiles.ntiles.data_ptr(), tiles.maxt, out.data_ptr(), _stream(xi))
    return out


def gather_qmm_int8_sorted_tiles(xi: torch.Tensor, sx: torch.Tensor, tw: TileWeights, tiles: TileTable,
                                 x_rows: torch.Tensor | None = None) -> torch.Tensor:
    """:func:`gather_qmm_int8_sorted` over tile-layout weights; same result."""
    _dev(xi, "xi")
    if xi.dtype != torch.int8:
        raise QmoeUnsupported(_lib.ERR_UNSUPPORTED, f"xi must be int8, got {xi.dtype}")
    xi = _ready(xi)
    sx = _f32(sx, "sx", xi.device)
    K = xi.shape[-1]
    if K != tw.K:
        raise ValueError(f"x has K={K}, the weights K={tw.K}")
    xr = None if x_rows is None else _i32(x_rows.reshape(-1), "x_rows", xi.device)
    if tiles.num_experts != tw.num_experts or tiles.tile_rows != tile_rows():
        raise ValueError("tile table does not match this call")
    out = torch.empty(tiles.rows, tw.N, dtype=torch.bfloat16, device=xi.device)
    _lib.call("qmoe_gather_qmm_int8_sorted_tiles", xi.data_ptr(), sx.data_ptr(), _ptr(xr), tiles.rows, K,
              tw.wp.data_ptr(), tw.sb.data_ptr(), tw.num_experts, tw.N, tiles.offsets.data_ptr(),
              tiles.tile_row.data_ptr(), tiles.tile_exp.data_ptr(), tiles.ntiles.data_ptr(), tiles.maxt,
              out.data_ptr(), _stream(xi))
    return out


def gather_qmm_swiglu_sorted_tiles(x: torch.Tensor, tw: TileWeights, tiles: TileTable,
                                   x_rows: torch.Tensor | None = None) -> torch.Tensor:
    """gate_up grouped GEMM with SwiGLU fused: h [rows, N/2] = silu(gate) * up
    over gate/up-paired tile weights (``repack_tiles(..., swiglu_pairs=True)``)."""
    if not tw.swiglu_pairs:
        raise ValueError("the SwiGLU GEMM needs weights repacked with swiglu_pairs=True")
    x = _bf16(x, "x")
    K = x.shape[-1]
    if K != tw.K:
        raise ValueError(f"x has K={K}, the weights K={tw.K}")
    if tiles.num_experts != tw.num_experts or tiles.tile_rows != tile_rows():
        raise ValueError("tile table does not match this call")
    x2 = x.reshape(-1, K)
    xr = None if x_rows is None else _i32(x_rows.reshape(-1), "x_rows", x.device)
    h = torch.empty(tiles.rows, tw.N // 2, dtype=torch.bfloat16, device=x.device)
    _lib.call("qmoe_gather_qmm_swiglu_sorted_tiles", x2.data_ptr(), _ptr(xr), tiles.rows, K, tw.wp.data_ptr(),
              tw.sb.data_ptr(), tw.num_experts, tw.N, tiles.offsets.data_ptr(), tiles.tile_row.data_ptr(),
              tiles.tile_exp.data_ptr(), tiles.ntiles.data_ptr(), tiles.maxt, h.data_ptr(), _stream(x))
    return h


def router_topk(logits: torch.Tensor, k: int, norm: bool = True):
    """Top-k experts per token from router logits, (idx int32 [T, k], scores
    float32 [T, k]); descending, ties to the lower expert index.  norm: the
    softmax renormalised over the chosen experts, else the full softmax
    (qwen3_5_moe/language.py:65-71, decode-fusion/fused_kernels.py:363-371)."""
    _dev(logits, "logits")
    lg = _ready(logits.float())
    E = lg.shape[-1]
    lg2 = lg.reshape(-1, E)
    T = lg2.shape[0]
    idx = torch.empty(T, k, dtype=torch.int32, device=lg.device)
    scores = torch.empty(T, k, dtype=torch.float32, device=lg.device)
    _lib.call("qmoe_router_topk", lg2.data_ptr(), T, E, k, int(bool(norm)), idx.data_ptr(), scores.data_ptr(),
              _stream(lg))
    return idx.reshape(*lg.shape[:-1], k), scores.reshape(*lg.shape[:-1], k)


def router_logits(x: torch.Tensor, router, group_size: int = GROUP, bits: int = BITS) -> torch.Tensor:
    """fp32 router logits [T, E] for tokens x [T, K]: ``router`` a dense bf16
    [E, K] weight, or an affine-quantized (w, scales, biases) triple, whose
    logits come straight from the codes (decode-fusion/fused_kernels.py:232-260)."""
    x = _bf16(x, "x")
    K = x.shape[-1]
    x2 = x.reshape(-1, K)
    T = x2.shape[0]
    if isinstance(router, torch.Tensor):
        w = _bf16(router, "router")
        E = w.shape[0]
        out = torch.empty(T, E, dtype=torch.float32, device=x.device)
        _lib.call("qmoe_router_logits_dense", x2.data_ptr(), T, K, w.data_ptr(), E, out.data_ptr(), _stream(x))
        return out
    w, scales, biases = _words(router[0], "w"), _bf16(router[1], "scales"), _bf16(router[2], "biases")
    if w.dim() != 2:
        raise QmoeUnsupported(_lib.ERR_UNSUPPORTED, f"router w must be [E, K*bits/32], got {tuple(w.shape)}")
    _check_quant(w, scales, group_size, bits, K)
    E = w.shape[0]
    out = torch.empty(T, E, dtype=torch.float32, device=x.device)
    _lib.call("qmoe_router_logits", x2.data_ptr(), T, K, w.data_ptr(), scales.data_ptr(), biases.data_ptr(), E,
              group_size, bits, out.data_ptr(), _stream(x))
    return out


__all__ = [
    "GROUP", "BITS", "QmoeError", "QmoeUnsupported", "TileTable", "TileWeights", "Routing", "build_tiles", "route",
    "repack_tiles", "gather_qmm_sorted_tiles", "gather_qmm_int8_sorted_tiles", "router_topk", "router_logits", "gather_qmm_swiglu_sorted_tiles", "swiglu_pair_order", "gather_qmv_tiles", "gate_up_silu_tiles",
    "down_wsum_tiles", "gate_up_silu_tiles_topk",
    "max_tiles", "tile_rows", "unpack", "dequantize", "gather_qmv", "gather_qmm_sorted", "gather_qmm",
    "gemm_supported", "quantized_matmul", "gate_up_silu", "down_wsum", "moe_weighted_sum",
    "quantize_act_int8", "gather_qmm_int8_sorted",
]
