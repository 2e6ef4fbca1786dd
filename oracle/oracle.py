"""numpy front end to the C oracle.  TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg
import this module; ``titan_amd`` never does.  It is the oracle the HIP path is
compared against, never a thing that is shipped or measured as the product.

Every wrapper forwards to ``oracle/qmoe_oracle.c``; the C file cites the
reference lines each function restates.  bf16 arrays are numpy ``uint16`` bit
patterns throughout.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libqmoe_oracle.so"

_lib = None


def build(force: bool = False) -> Path:
    """Compile the oracle with its Makefile (gcc, OpenMP)."""
    if force or not LIB_PATH.exists():
        subprocess.run(["make", "-C", str(HERE), "-s"], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        P = ctypes.c_void_p
        I64 = ctypes.c_int64
        I32 = ctypes.c_int32
        INT = ctypes.c_int
        L.orc_bf16_rne.restype = ctypes.c_uint16
        L.orc_bf16_rne.argtypes = [ctypes.c_float]
        L.orc_bf16_rne_f64.restype = ctypes.c_uint16
        L.orc_bf16_rne_f64.argtypes = [ctypes.c_double]
        L.orc_unpack.argtypes = [P, I64, INT, P]
        L.orc_pack.argtypes = [P, I64, INT, P]
        L.orc_dequantize_bf16.argtypes = [P, P, P, I64, I64, INT, INT, P]
        L.orc_gather_qmm_rows.argtypes = [P, I64, P, P, I64, P, P, P, I64, INT, INT,
                                          INT, P, P, INT]
        L.orc_route_sort.restype = INT
        L.orc_route_sort.argtypes = [P, I64, I32, P, P, P]
        L.orc_build_tiles.restype = I64
        L.orc_build_tiles.argtypes = [P, I64, I32, I32, P, P, P, I64]
        L.orc_swiglu.argtypes = [P, I64, I64, P, P]
        L.orc_weighted_sum.argtypes = [P, P, P, I64, I64, I64, INT, P]
        L.orc_down_wsum.argtypes = [P, P, P, I64, I64, I64, P, P, P, I64, INT, INT,
                                    P, P, INT]
        L.orc_quant_act_int8.argtypes = [P, I64, I64, P, P]
        L.orc_gather_qmm_int8_rows.argtypes = [P, P, I64, P, P, I64, P, P, P, I64,
                                               INT, INT, P, P, INT]
        L.orc_router_topk.argtypes = [P, I64, I64, I64, INT, P, P]
        L.orc_max_threads.restype = INT
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ------------------------------------------------------------------ bf16


def bf16_from_f32(a) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bit patterns (vectorised restatement
    of ``orc_bf16_rne``; tests check the two agree)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7F800000) == 0x7F800000
    nan &= (u & 0x007FFFFF) != 0
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r = np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)
    return r.astype(np.uint16)


def f32_from_bf16(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    return (h.astype(np.uint32) << 16).view(np.float32)


def bf16_rne_scalar(x: float) -> int:
    return int(lib().orc_bf16_rne(ctypes.c_float(x)))


def bf16_from_f64(a) -> np.ndarray:
    """Single rounding double -> bf16 (``orc_bf16_rne_f64``), elementwise."""
    a = np.ascontiguousarray(a, dtype=np.float64)
    f = lib().orc_bf16_rne_f64
    out = np.empty(a.shape, np.uint16)
    flat, of = a.reshape(-1), out.reshape(-1)
    for i in range(flat.size):
        of[i] = f(float(flat[i]))
    return out


# ----------------------------------------------------------- pack / dequant


def unpack(w, bits: int = 4) -> np.ndarray:
    w = _c(w, np.uint32)
    per = 32 // bits
    out = np.empty(w.shape[:-1] + (w.shape[-1] * per,), np.uint8)
    lib().orc_unpack(_p(w), w.size, bits, _p(out))
    return out


def pack(codes, bits: int = 4) -> np.ndarray:
    codes = _c(codes, np.uint8)
    per = 32 // bits
    out = np.empty(codes.shape[:-1] + (codes.shape[-1] // per,), np.uint32)
    lib().orc_pack(_p(codes), codes.size, bits, _p(out))
    return out


def dequantize_bf16(w, s, b, group_size: int = 64, bits: int = 4) -> np.ndarray:
    """bf16(fmaf(q, s, b)) for every element; leading dims are rows."""
    w, s, b = _c(w, np.uint32), _c(s, np.uint16), _c(b, np.uint16)
    K = w.shape[-1] * 32 // bits
    rows = int(np.prod(w.shape[:-1]))
    out = np.empty(w.shape[:-1] + (K,), np.uint16)
    lib().orc_dequantize_bf16(_p(w), _p(s), _p(b), rows, K, group_size, bits, _p(out))
    return out


# ------------------------------------------------------------- gather_qmm


def gather_qmm_rows(x, x_rows, experts, w, s, b, group_size=64, bits=4,
                    deq="exact", n_threads=0):
    """Row form of gather_qmm.  ``x`` bf16 [X, K]; ``x_rows`` int32 [R] or None;
    ``experts`` int32 [R]; ``w`` u32 [E, N, K*bits/32]; returns (f64 [R, N],
    bf16 [R, N])."""
    x = _c(x, np.uint16)
    K = x.shape[-1]
    x = x.reshape(-1, K)
    experts = _c(experts, np.int32).reshape(-1)
    xr = None if x_rows is None else _c(x_rows, np.int32).reshape(-1)
    w, s, b = _c(w, np.uint32), _c(s, np.uint16), _c(b, np.uint16)
    N = w.shape[-2]
    R = experts.size
    o64 = np.empty((R, N), np.float64)
    o16 = np.empty((R, N), np.uint16)
    mode = {"exact": 0, "bf16": 1}[deq]
    lib().orc_gather_qmm_rows(_p(x), K, _p(xr), _p(experts), R, _p(w), _p(s), _p(b),
                              N, group_size, bits, mode, _p(o64), _p(o16), n_threads)
    return o64, o16


def route_sort(ids, num_experts: int):
    ids = _c(ids, np.int32).reshape(-1)
    n = ids.size
    order = np.empty(n, np.int32)
    inv = np.empty(n, np.int32)
    srt = np.empty(n, np.int32)
    rc = lib().orc_route_sort(_p(ids), n, num_experts, _p(order), _p(inv), _p(srt))
    if rc != 0:
        raise ValueError("expert id out of range")
    return order, inv, srt


def max_tiles(rows: int, num_experts: int, tile_rows: int) -> int:
    return (rows + tile_rows - 1) // tile_rows + num_experts


def build_tiles(sorted_ids, num_experts: int, tile_rows: int):
    sorted_ids = _c(sorted_ids, np.int32).reshape(-1)
    n = sorted_ids.size
    mt = max_tiles(n, num_experts, tile_rows)
    offsets = np.empty(num_experts + 1, np.int32)
    trow = np.empty(mt, np.int32)
    texp = np.empty(mt, np.int32)
    nt = lib().orc_build_tiles(_p(sorted_ids), n, num_experts, tile_rows, _p(offsets),
                               _p(trow), _p(texp), mt)
    return offsets, trow, texp, int(nt)


def swiglu(gu_f64):
    gu = _c(gu_f64, np.float64)
    rows, two_i = gu.reshape(-1, gu.shape[-1]).shape
    I = two_i // 2
    h64 = np.empty((rows, I), np.float64)
    h16 = np.empty((rows, I), np.uint16)
    lib().orc_swiglu(_p(gu), rows, I, _p(h64), _p(h16))
    return h64, h16


MODES = {"fast": 0, "ops": 1, "clone": 2}


def weighted_sum(xs, inv, scores, rows: int, k: int, dim: int, mode="clone"):
    xs = _c(xs, np.uint16)
    inv = None if inv is None else _c(inv, np.int32).reshape(-1)
    scores = _c(scores, np.float32).reshape(-1)
    out = np.empty((rows, dim), np.uint16)
    lib().orc_weighted_sum(_p(xs), _p(inv), _p(scores), rows, k, dim, MODES[mode], _p(out))
    return out


def down_wsum(h, idx, scores, w, s, b, group_size=64, bits=4, n_threads=0):
    h = _c(h, np.uint16)
    T, k, I = h.shape
    idx = _c(idx, np.int32)
    scores = _c(scores, np.float32)
    w, s, b = _c(w, np.uint32), _c(s, np.uint16), _c(b, np.uint16)
    D = w.shape[-2]
    y64 = np.empty((T, D), np.float64)
    y16 = np.empty((T, D), np.uint16)
    lib().orc_down_wsum(_p(h), _p(idx), _p(scores), T, k, I, _p(w), _p(s), _p(b), D,
                        group_size, bits, _p(y64), _p(y16), n_threads)
    return y64, y16


def router_topk(logits, k: int, norm: bool = True):
    """Top-k experts per token by fp32 logit (ties to the lower index),
    descending; scores in float64 (fused_kernels.py:363-371)."""
    lg = _c(logits, np.float32)
    T, E = lg.reshape(-1, lg.shape[-1]).shape
    idx = np.empty((T, k), np.int32)
    sc = np.empty((T, k), np.float64)
    lib().orc_router_topk(_p(lg), T, E, k, int(norm), _p(idx), _p(sc))
    return idx, sc


def quant_act_int8(x):
    x = _c(x, np.uint16)
    K = x.shape[-1]
    x2 = x.reshape(-1, K)
    R = x2.shape[0]
    xi = np.empty((R, K), np.int8)
    sx = np.empty(R, np.float32)
    lib().orc_quant_act_int8(_p(x2), R, K, _p(xi), _p(sx))
    return xi, sx


def gather_qmm_int8_rows(xi, sx, x_rows, experts, w, s, b, group_size=64, bits=4,
                         n_threads=0):
    xi = _c(xi, np.int8)
    K = xi.shape[-1]
    sx = _c(sx, np.float32).reshape(-1)
    experts = _c(experts, np.int32).reshape(-1)
    xr = None if x_rows is None else _c(x_rows, np.int32).reshape(-1)
    w, s, b = _c(w, np.uint32), _c(s, np.uint16), _c(b, np.uint16)
    N = w.shape[-2]
    R = experts.size
    o64 = np.empty((R, N), np.float64)
    o16 = np.empty((R, N), np.uint16)
    lib().orc_gather_qmm_int8_rows(_p(xi), _p(sx), K, _p(xr), _p(experts), R, _p(w),
                                   _p(s), _p(b), N, group_size, bits, _p(o64), _p(o16),
                                   n_threads)
    return o64, o16


def max_threads() -> int:
    return int(lib().orc_max_threads())


# ------------------------------------------------------------ error metrics


def ordered(h) -> np.ndarray:
    """bf16 bit patterns onto a monotone signed integer line
    (tests/kernels/exactness.py:36-46)."""
    b = np.asarray(h, np.uint16).astype(np.int32)
    return np.where(b >= 0x8000, 0x8000 - 1 - b, b)


def ulp_distance(got, ref) -> np.ndarray:
    return np.abs(ordered(got) - ordered(ref))


def live_mask(ref_f64, frac: float = 1.0 / 256.0) -> np.ndarray:
    """Elements whose magnitude is at least max|ref|/256
    (engine/patches/round2/wsum10/test_exact.py:61-62)."""
    r = np.abs(np.asarray(ref_f64, np.float64))
    return r >= r.max() * frac


def err_report(got_bf16, ref_f64) -> dict:
    """max-abs, max-abs relative to max|ref| (decode-fusion/test_exact.py:53-57),
    rrmse (exactness.py:65-68) and ULP distances against the RNE golden."""
    g = f32_from_bf16(got_bf16).astype(np.float64)
    r = np.asarray(ref_f64, np.float64)
    d = np.abs(g - r)
    scale = max(np.abs(r).max(), 1e-30)
    ref16 = bf16_from_f64_fast(r)
    ulp = ulp_distance(got_bf16, ref16)
    live = live_mask(r)
    return {
        "max_abs": float(d.max()) if d.size else 0.0,
        "rel_to_max": float(d.max() / scale) if d.size else 0.0,
        "rrmse": float(np.sqrt((d ** 2).mean() / max((r ** 2).mean(), 1e-300))) if d.size else 0.0,
        "max_ulp_live": int(ulp[live].max()) if live.any() else 0,
        "max_ulp_all": int(ulp.max()) if ulp.size else 0,
        "n": int(d.size),
    }


def bf16_from_f64_fast(a) -> np.ndarray:
    """Vectorised single-rounding double -> bf16 for finite normal-range data;
    falls back to the scalar C routine for anything else."""
    a = np.asarray(a, np.float64)
    fin = np.isfinite(a) & ((np.abs(a) >= 2.0 ** -126) | (a == 0))
    fin &= np.abs(a) < 3.3e38
    if not fin.all():
        return bf16_from_f64(a)
    m, e = np.frexp(np.abs(a))
    q = np.rint(np.ldexp(m, 8))
    r = np.ldexp(q, e - 8) * np.sign(a)
    out = bf16_from_f32(r.astype(np.float32))
    out = np.where(a == 0, np.where(np.signbit(a), 0x8000, 0), out).astype(np.uint16)
    return out
