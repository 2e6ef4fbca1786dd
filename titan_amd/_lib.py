"""ctypes binding of libqmoe.so (declarations in include/qmoe.h).

The library is the product: every op in this package runs through it, and a
missing library is an error (:class:`QmoeLibraryMissing`), never a silent
switch to something else.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libqmoe.so"

OK = 0
ERR_INVALID = 1
ERR_UNSUPPORTED = 2
ERR_HIP = 3
ERR_WORKSPACE = 4

WSUM_MODES = {"fast": 0, "ops": 1, "clone": 2}


class QmoeError(RuntimeError):
    """A libqmoe entry point returned an error code."""

    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


class QmoeUnsupported(QmoeError):
    """No kernel for this shape / dtype / bit width / group size."""


class QmoeLibraryMissing(RuntimeError):
    """libqmoe.so is not built (run ``python -m titan_amd.build``)."""


P = ctypes.c_void_p
I32 = ctypes.c_int32
I64 = ctypes.c_int64
INT = ctypes.c_int
SZ = ctypes.c_size_t

# name -> (restype, argtypes); one entry per declaration in include/qmoe.h
SIGNATURES: dict[str, tuple] = {
    "qmoe_abi_version": (INT, []),
    "qmoe_last_error": (ctypes.c_char_p, []),
    "qmoe_unpack": (INT, [P, I64, INT, P, P]),
    "qmoe_dequantize": (INT, [P, P, P, I64, I64, INT, INT, P, P]),
    "qmoe_route_workspace_size": (SZ, [I64, I32]),
    "qmoe_route": (INT, [P, I64, I32, I32, P, P, P, P, P, P, P, I64, P, SZ, P]),
    "qmoe_route_noalloc": (INT, [P, I64, I32, I32, P, P, P, P, P, P, P, I64, P, P]),
    "qmoe_build_tiles": (INT, [P, I64, I32, I32, P, P, P, P, I64, P]),
    "qmoe_gather_qmv": (INT, [P, P, P, I64, I64, P, P, P, I32, I64, INT, INT, P, P]),
    "qmoe_quantized_matmul": (INT, [P, I64, I64, P, P, P, I64, INT, INT, P, P]),
    "qmoe_gemm_tile_rows": (INT, []),
    "qmoe_gather_qmm_sorted": (INT, [P, P, I64, I64, P, P, P, I32, I64, INT, INT, P, P, P, P, I64,
                                     P, P]),
    "qmoe_moe_gate_up_swiglu": (INT, [P, P, I64, I64, I64, P, P, P, I32, I64, INT, INT, P, P]),
    "qmoe_moe_down_wsum": (INT, [P, P, P, I64, I64, I64, P, P, P, I32, I64, INT, INT, P, P]),
    "qmoe_weighted_sum": (INT, [P, P, P, I64, I64, I64, INT, P, P]),
    "qmoe_repack_tiles": (INT, [P, P, P, I32, I64, I64, INT, INT, P, P, P]),
    "qmoe_gather_qmm_sorted_tiles": (INT, [P, P, I64, I64, P, P, I32, I64, P, P, P, P, I64, P, P]),
    "qmoe_gather_qmv_tiles": (INT, [P, P, P, I64, I64, P, P, I32, I64, P, P]),
    "qmoe_moe_gate_up_swiglu_tiles": (INT, [P, P, I64, I64, I64, P, P, I32, I64, P, P]),
    "qmoe_moe_down_wsum_tiles": (INT, [P, P, P, I64, I64, I64, P, P, I32, I64, P, P]),
    "qmoe_moe_gate_up_swiglu_tiles_topk": (INT, [P, P, INT, I64, I64, I64, P, P, I32, I64, P, P, P, P]),
    "qmoe_quantize_act_int8": (INT, [P, I64, I64, P, P, P]),
    "qmoe_gather_qmm_int8_sorted": (INT, [P, P, P, I64, I64, P, P, P, I32, I64, INT, INT, P, P, P, P,
                                          I64, P, P]),
    "qmoe_gather_qmm_int8_sorted_tiles": (INT, [P, P, P, I64, I64, P, P, I32, I64, P, P, P, P, I64, P, P]),
    "qmoe_router_topk": (INT, [P, I64, I64, I64, INT, P, P, P]),
    "qmoe_router_logits": (INT, [P, I64, I64, P, P, P, I64, INT, INT, P, P]),
    "qmoe_router_logits_dense": (INT, [P, I64, I64, P, I64, P, P]),
    "qmoe_gather_qmm_swiglu_sorted_tiles": (INT, [P, P, I64, I64, P, P, I32, I64, P, P, P, P, I64, P, P]),
}

_lock = threading.Lock()
_lib = None


def load() -> ctypes.CDLL:
    """The loaded library, with argument types set.  Raises QmoeLibraryMissing."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise QmoeLibraryMissing(
                f"{LIB_PATH} is not built; run `python -m titan_amd.build` (hipcc, gfx950)")
        L = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def available() -> bool:
    try:
        load()
        return True
    except QmoeLibraryMissing:
        return False


def last_error() -> str:
    msg = load().qmoe_last_error()
    return msg.decode() if msg else ""


def check(rc: int, what: str) -> None:
    if rc == OK:
        return
    msg = f"{what}: {last_error()} (code {rc})"
    if rc == ERR_UNSUPPORTED:
        raise QmoeUnsupported(rc, msg)
    raise QmoeError(rc, msg)


def call(name: str, *args) -> None:
    """Call entry point ``name`` and raise on a non-zero status."""
    check(getattr(load(), name)(*args), name)
