"""Per-weight-tensor prepared state for the grouped GEMMs: the tile-layout
repack of an MLX-affine expert tensor, built once and reused by every later
call on that tensor (the reference's ``_prepared`` cache,
engine/patches/moe-int8/kernel.py:452-463, filled ahead of time by the
patches' ``warmup(model)``, engine/patches/moe-int8/patch.py:179-198).

Entries are keyed by the identity of the (weight, scales, biases) tensors and
hold weak references to them: an entry whose tensors have been freed, or
modified in place since the repack (torch's version counter), is rebuilt, so
a reused address never serves stale weights.  The repacked copy is as large
as the MLX tensors (the layout is a permutation); callers of the drop-in
surface keep their MLX tensors for the stock path, so preparing a tensor adds
its size once.  ``TITAN_AMD_TILE_CACHE=0`` turns preparation off (the
MLX-layout kernels run instead).
"""

from __future__ import annotations

import os
import threading
import weakref

import torch

from .. import ops

__all__ = ["tile_weights", "lookup", "enabled", "clear_cache", "stats", "nbytes"]

_lock = threading.RLock()  # re-entrant: a weakref callback may run while it is held
_PREP: dict = {}
_STATS = {"built": 0, "hits": 0, "misses": 0}


def enabled() -> bool:
    return os.environ.get("TITAN_AMD_TILE_CACHE", "1") == "1"


def _key(w, scales, biases, swiglu_pairs):
    return (id(w), id(scales), id(biases), tuple(w.shape), bool(swiglu_pairs))


def lookup(w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, *,
           swiglu_pairs: bool = False):
    """The prepared tile-layout copy of (w, scales, biases), or None when none
    was built for these tensors as they are now (nothing is built here)."""
    key = _key(w, scales, biases, swiglu_pairs)
    versions = (w._version, scales._version, biases._version)
    with _lock:
        hit = _PREP.get(key)
        if hit is not None:
            refs, ver, tw = hit
            if all(r() is t for r, t in zip(refs, (w, scales, biases))) and ver == versions:
                _STATS["hits"] += 1
                return tw
        _STATS["misses"] += 1
    return None


def tile_weights(w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, *,
                 swiglu_pairs: bool = False) -> ops.TileWeights:
    """The tile-layout repack of (w, scales, biases): the cached copy, or a new
    one built and kept."""
    tw = lookup(w, scales, biases, swiglu_pairs=swiglu_pairs)
    if tw is not None:
        return tw
    key = _key(w, scales, biases, swiglu_pairs)
    versions = (w._version, scales._version, biases._version)
    tw = ops.repack_tiles(w, scales, biases, swiglu_pairs=swiglu_pairs)

    def _drop(_ref, key=key):
        with _lock:
            _PREP.pop(key, None)

    refs = tuple(weakref.ref(t, _drop) for t in (w, scales, biases))
    with _lock:
        _PREP[key] = (refs, versions, tw)
        _STATS["built"] += 1
    return tw


def clear_cache() -> None:
    with _lock:
        _PREP.clear()


def stats() -> dict:
    with _lock:
        return {**_STATS, "entries": len(_PREP)}


def nbytes() -> int:
    """Device bytes held by the prepared copies."""
    with _lock:
        return sum(tw.nbytes for _, _, tw in _PREP.values())
