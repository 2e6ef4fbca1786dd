"""The per-tensor prepared-weights cache (titan_amd/kernels/prepared.py), the
role of the reference's ``_prepared`` tables (engine/patches/moe-int8/
kernel.py:452-463): built once per (weight, scales, biases), rebuilt when a
tensor is modified in place, dropped when one is freed.  The repack itself is
a GPU kernel; here a stand-in counts the builds so the cache logic runs on the
CPU."""

import gc

import pytest
import torch

from titan_amd.kernels import prepared


class _Fake:
    def __init__(self, n, swiglu_pairs):
        self.nbytes = n
        self.swiglu_pairs = swiglu_pairs


@pytest.fixture
def builds(monkeypatch):
    calls = []

    def fake_repack(w, s, b, *, swiglu_pairs=False):
        calls.append((id(w), swiglu_pairs))
        return _Fake(w.numel() * w.element_size() + 2 * s.numel() * s.element_size(), swiglu_pairs)

    monkeypatch.setattr(prepared.ops, "repack_tiles", fake_repack)
    prepared.clear_cache()
    yield calls
    prepared.clear_cache()


def _trio(E=2, N=64, K=128):
    return (torch.zeros(E, N, K // 8, dtype=torch.int32), torch.zeros(E, N, K // 64, dtype=torch.bfloat16),
            torch.zeros(E, N, K // 64, dtype=torch.bfloat16))


def test_built_once_then_served(builds):
    w, s, b = _trio()
    a = prepared.tile_weights(w, s, b)
    assert prepared.tile_weights(w, s, b) is a
    st = prepared.stats()
    assert (st["built"], st["entries"]) == (1, 1) and st["hits"] >= 1 and len(builds) == 1
    assert prepared.nbytes() == a.nbytes


def test_pair_order_is_its_own_entry(builds):
    w, s, b = _trio()
    plain = prepared.tile_weights(w, s, b)
    paired = prepared.tile_weights(w, s, b, swiglu_pairs=True)
    assert plain is not paired and paired.swiglu_pairs and not plain.swiglu_pairs
    assert prepared.stats()["entries"] == 2


def test_in_place_modification_rebuilds(builds):
    w, s, b = _trio()
    first = prepared.tile_weights(w, s, b)
    s.add_(1)  # bumps the tensor's version counter
    second = prepared.tile_weights(w, s, b)
    assert second is not first and len(builds) == 2
    assert prepared.tile_weights(w, s, b) is second


def test_freed_tensors_drop_their_entry(builds):
    w, s, b = _trio()
    prepared.tile_weights(w, s, b)
    assert prepared.stats()["entries"] == 1
    del w, s, b
    gc.collect()
    assert prepared.stats()["entries"] == 0 and prepared.nbytes() == 0


def test_a_reused_address_is_not_served_stale(builds):
    """A new tensor that lands on a freed tensor's id gets its own repack."""
    w, s, b = _trio()
    prepared.tile_weights(w, s, b)
    del w, s, b
    gc.collect()
    w2, s2, b2 = _trio()  # may well reuse the freed tensors' ids
    prepared.tile_weights(w2, s2, b2)
    assert len(builds) == 2 and prepared.stats()["entries"] == 1


def test_cache_switch(monkeypatch):
    monkeypatch.setenv("TITAN_AMD_TILE_CACHE", "0")
    assert not prepared.enabled()
    monkeypatch.setenv("TITAN_AMD_TILE_CACHE", "1")
    assert prepared.enabled()
