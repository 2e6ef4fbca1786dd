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


def test_lookup_never_builds(builds):
    w, s, b = _trio()
    assert prepared.lookup(w, s, b) is None and len(builds) == 0
    a = prepared.tile_weights(w, s, b)
    assert prepared.lookup(w, s, b) is a and len(builds) == 1
    s.add_(1)
    assert prepared.lookup(w, s, b) is None and len(builds) == 1


class _Tiles:
    tile_rows = 128
    num_experts = 2
    rows = 64


def _dispatch_spy(monkeypatch, mod, names):
    seen = []
    for n in names:
        monkeypatch.setattr(mod.ops, n, lambda *a, _n=n, **k: (seen.append(_n), torch.zeros(64, 256))[1])
    monkeypatch.setattr(mod.ops, "tile_rows", lambda: 128)
    return seen


@pytest.mark.parametrize("cache", ["1", "0"])
def test_grouped_gemm_ops_read_only_prepared_copies(builds, monkeypatch, cache):
    """The bf16 and int8 grouped-GEMM ops take the tile-layout kernel only for a
    tensor prepared ahead of time (warmup), and the MLX-layout kernel
    otherwise -- no repack is built inside a call, and none at all with
    TITAN_AMD_TILE_CACHE=0."""
    from titan_amd.kernels import moe_gather_int8, moe_gather_ws

    monkeypatch.setenv("TITAN_AMD_TILE_CACHE", cache)
    w, s, b = _trio(E=2, N=256, K=128)
    x = torch.zeros(64, 1, 128, dtype=torch.bfloat16)
    ids = torch.zeros(64, dtype=torch.int32)
    seen = _dispatch_spy(monkeypatch, moe_gather_ws, ["gather_qmm_sorted", "gather_qmm_sorted_tiles"])
    moe_gather_ws.hip(x, w, s, b, ids, _Tiles())
    assert seen == ["gather_qmm_sorted"] and len(builds) == 0
    seen8 = _dispatch_spy(monkeypatch, moe_gather_int8, ["gather_qmm_int8_sorted", "gather_qmm_int8_sorted_tiles"])
    monkeypatch.setattr(moe_gather_int8, "quantize_activations", lambda x: (x, x))
    moe_gather_int8.hip(x, w, s, b, ids, None, _Tiles())
    assert seen8 == ["gather_qmm_int8_sorted"] and len(builds) == 0
    # prepared ahead of time (what warmup does): both ops read the copy
    tabs = moe_gather_int8.build_tables(w, s, b)
    assert len(builds) == (1 if cache == "1" else 0) and (tabs.tw is None) == (cache == "0")
    moe_gather_ws.hip(x, w, s, b, ids, _Tiles())
    moe_gather_int8.hip(x, w, s, b, ids, None, _Tiles())
    tiled = cache == "1"
    assert seen[-1] == ("gather_qmm_sorted_tiles" if tiled else "gather_qmm_sorted")
    assert seen8[-1] == ("gather_qmm_int8_sorted_tiles" if tiled else "gather_qmm_int8_sorted")
    assert len(builds) == (1 if tiled else 0)
