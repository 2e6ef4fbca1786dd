"""The overlay ``install()`` contract (mirrors the reference's
engine/patches/round3/gather-ws/test_patch.py:37-77): idempotent install,
env gate, fall-through, precedence against the int8 overlay, uninstall
identity.  Host logic only: the kernels are replaced by recording fakes, so
this runs on CPU."""

import types

import pytest
import torch

from titan_amd import core, patches, stock
from titan_amd.patches import gather_qmv, gather_ws, moe_int8
from titan_amd.switch_layers import SwitchGLU


@pytest.fixture
def ns():
    calls = []

    def base(x, w, *a, **kw):
        calls.append("stock")
        return "stock"

    n = types.SimpleNamespace(gather_qmm=base, quantized_matmul=base, calls=calls)
    yield n
    patches.uninstall()


@pytest.fixture
def fake_kernels(monkeypatch):
    """Shapes are always supported and the routes return a tag."""
    monkeypatch.setattr(gather_ws, "supported", lambda *a: True)
    monkeypatch.setattr(moe_int8, "supported", lambda *a: True)
    monkeypatch.setattr(gather_ws._OV, "targets", {"gather_qmm": (gather_ws._should_route, lambda *a: "ws")})
    monkeypatch.setattr(moe_int8._OV, "targets", {"gather_qmm": (moe_int8._should_route, lambda *a: "int8")})


def _call(ns_, rows=4096):
    x = torch.zeros(rows, 1, 8)
    return ns_.gather_qmm(x, None, None, None, rhs_indices=torch.zeros(rows), transpose=True, group_size=64,
                          bits=4, sorted_indices=True)


def test_install_is_idempotent_and_uninstall_restores(ns):
    base = ns.gather_qmm
    assert gather_ws.install(ns) is True
    assert gather_ws.install(ns) is False
    assert ns.gather_qmm is not base and getattr(ns.gather_qmm, gather_ws.MARKER)
    gather_ws.uninstall()
    assert ns.gather_qmm is base


def test_default_namespace_is_core_and_is_restored():
    before = SwitchGLU.__call__
    assert patches.install() is True
    assert patches.install() is False
    assert core.gather_qmm is not stock.gather_qmm
    patches.uninstall()
    assert core.gather_qmm is stock.gather_qmm and core.quantized_matmul is stock.quantized_matmul
    assert SwitchGLU.__call__ is before


def test_gate_off_does_not_route(ns, fake_kernels, monkeypatch):
    monkeypatch.setenv("TITAN_AMD_MOE_GATHER_WS", "0")
    gather_ws.install(ns)
    r0 = gather_ws.stats()["routed"]
    assert _call(ns) == "stock"
    assert gather_ws.stats()["routed"] == r0


def test_gate_on_routes(ns, fake_kernels, monkeypatch):
    monkeypatch.setenv("TITAN_AMD_MOE_GATHER_WS", "1")
    gather_ws.install(ns)
    r0 = gather_ws.stats()["routed"]
    assert _call(ns) == "ws"
    assert gather_ws.stats()["routed"] == r0 + 1


def test_unsorted_and_lhs_calls_fall_through(ns, fake_kernels, monkeypatch):
    monkeypatch.setenv("TITAN_AMD_MOE_GATHER_WS", "1")
    gather_ws.install(ns)
    x = torch.zeros(4096, 1, 8)
    assert ns.gather_qmm(x, None, None, None, rhs_indices=torch.zeros(4096)) == "stock"
    assert ns.gather_qmm(x, None, None, None, lhs_indices=torch.zeros(4096), rhs_indices=torch.zeros(4096),
                         sorted_indices=True) == "stock"


def test_row_floor_applies_without_a_token_count(ns, fake_kernels, monkeypatch):
    monkeypatch.setenv("TITAN_AMD_MOE_GATHER_WS", "1")
    monkeypatch.setenv("TITAN_AMD_MOE_GATHER_WS_MIN_ROWS", "100")
    gather_ws.install(ns)
    assert _call(ns, rows=99) == "stock"
    assert _call(ns, rows=100) == "ws"


def test_a_raising_kernel_falls_through_and_counts(ns, monkeypatch):
    monkeypatch.setenv("TITAN_AMD_MOE_GATHER_WS", "1")
    monkeypatch.setattr(gather_ws, "supported", lambda *a: True)

    def boom(*a):
        raise RuntimeError("kernel failed")

    monkeypatch.setattr(gather_ws._OV, "targets", {"gather_qmm": (gather_ws._should_route, boom)})
    gather_ws.install(ns)
    f0 = gather_ws.stats()["fallback"]
    assert _call(ns) == "stock"
    assert gather_ws.stats()["fallback"] == f0 + 1


def test_a_missing_library_is_not_handed_down(ns, monkeypatch):
    from titan_amd import _lib

    monkeypatch.setenv("TITAN_AMD_MOE_GATHER_WS", "1")
    monkeypatch.setattr(gather_ws, "supported", lambda *a: True)

    def missing(*a):
        raise _lib.QmoeLibraryMissing(-1, "not built")

    monkeypatch.setattr(gather_ws._OV, "targets", {"gather_qmm": (gather_ws._should_route, missing)})
    gather_ws.install(ns)
    with pytest.raises(_lib.QmoeLibraryMissing):
        _call(ns)


def test_int8_below_and_enabled_takes_precedence(ns, fake_kernels, monkeypatch):
    monkeypatch.setenv("TITAN_AMD_MOE_GATHER_WS", "1")
    monkeypatch.setenv("TITAN_AMD_MOE_INT8_PREFILL", "1")
    assert moe_int8.install(ns) is True
    assert gather_ws.install(ns) is True
    t0 = gather_ws.stats()["to_int8"]
    assert _call(ns) == "int8"
    assert gather_ws.stats()["to_int8"] == t0 + 1
    monkeypatch.setenv("TITAN_AMD_MOE_INT8_PREFILL", "0")
    assert _call(ns) == "ws"


def test_int8_on_top_takes_what_it_wants_first(ns, fake_kernels, monkeypatch):
    monkeypatch.setenv("TITAN_AMD_MOE_GATHER_WS", "1")
    monkeypatch.setenv("TITAN_AMD_MOE_INT8_PREFILL", "1")
    gather_ws.install(ns)
    moe_int8.install(ns)
    assert _call(ns) == "int8"
    monkeypatch.setenv("TITAN_AMD_MOE_INT8_PREFILL", "0")
    assert _call(ns) == "ws"


def test_token_floor_comes_from_the_switchglu_call(ns, fake_kernels, monkeypatch):
    """The SwitchGLU hook records T = indices.numel() / k for the call in
    progress; the floor is then in tokens, not rows."""
    monkeypatch.setenv("TITAN_AMD_MOE_GATHER_WS", "1")
    monkeypatch.setenv("TITAN_AMD_MOE_GATHER_WS_MIN_TOKENS", "50")
    gather_ws.install(ns)
    seen = []

    class Probe(SwitchGLU):
        def __init__(self):
            pass

    def inner(glu, x, indices):
        seen.append(_call(ns, rows=indices.numel()))
        return None

    monkeypatch.setattr(gather_ws._OV, "_switchglu_original", inner)
    wrapped = gather_ws._OV._switchglu_call()
    wrapped(Probe(), torch.zeros(1), torch.zeros(40, 10))  # 40 tokens, 400 rows: below the floor
    wrapped(Probe(), torch.zeros(1), torch.zeros(60, 10))
    assert seen == ["stock", "ws"]


def test_decode_overlay_declines_cpu_tensors(ns, monkeypatch):
    monkeypatch.setenv("TITAN_AMD_MOE_DECODE", "1")
    gather_qmv.install(ns)
    x = torch.zeros(1, 1, 1, 1, 8, dtype=torch.bfloat16)
    assert ns.gather_qmm(x, None, None, torch.zeros(1), rhs_indices=torch.zeros(1, 1, 2)) == "stock"
    assert ns.quantized_matmul(x, None, None, torch.zeros(1)) == "stock"
    assert gather_qmv.stats()["routed"] == 0


def test_stats_and_companions_exist():
    for m in (gather_ws, moe_int8, gather_qmv):
        assert set(m.stats()) >= {"routed", "fallback"}
        assert m.warmup() == 0
        m.clear_cache()
    assert set(patches.stats()) == {"gather_qmv", "gather_ws", "moe_int8"}


def test_switch_linears_finds_nested_layers():
    """warmup's walk: layers inside containers, attributes and named_modules."""
    from titan_amd.patches._overlay import switch_linears
    from titan_amd.switch_layers import QuantizedSwitchLinear, SwitchGLU

    z = torch.zeros(2, 64, 32, dtype=torch.int32)
    sc = torch.zeros(2, 64, 4, dtype=torch.bfloat16)
    a, b, c = (QuantizedSwitchLinear(z, sc, sc) for _ in range(3))
    glu = SwitchGLU(a, gate_up_proj=b)

    class Mod:
        def __init__(self, kids):
            self.kids = kids

        def named_modules(self):
            yield "", self
            for i, kd in enumerate(self.kids):
                yield str(i), kd

    import types

    # a Python module and a class as attributes are not entered (the walk
    # would otherwise cover the module's whole namespace)
    holder = types.SimpleNamespace(mod=torch, cls=QuantizedSwitchLinear, layer=c)
    model = {"blocks": [glu, Mod([c, glu])], "other": "x", "holder": holder}
    found = switch_linears(model)
    assert sorted(map(id, found)) == sorted(map(id, (a, b, c)))
    # CPU tensors: nothing to prepare, the walk still completes
    assert moe_int8.warmup(model) == 0 and gather_ws.warmup(model) == 0
