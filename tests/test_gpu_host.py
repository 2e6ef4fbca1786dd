"""The host-side interface on the GPU: registry dispatch reaches the HIP
kernels, and a SwitchGLU routed through the installed overlays matches the
oracle's per-pair chain at prefill and decode widths."""

import numpy as np
import pytest
import torch

from helpers import assert_close_bf16, bf16_t, bits, i32_t, words_t
from titan_amd import core, patches, stock, synth
from titan_amd.kernels import registry as R
from titan_amd.patches import gather_qmv
from titan_amd.switch_layers import QuantizedSwitchLinear, SwitchGLU

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[case] {msg}", flush=True)


def _quant(rng, E, N, K):
    return synth.quant_weights(rng, (E, N), K)


def test_registry_dispatch_runs_the_grouped_gemm(dev, orc):
    say("registry moe_gather_ws E=8 N=256 K=512 R=300")
    rng = np.random.default_rng(21)
    E, N, K, R_ = 8, 256, 512, 300
    w, s, b = _quant(rng, E, N, K)
    ids = np.sort(rng.integers(0, E, size=R_)).astype(np.int32)
    x = synth.bf16_bits(rng.normal(size=(R_, K)).astype(np.float32))
    reg = R.KernelRegistry(R.KernelConfig(fail_open=False))
    from titan_amd.kernels import moe_gather_ws

    reg.register(moe_gather_ws.OP)
    y = reg.call("moe_gather_ws", bf16_t(x, dev).reshape(R_, 1, K), words_t(w, dev), bf16_t(s, dev),
                 bf16_t(b, dev), i32_t(ids, dev))
    assert reg.counters().get("moe_gather_ws.fast") == 1
    ref64, _ = orc.gather_qmm_rows(x, None, ids, w, s, b, deq="bf16")
    assert_close_bf16(orc, bits(y).reshape(R_, N), ref64, what="registry ws")


def test_registry_dispatch_runs_the_weighted_sum(dev, orc):
    say("registry moe_weighted_sum rows=9 k=10 D=256 clone")
    rng = np.random.default_rng(22)
    rows, k, D = 9, 10, 256
    xs = synth.bf16_bits(rng.normal(size=(rows * k, D)).astype(np.float32))
    sc = rng.random((rows, k)).astype(np.float32)
    inv = rng.permutation(rows * k).astype(np.int32)
    reg = R.build_registry(R.KernelConfig(fail_open=False))
    out = reg.call("moe_weighted_sum", bf16_t(xs, dev), i32_t(inv, dev), torch.from_numpy(sc).to(dev),
                   (rows, D), "clone")
    assert reg.counters().get("moe_weighted_sum.fast") == 1
    want = orc.weighted_sum(xs, inv, sc, rows, k, D, "clone")
    assert np.array_equal(bits(out).reshape(-1), np.asarray(want).reshape(-1))


def _oracle_chain(orc, x16, ids, gu, dn):
    T, k = ids.shape
    rows = np.repeat(np.arange(T, dtype=np.int32), k)
    _, gu16 = orc.gather_qmm_rows(x16, rows, ids.reshape(-1), *gu, deq="bf16")
    g = orc.f32_from_bf16(gu16).astype(np.float32)
    I = g.shape[1] // 2
    h = g[:, :I] / (np.float32(1) + np.exp(-g[:, :I])) * g[:, I:]
    h16 = orc.bf16_from_f32(h.astype(np.float32))
    d64, _ = orc.gather_qmm_rows(h16, None, ids.reshape(-1), *dn, deq="bf16")
    return d64.reshape(T, k, -1)


@pytest.mark.parametrize("T", [1, 16])
def test_patched_switchglu_matches_the_oracle_chain(dev, orc, T):
    say(f"patched SwitchGLU T={T} E=16 K=256 I=256 k=10")
    rng = np.random.default_rng(300 + T)
    E, K, I, k = 16, 256, 256, 10
    gu = _quant(rng, E, 2 * I, K)
    dn = _quant(rng, E, K, I)
    x16 = synth.bf16_bits(rng.normal(size=(T, K)).astype(np.float32))
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    lin = lambda t: QuantizedSwitchLinear(words_t(t[0], dev), bf16_t(t[1], dev), bf16_t(t[2], dev))
    glu = SwitchGLU(lin(dn), gate_up_proj=lin(gu))
    from titan_amd import kernels

    kernels.reset()
    reg = R.build_registry(R.KernelConfig(fail_open=False))
    assert patches.install() is True
    try:
        r0 = gather_qmv.stats()["routed"]
        y = glu(bf16_t(x16, dev), i32_t(ids, dev))
        torch.cuda.synchronize()
        routed = gather_qmv.stats()["routed"] - r0
    finally:
        patches.uninstall()
        kernels.reset()
    assert core.gather_qmm is stock.gather_qmm
    assert y.shape == (T, k, K)
    ref = _oracle_chain(orc, x16, ids, gu, dn)
    got = orc.f32_from_bf16(bits(y)).astype(np.float64)
    err = np.abs(got - ref).max()
    print(f"[parity] SwitchGLU T={T}: max-abs {err:.3g} vs max|ref| {np.abs(ref).max():.3g}; routed {routed}")
    assert err <= 2.0 ** -7 * np.abs(ref).max()
    if T * k >= 64:
        # sorted: both projections through the registry's grouped GEMM
        assert reg.counters().get("moe_gather_ws.fast") == 2 and routed == 0
    else:
        # unsorted: both projections through the decode overlay's gather-GEMV
        assert routed == 2 and "moe_gather_ws.calls" not in reg.counters()


def test_warmup_prepares_tile_layouts_and_the_overlays_run_on_them(dev, orc, monkeypatch):
    """warmup(model) repacks each routed weight tensor into the tile layout once
    (engine/patches/moe-int8/patch.py:179-198); the prefill calls after it read
    those copies -- the bf16 registry path and the int8 overlay share them --
    and match the oracle."""
    from titan_amd import kernels
    from titan_amd.kernels import prepared
    from titan_amd.patches import gather_ws, moe_int8

    say("warmup + tile-layout prefill through the registry and the int8 overlay")
    rng = np.random.default_rng(77)
    E, K, I, k, T = 16, 512, 512, 10, 16
    gu, dn = _quant(rng, E, 2 * I, K), _quant(rng, E, K, I)
    x16 = synth.bf16_bits(rng.normal(size=(T, K)).astype(np.float32))
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    lin = lambda t: QuantizedSwitchLinear(words_t(t[0], dev), bf16_t(t[1], dev), bf16_t(t[2], dev))
    glu = SwitchGLU(lin(dn), gate_up_proj=lin(gu))
    model = {"layers": [{"mlp": glu}]}
    prepared.clear_cache()
    assert gather_ws.warmup(model) == 2
    st0 = prepared.stats()
    assert st0["built"] >= 2 and st0["entries"] == 2
    kernels.reset()
    R.build_registry(R.KernelConfig(fail_open=False))
    try:
        y = glu(bf16_t(x16, dev), i32_t(ids, dev))
        torch.cuda.synchronize()
    finally:
        kernels.reset()
    st1 = prepared.stats()
    assert st1["hits"] - st0["hits"] == 2 and st1["built"] == st0["built"]  # both projections, no rebuild
    ref = _oracle_chain(orc, x16, ids, gu, dn)
    err = np.abs(orc.f32_from_bf16(bits(y)).astype(np.float64) - ref).max()
    assert err <= 2.0 ** -7 * np.abs(ref).max()

    # the int8 overlay: its tables are the same prepared copies
    monkeypatch.setenv("TITAN_AMD_MOE_INT8_PREFILL", "1")
    monkeypatch.setenv("TITAN_AMD_MOE_INT8_MIN_ROWS", "64")
    assert moe_int8.warmup(model) == 2
    assert prepared.stats()["built"] == st1["built"]
    from titan_amd.kernels import moe_gather_int8

    tabs = moe_gather_int8.build_tables(glu.gate_up_proj.weight, glu.gate_up_proj.scales, glu.gate_up_proj.biases)
    assert tabs.nbytes == sum(a.nbytes for a in gu)
    ns = type("NS", (), {"gather_qmm": staticmethod(stock.gather_qmm),
                         "quantized_matmul": staticmethod(stock.quantized_matmul)})
    srt = np.sort(ids.reshape(-1)).astype(np.int32)
    xs = synth.bf16_bits(rng.normal(size=(srt.size, K)).astype(np.float32))
    assert moe_int8.install(ns) is True
    try:
        r0 = moe_int8.stats()["routed"]
        out = ns.gather_qmm(bf16_t(xs, dev).reshape(-1, 1, K), glu.gate_up_proj.weight, glu.gate_up_proj.scales,
                            glu.gate_up_proj.biases, rhs_indices=i32_t(srt, dev), sorted_indices=True)
        torch.cuda.synchronize()
        assert moe_int8.stats()["routed"] - r0 == 1
    finally:
        moe_int8.uninstall()
    rxi, rsx = orc.quant_act_int8(xs)
    ref64, _ = orc.gather_qmm_int8_rows(rxi, rsx, None, srt, *gu)
    assert_close_bf16(orc, bits(out).reshape(srt.size, -1), ref64, what="int8 overlay on prepared tiles")
