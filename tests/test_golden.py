"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py
from the oracle): the oracle must still reproduce them bit for bit, and the
HIP path must meet the parity bar on the same inputs."""

from pathlib import Path

import numpy as np
import pytest

from helpers import assert_close_bf16, bf16_t, bits, f32_t, i32_t, words_t

GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name):
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


# ------------------------------------------------------------------ oracle


def test_oracle_reproduces_unpack_dequant(orc):
    g = load("unpack_dequant")
    assert np.array_equal(orc.unpack(g["w"].reshape(-1), 4).reshape(g["codes"].shape), g["codes"])
    assert np.array_equal(orc.dequantize_bf16(g["w"], g["s"], g["b"], 64, 4).reshape(g["deq"].shape), g["deq"])


def test_oracle_reproduces_gather(orc):
    g = load("gather_sorted")
    y64, y16 = orc.gather_qmm_rows(g["x"], None, g["ids"], g["w"], g["s"], g["b"], deq="bf16")
    assert np.array_equal(y64, g["y64"]) and np.array_equal(y16, g["y16"])
    e64, _ = orc.gather_qmm_rows(g["x"], None, g["ids"], g["w"], g["s"], g["b"], deq="exact")
    assert np.array_equal(e64, g["e64"])


def test_oracle_reproduces_decode_gate_up(orc):
    g = load("decode_gate_up")
    k = g["idx"].size
    gu64, _ = orc.gather_qmm_rows(g["x"], np.zeros(k, np.int32), g["idx"].reshape(-1), g["w"], g["s"], g["b"])
    h64, _ = orc.swiglu(gu64)
    assert np.array_equal(h64.reshape(g["h64"].shape), g["h64"])


def test_oracle_reproduces_route(orc):
    g = load("route")
    order, inv, srt = orc.route_sort(g["ids"], 8)
    assert np.array_equal(order, g["order"]) and np.array_equal(inv, g["inv"]) and np.array_equal(srt, g["sorted"])
    offsets, trow, texp, nt = orc.build_tiles(srt, 8, int(g["tile_rows"]))
    assert nt == int(g["ntiles"]) and np.array_equal(offsets, g["offsets"])
    assert np.array_equal(trow, g["tile_row"]) and np.array_equal(texp, g["tile_exp"])
    # the closed forms the fixture must also satisfy
    assert np.array_equal(g["order"], np.argsort(g["ids"], kind="stable"))
    assert np.array_equal(g["offsets"], np.searchsorted(g["sorted"], np.arange(9), "left"))


def test_oracle_reproduces_weighted_sum(orc):
    g = load("weighted_sum")
    rows, D = g["clone"].shape
    k = g["scores"].shape[1]
    for m in ("clone", "ops", "fast"):
        got = np.asarray(orc.weighted_sum(g["xs"], g["inv"], g["scores"], rows, k, D, m)).reshape(rows, D)
        assert np.array_equal(got, g[m]), m


def test_oracle_reproduces_int8(orc):
    g = load("int8")
    xi, sx = orc.quant_act_int8(g["x"])
    assert np.array_equal(xi, g["xi"]) and np.array_equal(sx, g["sx"])
    y64, _ = orc.gather_qmm_int8_rows(xi, sx, None, g["ids"], g["w"], g["s"], g["b"])
    assert np.array_equal(y64, g["y64"])


# --------------------------------------------------------------------- GPU


@pytest.mark.gpu
def test_hip_matches_golden_unpack_dequant(dev):
    from titan_amd import ops

    g = load("unpack_dequant")
    w = words_t(g["w"], dev)
    assert np.array_equal(ops.unpack(w).cpu().numpy().reshape(g["codes"].shape), g["codes"])
    deq = ops.dequantize(w, bf16_t(g["s"], dev), bf16_t(g["b"], dev))
    assert np.array_equal(bits(deq).reshape(g["deq"].shape), g["deq"])


@pytest.mark.gpu
@pytest.mark.parametrize("tiled", [False, True])
def test_hip_matches_golden_gather(dev, orc, tiled):
    from titan_amd import ops

    g = load("gather_sorted")
    E = 4
    tiles = ops.build_tiles(i32_t(g["ids"], dev), E)
    w, s, b = words_t(g["w"], dev), bf16_t(g["s"], dev), bf16_t(g["b"], dev)
    if tiled:
        y = ops.gather_qmm_sorted_tiles(bf16_t(g["x"], dev), ops.repack_tiles(w, s, b), tiles)
    else:
        y = ops.gather_qmm_sorted(bf16_t(g["x"], dev), w, s, b, tiles)
    assert_close_bf16(orc, bits(y), g["y64"], what=f"golden gather tiled={tiled}")
    # the GEMV computes the exact affine form s*sum(x*q) + b*sum(x), as the decode kernels do
    yv = ops.gather_qmv(bf16_t(g["x"], dev), None, i32_t(g["ids"], dev), w, s, b)
    assert_close_bf16(orc, bits(yv), g["e64"], what="golden gather GEMV")


@pytest.mark.gpu
def test_hip_matches_golden_decode_gate_up(dev, orc):
    from titan_amd import ops

    g = load("decode_gate_up")
    h = ops.gate_up_silu(bf16_t(g["x"], dev), words_t(g["w"], dev), bf16_t(g["s"], dev), bf16_t(g["b"], dev),
                         i32_t(g["idx"], dev))
    assert_close_bf16(orc, bits(h).reshape(g["h64"].shape[1], -1), g["h64"].reshape(g["h64"].shape[1], -1),
                      what="golden decode gate_up")


@pytest.mark.gpu
def test_hip_matches_golden_route(dev):
    from titan_amd import ops

    g = load("route")
    r = ops.route(i32_t(g["ids"], dev), 8, int(g["tile_rows"]))
    assert np.array_equal(r.order.cpu().numpy(), g["order"])
    assert np.array_equal(r.inv_order.cpu().numpy(), g["inv"])
    assert np.array_equal(r.sorted_ids.cpu().numpy(), g["sorted"])
    assert np.array_equal(r.tiles.offsets.cpu().numpy(), g["offsets"])
    nt = int(r.tiles.ntiles.item())
    assert nt == int(g["ntiles"])
    assert np.array_equal(r.tiles.tile_row.cpu().numpy()[:nt], g["tile_row"][:nt])
    assert np.array_equal(r.tiles.tile_exp.cpu().numpy()[:nt], g["tile_exp"][:nt])


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["clone", "ops", "fast"])
def test_hip_matches_golden_weighted_sum(dev, mode):
    import torch

    from titan_amd import ops

    g = load("weighted_sum")
    rows, D = g[mode].shape
    out = ops.moe_weighted_sum(bf16_t(g["xs"], dev), i32_t(g["inv"], dev), torch.from_numpy(g["scores"]).to(dev),
                               (rows, D), mode)
    assert np.array_equal(bits(out), g[mode])


@pytest.mark.gpu
def test_hip_matches_golden_int8(dev, orc):
    from titan_amd import ops

    g = load("int8")
    xi, sx = ops.quantize_act_int8(bf16_t(g["x"], dev))
    assert np.array_equal(xi.cpu().numpy(), g["xi"]) and np.array_equal(sx.cpu().numpy(), g["sx"])
    tiles = ops.build_tiles(i32_t(g["ids"], dev), 2)
    y = ops.gather_qmm_int8_sorted(xi, sx, words_t(g["w"], dev), bf16_t(g["s"], dev), bf16_t(g["b"], dev), tiles)
    assert_close_bf16(orc, bits(y), g["y64"], what="golden int8")
