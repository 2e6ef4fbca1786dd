"""HIP path against the CPU oracle on the same seeded inputs.

Bars: unpack, dequant, routing indices and the weighted-sum modes are
bit-exact; matmul outputs are within 1 bf16 ULP of the RNE-rounded fp64 golden
on live elements (|ref| >= max|ref|/256, the rule of
engine/patches/round2/wsum10/test_exact.py:61-62) and within 2^-8 of max|ref|
in max-abs error everywhere (engine/patches/decode-fusion/test_exact.py:53-57).
"""

import numpy as np
import pytest
import torch

from helpers import assert_close_bf16, bf16_t, bits, f32_t, i32_t, words_t
from titan_amd import ops, synth

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[case] {msg}", flush=True)


# ------------------------------------------------------------------ layout


@pytest.mark.parametrize("bits_", [4, 8])
def test_unpack_bit_exact(dev, orc, bits_):
    say(f"unpack bits={bits_}")
    rng = np.random.default_rng(11)
    w = rng.integers(0, 2 ** 32, size=(64, 96), dtype=np.uint32)
    got = ops.unpack(words_t(w, dev), bits_).cpu().numpy()
    assert np.array_equal(got, orc.unpack(w, bits_))


@pytest.mark.parametrize("bits_,gs", [(4, 64), (4, 32), (8, 64), (4, 128)])
def test_dequantize_bit_exact(dev, orc, bits_, gs):
    say(f"dequantize bits={bits_} gs={gs}")
    rng = np.random.default_rng(12)
    K = 512
    w, s, b = synth.quant_weights(rng, (3, 40), K, gs, bits_)
    got = bits(ops.dequantize(words_t(w, dev), bf16_t(s, dev), bf16_t(b, dev), gs, bits_))
    assert np.array_equal(got, orc.dequantize_bf16(w, s, b, gs, bits_))


# ----------------------------------------------------------------- routing


def _route_cases():
    rng = np.random.default_rng(5)
    wl = synth.make(3, tokens=4096)
    yield "cfg3-zipf", wl["idx"], 256
    yield "one-expert", np.zeros(300, np.int32), 8
    yield "uniform", rng.integers(0, 32, size=200).astype(np.int32), 32
    yield "single", np.array([3], np.int32), 8
    yield "ragged", rng.integers(0, 1000, size=12345).astype(np.int32), 1000
    # the single-block path takes up to 4096 pairs and 512 experts
    yield "fused-max", rng.integers(0, 512, size=4096).astype(np.int32), 512
    yield "split-min", rng.integers(0, 512, size=4097).astype(np.int32), 512
    yield "zipf-700", synth.make(3, tokens=700)["idx"], 256
    yield "zipf-300-fused", synth.make(3, tokens=300)["idx"], 256
    yield "fused-ragged-waves", rng.integers(0, 40, size=1009).astype(np.int32), 40
    # more than 2048 experts: the separate scan and the one-wave-per-chunk scatter
    yield "many-experts", rng.integers(0, 3000, size=9000).astype(np.int32), 3000
    # more than 512 experts, up to 2048: the scatter that scans, whatever the size
    yield "scan-scatter-max", rng.integers(0, 2048, size=20000).astype(np.int32), 2048
    yield "one-chunk-many-experts", rng.integers(0, 1500, size=100).astype(np.int32), 1500
    yield "empty-many-experts", np.zeros(0, np.int32), 1000


@pytest.mark.parametrize("case", list(range(14)))
def test_route_matches_stable_sort(dev, orc, case):
    name, ids, E = list(_route_cases())[case]
    say(f"route {name} n={ids.size} E={E}")
    r = ops.route(i32_t(ids, dev), E)
    order, inv, srt = orc.route_sort(ids, E)
    assert np.array_equal(r.order.cpu().numpy(), order)
    assert np.array_equal(r.inv_order.cpu().numpy(), inv)
    assert np.array_equal(r.sorted_ids.cpu().numpy(), srt)
    assert np.array_equal(order, np.argsort(ids.reshape(-1), kind="stable"))
    off, trow, texp, nt = orc.build_tiles(srt, E, r.tiles.tile_rows)
    assert np.array_equal(r.tiles.offsets.cpu().numpy(), off)
    assert int(r.tiles.ntiles.item()) == nt
    assert np.array_equal(r.tiles.tile_row.cpu().numpy(), trow)
    assert np.array_equal(r.tiles.tile_exp.cpu().numpy(), texp)
    assert int(r.bad_ids.item()) == 0


@pytest.mark.parametrize("n", [7, 9000])
def test_route_clamps_out_of_range_ids(dev, orc, n):
    say(f"route out-of-range ids n={n}")
    ids = np.array([0, 5, 9, -1, 3, 12, 5], np.int32)
    if n > ids.size:
        ids = np.concatenate([ids, np.random.default_rng(n).integers(-2, 10, size=n - ids.size).astype(np.int32)])
    r = ops.route(i32_t(ids, dev), 8)
    assert int(r.bad_ids.item()) == int(((ids < 0) | (ids >= 8)).sum())
    clamped = np.clip(ids, 0, 7)
    order, inv, srt = orc.route_sort(clamped, 8)
    assert np.array_equal(r.order.cpu().numpy(), order)
    assert np.array_equal(r.sorted_ids.cpu().numpy(), srt)


def test_build_tiles_from_sorted(dev, orc):
    say("build_tiles sorted")
    rng = np.random.default_rng(9)
    ids = np.sort(rng.integers(0, 64, size=5000)).astype(np.int32)
    t = ops.build_tiles(i32_t(ids, dev), 64, 48)
    off, trow, texp, nt = orc.build_tiles(ids, 64, 48)
    assert np.array_equal(t.offsets.cpu().numpy(), off)
    assert int(t.ntiles.item()) == nt
    assert np.array_equal(t.tile_row.cpu().numpy(), trow)
    assert np.array_equal(t.tile_exp.cpu().numpy(), texp)


# ------------------------------------------------------------ decode GEMV


def test_quantized_matmul_cfg0(dev, orc):
    say("quantized_matmul workload 0 [1,2048]x[4096,2048]")
    wl = synth.make(0)
    y = ops.quantized_matmul(bf16_t(wl["x"], dev), words_t(wl["w"], dev), bf16_t(wl["s"], dev),
                             bf16_t(wl["b"], dev))
    ref64, _ = orc.gather_qmm_rows(wl["x"], None, np.zeros(1, np.int32), wl["w"][None], wl["s"][None],
                                   wl["b"][None])
    assert_close_bf16(orc, bits(y), ref64, what="cfg0")


@pytest.mark.parametrize("M,N,K", [(3, 256, 512), (5, 192, 2560), (2, 64, 640), (1, 100, 128)])
def test_quantized_matmul_shapes(dev, orc, M, N, K):
    say(f"quantized_matmul M={M} N={N} K={K}")
    rng = np.random.default_rng(M * 1000 + K)
    w, s, b = synth.quant_weights(rng, (N,), K)
    x = synth.bf16_bits(rng.normal(size=(M, K)).astype(np.float32))
    y = ops.quantized_matmul(bf16_t(x, dev), words_t(w, dev), bf16_t(s, dev), bf16_t(b, dev))
    ref64, _ = orc.gather_qmm_rows(x, None, np.zeros(M, np.int32), w[None], s[None], b[None])
    assert_close_bf16(orc, bits(y), ref64, what=f"qmm {M}x{N}x{K}")


def test_gate_up_swiglu_cfg1(dev, orc):
    say("gate_up + SwiGLU workload 1")
    wl = synth.make(1)
    h = ops.gate_up_silu(bf16_t(wl["x"], dev), words_t(wl["w"], dev), bf16_t(wl["s"], dev),
                         bf16_t(wl["b"], dev), i32_t(wl["idx"], dev))
    assert h.shape == (1, 10, 512)
    gu64, _ = orc.gather_qmm_rows(wl["x"], np.zeros(10, np.int32), wl["idx"].reshape(-1), wl["w"],
                                  wl["s"], wl["b"])
    h64, _ = orc.swiglu(gu64)
    assert_close_bf16(orc, bits(h).reshape(10, 512), h64, what="cfg1 swiglu")


def test_gather_qmm_decode_form(dev, orc):
    """x [T,1,1,K] with rhs [T,k] -> [T,k,1,N] (switch_layers.py:214 shapes)."""
    say("gather_qmm decode form T=3 k=4")
    rng = np.random.default_rng(21)
    E, N, K, T, k = 16, 128, 1024, 3, 4
    w, s, b = synth.quant_weights(rng, (E, N), K)
    x = synth.bf16_bits(rng.normal(size=(T, 1, 1, K)).astype(np.float32))
    idx = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    out = ops.gather_qmm(bf16_t(x, dev), words_t(w, dev), bf16_t(s, dev), bf16_t(b, dev),
                         rhs_indices=i32_t(idx, dev))
    assert out.shape == (T, k, 1, N)
    xr = np.repeat(np.arange(T), k).astype(np.int32)
    ref64, _ = orc.gather_qmm_rows(x.reshape(T, K), xr, idx.reshape(-1), w, s, b)
    assert_close_bf16(orc, bits(out).reshape(T * k, N), ref64, what="decode form")


def test_down_wsum_cfg2(dev, orc):
    say("down + weighted sum workload 2")
    wl = synth.make(2)
    y = ops.down_wsum(bf16_t(wl["h"], dev), words_t(wl["w"], dev), bf16_t(wl["s"], dev),
                      bf16_t(wl["b"], dev), i32_t(wl["idx"], dev), f32_t(wl["scores"], dev))
    y64, _ = orc.down_wsum(wl["h"], wl["idx"], wl["scores"], wl["w"], wl["s"], wl["b"])
    assert_close_bf16(orc, bits(y), y64, what="cfg2 down+wsum")


@pytest.mark.parametrize("T", [1, 3, 16])
def test_down_wsum_widths(dev, orc, T):
    say(f"down + weighted sum T={T}")
    wl = synth.make(2, seed=100 + T, tokens=T, experts=64)
    y = ops.down_wsum(bf16_t(wl["h"], dev), words_t(wl["w"], dev), bf16_t(wl["s"], dev),
                      bf16_t(wl["b"], dev), i32_t(wl["idx"], dev), f32_t(wl["scores"], dev))
    y64, _ = orc.down_wsum(wl["h"], wl["idx"], wl["scores"], wl["w"], wl["s"], wl["b"])
    assert_close_bf16(orc, bits(y), y64, what=f"down T={T}")


# ------------------------------------------------------------ weighted sum


@pytest.mark.parametrize("rows,dim", [(1, 256), (9, 256), (13, 2560), (128, 2560)])
@pytest.mark.parametrize("sorted_layout", [True, False])
@pytest.mark.parametrize("mode", ["clone", "ops", "fast"])
def test_weighted_sum_bit_exact(dev, orc, rows, dim, sorted_layout, mode):
    say(f"weighted_sum rows={rows} dim={dim} sorted={sorted_layout} mode={mode}")
    rng = np.random.default_rng(rows * 7 + dim)
    k = 10
    xs = synth.bf16_bits(rng.normal(size=(rows * k, dim)).astype(np.float32))
    sc = rng.uniform(size=(rows, k)).astype(np.float32)
    sc /= sc.sum(-1, keepdims=True)
    inv = rng.permutation(rows * k).astype(np.int32) if sorted_layout else None
    got = ops.moe_weighted_sum(bf16_t(xs, dev), None if inv is None else i32_t(inv, dev), f32_t(sc, dev),
                               (1, rows, dim), mode=mode)
    ref = orc.weighted_sum(xs, inv, sc, rows, k, dim, mode)
    assert np.array_equal(bits(got).reshape(rows, dim), ref)


@pytest.mark.parametrize("k", [1, 6, 8, 16, 17, 20, 33])
@pytest.mark.parametrize("mode", ["clone", "fast"])
def test_weighted_sum_other_top_k(dev, orc, k, mode):
    """Top-k below, at and past the kernel's batch of 16 slots (k = 33: three
    batches, the last with one slot), and a row of 65 eight-column groups."""
    say(f"weighted_sum k={k} mode={mode}")
    rng = np.random.default_rng(k)
    rows, dim = 32, 520
    xs = synth.bf16_bits(rng.normal(size=(rows * k, dim)).astype(np.float32))
    sc = rng.uniform(size=(rows, k)).astype(np.float32)
    inv = rng.permutation(rows * k).astype(np.int32)
    got = ops.moe_weighted_sum(bf16_t(xs, dev), i32_t(inv, dev), f32_t(sc, dev), (1, rows, dim), mode=mode)
    assert np.array_equal(bits(got).reshape(rows, dim), orc.weighted_sum(xs, inv, sc, rows, k, dim, mode))


# ------------------------------------------------------------- prefill GEMM


def _sorted_problem(seed, E, N, K, R, zipf=True, one_expert=False):
    rng = np.random.default_rng(seed)
    w, s, b = synth.quant_weights(rng, (E, N), K)
    if one_expert:
        ids = np.zeros(R, np.int32)
    elif zipf:
        p = 1.0 / np.arange(1, E + 1)
        ids = np.sort(rng.choice(E, size=R, p=p / p.sum())).astype(np.int32)
    else:
        ids = np.sort(rng.integers(0, E, size=R)).astype(np.int32)
    x = synth.bf16_bits(rng.normal(size=(R, K)).astype(np.float32))
    return w, s, b, ids, x


@pytest.mark.parametrize("E,N,K,R,kind", [
    (8, 256, 1024, 300, "zipf"),
    (32, 512, 2048, 700, "uniform"),
    (4, 256, 1024, 500, "one"),
    (16, 1024, 1024, 64, "zipf"),
    (16, 2048, 512, 700, "zipf"),    # the prefill down projection's shape (K = I = 512)
    (8, 768, 384, 333, "uniform"),   # K = 3 * 128, N = 3 * 256: the four-wave column block
])
def test_sorted_gemm_bf16(dev, orc, E, N, K, R, kind):
    say(f"sorted GEMM E={E} N={N} K={K} R={R} {kind}")
    w, s, b, ids, x = _sorted_problem(E * 31 + R, E, N, K, R, zipf=kind == "zipf", one_expert=kind == "one")
    xt = bf16_t(x, dev)
    tiles = ops.build_tiles(i32_t(ids, dev), E)
    y = ops.gather_qmm_sorted(xt, words_t(w, dev), bf16_t(s, dev), bf16_t(b, dev), tiles)
    got = bits(y)
    ref_b64, _ = orc.gather_qmm_rows(x, None, ids, w, s, b, deq="bf16")
    assert_close_bf16(orc, got, ref_b64, what=f"gemm bf16-deq {E}/{N}/{K}/{R}")
    ref_e64, _ = orc.gather_qmm_rows(x, None, ids, w, s, b, deq="exact")
    rep = orc.err_report(got, ref_e64)
    print(f"[parity] vs exact-affine golden: {rep}", flush=True)
    assert rep["rel_to_max"] <= 2.0 ** -8


@pytest.mark.parametrize("tiled", [False, True])
def test_sorted_gemm_dequant_bit_exact_one_hot(dev, orc, tiled):
    """Rows of x are one-hot, so y[r, n] = x[r, k_r] * deq(W)[n, k_r] with a
    single nonzero product: the GEMM output is the in-kernel dequantised
    weight itself, which must equal bf16_rne(fmaf(q, s, b)) bit for bit
    (moe_gather_ws.py:343-344) for every code position of every word."""
    say(f"sorted GEMM one-hot dequant tiled={tiled}")
    rng = np.random.default_rng(11)
    E, N, K = 2, 256, 256
    w, s, b = synth.quant_weights(rng, (E, N), K)
    R = 2 * K  # expert 0 and expert 1 each see every k once
    ids = np.repeat(np.arange(E), K).astype(np.int32)
    x = np.zeros((R, K), np.float32)
    x[np.arange(R), np.tile(np.arange(K), E)] = 1.0
    xb = synth.bf16_bits(x)
    tiles = ops.build_tiles(i32_t(ids, dev), E)
    if tiled:
        tw = ops.repack_tiles(words_t(w, dev), bf16_t(s, dev), bf16_t(b, dev))
        y = ops.gather_qmm_sorted_tiles(bf16_t(xb, dev), tw, tiles)
    else:
        y = ops.gather_qmm_sorted(bf16_t(xb, dev), words_t(w, dev), bf16_t(s, dev), bf16_t(b, dev), tiles)
    got = bits(y).reshape(E, K, N)
    deq = orc.dequantize_bf16(w, s, b, 64, 4)  # bf16 bits [E, N, K]
    assert np.array_equal(got, deq.transpose(0, 2, 1))


@pytest.mark.parametrize("tiled", [False, True])
def test_sorted_gemm_every_subtile_count(dev, orc, tiled):
    """Experts with 1, 33, 65, ... 225, 256 and 300 rows: tiles of every
    32-row subtile count 1..8, a full tile and a tile boundary inside an
    expert."""
    counts = [1, 33, 65, 97, 129, 161, 193, 225, 256, 300, 0, 31]
    E, N, K = len(counts), 512, 512
    say(f"sorted GEMM every subtile count tiled={tiled}")
    rng = np.random.default_rng(5)
    w, s, b = synth.quant_weights(rng, (E, N), K)
    ids = np.repeat(np.arange(E), counts).astype(np.int32)
    R = len(ids)
    x = synth.bf16_bits(rng.normal(size=(R, K)).astype(np.float32))
    tiles = ops.build_tiles(i32_t(ids, dev), E)
    if tiled:
        tw = ops.repack_tiles(words_t(w, dev), bf16_t(s, dev), bf16_t(b, dev))
        y = ops.gather_qmm_sorted_tiles(bf16_t(x, dev), tw, tiles)
    else:
        y = ops.gather_qmm_sorted(bf16_t(x, dev), words_t(w, dev), bf16_t(s, dev), bf16_t(b, dev), tiles)
    ref, _ = orc.gather_qmm_rows(x, None, ids, w, s, b, deq="bf16")
    assert_close_bf16(orc, bits(y), ref, what="gemm every subtile count")


def test_gather_qmm_sorted_with_lhs_indices(dev, orc):
    """The fused-gather form: x token-major, lhs_indices = order // k."""
    say("gather_qmm sorted with lhs_indices")
    wl = synth.make(3, seed=33, tokens=96, experts=16)
    T, k = wl["idx"].shape
    ids = wl["idx"].reshape(-1)
    order = np.argsort(ids, kind="stable").astype(np.int32)
    srt = ids[order]
    lhs = (order // k).astype(np.int32)
    x = wl["x"]
    out = ops.gather_qmm(bf16_t(x, dev).reshape(T, 1, -1), words_t(wl["w"], dev), bf16_t(wl["s"], dev),
                         bf16_t(wl["b"], dev), lhs_indices=i32_t(lhs, dev), rhs_indices=i32_t(srt, dev),
                         sorted_indices=True)
    assert out.shape == (T * k, 1, wl["w"].shape[1])
    ref64, _ = orc.gather_qmm_rows(x, lhs, srt, wl["w"], wl["s"], wl["b"], deq="bf16")
    assert_close_bf16(orc, bits(out).reshape(T * k, -1), ref64, what="lhs form")


def _sample_rows(offsets, R, n_random, rng):
    """Random rows plus the first and last row of every expert segment."""
    edges = set()
    for e in range(len(offsets) - 1):
        if offsets[e + 1] > offsets[e]:
            edges.add(int(offsets[e]))
            edges.add(int(offsets[e + 1] - 1))
            for j in range(offsets[e] + 127, offsets[e + 1], 128):
                edges.update((int(j), int(j + 1) if j + 1 < offsets[e + 1] else int(j)))
    rand = rng.choice(R, size=n_random, replace=False)
    return np.array(sorted(edges | set(int(v) for v in rand)), np.int64)


def test_sorted_gemm_cfg3_sampled(dev, orc):
    say("sorted GEMM workload 3 (full size, sampled rows checked)")
    wl = synth.make(3)
    T, k = wl["idx"].shape
    ids = wl["idx"]
    x = bf16_t(wl["x"], dev)
    r = ops.route(i32_t(ids, dev), 256)
    lhs = torch.div(r.order, k, rounding_mode="floor").to(torch.int32)
    y = ops.gather_qmm_sorted(x, words_t(wl["w"], dev), bf16_t(wl["s"], dev), bf16_t(wl["b"], dev), r.tiles,
                              x_rows=lhs)
    torch.cuda.synchronize()
    order, _, srt = orc.route_sort(ids, 256)
    off = np.searchsorted(srt, np.arange(257), side="left")
    rows = _sample_rows(off, T * k, 384, np.random.default_rng(0))
    got = bits(y)[rows]
    ref64, _ = orc.gather_qmm_rows(wl["x"], (order[rows] // k).astype(np.int32), srt[rows], wl["w"], wl["s"],
                                   wl["b"], deq="bf16")
    assert_close_bf16(orc, got, ref64, what=f"cfg3 {rows.size} rows")


# -------------------------------------------------------------------- int8


def test_quantize_act_int8_bit_exact(dev, orc):
    say("int8 quantizer workload 4 activations")
    wl = synth.make(4, tokens=512)
    x = wl["x"].copy()
    x[3] = 0  # an all-zero row
    xi, sx = ops.quantize_act_int8(bf16_t(x, dev))
    rxi, rsx = orc.quant_act_int8(x)
    assert np.array_equal(sx.cpu().numpy().view(np.uint32), rsx.view(np.uint32))
    assert np.array_equal(xi.cpu().numpy(), rxi)


@pytest.mark.parametrize("R,K", [(37, 512), (9, 1536), (5, 4096), (6, 5120), (3, 8192)])
def test_quantize_act_int8_row_lengths(dev, orc, R, K):
    """Rows of one to sixteen 512-element pieces per lane step, in registers
    (K <= 4096) and read twice (K > 4096); an all-zero row and a row whose
    maximum sits in its last element."""
    say(f"int8 quantizer R={R} K={K}")
    rng = np.random.default_rng(R * 31 + K)
    x = synth.bf16_bits(rng.normal(size=(R, K)).astype(np.float32))
    x[1] = 0
    x[2, -1] = synth.bf16_bits(np.array([40.0], np.float32))[0]
    xi, sx = ops.quantize_act_int8(bf16_t(x, dev))
    rxi, rsx = orc.quant_act_int8(x)
    assert np.array_equal(sx.cpu().numpy().view(np.uint32), rsx.view(np.uint32))
    assert np.array_equal(xi.cpu().numpy(), rxi)


@pytest.mark.parametrize("E,N,K,R", [(8, 256, 1024, 300), (16, 512, 2048, 640), (4, 768, 4096, 200),
                                     (8, 256, 1536, 90),
                                     (16, 2048, 512, 700)])  # the prefill down projection's shape (K = I = 512)
def test_sorted_gemm_int8(dev, orc, E, N, K, R):
    say(f"int8 sorted GEMM E={E} N={N} K={K} R={R}")
    w, s, b, ids, x = _sorted_problem(E * 17 + R, E, N, K, R)
    xi, sx = ops.quantize_act_int8(bf16_t(x, dev))
    tiles = ops.build_tiles(i32_t(ids, dev), E)
    rxi, rsx = orc.quant_act_int8(x)
    ref64, _ = orc.gather_qmm_int8_rows(rxi, rsx, None, ids, w, s, b)
    tw = ops.repack_tiles(words_t(w, dev), bf16_t(s, dev), bf16_t(b, dev))
    yt = ops.gather_qmm_int8_sorted_tiles(xi, sx, tw, tiles)
    assert_close_bf16(orc, bits(yt), ref64, what=f"int8 gemm tiles {E}/{N}/{K}/{R}")
    if K % 128 == 0:
        y = ops.gather_qmm_int8_sorted(xi, sx, words_t(w, dev), bf16_t(s, dev), bf16_t(b, dev), tiles)
        assert_close_bf16(orc, bits(y), ref64, what=f"int8 gemm {E}/{N}/{K}/{R}")
        # same rows, groups and summation order: the layouts agree bit for bit
        assert np.array_equal(bits(y), bits(yt))


def test_sorted_gemm_int8_every_subtile_count(dev, orc):
    """Experts with 1, 17, 33, ... rows: tiles of every 16- and 32-row subtile
    count, a full tile and a tile boundary inside an expert."""
    counts = [1, 17, 33, 49, 65, 81, 97, 113, 128, 200, 0, 31]
    E, N, K = len(counts), 512, 512
    say("int8 sorted GEMM every subtile count")
    rng = np.random.default_rng(6)
    w, s, b = synth.quant_weights(rng, (E, N), K)
    ids = np.repeat(np.arange(E), counts).astype(np.int32)
    x = synth.bf16_bits(rng.normal(size=(len(ids), K)).astype(np.float32))
    xi, sx = ops.quantize_act_int8(bf16_t(x, dev))
    tiles = ops.build_tiles(i32_t(ids, dev), E)
    tw = ops.repack_tiles(words_t(w, dev), bf16_t(s, dev), bf16_t(b, dev))
    y = ops.gather_qmm_int8_sorted_tiles(xi, sx, tw, tiles)
    rxi, rsx = orc.quant_act_int8(x)
    ref64, _ = orc.gather_qmm_int8_rows(rxi, rsx, None, ids, w, s, b)
    assert_close_bf16(orc, bits(y), ref64, what="int8 gemm every subtile count")
    # the MLX-layout kernel takes the same rows to the same bits
    ym = ops.gather_qmm_int8_sorted(xi, sx, words_t(w, dev), bf16_t(s, dev), bf16_t(b, dev), tiles)
    torch.cuda.synchronize()
    assert np.array_equal(bits(ym), bits(y))


def test_sorted_gemm_int8_cfg4_sampled(dev, orc):
    say("int8 sorted GEMM workload 4 (full size, sampled rows checked)")
    wl = synth.make(4)
    T, k = wl["idx"].shape
    ids = wl["idx"]
    xi, sx = ops.quantize_act_int8(bf16_t(wl["x"], dev))
    r = ops.route(i32_t(ids, dev), 256)
    lhs = torch.div(r.order, k, rounding_mode="floor").to(torch.int32)
    tw = ops.repack_tiles(words_t(wl["w"], dev), bf16_t(wl["s"], dev), bf16_t(wl["b"], dev))
    y = ops.gather_qmm_int8_sorted_tiles(xi, sx, tw, r.tiles, x_rows=lhs)
    torch.cuda.synchronize()
    order, _, srt = orc.route_sort(ids, 256)
    off = np.searchsorted(srt, np.arange(257), side="left")
    rows = _sample_rows(off, T * k, 256, np.random.default_rng(1))
    rxi, rsx = orc.quant_act_int8(wl["x"])
    ref64, _ = orc.gather_qmm_int8_rows(rxi, rsx, (order[rows] // k).astype(np.int32), srt[rows], wl["w"],
                                        wl["s"], wl["b"])
    assert_close_bf16(orc, bits(y)[rows], ref64, what=f"cfg4 {rows.size} rows")


def test_sorted_gemm_int8_down_prefill_sampled(dev, orc):
    """The int8 grouped GEMM on the prefill down projection at full size:
    4096 tokens x top-10 Zipf routed rows (40960, sorted by expert, no
    gather), h [40960, 512] -> [40960, 2048] with W [256, 2048, 512] int4 g64
    (K = I = 512), sampled rows against the fake-quant golden, and the bf16
    GEMM on the same rows against its fp64 golden."""
    say("int8 + bf16 sorted GEMM, down projection 40960 x 512 -> 2048, sampled rows")
    wl = synth.make(4)
    T, k = wl["idx"].shape
    rng = np.random.default_rng(512)
    w, s, b = synth.quant_weights(rng, (256, 2048), 512)
    order, _, srt = orc.route_sort(wl["idx"], 256)
    R = T * k
    h = synth.bf16_bits((rng.normal(size=(R, 512)) * 0.5).astype(np.float32))
    tiles = ops.build_tiles(i32_t(srt, dev), 256)
    ht = bf16_t(h, dev)
    tw = ops.repack_tiles(words_t(w, dev), bf16_t(s, dev), bf16_t(b, dev))
    hi, hs = ops.quantize_act_int8(ht)
    y8 = ops.gather_qmm_int8_sorted_tiles(hi, hs, tw, tiles)
    y16 = ops.gather_qmm_sorted_tiles(ht, tw, tiles)
    torch.cuda.synchronize()
    off = np.searchsorted(srt, np.arange(257), side="left")
    rows = _sample_rows(off, R, 256, np.random.default_rng(5))
    rxi, rsx = orc.quant_act_int8(h[rows])
    ref8, _ = orc.gather_qmm_int8_rows(rxi, rsx, None, srt[rows], w, s, b)
    assert_close_bf16(orc, bits(y8)[rows], ref8, what=f"int8 down {rows.size} rows")
    ref16, _ = orc.gather_qmm_rows(h[rows], None, srt[rows], w, s, b, deq="bf16")
    assert_close_bf16(orc, bits(y16)[rows], ref16, what=f"bf16 down {rows.size} rows")


# ---------------------------------------------------------------- tile layout


def _tile_layout_np(w, s, b):
    """The tile layout's index map restated in numpy (the header's formulas)."""
    E, N, KW = w.shape
    G = KW // 8
    wp = w.reshape(E, N // 64, 2, 32, G, 2, 4).transpose(0, 1, 4, 2, 5, 3, 6)  # e c g j h l t
    sb = (s.astype(np.uint32) | (b.astype(np.uint32) << 16)).reshape(E, N // 64, 64, G).transpose(0, 1, 3, 2)
    return np.ascontiguousarray(wp), np.ascontiguousarray(sb)


@pytest.mark.parametrize("E,N,K", [(3, 64, 64), (4, 256, 512), (2, 1024, 2048)])
def test_repack_tiles_is_the_documented_permutation(dev, E, N, K):
    say(f"repack E={E} N={N} K={K}")
    rng = np.random.default_rng(E * N + K)
    w, s, b = synth.quant_weights(rng, (E, N), K)
    tw = ops.repack_tiles(words_t(w, dev), bf16_t(s, dev), bf16_t(b, dev))
    want_wp, want_sb = _tile_layout_np(w, s, b)
    got_wp = tw.wp.cpu().numpy().view(np.uint32)
    got_sb = tw.sb.cpu().numpy().view(np.uint32)
    assert np.array_equal(got_wp, want_wp) and np.array_equal(got_sb, want_sb)


@pytest.mark.parametrize("E,N,K,R,kind", [
    (8, 256, 1024, 300, "zipf"),
    (16, 1024, 2048, 700, "uniform"),
    (16, 2048, 512, 500, "zipf"),
    (8, 768, 192, 333, "one"),   # K = 3 groups: no pair constraint in the tile layout
])
def test_sorted_gemm_tiles_is_bit_identical_to_mlx_layout(dev, orc, E, N, K, R, kind):
    say(f"sorted GEMM tile layout E={E} N={N} K={K} R={R} {kind}")
    w, s, b, ids, x = _sorted_problem(E * 17 + R, E, N, K, R, zipf=kind == "zipf", one_expert=kind == "one")
    xt = bf16_t(x, dev)
    tiles = ops.build_tiles(i32_t(ids, dev), E)
    tw = ops.repack_tiles(words_t(w, dev), bf16_t(s, dev), bf16_t(b, dev))
    y_t = ops.gather_qmm_sorted_tiles(xt, tw, tiles)
    ref64, _ = orc.gather_qmm_rows(x, None, ids, w, s, b, deq="bf16")
    assert_close_bf16(orc, bits(y_t), ref64, what=f"gemm tiles {E}/{N}/{K}/{R}")
    if K % 128 == 0:
        y_m = ops.gather_qmm_sorted(xt, words_t(w, dev), bf16_t(s, dev), bf16_t(b, dev), tiles)
        assert np.array_equal(bits(y_t), bits(y_m))


def test_gate_up_swiglu_tiles_cfg1_matches_mlx_layout(dev, orc):
    say("gate_up + SwiGLU tile layout, workload 1")
    wl = synth.make(1)
    w, s, b = words_t(wl["w"], dev), bf16_t(wl["s"], dev), bf16_t(wl["b"], dev)
    tw = ops.repack_tiles(w, s, b, swiglu_pairs=True)
    idx = i32_t(wl["idx"], dev)
    h_t = ops.gate_up_silu_tiles(bf16_t(wl["x"], dev), tw, idx)
    gu64, _ = orc.gather_qmm_rows(wl["x"], np.zeros(10, np.int32), wl["idx"].reshape(-1), wl["w"],
                                  wl["s"], wl["b"])
    h64, _ = orc.swiglu(gu64)
    assert_close_bf16(orc, bits(h_t).reshape(10, 512), h64, what="cfg1 swiglu tiles")


@pytest.mark.parametrize("T,k,E,I,K", [(3, 4, 16, 96, 2048), (1, 10, 16, 256, 4096), (2, 2, 4, 64, 6144),
                                       (2, 3, 4, 32, 8192), (16, 10, 64, 512, 2048)])
def test_gate_up_swiglu_tiles_shapes(dev, orc, T, k, E, I, K):
    say(f"gate_up tiles T={T} k={k} E={E} I={I} K={K}")
    rng = np.random.default_rng(T * 1000 + K)
    w, s, b = synth.quant_weights(rng, (E, 2 * I), K)
    x = synth.bf16_bits(rng.normal(size=(T, K)).astype(np.float32))
    idx = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    tw = ops.repack_tiles(words_t(w, dev), bf16_t(s, dev), bf16_t(b, dev), swiglu_pairs=True)
    h = ops.gate_up_silu_tiles(bf16_t(x, dev), tw, i32_t(idx, dev))
    rows = np.repeat(np.arange(T, dtype=np.int32), k)
    gu64, _ = orc.gather_qmm_rows(x, rows, idx.reshape(-1), w, s, b)
    h64, _ = orc.swiglu(gu64)
    assert_close_bf16(orc, bits(h).reshape(T * k, I), h64, what=f"gate_up tiles {T}/{k}/{E}/{I}/{K}")



@pytest.mark.parametrize("R,E,N,K", [(1, 1, 4096, 2048), (7, 8, 192, 4096), (5, 3, 64, 8192)])
def test_gather_qmv_tiles(dev, orc, R, E, N, K):
    say(f"gather_qmv tiles R={R} E={E} N={N} K={K}")
    rng = np.random.default_rng(R * 7 + N)
    w, s, b = synth.quant_weights(rng, (E, N), K)
    x = synth.bf16_bits(rng.normal(size=(3, K)).astype(np.float32))
    xr = rng.integers(0, 3, size=R).astype(np.int32)
    ex = rng.integers(0, E, size=R).astype(np.int32)
    tw = ops.repack_tiles(words_t(w, dev), bf16_t(s, dev), bf16_t(b, dev))
    y = ops.gather_qmv_tiles(bf16_t(x, dev), i32_t(xr, dev), i32_t(ex, dev), tw)
    ref64, _ = orc.gather_qmm_rows(x, xr, ex, w, s, b)
    assert_close_bf16(orc, bits(y), ref64, what=f"qmv tiles {R}/{E}/{N}/{K}")
    ym = ops.gather_qmv(bf16_t(x, dev), i32_t(xr, dev), i32_t(ex, dev), words_t(w, dev), bf16_t(s, dev),
                        bf16_t(b, dev))
    assert np.array_equal(bits(y), bits(ym))


@pytest.mark.parametrize("nbits,gs", [(8, 32), (8, 64), (8, 128), (4, 32), (4, 128)])
@pytest.mark.parametrize("M,N,K", [(1, 512, 2048), (3, 256, 1024), (16, 128, 4096), (2, 64, 512)])
def test_quantized_matmul_bits_and_groups(dev, orc, nbits, gs, M, N, K):
    """The small-M quantized matmul over 4- and 8-bit codes and group sizes
    32/64/128 (engine/patches/smallm/kernel.py:38, 319-327)."""
    say(f"quantized_matmul bits={nbits} gs={gs} M={M} N={N} K={K}")
    rng = np.random.default_rng(nbits * 7919 + gs * 31 + M * N + K)
    w, s, b = synth.quant_weights(rng, (N,), K, group_size=gs, bits=nbits)
    x = synth.bf16_bits(rng.normal(size=(M, K)).astype(np.float32))
    y = ops.quantized_matmul(bf16_t(x, dev), words_t(w, dev), bf16_t(s, dev), bf16_t(b, dev), group_size=gs,
                             bits=nbits)
    ref64, _ = orc.gather_qmm_rows(x, None, np.zeros(M, np.int32), w[None], s[None], b[None], group_size=gs,
                                   bits=nbits)
    assert_close_bf16(orc, bits(y), ref64, what=f"qmm{nbits} gs{gs} {M}x{N}x{K}")


@pytest.mark.parametrize("nbits,gs", [(8, 64), (8, 128), (4, 32)])
def test_gather_qmv_bits_and_groups(dev, orc, nbits, gs):
    say(f"gather_qmv bits={nbits} gs={gs}")
    rng = np.random.default_rng(nbits + gs)
    E, N, K, R = 6, 192, 2048, 13
    w, s, b = synth.quant_weights(rng, (E, N), K, group_size=gs, bits=nbits)
    x = synth.bf16_bits(rng.normal(size=(4, K)).astype(np.float32))
    xr = rng.integers(0, 4, size=R).astype(np.int32)
    ex = rng.integers(0, E, size=R).astype(np.int32)
    y = ops.gather_qmv(bf16_t(x, dev), i32_t(xr, dev), i32_t(ex, dev), words_t(w, dev), bf16_t(s, dev),
                       bf16_t(b, dev), gs, nbits)
    ref64, _ = orc.gather_qmm_rows(x, xr, ex, w, s, b, group_size=gs, bits=nbits)
    assert_close_bf16(orc, bits(y), ref64, what=f"qmv{nbits} gs{gs}")
    # through the mx.gather_qmm surface (decode form: rows of one token each)
    yg = ops.gather_qmm(bf16_t(x, dev)[:, None], words_t(w, dev), bf16_t(s, dev), bf16_t(b, dev),
                        lhs_indices=i32_t(xr, dev), rhs_indices=i32_t(ex, dev), group_size=gs, bits=nbits)
    assert np.array_equal(bits(yg).reshape(R, N), bits(y))


@pytest.mark.parametrize("gs", [64, 128])
@pytest.mark.parametrize("M,K", [(1, 6144), (3, 8192)])
def test_8bit_fast_gemv_wide_k(dev, orc, gs, M, K):
    """8-bit codes at K = 2048 * n beyond the lane split's reach (K > 4096) run
    on the 2048-chunk GEMV."""
    say(f"8-bit quantized_matmul gs={gs} M={M} K={K}")
    rng = np.random.default_rng(K + gs + M)
    N = 96
    w, s, b = synth.quant_weights(rng, (N,), K, group_size=gs, bits=8)
    x = synth.bf16_bits(rng.normal(size=(M, K)).astype(np.float32))
    y = ops.quantized_matmul(bf16_t(x, dev), words_t(w, dev), bf16_t(s, dev), bf16_t(b, dev), group_size=gs,
                             bits=8)
    ref64, _ = orc.gather_qmm_rows(x, None, np.zeros(M, np.int32), w[None], s[None], b[None], group_size=gs,
                                   bits=8)
    assert_close_bf16(orc, bits(y), ref64, what=f"qmm8 gs{gs} {M}x{N}x{K}")


def test_8bit_unsupported_shapes_are_declined(dev):
    """8-bit codes take K = 2048 * n (n <= 4) or a lane split (K <= 4096); the
    fused decode kernels take 4-bit only."""
    say("8-bit declines")
    rng = np.random.default_rng(5)
    w, s, b = synth.quant_weights(rng, (64,), 10240, bits=8)
    x = bf16_t(synth.bf16_bits(rng.normal(size=(1, 10240)).astype(np.float32)), dev)
    with pytest.raises(ops.QmoeUnsupported):
        ops.quantized_matmul(x, words_t(w, dev), bf16_t(s, dev), bf16_t(b, dev), bits=8)
    w, s, b = synth.quant_weights(rng, (4, 128), 2048, bits=8)
    x2 = bf16_t(synth.bf16_bits(rng.normal(size=(1, 2048)).astype(np.float32)), dev)
    with pytest.raises(ops.QmoeUnsupported):
        ops.gate_up_silu(x2, words_t(w, dev), bf16_t(s, dev), bf16_t(b, dev),
                         i32_t(np.zeros((1, 2), np.int32), dev), bits=8)


@pytest.mark.parametrize("K", [2560, 3584, 5120, 7680])
def test_decode_gemv_tail_chunk_shapes(dev, orc, K):
    """K = 2048 n + 512 t: the 2048-chunk GEMV with a partial last chunk
    (the reference model's hidden size 2560 among them)."""
    say(f"decode GEMV tail shapes K={K}")
    rng = np.random.default_rng(K)
    E, I, k = 16, 256, 4
    w, s, b = synth.quant_weights(rng, (E, 2 * I), K)
    x = synth.bf16_bits(rng.normal(size=(2, K)).astype(np.float32))
    idx = np.stack([rng.choice(E, k, replace=False) for _ in range(2)]).astype(np.int32)
    h = ops.gate_up_silu(bf16_t(x, dev), words_t(w, dev), bf16_t(s, dev), bf16_t(b, dev), i32_t(idx, dev))
    gu64, _ = orc.gather_qmm_rows(x, np.repeat(np.arange(2), k).astype(np.int32), idx.reshape(-1), w, s, b)
    h64, _ = orc.swiglu(gu64)
    assert_close_bf16(orc, bits(h).reshape(2 * k, I), h64, what=f"gate_up K={K}")
    xr = rng.integers(0, 2, size=9).astype(np.int32)
    ex = rng.integers(0, E, size=9).astype(np.int32)
    y = ops.gather_qmv(bf16_t(x, dev), i32_t(xr, dev), i32_t(ex, dev), words_t(w, dev), bf16_t(s, dev),
                       bf16_t(b, dev))
    ref64, _ = orc.gather_qmm_rows(x, xr, ex, w, s, b)
    assert_close_bf16(orc, bits(y), ref64, what=f"gather_qmv K={K}")
    yq = ops.quantized_matmul(bf16_t(x, dev), words_t(w[0], dev), bf16_t(s[0], dev), bf16_t(b[0], dev))
    refq, _ = orc.gather_qmm_rows(x, None, np.zeros(2, np.int32), w[:1], s[:1], b[:1])
    assert_close_bf16(orc, bits(yq), refq, what=f"quantized_matmul K={K}")


# ------------------------------------- timed kernels at their timed shapes


def _prefill_routed(dev, orc, tokens, cfg=3):
    """A Zipf-routed prefill workload, routed on the device: (workload, routing,
    x_rows = order // k, host order, host sorted ids, host offsets)."""
    wl = synth.make(cfg, tokens=tokens)
    k = wl["idx"].shape[1]
    r = ops.route(i32_t(wl["idx"], dev), 256)
    lhs = torch.div(r.order, k, rounding_mode="floor").to(torch.int32)
    order, _, srt = orc.route_sort(wl["idx"], 256)
    off = np.searchsorted(srt, np.arange(257), side="left")
    return wl, r, lhs, order, srt, off


@pytest.mark.parametrize("tokens", [4096, 8192])
def test_sorted_gemm_tiles_prefill_sampled(dev, orc, tokens):
    """The tile-layout grouped GEMM the bench times for workload 3, at its
    full size (4096 tokens, 479 tiles) and at 8192 tokens, where the tile
    count passes the 512 the heavy-first ranking holds and the kernel walks
    tiles in table order."""
    say(f"sorted GEMM tiles, {tokens} tokens x top-10 Zipf, sampled rows")
    wl, r, lhs, order, srt, off = _prefill_routed(dev, orc, tokens)
    T, k = wl["idx"].shape
    nt = int(r.tiles.ntiles.item())
    assert (nt > 512) == (tokens == 8192), nt
    tw = ops.repack_tiles(words_t(wl["w"], dev), bf16_t(wl["s"], dev), bf16_t(wl["b"], dev))
    y = ops.gather_qmm_sorted_tiles(bf16_t(wl["x"], dev), tw, r.tiles, x_rows=lhs)
    torch.cuda.synchronize()
    rows = _sample_rows(off, T * k, 384, np.random.default_rng(tokens))
    ref64, _ = orc.gather_qmm_rows(wl["x"], (order[rows] // k).astype(np.int32), srt[rows], wl["w"], wl["s"],
                                   wl["b"], deq="bf16")
    assert_close_bf16(orc, bits(y)[rows], ref64, what=f"gemm tiles {tokens} tokens, {nt} tiles, {rows.size} rows")
    if tokens == 8192:
        # the MLX-layout kernel's unranked branch, same rows and summation order
        ym = ops.gather_qmm_sorted(bf16_t(wl["x"], dev), words_t(wl["w"], dev), bf16_t(wl["s"], dev),
                                   bf16_t(wl["b"], dev), r.tiles, x_rows=lhs)
        assert torch.equal(ym, y)


def test_grouped_gemms_repeat_and_replay(dev, orc):
    """Back-to-back calls of the grouped GEMMs on one tile table (bf16,
    SwiGLU, int8, as a block's projections share it) give identical results,
    and a captured graph of the GEMM replays to the eager result every time,
    with eager work on the same table between replays."""
    say("grouped GEMMs: repeat calls and graph replays")
    wl, r, lhs, order, srt, off = _prefill_routed(dev, orc, 1024)
    t = r.tiles
    xt = bf16_t(wl["x"], dev)
    tw = ops.repack_tiles(words_t(wl["w"], dev), bf16_t(wl["s"], dev), bf16_t(wl["b"], dev))
    twp = ops.repack_tiles(words_t(wl["w"], dev), bf16_t(wl["s"], dev), bf16_t(wl["b"], dev), swiglu_pairs=True)
    xi, sx = ops.quantize_act_int8(xt)
    runs = {
        "bf16": lambda: ops.gather_qmm_sorted_tiles(xt, tw, t, x_rows=lhs),
        "swiglu": lambda: ops.gather_qmm_swiglu_sorted_tiles(xt, twp, t, x_rows=lhs),
        "int8": lambda: ops.gather_qmm_int8_sorted_tiles(xi, sx, tw, t, x_rows=lhs),
    }
    first = {}
    for rep in range(3):
        for name, f in runs.items():
            y = f()
            torch.cuda.synchronize()
            if rep == 0:
                first[name] = y.clone()
            else:
                assert torch.equal(y, first[name]), (name, rep)
    rows = _sample_rows(off, int(wl["idx"].size), 128, np.random.default_rng(9))
    k = wl["idx"].shape[1]
    ref64, _ = orc.gather_qmm_rows(wl["x"], (order[rows] // k).astype(np.int32), srt[rows], wl["w"], wl["s"],
                                   wl["b"], deq="bf16")
    assert_close_bf16(orc, bits(first["bf16"])[rows], ref64, what="gemm tiles 1024 tokens")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        runs["bf16"]()  # warm the allocator off the capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        yg = runs["bf16"]()
    for rep in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(yg, first["bf16"]), rep
        runs["int8"]()  # eager work on the same table between replays
        torch.cuda.synchronize()


def test_grouped_gemm_many_launches_in_a_row(dev, orc):
    """150 launches of the bf16 grouped GEMM queued back to back (more than
    the kernel's 64 unit-queue slots, so every slot is reused, and each launch
    starts right after the previous one clears its slot) all give the first
    launch's output bit for bit: no unit is skipped or taken twice."""
    say("grouped GEMM: 150 launches in a row")
    wl, r, lhs, order, srt, off = _prefill_routed(dev, orc, 1024)
    t = r.tiles
    xt = bf16_t(wl["x"], dev)
    tw = ops.repack_tiles(words_t(wl["w"], dev), bf16_t(wl["s"], dev), bf16_t(wl["b"], dev))
    twp = ops.repack_tiles(words_t(wl["w"], dev), bf16_t(wl["s"], dev), bf16_t(wl["b"], dev), swiglu_pairs=True)
    ref = ops.gather_qmm_sorted_tiles(xt, tw, t, x_rows=lhs)
    ref_h = ops.gather_qmm_swiglu_sorted_tiles(xt, twp, t, x_rows=lhs)
    torch.cuda.synchronize()
    for batch in range(5):
        outs = []
        for i in range(30):
            if i % 3 == 2:
                outs.append(("swiglu", ops.gather_qmm_swiglu_sorted_tiles(xt, twp, t, x_rows=lhs)))
            else:
                outs.append(("bf16", ops.gather_qmm_sorted_tiles(xt, tw, t, x_rows=lhs)))
        torch.cuda.synchronize()
        for i, (kind, y) in enumerate(outs):
            assert torch.equal(y, ref if kind == "bf16" else ref_h), (batch, i, kind)
    rows = _sample_rows(off, int(wl["idx"].size), 128, np.random.default_rng(11))
    k = wl["idx"].shape[1]
    ref64, _ = orc.gather_qmm_rows(wl["x"], (order[rows] // k).astype(np.int32), srt[rows], wl["w"], wl["s"],
                                   wl["b"], deq="bf16")
    assert_close_bf16(orc, bits(ref)[rows], ref64, what="gemm tiles 1024 tokens, first launch")


@pytest.mark.parametrize("tokens", [4096, 8192])
def test_swiglu_gemm_tiles_prefill_sampled(dev, orc, tokens):
    """The SwiGLU-epilogue grouped GEMM (the block's prefill gate_up) at the
    workload-3 shape and past 512 tiles: h = silu(gate) * up against the
    fp64 closed form over bf16-dequantised weights."""
    say(f"SwiGLU GEMM tiles, {tokens} tokens x top-10 Zipf, sampled rows")
    wl, r, lhs, order, srt, off = _prefill_routed(dev, orc, tokens)
    T, k = wl["idx"].shape
    tw = ops.repack_tiles(words_t(wl["w"], dev), bf16_t(wl["s"], dev), bf16_t(wl["b"], dev), swiglu_pairs=True)
    h = ops.gather_qmm_swiglu_sorted_tiles(bf16_t(wl["x"], dev), tw, r.tiles, x_rows=lhs)
    torch.cuda.synchronize()
    assert h.shape == (T * k, 512)
    rows = _sample_rows(off, T * k, 256, np.random.default_rng(tokens + 1))
    gu64, _ = orc.gather_qmm_rows(wl["x"], (order[rows] // k).astype(np.int32), srt[rows], wl["w"], wl["s"],
                                  wl["b"], deq="bf16")
    h64, _ = orc.swiglu(gu64)
    assert_close_bf16(orc, bits(h)[rows], h64, what=f"swiglu gemm {tokens} tokens, {rows.size} rows")


def test_sorted_gemm_int8_tiles_past_512_tiles(dev, orc):
    """The int8 grouped GEMM over 8192 tokens (more than 512 tiles: tiles in
    table order), sampled rows against the fake-quant golden."""
    say("int8 sorted GEMM tiles, 8192 tokens, sampled rows")
    wl, r, lhs, order, srt, off = _prefill_routed(dev, orc, 8192, cfg=4)
    T, k = wl["idx"].shape
    assert int(r.tiles.ntiles.item()) > 512
    xi, sx = ops.quantize_act_int8(bf16_t(wl["x"], dev))
    tw = ops.repack_tiles(words_t(wl["w"], dev), bf16_t(wl["s"], dev), bf16_t(wl["b"], dev))
    y = ops.gather_qmm_int8_sorted_tiles(xi, sx, tw, r.tiles, x_rows=lhs)
    torch.cuda.synchronize()
    rows = _sample_rows(off, T * k, 256, np.random.default_rng(3))
    rxi, rsx = orc.quant_act_int8(wl["x"])
    ref64, _ = orc.gather_qmm_int8_rows(rxi, rsx, (order[rows] // k).astype(np.int32), srt[rows], wl["w"],
                                        wl["s"], wl["b"])
    assert_close_bf16(orc, bits(y)[rows], ref64, what=f"int8 gemm 8192 tokens, {rows.size} rows")


@pytest.mark.parametrize("gs", [32, 128])
def test_fused_decode_group_sizes(dev, orc, gs):
    """The fused decode kernels (gate_up + SwiGLU, down + weighted sum) with
    group sizes 32 and 128 at the workload shapes: the reference's fused decode
    path takes group 64 and 128 (engine/patches/decode-fusion/kernel.py:50-60)."""
    say(f"fused decode gate_up / down group_size={gs}")
    rng = np.random.default_rng(gs)
    E, I, K, T, k = 256, 512, 2048, 3, 10
    w, s, b = synth.quant_weights(rng, (E, 2 * I), K, group_size=gs)
    x = synth.bf16_bits(rng.normal(size=(T, K)).astype(np.float32))
    idx = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    h = ops.gate_up_silu(bf16_t(x, dev), words_t(w, dev), bf16_t(s, dev), bf16_t(b, dev), i32_t(idx, dev),
                         group_size=gs)
    gu64, _ = orc.gather_qmm_rows(x, np.repeat(np.arange(T), k).astype(np.int32), idx.reshape(-1), w, s, b,
                                  group_size=gs)
    h64, _ = orc.swiglu(gu64)
    assert_close_bf16(orc, bits(h).reshape(T * k, I), h64, what=f"gate_up gs{gs}")
    wd, sd, bd = synth.quant_weights(rng, (E, K), I, group_size=gs)
    sc = synth.softmax(rng.normal(size=(T, k)))
    for TT in (1, T):  # one token: the 8-row variant; more: the 16-row one
        y = ops.down_wsum(h[:TT], words_t(wd, dev), bf16_t(sd, dev), bf16_t(bd, dev), i32_t(idx[:TT], dev),
                          f32_t(sc[:TT], dev), group_size=gs)
        y64, _ = orc.down_wsum(bits(h[:TT]), idx[:TT], sc[:TT], wd, sd, bd, group_size=gs)
        assert_close_bf16(orc, bits(y), y64, what=f"down gs{gs} T={TT}")


@pytest.mark.parametrize("k,K,gs", [(10, 2048, 64), (9, 2048, 64), (10, 2048, 32), (9, 2048, 128),
                                    (10, 4096, 64), (10, 6144, 128), (9, 6144, 32), (9, 8192, 64),
                                    (10, 8192, 128)])
def test_gate_up_one_token_flat_waves(dev, orc, k, K, gs, monkeypatch):
    """One token's fused gate_up + SwiGLU runs on waves of five consecutive
    (pair, index) slots (qmv64_flat_kernel, four waves per workgroup: ten
    experts x 512 indices make 1024 waves, some spanning two experts; k = 9
    leaves a partial last wave and a workgroup with waves past the list).
    QMOE_DECODE_FLAT=1 takes that kernel whatever the part's SIMD count, =0 the
    four-index waves; the same token given twice also takes the four-index
    waves.  All must match bit for bit and stay within the bar of the oracle."""
    say(f"gate_up one token flat waves k={k} K={K} gs={gs}")
    rng = np.random.default_rng(1000 + k + K + gs)
    E, I = (256 if K <= 4096 else 32), 512
    w, s, b = synth.quant_weights(rng, (E, 2 * I), K, group_size=gs)
    x = synth.bf16_bits(rng.normal(size=(1, K)).astype(np.float32))
    idx = rng.choice(E, k, replace=False).astype(np.int32)[None]
    wt, st, bt = words_t(w, dev), bf16_t(s, dev), bf16_t(b, dev)
    monkeypatch.setenv("QMOE_DECODE_FLAT", "1")
    h1 = ops.gate_up_silu(bf16_t(x, dev), wt, st, bt, i32_t(idx, dev), group_size=gs)
    monkeypatch.setenv("QMOE_DECODE_FLAT", "0")
    h0 = ops.gate_up_silu(bf16_t(x, dev), wt, st, bt, i32_t(idx, dev), group_size=gs)
    monkeypatch.delenv("QMOE_DECODE_FLAT")
    h2 = ops.gate_up_silu(bf16_t(np.repeat(x, 2, axis=0), dev), wt, st, bt, i32_t(np.repeat(idx, 2, axis=0), dev),
                          group_size=gs)
    assert torch.equal(h1, h0) and torch.equal(h1[0], h2[0]) and torch.equal(h2[0], h2[1])
    gu64, _ = orc.gather_qmm_rows(x, np.zeros(k, np.int32), idx.reshape(-1), w, s, b, group_size=gs)
    h64, _ = orc.swiglu(gu64)
    assert_close_bf16(orc, bits(h1).reshape(k, I), h64, what=f"gate_up flat k={k} K={K} gs{gs}")


@pytest.mark.parametrize("T,E,D", [(1, 256, 2048), (3, 64, 2048), (8, 256, 2048), (16, 32, 192)])
def test_down_wsum_tiles_matches_mlx_layout(dev, orc, T, E, D):
    """The fused down + weighted sum over tile-layout down weights: bit-identical
    to the MLX-layout kernel (the same 32 codes per lane, the same reduction)
    and within the bar of the oracle."""
    say(f"down + weighted sum tiles T={T} E={E} D={D}")
    wl = synth.make(2, seed=300 + T, tokens=T, experts=E)
    if D != 2048:
        rng = np.random.default_rng(D)
        w, s_, b = synth.quant_weights(rng, (E, D), 512)
    else:
        w, s_, b = wl["w"], wl["s"], wl["b"]
    tw = ops.repack_tiles(words_t(w, dev), bf16_t(s_, dev), bf16_t(b, dev))
    h, idx, sc = bf16_t(wl["h"], dev), i32_t(wl["idx"], dev), f32_t(wl["scores"], dev)
    yt = ops.down_wsum_tiles(h, tw, idx, sc)
    ym = ops.down_wsum(h, words_t(w, dev), bf16_t(s_, dev), bf16_t(b, dev), idx, sc)
    assert torch.equal(yt, ym)
    y64, _ = orc.down_wsum(wl["h"], wl["idx"], wl["scores"], w, s_, b)
    assert_close_bf16(orc, bits(yt), y64, what=f"down tiles T={T}")
