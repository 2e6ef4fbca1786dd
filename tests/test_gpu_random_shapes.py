"""Seeded random shapes for the grouped GEMMs against the oracle: expert
counts, column counts and K drawn from each kernel's envelope, rows routed
uniformly, Zipf-skewed, onto one expert or with empty experts, and gathered
through x_rows -- the combinations the hand-picked cases do not pin down."""

import numpy as np
import pytest
import torch

from helpers import assert_close_bf16, bf16_t, bits, i32_t, words_t
from titan_amd import ops, synth

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[case] {msg}", flush=True)


def _case(seed):
    rng = np.random.default_rng(1000 + seed)
    E = int(rng.choice([1, 3, 17, 64, 256]))
    N = int(256 * rng.integers(1, 7))
    K = int(128 * rng.integers(1, 17))
    R = int(rng.integers(64, 2500))
    kind = ["uniform", "zipf", "one", "sparse"][seed % 4]
    w, s, b = synth.quant_weights(rng, (E, N), K)
    if kind == "one":
        ids = np.full(R, E - 1, np.int32)
    elif kind == "zipf":
        p = 1.0 / np.arange(1, E + 1) ** 1.2
        ids = rng.choice(E, size=R, p=p / p.sum()).astype(np.int32)
    elif kind == "sparse":  # most experts empty
        live = rng.choice(E, size=max(1, E // 8), replace=False)
        ids = rng.choice(live, size=R).astype(np.int32)
    else:
        ids = rng.integers(0, E, size=R).astype(np.int32)
    ids = np.sort(ids).astype(np.int32)
    T = int(rng.integers(1, R + 1))
    x_rows = rng.integers(0, T, size=R).astype(np.int32)  # rows gathered from a [T, K] matrix
    x = synth.bf16_bits(rng.normal(size=(T, K)).astype(np.float32))
    return dict(E=E, N=N, K=K, R=R, T=T, kind=kind, w=w, s=s, b=b, ids=ids, x=x, x_rows=x_rows)


@pytest.mark.parametrize("seed", range(12))
def test_grouped_gemms_random_shapes(dev, orc, seed):
    c = _case(seed)
    say(f"random grouped GEMM seed={seed}: E={c['E']} N={c['N']} K={c['K']} R={c['R']} T={c['T']} {c['kind']}")
    wt, st, bt = words_t(c["w"], dev), bf16_t(c["s"], dev), bf16_t(c["b"], dev)
    xt, xr = bf16_t(c["x"], dev), i32_t(c["x_rows"], dev)
    tiles = ops.build_tiles(i32_t(c["ids"], dev), c["E"])
    tw = ops.repack_tiles(wt, st, bt)
    y_t = ops.gather_qmm_sorted_tiles(xt, tw, tiles, x_rows=xr)
    y_m = ops.gather_qmm_sorted(xt, wt, st, bt, tiles, x_rows=xr)
    torch.cuda.synchronize()
    ref, _ = orc.gather_qmm_rows(c["x"], c["x_rows"], c["ids"], c["w"], c["s"], c["b"], deq="bf16")
    assert_close_bf16(orc, bits(y_t), ref, what=f"tiles seed {seed}")
    # the two layouts feed the same MFMAs in the same order
    assert torch.equal(y_t, y_m)
    if c["K"] % 512 == 0 and c["K"] <= 4096:
        xi, sx = ops.quantize_act_int8(xt)
        y8 = ops.gather_qmm_int8_sorted_tiles(xi, sx, tw, tiles, x_rows=xr)
        torch.cuda.synchronize()
        rxi, rsx = orc.quant_act_int8(c["x"])
        ref8, _ = orc.gather_qmm_int8_rows(rxi, rsx, c["x_rows"], c["ids"], c["w"], c["s"], c["b"])
        assert_close_bf16(orc, bits(y8), ref8, what=f"int8 seed {seed}")


@pytest.mark.parametrize("seed", range(6))
def test_swiglu_gemm_random_shapes(dev, orc, seed):
    c = _case(100 + seed)
    say(f"random SwiGLU GEMM seed={seed}: E={c['E']} N={c['N']} K={c['K']} R={c['R']} {c['kind']}")
    wt, st, bt = words_t(c["w"], dev), bf16_t(c["s"], dev), bf16_t(c["b"], dev)
    tiles = ops.build_tiles(i32_t(c["ids"], dev), c["E"])
    twp = ops.repack_tiles(wt, st, bt, swiglu_pairs=True)
    h = ops.gather_qmm_swiglu_sorted_tiles(bf16_t(c["x"], dev), twp, tiles, x_rows=i32_t(c["x_rows"], dev))
    torch.cuda.synchronize()
    gu, _ = orc.gather_qmm_rows(c["x"], c["x_rows"], c["ids"], c["w"], c["s"], c["b"], deq="bf16")
    h64, _ = orc.swiglu(gu)
    assert_close_bf16(orc, bits(h), h64, what=f"swiglu seed {seed}")
