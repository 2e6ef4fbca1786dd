"""Write the golden fixtures of tests/golden/ from the oracle.

    python tests/golden/make_golden.py

Each fixture is a small .npz (inputs and expected outputs, no pickles) for
one function of the path.  The expected outputs come from the C oracle; the
tests re-derive them (to catch a drifting oracle) and run the HIP path on the
same inputs.  Inputs are seeded (numpy PCG64), so re-running this script
reproduces the files bit for bit.
"""

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "oracle"))

import oracle  # noqa: E402
from titan_amd import synth  # noqa: E402


def _save(name, **arrays):
    np.savez_compressed(HERE / f"{name}.npz", **arrays)


def unpack_dequant():
    rng = np.random.default_rng(11)
    w, s, b = synth.quant_weights(rng, (3, 32), 128)
    codes = oracle.unpack(w.reshape(-1), 4).reshape(3, 32, 128)
    deq = oracle.dequantize_bf16(w, s, b, 64, 4).reshape(3, 32, 128)
    _save("unpack_dequant", w=w, s=s, b=b, codes=codes, deq=deq)


def gather_sorted():
    rng = np.random.default_rng(12)
    E, N, K, R = 4, 256, 256, 64
    w, s, b = synth.quant_weights(rng, (E, N), K)
    ids = np.sort(rng.integers(0, E, size=R)).astype(np.int32)
    x = synth.bf16_bits(rng.normal(size=(R, K)).astype(np.float32))
    # materialised bf16 weights (the grouped GEMM) and the exact affine form (the GEMV)
    y64, y16 = oracle.gather_qmm_rows(x, None, ids, w, s, b, deq="bf16")
    e64, _ = oracle.gather_qmm_rows(x, None, ids, w, s, b, deq="exact")
    _save("gather_sorted", w=w, s=s, b=b, ids=ids, x=x, y64=y64, y16=y16, e64=e64)


def decode_gate_up():
    rng = np.random.default_rng(13)
    E, I, K, k = 8, 64, 256, 4
    w, s, b = synth.quant_weights(rng, (E, 2 * I), K)
    idx = rng.permutation(E)[:k].astype(np.int32).reshape(1, k)
    x = synth.bf16_bits(rng.normal(size=(1, K)).astype(np.float32))
    gu64, _ = oracle.gather_qmm_rows(x, np.zeros(k, np.int32), idx.reshape(-1), w, s, b, deq="exact")
    h64, _ = oracle.swiglu(gu64)
    _save("decode_gate_up", w=w, s=s, b=b, idx=idx, x=x, h64=h64.reshape(1, k, I))


def route():
    rng = np.random.default_rng(14)
    E, n, tr = 8, 45, 8
    ids = rng.integers(0, E, size=n).astype(np.int32)
    ids[ids == 5] = 6  # an empty expert
    order, inv, srt = oracle.route_sort(ids, E)
    offsets, trow, texp, nt = oracle.build_tiles(srt, E, tr)
    _save("route", ids=ids, tile_rows=np.int32(tr), order=order, inv=inv, sorted=srt, offsets=offsets,
          tile_row=trow, tile_exp=texp, ntiles=np.int32(nt))


def weighted_sum():
    rng = np.random.default_rng(15)
    rows, k, D = 3, 10, 64
    xs = synth.bf16_bits(rng.normal(size=(rows * k, D)).astype(np.float32))
    inv = rng.permutation(rows * k).astype(np.int32)
    sc = rng.random((rows, k)).astype(np.float32)
    sc /= sc.sum(1, keepdims=True)
    out = {m: np.asarray(oracle.weighted_sum(xs, inv, sc, rows, k, D, m)).reshape(rows, D)
           for m in ("clone", "ops", "fast")}
    _save("weighted_sum", xs=xs, inv=inv, scores=sc, clone=out["clone"], ops=out["ops"], fast=out["fast"])


def int8():
    rng = np.random.default_rng(16)
    E, N, K, R = 2, 256, 1024, 40
    w, s, b = synth.quant_weights(rng, (E, N), K)
    xf = rng.normal(size=(R, K)).astype(np.float32)
    xf[rng.random((R, K)) < 0.001] *= 20
    x = synth.bf16_bits(xf)
    xi, sx = oracle.quant_act_int8(x)
    ids = np.sort(rng.integers(0, E, size=R)).astype(np.int32)
    y64, _ = oracle.gather_qmm_int8_rows(xi, sx, None, ids, w, s, b)
    _save("int8", w=w, s=s, b=b, x=x, xi=xi, sx=sx, ids=ids, y64=y64)


if __name__ == "__main__":
    oracle.build()
    for f in (unpack_dequant, gather_sorted, decode_gate_up, route, weighted_sum, int8):
        f()
        print("wrote", f.__name__)
