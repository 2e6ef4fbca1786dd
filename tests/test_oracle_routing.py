"""Pins the oracle's routing (stable sort, inverse, offsets, tile list) and
weighted-sum modes.

Routing is checked against numpy's stable argsort and searchsorted and
against structural properties of the tile list (coverage, counts, order)
including the reference's special cases (one expert takes every row,
uniform routing, empty experts: tests/kernels/test_moe_gather_ws.py:67-89).
The weighted sum is checked against the same arithmetic carried out by
torch's bf16 ops where a closed form exists (k <= 8 and k = 10), and against
float64 for the fp32 mode.
"""

import numpy as np
import pytest
import torch

from titan_amd import synth


def check_tiles(ids_sorted, E, TM, off, trow, texp, nt):
    n = ids_sorted.size
    assert np.array_equal(off, np.searchsorted(ids_sorted, np.arange(E + 1), side="left"))
    counts = np.diff(off)
    assert nt == int(np.sum((counts + TM - 1) // TM))
    seen = []
    for t in range(nt):
        e, r0 = texp[t], trow[t]
        assert off[e] <= r0 < off[e + 1]
        assert (r0 - off[e]) % TM == 0
        seen.append((e, r0))
    assert seen == sorted(seen), "tiles must be expert-major, rows ascending"
    covered = np.zeros(n, np.int32)
    for e, r0 in seen:
        covered[r0:min(r0 + TM, off[e + 1])] += 1
    assert np.all(covered == 1)
    assert not trow[nt:].any() and not texp[nt:].any()


@pytest.mark.parametrize("case", ["zipf", "one", "uniform", "empty-experts", "single"])
def test_route_and_tiles(orc, case):
    rng = np.random.default_rng(20)
    E, TM = 32, 48
    if case == "zipf":
        ids = synth.make(3, tokens=300, experts=E)["idx"]
    elif case == "one":
        ids = np.zeros(256, np.int32)
    elif case == "uniform":
        ids = rng.integers(0, E, size=200).astype(np.int32)
    elif case == "empty-experts":
        ids = rng.choice([3, 9, 30], size=150).astype(np.int32)
    else:
        ids = np.array([5], np.int32)
    order, inv, srt = orc.route_sort(ids, E)
    flat = ids.reshape(-1)
    assert np.array_equal(order, np.argsort(flat, kind="stable"))
    assert np.array_equal(inv, np.argsort(order, kind="stable"))
    assert np.array_equal(srt, flat[order])
    off, trow, texp, nt = orc.build_tiles(srt, E, TM)
    check_tiles(srt, E, TM, off, trow, texp, nt)


def test_route_rejects_out_of_range(orc):
    with pytest.raises(ValueError):
        orc.route_sort(np.array([0, 8], np.int32), 8)


def test_tiles_for_one_heavy_expert(orc):
    ids = np.zeros(1000, np.int32)
    off, trow, texp, nt = orc.build_tiles(ids, 8, 128)
    assert nt == 8 and trow[:8].tolist() == list(range(0, 1000, 128)) and not texp[:8].any()
    assert off.tolist() == [0] + [1000] * 8


def t16(a):
    return torch.from_numpy(np.asarray(a, np.uint16).view(np.int16)).view(torch.bfloat16)


def torch_clone_reference(xs, inv, sc, rows, k, dim):
    """The clone-mode sequence (titan/kernels/moe_weighted_sum.py:71-96) on
    torch bf16 tensors: every product and sum rounds to bf16 in torch."""
    src = np.arange(rows * k) if inv is None else inv
    x = t16(xs)[torch.from_numpy(src.astype(np.int64))].reshape(rows, k, dim)
    s = torch.from_numpy(sc.reshape(rows, k)).to(torch.bfloat16)
    prods = x * s[:, :, None]
    acc = [torch.zeros(rows, dim, dtype=torch.bfloat16) for _ in range(8)]
    for j in range(k):
        acc[j % 8] = acc[j % 8] + prods[:, j]
    a = acc[0]
    for j in range(1, 8):
        a = a + acc[j]
    return a.view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("k", [1, 6, 8, 10])
@pytest.mark.parametrize("permuted", [False, True])
def test_weighted_sum_clone_matches_torch_bf16(orc, k, permuted):
    rng = np.random.default_rng(k)
    rows, dim = 7, 96
    xs = synth.bf16_bits(rng.normal(size=(rows * k, dim)).astype(np.float32))
    sc = rng.uniform(size=(rows, k)).astype(np.float32)
    inv = rng.permutation(rows * k).astype(np.int32) if permuted else None
    got = orc.weighted_sum(xs, inv, sc, rows, k, dim, "clone")
    assert np.array_equal(got, torch_clone_reference(xs, inv, sc, rows, k, dim))


def test_weighted_sum_fast_and_ops_near_float64(orc):
    rng = np.random.default_rng(30)
    rows, k, dim = 16, 10, 128
    xs = synth.bf16_bits(rng.normal(size=(rows * k, dim)).astype(np.float32))
    sc = synth.softmax(rng.normal(size=(rows, k)))
    inv = rng.permutation(rows * k).astype(np.int32)
    exact = np.einsum("rk,rkd->rd", sc.astype(np.float64),
                      synth.bf16_to_f32(xs)[inv].reshape(rows, k, dim).astype(np.float64))
    for mode, tol in (("fast", 2.0 ** -8), ("ops", 2.0 ** -6)):
        got = synth.bf16_to_f32(orc.weighted_sum(xs, inv, sc, rows, k, dim, mode)).astype(np.float64)
        assert np.abs(got - exact).max() <= tol * np.abs(exact).max()


def test_weighted_sum_identity_permutation(orc):
    rng = np.random.default_rng(31)
    rows, k, dim = 5, 10, 64
    xs = synth.bf16_bits(rng.normal(size=(rows * k, dim)).astype(np.float32))
    sc = rng.uniform(size=(rows, k)).astype(np.float32)
    for mode in ("fast", "ops", "clone"):
        a = orc.weighted_sum(xs, None, sc, rows, k, dim, mode)
        b = orc.weighted_sum(xs, np.arange(rows * k, dtype=np.int32), sc, rows, k, dim, mode)
        assert np.array_equal(a, b)
