"""Pins the oracle's gather_qmm, SwiGLU, fused down + weighted sum and int8
goldens.

Expected values come from numpy/float64 compositions built from numpy bit
operations (not the oracle's unpack), closed forms (bias-only weights,
scaling by two), and invariants (row-permutation equivariance, dense
reduction at E = 1).  A transposed operand, a swapped nibble order or a
dropped bias term each fails one of these.
"""

import numpy as np
import pytest

from titan_amd import synth


def np_dequant(w, s, b, gs=64, bits=4, bf16=False):
    """float64 weights [..., N, K] from packed words by numpy shifts."""
    per = 32 // bits
    mask = (1 << bits) - 1
    q = np.stack([(w >> (bits * t)) & mask for t in range(per)], axis=-1).reshape(*w.shape[:-1], -1)
    K = q.shape[-1]
    g = np.arange(K) // gs
    sf = synth.bf16_to_f32(s).astype(np.float64)[..., g]
    bf = synth.bf16_to_f32(b).astype(np.float64)[..., g]
    W = q.astype(np.float64) * sf + bf
    if bf16:
        W = synth.bf16_to_f32(synth.bf16_bits(W.astype(np.float32))).astype(np.float64)
    return W


def xf(x):
    return synth.bf16_to_f32(x).astype(np.float64)


@pytest.fixture(scope="module")
def problem():
    rng = np.random.default_rng(10)
    E, N, K, R = 5, 48, 256, 17
    w, s, b = synth.quant_weights(rng, (E, N), K)
    x = synth.bf16_bits(rng.normal(size=(9, K)).astype(np.float32))
    xr = rng.integers(0, 9, size=R).astype(np.int32)
    ex = rng.integers(0, E, size=R).astype(np.int32)
    return w, s, b, x, xr, ex


@pytest.mark.parametrize("deq", ["exact", "bf16"])
def test_gather_rows_matches_numpy(orc, problem, deq):
    w, s, b, x, xr, ex = problem
    got, got16 = orc.gather_qmm_rows(x, xr, ex, w, s, b, deq=deq)
    W = np_dequant(w, s, b, bf16=deq == "bf16")
    want = np.einsum("rk,rnk->rn", xf(x)[xr], W[ex])
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)
    assert np.array_equal(got16, orc.bf16_from_f64(got))


def test_dense_reduction_at_one_expert(orc):
    rng = np.random.default_rng(11)
    w, s, b = synth.quant_weights(rng, (64,), 512)
    x = synth.bf16_bits(rng.normal(size=(3, 512)).astype(np.float32))
    got, _ = orc.gather_qmm_rows(x, None, np.zeros(3, np.int32), w[None], s[None], b[None])
    np.testing.assert_allclose(got, xf(x) @ np_dequant(w, s, b).T, rtol=1e-12)


def test_bias_only_weights(orc):
    """q == 0 everywhere: y[n] = sum_g b[n,g] * sum_{k in g} x[k]."""
    rng = np.random.default_rng(12)
    N, K = 32, 256
    _, s, b = synth.quant_weights(rng, (N,), K)
    w = np.zeros((N, K // 8), np.uint32)
    x = synth.bf16_bits(rng.normal(size=(2, K)).astype(np.float32))
    got, _ = orc.gather_qmm_rows(x, None, np.zeros(2, np.int32), w[None], s[None], b[None])
    xs = xf(x).reshape(2, K // 64, 64).sum(-1)
    want = xs @ synth.bf16_to_f32(b).astype(np.float64).T
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-13)


def test_scaling_and_permutation(orc, problem):
    w, s, b, x, xr, ex = problem
    base, _ = orc.gather_qmm_rows(x, xr, ex, w, s, b)
    x2 = synth.bf16_bits(2 * synth.bf16_to_f32(x))
    twice, _ = orc.gather_qmm_rows(x2, xr, ex, w, s, b)
    np.testing.assert_array_equal(twice, 2 * base)
    perm = np.random.default_rng(0).permutation(xr.size)
    p, _ = orc.gather_qmm_rows(x, xr[perm], ex[perm], w, s, b)
    np.testing.assert_array_equal(p, base[perm])


def test_swapped_nibble_order_is_detected(orc, problem):
    """The plausible packing mistake (high nibble first) moves the result."""
    w, s, b, x, xr, ex = problem
    swapped = ((w & 0x0F0F0F0F) << 4) | ((w >> 4) & 0x0F0F0F0F)
    a, _ = orc.gather_qmm_rows(x, xr, ex, w, s, b)
    c, _ = orc.gather_qmm_rows(x, xr, ex, swapped.astype(np.uint32), s, b)
    assert np.abs(a - c).max() > 1e-3


def test_swiglu_closed_form(orc):
    rng = np.random.default_rng(13)
    gu = rng.normal(size=(6, 2 * 40)) * 3
    h64, h16 = orc.swiglu(gu)
    g, u = gu[:, :40], gu[:, 40:]
    np.testing.assert_allclose(h64, g / (1 + np.exp(-g)) * u, rtol=1e-14)
    assert np.array_equal(h16, orc.bf16_from_f64(h64))


def test_down_wsum_matches_composition(orc):
    rng = np.random.default_rng(14)
    E, D, I, T, k = 12, 40, 128, 3, 4
    w, s, b = synth.quant_weights(rng, (E, D), I)
    h = synth.bf16_bits(rng.normal(size=(T, k, I)).astype(np.float32))
    idx = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    sc = synth.softmax(rng.normal(size=(T, k)))
    y64, _ = orc.down_wsum(h, idx, sc, w, s, b)
    W = np_dequant(w, s, b)
    want = np.zeros((T, D))
    for t in range(T):
        for j in range(k):
            want[t] += float(sc[t, j]) * (W[idx[t, j]] @ xf(h[t, j]))
    np.testing.assert_allclose(y64, want, rtol=1e-12, atol=1e-12)


def test_quant_act_int8_matches_numpy_float32(orc):
    wl = synth.make(4, tokens=64)
    x = wl["x"].copy()
    x[5] = 0
    xi, sx = orc.quant_act_int8(x)
    f = synth.bf16_to_f32(x)
    amax = np.abs(f).max(-1)
    want_sx = (amax / np.float32(127)).astype(np.float32)
    assert np.array_equal(sx.view(np.uint32), want_sx.view(np.uint32))
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.rint(f / want_sx[:, None])
    q = np.where(want_sx[:, None] == 0, 0, np.clip(q, -127, 127))
    assert np.array_equal(xi, q.astype(np.int8))
    nz = amax > 0
    assert np.all(np.abs(xi[nz].astype(np.int32)).max(-1) == 127)
    assert sx[5] == 0 and not xi[5].any()


def test_int8_golden_is_fake_quant(orc):
    rng = np.random.default_rng(15)
    E, N, K, R = 4, 32, 256, 9
    w, s, b = synth.quant_weights(rng, (E, N), K)
    x = synth.bf16_bits(rng.normal(size=(R, K)).astype(np.float32))
    xi, sx = orc.quant_act_int8(x)
    ex = rng.integers(0, E, size=R).astype(np.int32)
    got, _ = orc.gather_qmm_int8_rows(xi, sx, None, ex, w, s, b)
    xhat = xi.astype(np.float64) * sx.astype(np.float64)[:, None]
    want = np.einsum("rk,rnk->rn", xhat, np_dequant(w, s, b)[ex])
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("bits,gs", [(8, 32), (8, 64), (8, 128), (4, 32), (4, 128)])
@pytest.mark.parametrize("deq", ["exact", "bf16"])
def test_gather_rows_other_widths_and_groups(orc, bits, gs, deq):
    """8-bit codes (4 per word, low byte first) and group sizes 32 / 128
    against the numpy shift-based dequant."""
    rng = np.random.default_rng(bits * 1000 + gs)
    E, N, K, R = 3, 24, 512, 11
    w, s, b = synth.quant_weights(rng, (E, N), K, group_size=gs, bits=bits)
    x = synth.bf16_bits(rng.normal(size=(5, K)).astype(np.float32))
    xr = rng.integers(0, 5, size=R).astype(np.int32)
    ex = rng.integers(0, E, size=R).astype(np.int32)
    got, _ = orc.gather_qmm_rows(x, xr, ex, w, s, b, group_size=gs, bits=bits, deq=deq)
    W = np_dequant(w, s, b, gs=gs, bits=bits, bf16=deq == "bf16")
    want = np.einsum("rk,rnk->rn", xf(x)[xr], W[ex])
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)
    # the 8-bit byte order: a wrong (high byte first) order moves the result
    if bits == 8:
        swapped = ((w & 0x00FF00FF) << 8) | ((w >> 8) & 0x00FF00FF)
        bad, _ = orc.gather_qmm_rows(x, xr, ex, swapped, s, b, group_size=gs, bits=bits, deq=deq)
        assert np.abs(bad - want).max() > 1e-3
