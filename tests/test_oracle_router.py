"""Pins the oracle's router top-k (a14) without the reference: against a
numpy restatement by stable sort, the softmax closed form, the invariants the
scores must satisfy, and a planted tie."""

import numpy as np
import pytest


def _np_topk(lg, k, norm):
    # stable sort on -logit: larger first, equal logits by lower index
    order = np.argsort(-lg.astype(np.float64), axis=-1, kind="stable")[:, :k]
    top = np.take_along_axis(lg.astype(np.float64), order, axis=-1)
    if norm:
        p = np.exp(top - top[:, :1])
        sc = p / p.sum(-1, keepdims=True)
    else:
        m = lg.max(-1, keepdims=True).astype(np.float64)
        sc = np.exp(top - m) / np.exp(lg.astype(np.float64) - m).sum(-1, keepdims=True)
    return order.astype(np.int32), sc


@pytest.mark.parametrize("T,E,k", [(1, 256, 10), (37, 256, 10), (8, 128, 8), (5, 512, 4), (3, 64, 64)])
@pytest.mark.parametrize("norm", [True, False])
def test_router_topk_matches_stable_sort(orc, T, E, k, norm):
    rng = np.random.default_rng(T * 131 + E + k)
    lg = rng.normal(size=(T, E)).astype(np.float32)
    idx, sc = orc.router_topk(lg, k, norm)
    ridx, rsc = _np_topk(lg, k, norm)
    assert np.array_equal(idx, ridx)
    np.testing.assert_allclose(sc, rsc, rtol=1e-12, atol=0)


def test_router_topk_ties_take_lower_index(orc):
    lg = np.zeros((2, 16), np.float32)
    lg[0, [3, 7, 9]] = 1.0       # three-way tie at the top
    lg[1, :] = 0.5               # everything tied
    idx, sc = orc.router_topk(lg, 4, True)
    assert idx[0].tolist() == [3, 7, 9, 0]
    assert idx[1].tolist() == [0, 1, 2, 3]
    np.testing.assert_allclose(sc[1], 0.25, rtol=0, atol=1e-15)


def test_router_topk_scores_are_renormalised_softmax(orc):
    rng = np.random.default_rng(3)
    lg = rng.normal(size=(16, 256)).astype(np.float32) * 3
    idx, sn = orc.router_topk(lg, 10, True)
    _, sa = orc.router_topk(lg, 10, False)
    # norm: sums to one, descending, and proportional to the full softmax's top-k
    np.testing.assert_allclose(sn.sum(-1), 1.0, rtol=0, atol=1e-12)
    assert np.all(np.diff(sn, axis=-1) <= 0)
    np.testing.assert_allclose(sn, sa / sa.sum(-1, keepdims=True), rtol=1e-12)
    # the softmax over all experts, restricted: full softmax computed independently
    full = np.exp(lg.astype(np.float64) - lg.max(-1, keepdims=True))
    full /= full.sum(-1, keepdims=True)
    np.testing.assert_allclose(sa, np.take_along_axis(full, idx, -1), rtol=1e-12)
