"""The router top-k kernel, the SwiGLU-epilogue grouped GEMM and the whole
routed MoE block (titan_amd.moe_block) against the CPU oracle.

Bars: router indices exact (ties to the lower index) and scores within fp32
rounding of the float64 oracle; h and the block output within 1 bf16 ULP of
the fp64 golden chain on live elements (the rule of the other parity tests),
with the weights exact for the decode kernels and bf16-materialised for the
grouped GEMMs (the MLX qmv / qmm split).
The block is checked stage by stage: its expert selection against the oracle
on the GPU's own fp32 logits, then its output against an oracle chain that
takes the same selection, so a near-tie in routing cannot mask or fake an
arithmetic error.  The shared-expert branch adds two bf16 roundings (its
gated output, then the sum with the routed output) and is held to 2^-7 of
max|y| against the fp64 chain.
"""

import numpy as np
import pytest
import torch

from helpers import assert_close_bf16, bf16_t, bits, f32_t, words_t
from titan_amd import moe_block, ops, synth

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[case] {msg}", flush=True)


@pytest.mark.parametrize("T,E,k", [(1, 256, 10), (4096, 256, 10), (7, 512, 8), (5, 100, 6), (3, 64, 64)])
@pytest.mark.parametrize("norm", [True, False])
def test_router_topk_matches_oracle(dev, orc, T, E, k, norm):
    say(f"router top-k T={T} E={E} k={k} norm={norm}")
    rng = np.random.default_rng(T + E + k)
    lg = (rng.normal(size=(T, E)) * 2).astype(np.float32)
    idx, sc = ops.router_topk(f32_t(lg, dev), k, norm)
    ridx, rsc = orc.router_topk(lg, k, norm)
    assert np.array_equal(idx.cpu().numpy(), ridx)
    np.testing.assert_allclose(sc.cpu().numpy(), rsc, rtol=4e-6, atol=1e-7)


def test_router_topk_ties_take_lower_index(dev, orc):
    say("router top-k ties")
    lg = np.zeros((3, 256), np.float32)
    lg[0, [3, 70, 9]] = 1.0
    lg[1, :] = 0.5
    lg[2, 200:] = 2.0
    idx, sc = ops.router_topk(f32_t(lg, dev), 10, True)
    ridx, rsc = orc.router_topk(lg, 10, True)
    assert np.array_equal(idx.cpu().numpy(), ridx)
    assert idx[0, :4].tolist() == [3, 9, 70, 0]
    np.testing.assert_allclose(sc.cpu().numpy(), rsc, rtol=4e-6, atol=1e-7)


@pytest.mark.parametrize("E,k", [(64, 64), (100, 33), (256, 10), (256, 64), (512, 8), (1024, 64)])
def test_router_topk_many_ties(dev, orc, E, k):
    """Logits drawn from seven values (and signed zeros), so most rounds pick
    among equal logits held by several lanes and columns: ties go to the
    lower expert index."""
    say(f"router top-k, many ties, E={E} k={k}")
    rng = np.random.default_rng(E * 131 + k)
    T = 64
    lg = rng.integers(-3, 4, size=(T, E)).astype(np.float32)
    lg[T // 2:] = np.where(rng.random((T - T // 2, E)) < 0.5, -0.0, 0.0).astype(np.float32)
    for norm in (True, False):
        idx, sc = ops.router_topk(f32_t(lg, dev), k, norm)
        ridx, rsc = orc.router_topk(lg, k, norm)
        assert np.array_equal(idx.cpu().numpy(), ridx)
        np.testing.assert_allclose(sc.cpu().numpy(), rsc, rtol=4e-6, atol=1e-7)


@pytest.mark.parametrize("E", [100, 600])
def test_router_topk_nan_logits_rank_last(dev, E):
    """Logits are expected finite; a NaN ranks below every number: the
    choices are the finite logits in descending order (ties to the lower
    index), then the NaN entries in index order, and -0 ties with +0.  Pinned
    against a numpy sort of (-value, index) with NaN mapped below -inf."""
    say(f"router top-k with NaN logits E={E}")
    rng = np.random.default_rng(E)
    T, k = 3, 16
    lg = rng.normal(size=(T, E)).astype(np.float32)
    lg[0, [5, 17, 63]] = np.nan
    lg[1, :] = np.nan
    lg[1, [9, 2, 70]] = [1.0, 3.0, -np.inf]  # three numbers, then NaN in index order
    lg[2, :] = -np.abs(lg[2, :]) - 1.0
    lg[2, [8, 4]] = [-0.0, 0.0]  # signed zeros tie: index 4 first
    lg[2, [1, 3]] = [7.0, 7.0]
    idx, sc = ops.router_topk(f32_t(lg, dev), k, True)
    idx = idx.cpu().numpy()
    for t in range(T):
        v = lg[t].astype(np.float64)
        rank = np.where(np.isnan(v), -np.inf, v)
        order = np.lexsort((np.arange(E), np.isnan(v), -rank))  # finite first by value, NaN after, then index
        assert idx[t].tolist() == order[:k].tolist(), t
    assert idx[1, :3].tolist() == [2, 9, 70] and idx[1, 3:6].tolist() == [0, 1, 3]
    assert idx[2, :4].tolist() == [1, 3, 4, 8]
    assert np.all(np.isfinite(sc.cpu().numpy()[[0, 2]]))


def _assert_logits(got, ref64, absx_absw):
    """fp32 accumulation bound: |got - ref| <= 2^-14 * sum_k |x_k||w_k| per
    element, i.e. n * 2^-24 for n = 1024 sequential roundings.  The GEMV
    kernel's lane chains take K/512 + 8 of them; the tiled MFMA kernel's two
    accumulators K/32 steps of 16 products each (at most 5 roundings a step),
    plus one.  One dropped or doubled product moves a logit by ~1/K of that
    sum, 4x the bound and more for K <= 4096."""
    err = np.abs(got.astype(np.float64) - ref64)
    bound = 2.0 ** -14 * absx_absw
    print(f"[parity] logits max err/bound {np.max(err / bound):.3g}", flush=True)
    assert np.all(err <= bound)


@pytest.mark.parametrize("T,E,K", [
    # one wave per logit (T < 48, E < 32 or K % 128 != 0)
    (1, 256, 2048), (5, 128, 1024), (16, 512, 4096), (3, 64, 200), (47, 256, 2048), (500, 1, 2048),
    (400, 31, 256), (300, 64, 200),
    # tiled MFMA GEMM, 32 x 32 tiles (T >= 48, E >= 32, K % 128 == 0, fewer
    # than 128 tiles of 64 x 64), ragged tiles included
    (48, 32, 128), (300, 256, 2048), (1000, 200, 1024), (129, 1024, 4096), (77, 130, 384),
    # 64 x 64 tiles
    (4096, 256, 2048), (2050, 256, 2048), (8191, 100, 256)])
def test_router_logits_dense(dev, orc, T, E, K):
    say(f"router logits dense T={T} E={E} K={K}")
    rng = np.random.default_rng(T * E + K)
    x = synth.bf16_bits(rng.normal(size=(T, K)).astype(np.float32))
    w = synth.bf16_bits((rng.normal(size=(E, K)) * 0.05).astype(np.float32))
    got = ops.router_logits(bf16_t(x, dev), bf16_t(w, dev)).cpu().numpy()
    xf, wf = orc.f32_from_bf16(x).astype(np.float64), orc.f32_from_bf16(w).astype(np.float64)
    _assert_logits(got, xf @ wf.T, np.abs(xf) @ np.abs(wf).T)


@pytest.mark.parametrize("seed", range(8))
def test_router_logits_dense_random_shapes(dev, orc, seed):
    """Seeded random token and expert counts and K (a multiple of 8, half of
    them multiples of 128), so both kernels and both tile sizes of the tiled
    one meet ragged edges."""
    rng = np.random.default_rng(500 + seed)
    T = int(rng.integers(1, 3000))
    E = int(rng.integers(1, 600))
    K = int(128 * rng.integers(1, 24)) if seed % 2 == 0 else int(8 * rng.integers(1, 300))
    say(f"router logits dense random seed={seed}: T={T} E={E} K={K}")
    x = synth.bf16_bits(rng.normal(size=(T, K)).astype(np.float32))
    w = synth.bf16_bits((rng.normal(size=(E, K)) * 0.05).astype(np.float32))
    got = ops.router_logits(bf16_t(x, dev), bf16_t(w, dev)).cpu().numpy()
    xf, wf = orc.f32_from_bf16(x).astype(np.float64), orc.f32_from_bf16(w).astype(np.float64)
    _assert_logits(got, xf @ wf.T, np.abs(xf) @ np.abs(wf).T)


@pytest.mark.parametrize("nbits,gs", [(4, 64), (8, 64), (8, 32), (4, 128)])
def test_router_logits_quantized(dev, orc, nbits, gs):
    say(f"router logits quantized bits={nbits} gs={gs}")
    T, E, K = 3, 256, 2048
    rng = np.random.default_rng(nbits * gs)
    w, s, b = synth.quant_weights(rng, (E,), K, group_size=gs, bits=nbits)
    x = synth.bf16_bits(rng.normal(size=(T, K)).astype(np.float32))
    got = ops.router_logits(bf16_t(x, dev), (words_t(w, dev), bf16_t(s, dev), bf16_t(b, dev)), gs, nbits)
    ref64 = np.stack([orc.gather_qmm_rows(x[t:t + 1], None, np.zeros(1, np.int32), w[None], s[None], b[None],
                                          group_size=gs, bits=nbits)[0][0] for t in range(T)])
    # the kernel sums x * (128 + q) per chunk before the affine correction
    # (qmoe_router_logits), so its rounding scales with those magnitudes:
    # sum_g s_g * (128 + 2^bits) * sum_{k in g} |x_k| + |b_g| * sum_{k in g} |x_k|
    xg = np.abs(orc.f32_from_bf16(x).astype(np.float64)).reshape(T, K // gs, gs).sum(-1)
    sf = np.abs(orc.f32_from_bf16(s).astype(np.float64))
    bf = np.abs(orc.f32_from_bf16(b).astype(np.float64))
    mag = xg @ (sf * (128 + 2 ** nbits) + bf).T
    _assert_logits(got.cpu().numpy(), ref64, mag)


@pytest.mark.parametrize("E,I,K,counts", [
    (4, 512, 2048, [1, 129, 300, 64]),
    (8, 128, 1024, [7, 0, 33, 97, 128, 200, 2, 65]),
    (3, 256, 512, [256, 5, 100]),
])
def test_swiglu_gemm_matches_oracle(dev, orc, E, I, K, counts):
    say(f"SwiGLU grouped GEMM E={E} I={I} K={K}")
    rng = np.random.default_rng(E * I + K)
    w, s, b = synth.quant_weights(rng, (E, 2 * I), K)
    ids = np.repeat(np.arange(E), counts).astype(np.int32)
    x = synth.bf16_bits(rng.normal(size=(len(ids), K)).astype(np.float32))
    tw = ops.repack_tiles(words_t(w, dev), bf16_t(s, dev), bf16_t(b, dev), swiglu_pairs=True)
    tiles = ops.build_tiles(torch.from_numpy(ids).to(dev), E)
    h = ops.gather_qmm_swiglu_sorted_tiles(bf16_t(x, dev), tw, tiles)
    gu64, _ = orc.gather_qmm_rows(x, None, ids, w, s, b, deq="bf16")  # the GEMM's bf16 weights
    h64, _ = orc.swiglu(gu64)
    assert_close_bf16(orc, bits(h), h64, what=f"swiglu gemm {E}/{I}/{K}")


def _block_problem(seed, E, H, I, with_shared=False):
    rng = np.random.default_rng(seed)
    gu = synth.quant_weights(rng, (E, 2 * I), H)
    dn = synth.quant_weights(rng, (E, H), I)
    router = synth.bf16_bits((rng.normal(size=(E, H)) * 0.05).astype(np.float32))
    shared = None
    if with_shared:
        sgu = synth.quant_weights(rng, (1, 2 * I), H)
        sdn = synth.quant_weights(rng, (1, H), I)
        sg = synth.bf16_bits((rng.normal(size=(1, H)) * 0.05).astype(np.float32))
        shared = (sgu, sdn, sg)
    return gu, dn, router, shared


def _dev_w(t, dev):
    w, s, b = t
    return words_t(w, dev), bf16_t(s, dev), bf16_t(b, dev)


@pytest.mark.parametrize("T,smp", [(1, 64), (3, 64), (6, 64), (7, 64), (300, 64), (7, 1000), (16, 1000)])
def test_moe_block_matches_oracle_chain(dev, orc, T, smp):
    E, H, I, k = 64, 2048, 512, 10
    say(f"MoE block T={T} E={E} H={H} I={I} k={k} sort_min_pairs={smp}")
    gu, dn, router, _ = _block_problem(T + 5, E, H, I)
    rng = np.random.default_rng(T)
    x = synth.bf16_bits(rng.normal(size=(T, H)).astype(np.float32))
    blk = moe_block.SparseMoeBlock(bf16_t(router, dev), _dev_w(gu, dev), _dev_w(dn, dev), k, sort_min_pairs=smp)
    xt = bf16_t(x, dev)
    y = bits(blk(xt))
    # stage 1: the logits, then the selection on the block's own fp32 logits
    logits = blk.route_logits(xt).cpu().numpy()
    xf, wf = orc.f32_from_bf16(x).astype(np.float64), orc.f32_from_bf16(router).astype(np.float64)
    _assert_logits(logits, xf @ wf.T, np.abs(xf) @ np.abs(wf).T)
    idx, sc = blk.route(xt)
    ridx, rsc = orc.router_topk(logits, k, True)
    assert np.array_equal(idx.cpu().numpy(), ridx)
    np.testing.assert_allclose(sc.cpu().numpy(), rsc, rtol=4e-6, atol=1e-7)
    sc32 = sc.cpu().numpy()
    if T * k < blk.sort_min_pairs and T <= 16:
        # stage 2: h = silu(gate) * up per (token, slot); stage 3: the fused
        # down + weighted sum, the oracle fed the kernel's own h
        # the block keeps one resident copy, in the tile layout, and decodes from it
        assert blk.decode_tiles and blk.gate_up is None and blk.down is None
        h = ops.gate_up_silu_tiles(xt, blk.gu_tiles, idx)
        tok = np.repeat(np.arange(T), k).astype(np.int32)
        gu64, _ = orc.gather_qmm_rows(x, tok, ridx.reshape(-1), *gu)
        h64, _ = orc.swiglu(gu64)
        assert_close_bf16(orc, bits(h).reshape(T * k, I), h64, what=f"block h T={T}")
        y64, _ = orc.down_wsum(bits(h), ridx, sc32, *dn)
        assert_close_bf16(orc, y, y64, what=f"block y T={T}")
        want = bits(ops.down_wsum_tiles(h, blk.down_tiles, idx, sc))
    else:
        # stage 2: routing sort + SwiGLU gate_up GEMM; stage 3: down GEMM on
        # the kernel's own h; stage 4: un-permute + weighted sum, bit-exact
        r = ops.route(idx, E)
        order = r.order.cpu().numpy()
        srt = r.sorted_ids.cpu().numpy()
        assert np.array_equal(srt, ridx.reshape(-1)[order])
        lhs = torch.div(r.order, k, rounding_mode="floor").to(torch.int32)
        h = ops.gather_qmm_swiglu_sorted_tiles(xt, blk.gu_tiles, r.tiles, x_rows=lhs)
        gu64, _ = orc.gather_qmm_rows(x, order // k, srt, *gu, deq="bf16")
        h64, _ = orc.swiglu(gu64)
        assert_close_bf16(orc, bits(h), h64, what=f"block h T={T}")
        yd = ops.gather_qmm_sorted_tiles(h, blk.down_tiles, r.tiles)
        yd64, _ = orc.gather_qmm_rows(bits(h), None, srt, *dn, deq="bf16")
        assert_close_bf16(orc, bits(yd), yd64, what=f"block down T={T}")
        want = orc.weighted_sum(bits(yd), r.inv_order.cpu().numpy(), sc32, T, k, H, blk.wsum_mode)
    assert np.array_equal(y, want), f"block output differs from its stages (T={T})"


@pytest.mark.parametrize("T", [2, 200])
def test_moe_block_shared_expert(dev, orc, T):
    E, H, I, k = 32, 2048, 512, 4
    say(f"MoE block with shared expert T={T}")
    gu, dn, router, (sgu, sdn, sg) = _block_problem(T + 9, E, H, I, with_shared=True)
    rng = np.random.default_rng(T + 1)
    x = synth.bf16_bits(rng.normal(size=(T, H)).astype(np.float32))
    shared = moe_block.SharedExpert(_dev_w(sgu, dev), _dev_w(sdn, dev), bf16_t(sg, dev))
    blk = moe_block.SparseMoeBlock(bf16_t(router, dev), _dev_w(gu, dev), _dev_w(dn, dev), k, shared=shared)
    xt = bf16_t(x, dev)
    y = blk(xt).float().cpu().numpy()
    routed = blk.experts(xt, *blk.route(xt)).float().cpu().numpy()
    # shared branch: the oracle's dense SwiGLU MLP on the same x, gated
    zero = np.zeros(T, np.int32)
    deq = "exact" if T <= 16 else "bf16"  # decode kernels vs the GEMMs
    gu64, _ = orc.gather_qmm_rows(x, None, zero, *sgu, deq=deq)
    _, h16 = orc.swiglu(gu64)
    sh64, _ = orc.gather_qmm_rows(h16, None, zero, *sdn, deq=deq)
    g = 1.0 / (1.0 + np.exp(-(orc.f32_from_bf16(x).astype(np.float64) @ orc.f32_from_bf16(sg)[0].astype(np.float64))))
    want = routed.astype(np.float64) + g[:, None] * sh64
    err = np.abs(y - want).max() / np.abs(want).max()
    print(f"[parity] shared block rel_to_max {err:.3g}", flush=True)
    assert err <= 2.0 ** -7


@pytest.mark.parametrize("resident", ["tiles", "both"])
def test_moe_block_resident_copies(dev, orc, resident):
    """resident="tiles": one tile-layout copy, the same bytes as the MLX tensors
    it was built from (the layout is a permutation); "both": twice that.  The
    two blocks' decode outputs both meet the oracle's bar."""
    E, H, I, k, T = 16, 2048, 512, 4, 2
    say(f"MoE block resident={resident}")
    gu, dn, router, (sgu, sdn, sg) = _block_problem(3, E, H, I, with_shared=True)
    shared = moe_block.SharedExpert(_dev_w(sgu, dev), _dev_w(sdn, dev), bf16_t(sg, dev))
    blk = moe_block.SparseMoeBlock(bf16_t(router, dev), _dev_w(gu, dev), _dev_w(dn, dev), k, shared=shared,
                                   resident=resident)
    mlx_bytes = sum(a.nbytes for grp in (gu, dn, sgu, sdn) for a in grp)
    assert blk.nbytes == (1 if resident == "tiles" else 2) * mlx_bytes, (blk.nbytes, mlx_bytes)
    assert blk.decode_tiles == (resident == "tiles")
    rng = np.random.default_rng(5)
    x = synth.bf16_bits(rng.normal(size=(T, H)).astype(np.float32))
    xt = bf16_t(x, dev)
    idx, sc = blk.route(xt)
    y = bits(blk.experts(xt, idx, sc))
    ridx = idx.cpu().numpy()
    tok = np.repeat(np.arange(T), k).astype(np.int32)
    gu64, _ = orc.gather_qmm_rows(x, tok, ridx.reshape(-1), *gu)
    _, h16 = orc.swiglu(gu64)
    y64, _ = orc.down_wsum(h16.reshape(T, k, I), ridx, sc.cpu().numpy(), *dn)
    rep = orc.err_report(y, y64)
    print(f"[parity] block resident={resident}: {rep}", flush=True)
    assert rep["rel_to_max"] <= 2.0 ** -7


def _dev_tiles(E, N, K, dev, pairs, seed):
    """Random tile-layout weights [E, N, K] made on the device (the two paths
    compared below read the same bytes; the values only need to be varied)."""
    g = torch.Generator(device=dev).manual_seed(seed)
    w = torch.randint(-2 ** 31, 2 ** 31 - 1, (E, N, K // 8), dtype=torch.int32, device=dev, generator=g)
    s = (torch.rand(E, N, K // 64, device=dev, generator=g) * 0.015 + 0.005).to(torch.bfloat16)
    b = (torch.randn(E, N, K // 64, device=dev, generator=g) * 0.05).to(torch.bfloat16)
    return ops.repack_tiles(w, s, b, swiglu_pairs=pairs)


@pytest.mark.parametrize("T,E,k,norm,K", [(1, 256, 10, True, 2048), (3, 64, 8, False, 2048),
                                          (6, 300, 10, True, 4096), (16, 32, 4, True, 2048),
                                          (2, 1024, 16, False, 2048), (1, 256, 10, True, 6144),
                                          (4, 128, 8, False, 8192)])
def test_decode_topk_kernels_match_router_topk(dev, T, E, k, norm, K):
    """The gate_up decode kernel that selects its own experts from the logits
    equals router_topk followed by the id-taking kernel, bit for bit, in h and
    in the ids and scores it hands on, on both in-kernel top-k instances
    (E <= 256, E > 256) and with planted ties."""
    say(f"decode top-k kernels T={T} E={E} k={k} norm={norm} K={K}")
    I, D = 512, K
    gu = _dev_tiles(E, 2 * I, K, dev, True, 11 + E)
    dn = _dev_tiles(E, D, I, dev, False, 12 + E)
    g = torch.Generator(device=dev).manual_seed(T * 131 + E)
    x = torch.randn(T, K, device=dev, generator=g).to(torch.bfloat16)
    logits = torch.randn(T, E, device=dev, generator=g)
    logits[:, E // 3] = logits[:, E // 5]  # ties: the lower index goes first
    logits[0, 1] = logits[0, 0]
    idx_ref, sc_ref = ops.router_topk(logits, k, norm)
    h_ref = ops.gate_up_silu_tiles(x, gu, idx_ref)
    h, idx, sc = ops.gate_up_silu_tiles_topk(x, gu, logits, k, norm)
    y_ref = ops.down_wsum_tiles(h_ref, dn, idx_ref, sc_ref)
    y = ops.down_wsum_tiles(h, dn, idx, sc)
    torch.cuda.synchronize()
    assert torch.equal(idx, idx_ref), "ids from the gate_up kernel differ from router_topk's"
    assert torch.equal(sc, sc_ref), "scores from the gate_up kernel differ from router_topk's"
    assert torch.equal(h, h_ref), "gate_up from logits differs from router_topk + gate_up"
    assert torch.equal(y, y_ref)


@pytest.mark.parametrize("E,k", [(256, 10), (1024, 16)])
def test_decode_topk_kernels_many_ties(dev, orc, E, k):
    """As above with logits from five values, so most choices are decided by
    the index: every wave's own choice (h), the written ids and the router
    top-k agree with the oracle's ids."""
    say(f"decode top-k kernels, many ties, E={E} k={k}")
    T, K, I = 4, 2048, 512
    gu = _dev_tiles(E, 2 * I, K, dev, True, 21 + E)
    rng = np.random.default_rng(E + k)
    lg = rng.integers(-2, 3, size=(T, E)).astype(np.float32)
    logits = f32_t(lg, dev)
    x = torch.randn(T, K, device=dev, generator=torch.Generator(device=dev).manual_seed(E)).to(torch.bfloat16)
    ridx, rsc = orc.router_topk(lg, k, True)
    h, idx, sc = ops.gate_up_silu_tiles_topk(x, gu, logits, k, True)
    h_ref = ops.gate_up_silu_tiles(x, gu, torch.from_numpy(ridx).to(dev))
    torch.cuda.synchronize()
    assert np.array_equal(idx.cpu().numpy(), ridx)
    np.testing.assert_allclose(sc.cpu().numpy(), rsc, rtol=4e-6, atol=1e-7)
    assert torch.equal(h, h_ref)


def test_block_decode_takes_the_topk_kernels(dev, orc):
    """A tile-resident block decodes through the top-k kernels, and its output
    equals the id-taking path's."""
    E, H, I, k = 64, 2048, 512, 10
    gu, dn, router, _ = _block_problem(9, E, H, I)
    blk = moe_block.SparseMoeBlock(bf16_t(router, dev), _dev_w(gu, dev), _dev_w(dn, dev), k)
    rng = np.random.default_rng(9)
    for T in (1, 3, 6):
        assert blk.decodes_with_topk(T)
        xt = bf16_t(synth.bf16_bits(rng.normal(size=(T, H)).astype(np.float32)), dev)
        y = blk(xt)
        idx, sc = blk.route(xt)
        want = blk.experts(xt, idx, sc)
        torch.cuda.synchronize()
        assert torch.equal(y, want), f"T={T}"
    assert not blk.decodes_with_topk(7)  # 70 pairs: the sorted path


@pytest.mark.parametrize("T", [1, 3])
def test_moe_block_decode_top_k_past_tile_kernels(dev, orc, T):
    """top_k = 20 is past the tile-layout down kernel's 16 experts per token
    (qmoe_moe_down_wsum_tiles), so the block keeps the MLX tensors resident
    and decodes from them (qmoe_moe_down_wsum takes up to 64); at T * k < 64
    the call is a decode and must meet the oracle's bar."""
    E, H, I, k = 64, 2048, 512, 20
    say(f"MoE block decode top_k={k} T={T}")
    gu, dn, router, _ = _block_problem(40 + T, E, H, I)
    rng = np.random.default_rng(60 + T)
    x = synth.bf16_bits(rng.normal(size=(T, H)).astype(np.float32))
    blk = moe_block.SparseMoeBlock(bf16_t(router, dev), _dev_w(gu, dev), _dev_w(dn, dev), k)
    assert not moe_block.tile_decode_supported(H, I, top_k=k)
    assert not blk.decode_tiles and blk.gate_up is not None and blk.down is not None
    assert T * k < blk.sort_min_pairs and not blk.decodes_with_topk(T)
    xt = bf16_t(x, dev)
    y = bits(blk(xt))
    idx, sc = blk.route(xt)
    ridx = idx.cpu().numpy()
    tok = np.repeat(np.arange(T), k).astype(np.int32)
    gu64, _ = orc.gather_qmm_rows(x, tok, ridx.reshape(-1), *gu)
    _, h16 = orc.swiglu(gu64)
    y64, _ = orc.down_wsum(h16.reshape(T, k, I), ridx, sc.cpu().numpy(), *dn)
    rep = orc.err_report(y, y64)
    print(f"[parity] block decode top_k={k} T={T}: {rep}", flush=True)
    assert rep["rel_to_max"] <= 2.0 ** -7


@pytest.mark.parametrize("T,with_shared", [(1, False), (4, False), (1, True), (256, False), (256, True)])
def test_moe_block_graph_replays(dev, T, with_shared):
    """The whole block captured into a graph (the serving pattern: a static
    input, new tokens copied in, the graph replayed) gives the eager result
    bit for bit on every replay, with eager work between replays: decode
    (the top-k gate_up and fused down kernels) and prefill (router top-k,
    routing sort, the grouped GEMMs, the weighted sum), with and without the
    shared expert."""
    E, H, I, k = 64, 2048, 512, 8
    say(f"MoE block graph replays T={T} shared={with_shared}")
    gu, dn, router, sh = _block_problem(T + 31, E, H, I, with_shared=with_shared)
    shared = None
    if with_shared:
        sgu, sdn, sg = sh
        shared = moe_block.SharedExpert(_dev_w(sgu, dev), _dev_w(sdn, dev), bf16_t(sg, dev))
    blk = moe_block.SparseMoeBlock(bf16_t(router, dev), _dev_w(gu, dev), _dev_w(dn, dev), k, shared=shared)
    rng = np.random.default_rng(T + 77)
    xs = [bf16_t(synth.bf16_bits(rng.normal(size=(T, H)).astype(np.float32)), dev) for _ in range(4)]
    want = [blk(x).clone() for x in xs]
    torch.cuda.synchronize()
    static_x = xs[0].clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        blk(static_x)  # warm the allocator off the capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        static_y = blk(static_x)
    for rep in range(8):
        i = (rep * 3) % len(xs)
        static_x.copy_(xs[i])
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(static_y, want[i]), (T, with_shared, rep)
        blk(xs[(i + 1) % len(xs)])  # eager work between replays
        torch.cuda.synchronize()
