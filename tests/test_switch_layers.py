"""SwitchGLU / QuantizedSwitchLinear semantics on CPU tensors (stock path):
sort threshold, fused gate_up split, SwiGLU, un-sort; checked against the
oracle's per-pair chain."""

import numpy as np
import pytest
import torch

from helpers import bf16_t, bits, words_t
from titan_amd.switch_layers import QuantizedSwitchLinear, SwitchGLU, _gather_sort, swiglu


def _layer(orc, rng, E, N, K):
    w = rng.integers(0, 2**32, size=(E, N, K // 8), dtype=np.uint64).astype(np.uint32)
    s = orc.bf16_from_f32(rng.uniform(0.005, 0.02, size=(E, N, K // 64)).astype(np.float32))
    b = orc.bf16_from_f32(rng.normal(0, 0.05, size=(E, N, K // 64)).astype(np.float32))
    return (w, s, b), QuantizedSwitchLinear(words_t(w), bf16_t(s), bf16_t(b))


def _oracle_chain(orc, x16, ids, gu, dn):
    """Per (token, slot): gate_up row -> bf16, swiglu in fp32 of the bf16 halves
    -> bf16, down -> bf16 (the stock layer's rounding points)."""
    T, k = ids.shape
    rows = np.repeat(np.arange(T, dtype=np.int32), k)
    _, gu16 = orc.gather_qmm_rows(x16, rows, ids.reshape(-1), *gu, deq="bf16")
    g = orc.f32_from_bf16(gu16).astype(np.float32)
    I = g.shape[1] // 2
    gate, up = g[:, :I], g[:, I:]
    h = gate / (np.float32(1) + np.exp(-gate)) * up
    h16 = orc.bf16_from_f32(h.astype(np.float32))
    d64, _ = orc.gather_qmm_rows(h16, None, ids.reshape(-1), *dn, deq="bf16")
    return d64.reshape(T, k, -1)


@pytest.mark.parametrize("T", [1, 3, 9])
def test_switch_glu_matches_the_oracle_chain(orc, T):
    rng = np.random.default_rng(100 + T)
    E, K, I, k = 8, 128, 64, 4
    gu, gu_layer = _layer(orc, rng, E, 2 * I, K)
    dn, dn_layer = _layer(orc, rng, E, K, I)
    x16 = orc.bf16_from_f32(rng.normal(size=(T, K)).astype(np.float32))
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    glu = SwitchGLU(dn_layer, gate_up_proj=gu_layer)
    y = glu(bf16_t(x16), torch.from_numpy(ids))
    assert y.shape == (T, k, K)
    ref = _oracle_chain(orc, x16, ids, gu, dn)
    # one rounding of h may differ by an ULP between fp32 paths; compare at the layer's bar
    err = np.abs(orc.f32_from_bf16(bits(y)).astype(np.float64) - ref).max()
    assert err <= 2.0 ** -7 * np.abs(ref).max(), err


def test_sorted_and_unsorted_paths_agree():
    """Row-permutation equivariance: the 64-pair sort must not change results."""
    gen = torch.Generator().manual_seed(0)
    E, K, N = 4, 128, 32
    w = torch.randint(-2**31, 2**31 - 1, (E, N, K // 8), generator=gen, dtype=torch.int32)
    s = (torch.rand(E, N, K // 64, generator=gen) * 0.01 + 0.005).to(torch.bfloat16)
    b = (torch.randn(E, N, K // 64, generator=gen) * 0.05).to(torch.bfloat16)
    lin = QuantizedSwitchLinear(w, s, b)
    x = torch.randn(16, 1, 1, K, generator=gen).to(torch.bfloat16)
    ids = torch.randint(0, E, (16, 4), generator=gen)
    unsorted = lin(x, ids)
    xs, sid, inv, _ = _gather_sort(x, ids, E)
    srt = lin(xs, sid, sorted_indices=True)
    assert torch.equal(srt[inv].reshape(unsorted.shape), unsorted)


def test_gather_sort_is_stable():
    ids = torch.tensor([[3, 1], [1, 3], [0, 1]])
    x = torch.arange(3).reshape(3, 1, 1, 1).float()
    xs, sid, inv, tiles = _gather_sort(x, ids, 4)
    assert sid.tolist() == [0, 1, 1, 1, 3, 3]
    assert xs.flatten().tolist() == [2, 0, 1, 2, 0, 1]
    assert tiles is None and torch.equal(sid[inv], ids.reshape(-1))


def test_per_expert_bias_is_added_after_the_gather():
    gen = torch.Generator().manual_seed(1)
    E, K, N = 3, 128, 16
    w = torch.randint(-2**31, 2**31 - 1, (E, N, K // 8), generator=gen, dtype=torch.int32)
    s = (torch.rand(E, N, K // 64, generator=gen) * 0.01).to(torch.bfloat16)
    b = torch.zeros(E, N, K // 64, dtype=torch.bfloat16)
    bias = torch.randn(E, N, generator=gen).to(torch.bfloat16)
    x = torch.randn(2, 1, 1, K, generator=gen).to(torch.bfloat16)
    ids = torch.tensor([[0, 2], [1, 0]])
    plain = QuantizedSwitchLinear(w, s, b)(x, ids)
    biased = QuantizedSwitchLinear(w, s, b, bias=bias)(x, ids)
    torch.testing.assert_close(biased.float(), (plain + bias[ids].unsqueeze(-2)).float())


def test_swiglu_is_silu_gate_times_up():
    g = torch.tensor([-2.0, 0.0, 1.5]).to(torch.bfloat16)
    u = torch.tensor([1.0, 3.0, -2.0]).to(torch.bfloat16)
    want = (g.float() * torch.sigmoid(g.float()) * u.float()).to(torch.bfloat16)
    assert torch.equal(swiglu(g, u), want)


def test_custom_activation_gets_up_then_gate(orc):
    """SwitchGLU calls activation(x_up, x_gate), as the reference does
    (switch_layers.py:237, with SwiGLU.__call__(x, gate) at :189-194): an
    asymmetric activation sees the up half first."""
    from titan_amd.switch_layers import SwiGLU

    rng = np.random.default_rng(3)
    E, K, I, k = 4, 128, 64, 2
    gu, gu_layer = _layer(orc, rng, E, 2 * I, K)
    dn, dn_layer = _layer(orc, rng, E, K, I)
    x = bf16_t(orc.bf16_from_f32(rng.normal(size=(2, K)).astype(np.float32)))
    ids = torch.tensor([[0, 1], [2, 3]])
    seen = {}

    def take_first(a, b):
        seen["first"], seen["second"] = a, b
        return a

    SwitchGLU(dn_layer, gate_up_proj=gu_layer, activation=take_first)(x, ids)
    up_then_gate = gu_layer(x.unsqueeze(-2).unsqueeze(-2), ids).chunk(2, dim=-1)
    assert torch.equal(seen["first"], up_then_gate[1]) and torch.equal(seen["second"], up_then_gate[0])
    # the default module computes silu(gate) * up from that order
    g, u = up_then_gate[0], up_then_gate[1]
    assert torch.equal(SwiGLU()(u, g), swiglu(g, u))


def test_passing_the_swiglu_function_matches_the_default(orc):
    """The bare swiglu function takes (gate, x); given as the activation it is
    wrapped in the SwiGLU module (called with (x_up, x_gate)), so the layer
    computes silu(gate) * up either way."""
    rng = np.random.default_rng(5)
    E, K, I, k = 4, 128, 64, 2
    gu, gu_layer = _layer(orc, rng, E, 2 * I, K)
    dn, dn_layer = _layer(orc, rng, E, K, I)
    x = bf16_t(orc.bf16_from_f32(rng.normal(size=(3, K)).astype(np.float32)))
    ids = torch.tensor([[0, 1], [2, 3], [1, 2]])
    want = SwitchGLU(dn_layer, gate_up_proj=gu_layer)(x, ids)
    got = SwitchGLU(dn_layer, gate_up_proj=gu_layer, activation=swiglu)(x, ids)
    assert torch.equal(got, want)


def test_tile_decode_envelope_includes_top_k():
    """The block decodes from its one tile-layout copy only where the tile
    decode kernels take the shape: hidden 2048 n (n <= 4), intermediate 512,
    group 64 4-bit codes and at most 16 experts per token
    (qmoe_moe_down_wsum_tiles); otherwise it keeps the MLX tensors."""
    from titan_amd.moe_block import TILE_DECODE_MAX_K, tile_decode_supported

    assert TILE_DECODE_MAX_K == 16
    assert tile_decode_supported(2048, 512, top_k=10)
    assert tile_decode_supported(8192, 512, top_k=16)
    assert not tile_decode_supported(2048, 512, top_k=17)
    assert not tile_decode_supported(2048, 512, top_k=20)
    assert not tile_decode_supported(2560, 512, top_k=8)
    assert not tile_decode_supported(2048, 768, top_k=8)
    assert not tile_decode_supported(2048, 512, group_size=32, top_k=8)
