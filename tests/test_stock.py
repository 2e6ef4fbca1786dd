"""The stock torch path (the registry's reference and the un-patched
namespace) against the oracle, on CPU tensors."""

import numpy as np
import pytest
import torch

from helpers import bf16_t, bits, words_t
from titan_amd import stock


def _quant(rng, E, N, K, bits_=4):
    w = rng.integers(0, 2**32, size=(E, N, K * bits_ // 32), dtype=np.uint64).astype(np.uint32)
    s = (rng.uniform(0.005, 0.02, size=(E, N, K // 64))).astype(np.float32)
    b = rng.normal(0, 0.05, size=(E, N, K // 64)).astype(np.float32)
    return w, s, b


@pytest.mark.parametrize("bits_", [4, 8])
def test_stock_dequantize_is_bit_exact_with_the_oracle(orc, bits_):
    rng = np.random.default_rng(7)
    w, s, b = _quant(rng, 2, 16, 256, bits_)
    s16, b16 = orc.bf16_from_f32(s), orc.bf16_from_f32(b)
    want = orc.dequantize_bf16(w, s16, b16, 64, bits_)
    got = stock.dequantize(words_t(w), bf16_t(s16), bf16_t(b16), 64, bits_)
    assert np.array_equal(bits(got), want.reshape(bits(got).shape))


def test_stock_unpack_matches_the_oracle(orc):
    rng = np.random.default_rng(3)
    w = rng.integers(0, 2**32, size=(5, 12), dtype=np.uint64).astype(np.uint32)
    for b_ in (4, 8):
        assert np.array_equal(stock.unpack(words_t(w), b_).numpy(), orc.unpack(w, b_).reshape(5, -1))


def test_stock_gather_qmm_is_within_one_ulp_of_the_fp64_golden(orc):
    from helpers import assert_close_bf16

    rng = np.random.default_rng(11)
    E, N, K, R = 6, 64, 256, 40
    w, s, b = _quant(rng, E, N, K)
    s16, b16 = orc.bf16_from_f32(s), orc.bf16_from_f32(b)
    x16 = orc.bf16_from_f32(rng.normal(size=(R, K)).astype(np.float32))
    ids = np.sort(rng.integers(0, E, size=R)).astype(np.int32)
    ref64, _ = orc.gather_qmm_rows(x16, None, ids, w, s16, b16, deq="bf16")
    got = stock.gather_qmm(bf16_t(x16).reshape(R, 1, K), words_t(w), bf16_t(s16), bf16_t(b16),
                           rhs_indices=torch.from_numpy(ids), sorted_indices=True)
    assert got.shape == (R, 1, N)
    assert_close_bf16(orc, bits(got).reshape(R, N), ref64, what="stock gather_qmm")


def test_stock_gather_qmm_broadcasts_like_the_decode_call(orc):
    """x [1,1,1,1,K] against ids [1,1,k] -> [1,1,k,1,N] (compiled.py:500-512)."""
    rng = np.random.default_rng(5)
    E, N, K, k = 8, 32, 128, 3
    w, s, b = _quant(rng, E, N, K)
    s16, b16 = orc.bf16_from_f32(s), orc.bf16_from_f32(b)
    x16 = orc.bf16_from_f32(rng.normal(size=(1, K)).astype(np.float32))
    ids = rng.permutation(E)[:k].astype(np.int32)
    got = stock.gather_qmm(bf16_t(x16).reshape(1, 1, 1, 1, K), words_t(w), bf16_t(s16), bf16_t(b16),
                           rhs_indices=torch.from_numpy(ids).reshape(1, 1, k))
    assert got.shape == (1, 1, k, 1, N)
    ref64, _ = orc.gather_qmm_rows(x16, np.zeros(k, np.int32), ids, w, s16, b16, deq="bf16")
    from helpers import assert_close_bf16

    assert_close_bf16(orc, bits(got).reshape(k, N), ref64, what="stock decode broadcast")


def test_stock_quantized_matmul_transposed_and_not(orc):
    rng = np.random.default_rng(9)
    w, s, b = _quant(rng, 1, 48, 128)
    s16, b16 = orc.bf16_from_f32(s[0]), orc.bf16_from_f32(b[0])
    x = torch.randn(3, 128, generator=torch.Generator().manual_seed(0)).to(torch.bfloat16)
    y = stock.quantized_matmul(x, words_t(w[0]), bf16_t(s16), bf16_t(b16))
    wd = stock.dequantize(words_t(w[0]), bf16_t(s16), bf16_t(b16), 64, 4).float()
    torch.testing.assert_close(y.float(), (x.float() @ wd.T).to(torch.bfloat16).float(), rtol=0, atol=0)
    # transpose=False: W stored [K, N/8] with groups along N
    y2 = stock.quantized_matmul(torch.randn(2, 48).to(torch.bfloat16), words_t(w[0]), bf16_t(s16),
                                bf16_t(b16), transpose=False)
    assert y2.shape == (2, 128)
