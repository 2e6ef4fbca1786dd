"""Pins the oracle's bf16 rounding, unpack/pack and dequant.

Each check reaches the expected value by a route independent of the oracle's
C code: torch's own fp32->bf16 conversion, exact rational arithmetic, numpy
bit operations, and the reference's host nibble count
(tests/kernels/test_moe_gather_int8.py:104-115).
"""

from fractions import Fraction

import numpy as np
import pytest
import torch

from titan_amd import synth


def torch_bf16_bits(a):
    return torch.from_numpy(np.asarray(a, np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


SPECIALS = np.array([0.0, -0.0, 1.0, -1.0, 1.00390625, 1.0 + 2 ** -9, 1.0 + 3 * 2 ** -9, 3.4e38, -3.4e38,
                     1e-40, -1e-40, 2 ** -126, 2 ** -133, 65504.0, 1.0 / 3], np.float32)


def test_bf16_rne_matches_torch(orc):
    rng = np.random.default_rng(0)
    vals = np.concatenate([SPECIALS, rng.normal(size=5000).astype(np.float32),
                           (rng.normal(size=2000) * 1e-38).astype(np.float32),
                           rng.uniform(-1e30, 1e30, size=2000).astype(np.float32),
                           np.array([np.inf, -np.inf], np.float32)])
    want = torch_bf16_bits(vals)
    assert np.array_equal(orc.bf16_from_f32(vals), want)
    assert all(orc.bf16_rne_scalar(float(v)) == int(w) for v, w in zip(vals[:300], want[:300]))


def _bf16_value(h):
    return Fraction(float(np.array([h], np.uint16).astype(np.uint32).__lshift__(16).view(np.float32)[0]))


def test_bf16_from_f64_is_nearest_even(orc):
    """Single rounding of a double: the result is a nearest bf16, ties to an
    even significand -- checked against both neighbours in exact arithmetic."""
    rng = np.random.default_rng(1)
    ds = np.concatenate([rng.normal(size=300) * 10 ** rng.uniform(-30, 30, size=300),
                         [1 + 2 ** -8, 1 + 3 * 2 ** -8, -(1 + 2 ** -8), 2 ** -130 * 1.5, 1e-45]])
    got = orc.bf16_from_f64(ds)
    for d, h in zip(ds, got):
        h = int(h)
        v = _bf16_value(h)
        exact = Fraction(float(d))
        for nb in (h - 1, h + 1):
            if nb & 0x7F80 == 0x7F80 or nb < 0 or (h & 0x7FFF) == 0 and nb == h - 1:
                continue
            w = _bf16_value(nb & 0xFFFF)
            assert abs(exact - v) <= abs(exact - w), (d, hex(h), hex(nb))
            if abs(exact - v) == abs(exact - w):
                assert h % 2 == 0, (d, hex(h))
    fast = orc.bf16_from_f64_fast(ds[np.abs(ds) > 2.0 ** -126])
    assert np.array_equal(fast, got[np.abs(ds) > 2.0 ** -126])


def test_unpack_known_answers(orc):
    assert orc.unpack(np.array([0x76543210], np.uint32), 4).tolist() == list(range(8))
    assert orc.unpack(np.array([0xFEDCBA98], np.uint32), 4).tolist() == list(range(8, 16))
    assert orc.unpack(np.array([0x04030201], np.uint32), 8).tolist() == [1, 2, 3, 4]


@pytest.mark.parametrize("bits", [4, 8])
def test_pack_unpack_round_trip(orc, bits):
    rng = np.random.default_rng(bits)
    w = rng.integers(0, 2 ** 32, size=(7, 33), dtype=np.uint32)
    assert np.array_equal(orc.pack(orc.unpack(w, bits), bits), w)
    codes = rng.integers(0, 2 ** bits, size=(5, 64), dtype=np.uint8)
    assert np.array_equal(orc.unpack(orc.pack(codes, bits), bits), codes)


def test_unpack_matches_reference_host_nibble_count(orc):
    """tests/kernels/test_moe_gather_int8.py:104-115 builds nibbles as
    stack([(packed >> 4t) & 0xF for t in range(8)], -1); group sums of 64."""
    rng = np.random.default_rng(3)
    packed = rng.integers(0, 2 ** 32, size=(4, 128, 32), dtype=np.uint32)
    nibbles = np.stack([(packed >> (4 * t)) & 0xF for t in range(8)], axis=-1)
    assert np.array_equal(orc.unpack(packed, 4), nibbles.reshape(4, 128, 256))
    qsum = nibbles.reshape(4, 128, 4, 64).sum(-1)
    assert np.array_equal(orc.unpack(packed, 4).reshape(4, 128, 4, 64).sum(-1, dtype=np.int64), qsum)


def test_dequant_exhaustive_codes(orc):
    """All 16 codes x sampled (s, b): bf16(fmaf(q, s, b)).  q*s + b is exact in
    double for bf16 s, b, so numpy's double->float32 cast is the one fp32
    rounding fmaf makes; torch then rounds to bf16."""
    rng = np.random.default_rng(4)
    n = 600
    s = synth.bf16_bits(np.concatenate([rng.uniform(0.001, 0.05, n // 2),
                                        rng.normal(size=n // 2) * 10.0 ** rng.integers(-20, 20, n // 2)])
                        .astype(np.float32))
    b = synth.bf16_bits((rng.normal(size=n) * 10.0 ** rng.integers(-20, 20, n)).astype(np.float32))
    codes = np.tile(np.arange(16, dtype=np.uint8), (n, 4))  # [n, 64]
    w = orc.pack(codes, 4)
    got = orc.dequantize_bf16(w, s[:, None], b[:, None], 64, 4)
    sf = synth.bf16_to_f32(s).astype(np.float64)[:, None]
    bf = synth.bf16_to_f32(b).astype(np.float64)[:, None]
    want = torch_bf16_bits((codes.astype(np.float64) * sf + bf).astype(np.float32))
    assert np.array_equal(got, want)


def test_dequant_groups_and_8bit(orc):
    rng = np.random.default_rng(5)
    for bits, gs in ((4, 32), (4, 128), (8, 64)):
        K = 256
        w, s, b = synth.quant_weights(rng, (6,), K, gs, bits)
        q = orc.unpack(w, bits).astype(np.float64)
        g = np.arange(K) // gs
        want = torch_bf16_bits((q * synth.bf16_to_f32(s)[:, g] + synth.bf16_to_f32(b)[:, g]).astype(np.float32))
        assert np.array_equal(orc.dequantize_bf16(w, s, b, gs, bits), want)
