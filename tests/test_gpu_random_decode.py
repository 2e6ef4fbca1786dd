"""Seeded random shapes for the fused decode kernels against the oracle:
gate_up + SwiGLU and down + weighted sum over random expert counts, widths,
top-k, hidden and intermediate sizes and group sizes within their envelope,
with repeated experts across tokens."""

import numpy as np
import pytest
import torch

from helpers import assert_close_bf16, bf16_t, bits, f32_t, i32_t, words_t
from titan_amd import ops, synth

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[case] {msg}", flush=True)


@pytest.mark.parametrize("seed", range(10))
def test_fused_decode_random_shapes(dev, orc, seed):
    rng = np.random.default_rng(2000 + seed)
    gs = int(rng.choice([32, 64, 128]))
    E = int(rng.choice([8, 64, 256, 512]))
    T = int(rng.integers(1, 17))
    k = int(rng.integers(1, min(E, 16) + 1))
    K = int(rng.choice([1024, 2048, 2560, 4096, 512 * int(rng.integers(1, 9))]))
    I = int(rng.choice([256, 512, 640, 768]))
    say(f"fused decode seed={seed}: gs={gs} E={E} T={T} k={k} K={K} I={I}")
    w, s, b = synth.quant_weights(rng, (E, 2 * I), K, group_size=gs)
    wd, sd, bd = synth.quant_weights(rng, (E, K), I, group_size=gs)
    x = synth.bf16_bits(rng.normal(size=(T, K)).astype(np.float32))
    idx = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    sc = synth.softmax(rng.normal(size=(T, k)))
    try:
        h = ops.gate_up_silu(bf16_t(x, dev), words_t(w, dev), bf16_t(s, dev), bf16_t(b, dev), i32_t(idx, dev),
                             group_size=gs)
    except ops.QmoeUnsupported as exc:
        pytest.skip(f"outside the gate_up kernel's envelope: {exc}")
    gu64, _ = orc.gather_qmm_rows(x, np.repeat(np.arange(T), k).astype(np.int32), idx.reshape(-1), w, s, b,
                                  group_size=gs)
    h64, _ = orc.swiglu(gu64)
    assert_close_bf16(orc, bits(h).reshape(T * k, I), h64, what=f"gate_up seed {seed}")
    try:
        y = ops.down_wsum(h, words_t(wd, dev), bf16_t(sd, dev), bf16_t(bd, dev), i32_t(idx, dev), f32_t(sc, dev),
                          group_size=gs)
    except ops.QmoeUnsupported as exc:
        pytest.skip(f"outside the down kernel's envelope: {exc}")
    torch.cuda.synchronize()
    y64, _ = orc.down_wsum(bits(h), idx, sc, wd, sd, bd, group_size=gs)
    assert_close_bf16(orc, bits(y), y64, what=f"down seed {seed}")
