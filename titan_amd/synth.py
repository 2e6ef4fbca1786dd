"""Seeded synthetic inputs for the five benchmark workloads.

numpy PCG64 with a fixed seed per workload (default: the workload number), so
the GPU path, the tests and the CPU baseline all see the same bytes.  bf16
tensors are returned as ``uint16`` bit patterns (round to nearest even from
fp32), packed weights as ``uint32``.  Uniform 4-bit codes packed eight to a
word are uniform 32-bit words, which is how they are drawn.

Workloads (hidden H=2048, experts E=256, top_k=10, expert intermediate I=512):

0. dense quantized_matmul: x [1,2048], W [4096,2048] 4-bit group 64.
1. decode gate_up: 1 token, 10 experts drawn without replacement,
   W [E,1024,2048]; output [10,1024] then SwiGLU [10,512].
2. decode down + weighted sum: 8 tokens, 10 distinct experts each, router
   weights softmax of N(0,1) logits; h [8,10,512]; W [E,2048,512].
3. prefill grouped GEMM: 4096 tokens, logits N(0,1) + log p_e with
   p_e ~ rank^-1.1 over a seeded expert permutation, top-10 per token,
   W [E,1024,2048]; 40960 routed rows.
4. as 3 with 0.1% activation outliers at x20, per-token int8 activations.

Routed expert order within a token is by descending logit (ties by expert id),
which fixes the pair index t*k + j.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

HIDDEN = 2048
EXPERTS = 256
TOP_K = 10
INTER = 512
GROUP = 64
BITS = 4


def bf16_bits(a) -> np.ndarray:
    """fp32 -> bf16 bit patterns, round to nearest even."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return r.astype(np.uint16)


def bf16_to_f32(h) -> np.ndarray:
    return (np.ascontiguousarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def rng_for(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def quant_weights(rng, rows_shape, K, group_size=GROUP, bits=BITS):
    """Packed codes (uniform), bf16 scales ~U(0.005, 0.02), bf16 biases ~N(0, 0.05)."""
    words = K * bits // 32
    w = rng.integers(0, 2 ** 32, size=tuple(rows_shape) + (words,), dtype=np.uint32)
    G = K // group_size
    s = bf16_bits(rng.uniform(0.005, 0.02, size=tuple(rows_shape) + (G,)).astype(np.float32))
    b = bf16_bits(rng.normal(0.0, 0.05, size=tuple(rows_shape) + (G,)).astype(np.float32))
    return w, s, b


def softmax(z):
    z = np.asarray(z, np.float32)
    m = z.max(axis=-1, keepdims=True)
    e = np.exp(z - m)
    return (e / e.sum(axis=-1, keepdims=True)).astype(np.float32)


def zipf_topk(rng, tokens, experts=EXPERTS, k=TOP_K, s=1.1):
    """Router logits N(0,1) + log p_e, p_e ~ rank(e)^-s over a seeded
    permutation; top-k by logit (descending, ties by expert id); weights are
    the softmax over the chosen k."""
    perm = rng.permutation(experts)
    rank = np.empty(experts, np.float64)
    rank[perm] = np.arange(1, experts + 1)
    logp = -s * np.log(rank)
    logp -= np.log(np.exp(logp).sum())
    z = (rng.normal(0.0, 1.0, size=(tokens, experts)) + logp[None, :]).astype(np.float32)
    idx = np.argsort(-z, axis=-1, kind="stable")[:, :k].astype(np.int32)
    chosen = np.take_along_axis(z, idx, axis=-1)
    return idx, softmax(chosen)


@dataclass
class Workload:
    cfg: int
    seed: int
    arrays: dict = field(default_factory=dict)
    meta: dict = field(default_factory=dict)

    def __getitem__(self, k):
        return self.arrays[k]


def make(cfg: int, seed: int | None = None, *, tokens: int | None = None,
         experts: int = EXPERTS) -> Workload:
    """Build workload ``cfg`` (0..4; 5: workload 0 with 8-bit codes).  ``tokens`` shrinks the prefill workloads
    for tests; ``experts`` shrinks E (the ids stay in range)."""
    seed = cfg if seed is None else seed
    rng = rng_for(seed)
    wl = Workload(cfg=cfg, seed=seed)
    A, M = wl.arrays, wl.meta
    if cfg == 0:
        A["w"], A["s"], A["b"] = quant_weights(rng, (4096,), HIDDEN)
        A["x"] = bf16_bits(rng.normal(0.0, 1.0, size=(1, HIDDEN)).astype(np.float32))
        M.update(M=1, N=4096, K=HIDDEN)
    elif cfg == 1:
        A["w"], A["s"], A["b"] = quant_weights(rng, (experts, 2 * INTER), HIDDEN)
        A["x"] = bf16_bits(rng.normal(0.0, 1.0, size=(1, HIDDEN)).astype(np.float32))
        A["idx"] = rng.choice(experts, size=TOP_K, replace=False).astype(np.int32)[None, :]
        M.update(T=1, k=TOP_K, K=HIDDEN, I=INTER, E=experts)
    elif cfg == 2:
        T = 8 if tokens is None else tokens
        A["w"], A["s"], A["b"] = quant_weights(rng, (experts, HIDDEN), INTER)
        A["idx"] = np.stack([rng.choice(experts, size=TOP_K, replace=False)
                             for _ in range(T)]).astype(np.int32)
        A["scores"] = softmax(rng.normal(0.0, 1.0, size=(T, TOP_K)))
        A["h"] = bf16_bits(rng.normal(0.0, 1.0, size=(T, TOP_K, INTER)).astype(np.float32))
        M.update(T=T, k=TOP_K, I=INTER, D=HIDDEN, E=experts,
                 distinct=int(np.unique(A["idx"]).size))
    elif cfg in (3, 4):
        T = 4096 if tokens is None else tokens
        A["w"], A["s"], A["b"] = quant_weights(rng, (experts, 2 * INTER), HIDDEN)
        A["idx"], A["scores"] = zipf_topk(rng, T, experts)
        x = rng.normal(0.0, 1.0, size=(T, HIDDEN)).astype(np.float32)
        if cfg == 4:
            out = rng.random(size=x.shape) < 0.001
            x = np.where(out, x * 20.0, x).astype(np.float32)
        A["x"] = bf16_bits(x)
        M.update(T=T, k=TOP_K, K=HIDDEN, N=2 * INTER, E=experts)
    elif cfg == 5:
        A["w"], A["s"], A["b"] = quant_weights(rng, (4096,), HIDDEN, bits=8)
        A["x"] = bf16_bits(rng.normal(0.0, 1.0, size=(1, HIDDEN)).astype(np.float32))
        M.update(M=1, N=4096, K=HIDDEN, bits=8)
    else:
        raise ValueError(f"no workload {cfg}")
    return wl


def algorithmic_bytes(cfg: int, wl: Workload | None = None) -> int:
    """HBM bytes one call must move at minimum (each touched expert once)."""
    row_bytes = lambda K: K // 2 + (K // GROUP) * 4  # packed codes + bf16 scale & bias
    if cfg == 0:
        return 4096 * row_bytes(HIDDEN) + HIDDEN * 2 + 4096 * 2
    if cfg == 5:  # 8-bit codes: one byte per element
        return 4096 * (HIDDEN + (HIDDEN // GROUP) * 4) + HIDDEN * 2 + 4096 * 2
    if cfg == 1:
        return TOP_K * 2 * INTER * row_bytes(HIDDEN) + HIDDEN * 2 + TOP_K * INTER * 2 * 2
    if cfg == 2:
        assert wl is not None
        T = wl.meta["T"]
        return (wl.meta["distinct"] * HIDDEN * row_bytes(INTER) + T * TOP_K * INTER * 2
                + T * HIDDEN * 2 + T * TOP_K * 4)
    raise ValueError("prefill workloads are priced in flops")


def algorithmic_flops(cfg: int, wl: Workload | None = None) -> int:
    if cfg in (0, 5):
        return 2 * 4096 * HIDDEN
    if cfg == 1:
        return 2 * TOP_K * 2 * INTER * HIDDEN
    if cfg == 2:
        T = wl.meta["T"] if wl is not None else 8
        return 2 * T * TOP_K * HIDDEN * INTER
    T = wl.meta["T"] if wl is not None else 4096
    return 2 * T * TOP_K * 2 * INTER * HIDDEN
