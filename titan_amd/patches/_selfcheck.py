"""Install-time self-checks: one small call through the kernel against the
implementation an overlay is about to replace (the compile-and-verify step of
engine/patches/round2/wsum10/kernel.py:378-449)."""

from __future__ import annotations

import torch

# bf16 has 8 significant bits: two paths that both accumulate in fp32 and
# round once agree to about one ULP of the largest output.
_REL = 2.0 ** -7


def _quant(E, N, K, gen, dev):
    w = torch.randint(-2**31, 2**31 - 1, (E, N, K // 8), generator=gen, dtype=torch.int32).to(dev)
    s = (torch.rand(E, N, K // 64, generator=gen) * 0.015 + 0.005).to(torch.bfloat16).to(dev)
    b = (torch.randn(E, N, K // 64, generator=gen) * 0.05).to(torch.bfloat16).to(dev)
    return w, s, b


def _close(a: torch.Tensor, b: torch.Tensor) -> bool:
    a32, b32 = a.float(), b.float()
    scale = b32.abs().max().item()
    return bool(torch.isfinite(a32).all()) and (a32 - b32).abs().max().item() <= _REL * max(scale, 1e-30)


def sorted_gather_matches(previous, fast) -> bool:
    dev = torch.device("cuda:0")
    gen = torch.Generator().manual_seed(1234)
    E, R, K, N = 4, 96, 256, 256
    w, s, b = _quant(E, N, K, gen, dev)
    idx = torch.sort(torch.randint(0, E, (R,), generator=gen)).values.to(torch.int32).to(dev)
    x = torch.randn(R, 1, K, generator=gen).to(torch.bfloat16).to(dev)
    ref = previous(x, w, s, b, rhs_indices=idx, transpose=True, group_size=64, bits=4, sorted_indices=True)
    got = fast(x, w, s, b, idx, group_size=64, bits=4)
    torch.cuda.synchronize()
    return _close(got.reshape(ref.shape), ref)


def decode_gather_matches(previous, fast) -> bool:
    dev = torch.device("cuda:0")
    gen = torch.Generator().manual_seed(4321)
    E, K, N, k = 8, 512, 128, 4
    w, s, b = _quant(E, N, K, gen, dev)
    idx = torch.randperm(E, generator=gen)[:k].reshape(1, 1, k).to(torch.int32).to(dev)
    x = torch.randn(1, 1, 1, 1, K, generator=gen).to(torch.bfloat16).to(dev)
    ref = previous(x, w, s, b, rhs_indices=idx, transpose=True, group_size=64, bits=4)
    got = fast(x, w, s, b, rhs_indices=idx, transpose=True, group_size=64, bits=4)
    torch.cuda.synchronize()
    return _close(got, ref)
