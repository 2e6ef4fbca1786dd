"""Whole outputs of the prefill grouped GEMMs at the full workload size.

The parity tests against the fp64 oracle check configs 3 and 4 on sampled
rows (every segment edge plus random rows), because the oracle's row-wise
fp64 gather takes minutes for 40,960 rows.  Here every output is compared,
under the same bar, with a PyTorch fp32 reference of the same op on the GPU,
at 4096 tokens x top-10 Zipf(1.1) routing over 256 experts:

* gate_up, W [256, 1024, 2048] int4 g64: the bf16 GEMM and its SwiGLU
  epilogue on workload 3's activations, the int8 GEMM on workload 4's
  (per-token int8 with 0.1% outliers at x20);
* the down projection, W [256, 2048, 512], over the 40,960 sorted rows of
  h, bf16 and int8.

The reference:

* the weights dequantised in torch as (q * s + b) rounded to bf16, which is
  bf16_rne(fmaf(q, s, b)) bit for bit (q * s is exact in fp32: 4 x 8
  significant bits); checked against the oracle's dequantiser on one expert
  before it is used;
* each expert's gathered rows times its weights in fp32 (no
  reduced-precision matmul modes);
* bf16: y = x . deq(W)^T; SwiGLU: h = silu(gate) * up from the fp32
  products, in fp64; int8: the fake-quant golden (sx * xi) . (s q + b)^T
  over the affine weights themselves, not rounded to bf16, as the int8
  kernel's integer accumulation and rescale compute it
  (moe_gather_int8.py:15-33, the oracle's gather_qmm_int8_rows).

Bar (tests/helpers.py): within 1 bf16 ULP of the rounded reference on live
elements and max-abs within 2^-8 of max|ref| everywhere.  The fp32
reference's own accumulation error (~1e-6 relative) is far below an ULP;
near a rounding boundary it can move the rounded reference by one ULP, and
the kernel's output then sits on the same boundary, so the distance stays
within one ULP.
"""

import numpy as np
import pytest
import torch

from helpers import assert_close_bf16, bf16_t, bits, i32_t, words_t
from titan_amd import ops, synth

pytestmark = pytest.mark.gpu

E, GS = 256, 64


def say(msg):
    print(f"[case] {msg}", flush=True)


def _dequant_expert(w, s, b, e, rounded=True):
    """Expert e's weights as fp32 [N, K] (w int32 [E, N, K/8] words, s/b bf16
    [E, N, K/64]): bf16(q * s + b), or (rounded=False) q * s + b itself, the
    affine weights the int8 golden multiplies (one fp32 rounding, 2^-24)."""
    N, KW = w.shape[1], w.shape[2]
    we = w[e].view(torch.int32)
    sh = torch.arange(0, 32, 4, device=w.device, dtype=torch.int32)
    q = ((we.unsqueeze(-1) >> sh) & 15).reshape(N, KW * 8).float()
    se = s[e].float().repeat_interleave(GS, dim=1)
    be = b[e].float().repeat_interleave(GS, dim=1)
    wf = q * se + be
    return wf.to(torch.bfloat16).float() if rounded else wf


def _reference(xs, w, s, b, off, rounded=True):
    """fp32 products of the sorted rows xs [R, K] (fp32) with their experts'
    weights: [R, N] fp32."""
    out = torch.empty(xs.shape[0], w.shape[1], dtype=torch.float32, device=xs.device)
    for e in range(E):
        lo, hi = int(off[e]), int(off[e + 1])
        if hi > lo:
            out[lo:hi] = xs[lo:hi] @ _dequant_expert(w, s, b, e, rounded).t()
    return out


_cache = {}


def _routed(dev, orc, cfg):
    """Workload cfg's inputs routed on the device (and the reference's rows
    through the oracle's stable sort, which the device routing must equal),
    the gate_up weights on the device, and the torch dequantiser pinned
    against the oracle's on one expert."""
    if cfg in _cache:
        return _cache[cfg]
    torch.backends.cuda.matmul.allow_tf32 = False
    wl = synth.make(cfg)
    T, k = wl["idx"].shape
    r = ops.route(i32_t(wl["idx"], dev), E)
    lhs = torch.div(r.order, k, rounding_mode="floor").to(torch.int32)
    w, s, b = words_t(wl["w"], dev), bf16_t(wl["s"], dev), bf16_t(wl["b"], dev)
    e0 = 17
    got = _dequant_expert(w, s, b, e0).to(torch.bfloat16).cpu().view(torch.int16).numpy().view(np.uint16)
    ref = orc.dequantize_bf16(wl["w"][e0], wl["s"][e0], wl["b"][e0], GS, 4)
    assert np.array_equal(got, ref.reshape(got.shape)), "torch dequant differs from the oracle's"
    order, _, srt = orc.route_sort(wl["idx"], E)
    assert np.array_equal(r.order.cpu().numpy(), order)
    off = np.searchsorted(srt, np.arange(E + 1), side="left")
    rows = torch.from_numpy((order // k).astype(np.int64)).to(dev)
    _cache[cfg] = (wl, r, lhs, (w, s, b), off, rows)
    return _cache[cfg]


@pytest.mark.parametrize("kind", ["bf16", "swiglu", "int8"])
def test_prefill_gate_up_whole_output_full_size(dev, orc, kind):
    cfg = 4 if kind == "int8" else 3
    wl, r, lhs, (w, s, b), off, rows = _routed(dev, orc, cfg)
    t = r.tiles
    xt = bf16_t(wl["x"], dev)
    N = w.shape[1]
    say(f"{kind} gate_up grouped GEMM, every output at 4096 tokens (config {cfg})")
    if kind == "int8":
        xi, sx = ops.quantize_act_int8(xt)
        xs = (xi.float() * sx.unsqueeze(1))[rows]
    else:
        xs = xt.float()[rows]
    if kind == "swiglu":
        twp = ops.repack_tiles(w, s, b, swiglu_pairs=True)
        got = ops.gather_qmm_swiglu_sorted_tiles(xt, twp, t, x_rows=lhs)
        gu = _reference(xs, w, s, b, off).double()
        g, u = gu[:, : N // 2], gu[:, N // 2:]
        ref = g / (1.0 + torch.exp(-g)) * u
    else:
        tw = ops.repack_tiles(w, s, b)
        if kind == "int8":
            got = ops.gather_qmm_int8_sorted_tiles(xi, sx, tw, t, x_rows=lhs)
        else:
            got = ops.gather_qmm_sorted_tiles(xt, tw, t, x_rows=lhs)
        ref = _reference(xs, w, s, b, off, rounded=kind != "int8")
    torch.cuda.synchronize()
    assert_close_bf16(orc, bits(got), ref.double().cpu().numpy(), what=f"{kind} gate_up, every output")


@pytest.mark.parametrize("kind", ["bf16", "int8"])
def test_prefill_down_whole_output_full_size(dev, orc, kind):
    """The down projection over the sorted h rows (K = I = 512, N = 2048), as
    the MoE block runs it at 4096 tokens: no row gather."""
    wl, r, lhs, _, off, _ = _routed(dev, orc, 3)
    t = r.tiles
    R = int(wl["idx"].size)
    rng = np.random.default_rng(23)
    wd, sd, bd = synth.quant_weights(rng, (E, 2048), 512)
    w, s, b = words_t(wd, dev), bf16_t(sd, dev), bf16_t(bd, dev)
    h = bf16_t(synth.bf16_bits(rng.normal(size=(R, 512)).astype(np.float32)), dev)
    say(f"{kind} down grouped GEMM, every output: {R} rows x 2048, K = 512")
    tw = ops.repack_tiles(w, s, b)
    if kind == "int8":
        hq, sh = ops.quantize_act_int8(h)
        got = ops.gather_qmm_int8_sorted_tiles(hq, sh, tw, t)
        xs = hq.float() * sh.unsqueeze(1)
    else:
        got = ops.gather_qmm_sorted_tiles(h, tw, t)
        xs = h.float()
    ref = _reference(xs, w, s, b, off, rounded=kind != "int8")
    torch.cuda.synchronize()
    assert_close_bf16(orc, bits(got), ref.double().cpu().numpy(), what=f"{kind} down, every output")
