"""A MoE block loaded from an MLX-affine safetensors checkpoint
(titan_amd.loader) against the same block built from the arrays directly:
bit-identical outputs in decode and prefill form, the 8-bit router
dequantised bit-exactly, and the shared expert bound."""

import numpy as np
import pytest
import torch

from helpers import bf16_t, bits, words_t
from synth_ckpt import ROOT, make_checkpoint
from titan_amd import loader, moe_block, synth

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[case] {msg}", flush=True)


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    d = tmp_path_factory.mktemp("ckpt")
    layers, config = make_checkpoint(d)
    return d, layers, config


def _direct(a, dev, k):
    def trio(t):
        return words_t(t[0], dev), bf16_t(t[1], dev), bf16_t(t[2], dev)

    gu = tuple(np.concatenate([g, u], axis=1) for g, u in zip(a["gate"], a["up"]))
    shared = None
    if "sg" in a:
        sgu = tuple(np.concatenate([g, u], axis=1) for g, u in zip(a["sg"], a["su"]))
        shared = moe_block.SharedExpert(trio(sgu), trio(a["sd"]), bf16_t(a["sgate"], dev))
    if "router_q" in a:
        return moe_block.SparseMoeBlock(trio(a["router_q"]), trio(gu), trio(a["down"]), k, shared=shared,
                                        router_quant=(64, 8))
    return moe_block.SparseMoeBlock(bf16_t(a["router"], dev), trio(gu), trio(a["down"]), k, shared=shared)


@pytest.mark.parametrize("layer", [0, 1])
@pytest.mark.parametrize("T", [2, 64])
def test_loaded_block_matches_direct_block(dev, orc, ckpt, layer, T):
    d, layers, config = ckpt
    prefix = f"{ROOT}.{layer}.mlp"
    say(f"loaded MoE block {prefix} T={T}")
    a = layers[prefix]
    blk = loader.load_moe_block(d, prefix, device=dev)
    k = config["text_config"]["num_experts_per_tok"]
    assert blk.top_k == k and blk.num_experts == a["gate"][0].shape[0]
    if "router_q" in a:
        # kept quantised; the prefill GEMM's copy is the bf16 dequantisation
        w, s, b = a["router_q"]
        assert blk.router_quant == (64, 8)
        assert np.array_equal(blk.router_weight[0].cpu().numpy().view(np.uint32), w)
        want_router = orc.dequantize_bf16(w, s, b, 64, 8)
    else:
        assert np.array_equal(bits(blk.router_weight), a["router"])
        want_router = a["router"]
    assert np.array_equal(bits(blk._router_dense), want_router)
    assert (blk.shared is not None) == ("sg" in a)
    ref = _direct(a, dev, k)
    rng = np.random.default_rng(T + layer)
    x = bf16_t(synth.bf16_bits(rng.normal(size=(T, a["gate"][0].shape[2] * 8)).astype(np.float32)), dev)
    y, yr = blk(x), ref(x)
    torch.cuda.synchronize()
    assert np.array_equal(bits(y), bits(yr))
    assert torch.isfinite(y.float()).all()


def test_loader_passes_the_residency_choice(dev, ckpt):
    """``load_moe_block(resident=...)`` reaches the block: "both" keeps the
    MLX tensors beside the tile-layout copy and decodes from them; "tiles"
    (the default) keeps one copy where the tile-layout decode kernels take the
    shape -- not this checkpoint's (H = 1024, I = 256), so both keep both."""
    d, layers, config = ckpt
    prefix = f"{ROOT}.0.mlp"
    say(f"loaded MoE block {prefix}: resident tiles / both")
    one = loader.load_moe_block(d, prefix, device=dev)
    two = loader.load_moe_block(d, prefix, device=dev, resident="both")
    assert one.resident == "tiles" and two.resident == "both"
    assert not two.decode_tiles and not one.decode_tiles
    assert two.nbytes == one.nbytes
