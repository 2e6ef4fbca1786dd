"""A small synthetic MLX-affine checkpoint on disk for the loader tests:
two MoE layers over two shards with an index, non-MoE tensors beside them,
an 8-bit router in layer 1 and a shared expert in layer 1."""

import json
from pathlib import Path

import numpy as np

from titan_amd import loader, synth

ROOT = "language_model.model.layers"


def layer_arrays(rng, E, H, I, S=0, router_bits=None):
    """numpy arrays of one layer: the routed experts as separate gate / up /
    down trios, the router, and (S > 0) a shared expert of width S."""
    g = synth.quant_weights(rng, (E, I), H)
    u = synth.quant_weights(rng, (E, I), H)
    d = synth.quant_weights(rng, (E, H), I)
    out = {"gate": g, "up": u, "down": d}
    rw = synth.bf16_bits((rng.normal(size=(E, H)) * 0.05).astype(np.float32))
    if router_bits:
        rq = synth.quant_weights(rng, (E,), H, bits=router_bits)
        out["router_q"] = rq
    out["router"] = rw
    if S:
        out["sg"] = synth.quant_weights(rng, (1, S), H)
        out["su"] = synth.quant_weights(rng, (1, S), H)
        out["sd"] = synth.quant_weights(rng, (1, H), S)
        out["sgate"] = synth.bf16_bits((rng.normal(size=(1, H)) * 0.05).astype(np.float32))
    return out


def _trio(prefix, t, squeeze=False):
    w, s, b = t
    if squeeze:
        w, s, b = w[0], s[0], b[0]
    return {f"{prefix}.weight": ("U32", w), f"{prefix}.scales": ("BF16", s), f"{prefix}.biases": ("BF16", b)}


def make_checkpoint(tmp: Path, E=8, H=1024, I=256, S=256, k=4, seed=0, router_bits=8):
    """Writes the checkpoint under tmp; returns (layers, config) where layers
    maps each MoE prefix to its numpy arrays."""
    tmp = Path(tmp)
    rng = np.random.default_rng(seed)
    layers = {}
    shards = [{}, {}]
    for li in (0, 1):
        prefix = f"{ROOT}.{li}.mlp"
        a = layer_arrays(rng, E, H, I, S=S if li == 1 else 0, router_bits=router_bits if li == 1 else None)
        layers[prefix] = a
        t = {}
        t.update(_trio(f"{prefix}.switch_mlp.gate_proj", a["gate"]))
        t.update(_trio(f"{prefix}.switch_mlp.up_proj", a["up"]))
        t.update(_trio(f"{prefix}.switch_mlp.down_proj", a["down"]))
        if "router_q" in a:
            t.update(_trio(f"{prefix}.gate", a["router_q"]))
        else:
            t[f"{prefix}.gate.weight"] = ("BF16", a["router"])
        if "sg" in a:
            t.update(_trio(f"{prefix}.shared_expert.gate_proj", a["sg"], squeeze=True))
            t.update(_trio(f"{prefix}.shared_expert.up_proj", a["su"], squeeze=True))
            t.update(_trio(f"{prefix}.shared_expert.down_proj", a["sd"], squeeze=True))
            t[f"{prefix}.shared_expert_gate.weight"] = ("BF16", a["sgate"])
        # non-MoE neighbours the plan must leave alone
        t[f"{ROOT}.{li}.input_layernorm.weight"] = ("BF16", np.full(H, 0x3F80, np.uint16))
        t[f"{ROOT}.{li}.self_attn.q_proj.weight"] = ("U32", rng.integers(0, 2**32, (16, H // 8), dtype=np.uint32))
        # gate and up of a layer in different shards: the fuse crosses shards
        for name, v in t.items():
            shards[(li + ("up_proj" in name)) % 2][name] = v
    names = ["model-00001-of-00002.safetensors", "model-00002-of-00002.safetensors"]
    weight_map = {}
    for sh, fn in zip(shards, names):
        loader.write_safetensors(tmp / fn, sh, {"format": "mlx"})
        weight_map.update({n: fn for n in sh})
    (tmp / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": weight_map}))
    config = {
        "model_type": "qwen3_5_moe",
        "text_config": {"hidden_size": H, "moe_intermediate_size": I, "num_experts": E,
                        "num_experts_per_tok": k, "norm_topk_prob": True,
                        "shared_expert_intermediate_size": S},
        "quantization": {"group_size": 64, "bits": 4,
                         f"{ROOT}.1.mlp.gate": {"group_size": 64, "bits": router_bits or 4}},
    }
    (tmp / "config.json").write_text(json.dumps(config))
    return layers, config
