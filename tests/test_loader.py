"""The safetensors loader of the MoE path (titan_amd.loader) on the CPU:
headers, the per-layer plan, quantisation overrides and the fused gate_up
layout (titan/adapters/mlx/loader.py:19-27, 125-146, 244-275;
titan/adapters/mlx/checkpoint.py:68-106)."""

import json
import re
import struct

import numpy as np
import pytest
import torch

from synth_ckpt import ROOT, make_checkpoint
from titan_amd import loader


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    d = tmp_path_factory.mktemp("ckpt")
    layers, config = make_checkpoint(d)
    return d, layers, config


def test_headers_round_trip(ckpt):
    d, layers, _ = ckpt
    t = loader.checkpoint_tensors(d)
    p = f"{ROOT}.0.mlp"
    m = t[f"{p}.switch_mlp.gate_proj.weight"]
    assert m.dtype == "U32" and m.shape == layers[p]["gate"][0].shape
    assert m.nbytes == layers[p]["gate"][0].nbytes
    # every tensor's bytes read back bit for bit
    got = loader.read_tensor(t[f"{p}.switch_mlp.down_proj.scales"])
    assert got.dtype == torch.bfloat16
    assert np.array_equal(got.view(torch.int16).numpy().view(np.uint16), layers[p]["down"][1])
    w = loader.read_tensor(m)
    assert w.dtype == torch.int32 and np.array_equal(w.numpy().view(np.uint32), layers[p]["gate"][0])


def test_reader_agrees_with_the_safetensors_library(tmp_path):
    from safetensors.torch import load_file, save_file

    rng = np.random.default_rng(3)
    a = torch.from_numpy(rng.integers(-2**31, 2**31 - 1, (5, 7), dtype=np.int64).astype(np.int32))
    b = torch.randn(3, 64).to(torch.bfloat16)
    c = torch.randn(2, 3, 4)
    save_file({"a": a, "b.x": b, "c": c}, str(tmp_path / "lib.safetensors"))
    t = loader.checkpoint_tensors(tmp_path)
    assert torch.equal(loader.read_tensor(t["a"]), a)
    assert torch.equal(loader.read_tensor(t["b.x"]).view(torch.int16), b.view(torch.int16))
    assert torch.equal(loader.read_tensor(t["c"]), c)
    # and the library reads what this module writes
    loader.write_safetensors(tmp_path / "own.safetensors",
                             {"w": ("U32", np.arange(12, dtype=np.uint32).reshape(3, 4)),
                              "s": ("BF16", np.array([0x3F80, 0xC000], np.uint16))})
    back = load_file(str(tmp_path / "own.safetensors"))
    assert back["w"].view(torch.int32).tolist() == np.arange(12).reshape(3, 4).tolist()
    assert back["s"].float().tolist() == [1.0, -2.0]


def test_bad_headers_are_errors(tmp_path):
    p = tmp_path / "bad.safetensors"
    hdr = json.dumps({"x": {"dtype": "F32", "shape": [4], "data_offsets": [0, 12]}}).encode()
    p.write_bytes(struct.pack("<Q", len(hdr)) + hdr + b"\0" * 16)
    with pytest.raises(ValueError, match="do not fit"):
        loader.checkpoint_tensors(tmp_path)
    p.write_bytes(struct.pack("<Q", 1 << 40) + b"{}")
    with pytest.raises(ValueError, match="implausible"):
        loader.checkpoint_tensors(tmp_path)
    q = tmp_path / "dup"
    q.mkdir()
    for i in range(2):
        loader.write_safetensors(q / f"s{i}.safetensors", {"x": ("F32", np.zeros(2, np.float32))})
    with pytest.raises(ValueError, match="two shards"):
        loader.checkpoint_tensors(q)


def test_plan_claims_every_moe_tensor_once(ckpt):
    d, _, config = ckpt
    t = loader.checkpoint_tensors(d)
    plans = loader.plan_moe_layers(t, config)
    assert sorted(plans) == [f"{ROOT}.0.mlp", f"{ROOT}.1.mlp"]
    src = [n for p in plans.values() for n in p.sources()]
    assert len(src) == len(set(src))
    moe = {n for n in t if re.search(r"\.mlp\.", n)}
    assert set(src) == moe
    assert not any("self_attn" in n or "layernorm" in n for n in src)
    p0, p1 = plans[f"{ROOT}.0.mlp"], plans[f"{ROOT}.1.mlp"]
    assert p0.gate_up["weight"] == (f"{ROOT}.0.mlp.switch_mlp.gate_proj.weight",
                                    f"{ROOT}.0.mlp.switch_mlp.up_proj.weight")
    assert set(p0.router) == {"weight"} and not p0.shared
    assert set(p1.router) == {"weight", "scales", "biases"}
    assert set(p1.shared) == {"gate_proj", "up_proj", "down_proj"} and set(p1.shared_gate) == {"weight"}
    assert p1.quant[f"{ROOT}.1.mlp.gate"] == {"group_size": 64, "bits": 8}
    assert p1.quant[f"{ROOT}.1.mlp.switch_mlp.gate_up_proj"] == {"group_size": 64, "bits": 4}


def test_quant_override_spellings():
    cfg = {"quantization": {"group_size": 64, "bits": 4,
                            "language_model.model.layers.3.mlp.gate": {"group_size": 64, "bits": 8},
                            "model.layers.5.mlp.switch_mlp.gate_proj": {"group_size": 32, "bits": 4}}}
    assert loader.quant_spec(cfg, "model.layers.3.mlp.gate") == {"group_size": 64, "bits": 8}
    assert loader.quant_spec(cfg, "language_model.model.layers.3.mlp.gate") == {"group_size": 64, "bits": 8}
    assert loader.quant_spec(cfg, "model.language_model.layers.3.mlp.gate") == {"group_size": 64, "bits": 8}
    assert loader.quant_spec(cfg, "model.layers.4.mlp.gate") == {"group_size": 64, "bits": 4}
    assert loader.quant_spec({}, "x") == {"group_size": 64, "bits": 4}
    # the fused module takes its gate half's override
    names = {f"model.layers.5.mlp.switch_mlp.{p}.{s}" for p in ("gate_proj", "up_proj", "down_proj")
             for s in ("weight", "scales", "biases")} | {"model.layers.5.mlp.gate.weight"}
    t = {n: None for n in names}
    for n in names:
        shape = (2, 4, 8) if "switch_mlp" in n else (2, 64)
        t[n] = loader.TensorMeta(n, "U32", shape, None, 0, 0)
    plans = loader.plan_moe_layers(t, cfg)
    assert plans["model.layers.5.mlp"].quant["model.layers.5.mlp.switch_mlp.gate_up_proj"] == \
        {"group_size": 32, "bits": 4}


def test_plan_errors(ckpt):
    d, _, config = ckpt
    t = loader.checkpoint_tensors(d)
    no_up = {n: m for n, m in t.items() if ".0.mlp.switch_mlp.up_proj" not in n}
    with pytest.raises(ValueError, match="missing"):
        loader.plan_moe_layers(no_up, config)
    no_router = {n: m for n, m in t.items() if n != f"{ROOT}.0.mlp.gate.weight"}
    with pytest.raises(ValueError, match="router"):
        loader.plan_moe_layers(no_router, config)
    no_sgate = {n: m for n, m in t.items() if "shared_expert_gate" not in n}
    with pytest.raises(ValueError, match="shared_expert_gate"):
        loader.plan_moe_layers(no_sgate, config)


def test_fused_gate_up_is_the_concatenation(ckpt):
    d, layers, config = ckpt
    t = loader.checkpoint_tensors(d)
    plans = loader.plan_moe_layers(t, config)
    for prefix, a in layers.items():
        got = loader.load_moe_tensors(t, plans[prefix], "cpu")
        for i, (gu, dn) in enumerate(zip(got["gate_up"], got["down"])):
            want = np.concatenate([a["gate"][i], a["up"][i]], axis=1)
            assert np.array_equal(gu.view(torch.int16 if i else torch.int32).numpy().view(want.dtype), want)
            assert np.array_equal(dn.view(torch.int16 if i else torch.int32).numpy().view(a["down"][i].dtype),
                                  a["down"][i])
        if "sg" in a:
            sgu = got["shared_gate_up"][0].numpy().view(np.uint32)
            assert sgu.shape[0] == 1
            assert np.array_equal(sgu[0], np.concatenate([a["sg"][0][0], a["su"][0][0]], axis=0))
