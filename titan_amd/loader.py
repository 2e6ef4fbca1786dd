"""MLX-affine safetensors checkpoints -> MoE blocks on the device.

Scope: the tensors of the routed MoE path (titan/adapters/mlx/loader.py,
restricted to what the quantized-MoE block binds).  Two steps, as in the
reference (loader.py:1-31):

* :func:`plan_moe_layers` reads nothing but the safetensors headers and
  ``config.json``: for every MoE layer it names the checkpoint tensors of the
  routed experts (``switch_mlp.{gate,up,down}_proj.{weight,scales,biases}``,
  or an already fused ``gate_up_proj``), the router (``gate``), the optional
  shared expert and its gate, and the quantisation spec of each module
  (per-module override in ``config.json`` under any of its spellings, else
  the global block; loader.py:125-146, 264-275).
* :func:`load_moe_block` reads those tensors through a memory map of the
  shard, moves them to the device, fuses gate and up on the output axis
  (``concatenate([gate, up], axis=1)`` over weight, scales and biases alike:
  exact, because affine groups run along the input axis; loader.py:19-27,
  244-262) and builds a :class:`~titan_amd.moe_block.SparseMoeBlock`, whose
  constructor repacks the prefill copies into the tile layout once.  A
  quantised router stays quantised (its decode logits come from the codes);
  a quantised shared-expert gate is dequantised.

The header format is the published safetensors one: an 8-byte little-endian
header length, a JSON header mapping each tensor name to ``dtype``, ``shape``
and ``data_offsets`` (relative to the end of the header), then the data.
"""

from __future__ import annotations

import json
import re
import struct
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

__all__ = [
    "TensorMeta", "MoeLayerPlan", "read_safetensors_header", "shard_paths", "checkpoint_tensors", "load_config",
    "quant_spec", "plan_moe_layers", "read_tensor", "load_moe_tensors", "load_moe_block", "write_safetensors",
]

_DTYPES = {
    "BF16": (np.uint16, 2), "F16": (np.float16, 2), "F32": (np.float32, 4), "F64": (np.float64, 8),
    "U32": (np.uint32, 4), "I32": (np.int32, 4), "U16": (np.uint16, 2), "I16": (np.int16, 2),
    "U8": (np.uint8, 1), "I8": (np.int8, 1), "I64": (np.int64, 8), "U64": (np.uint64, 8),
}
_MAX_HEADER = 256 << 20
QUANT_SUFFIXES = ("weight", "scales", "biases")

# ``<prefix>.switch_mlp.<proj>.<suffix>`` (the routed experts of one MoE layer)
_SWITCH_RE = re.compile(r"^(.*)\.switch_mlp\.(gate_proj|up_proj|down_proj|gate_up_proj)\.(weight|scales|biases)$")


@dataclass(frozen=True)
class TensorMeta:
    """One tensor as a shard header declares it (checkpoint.py:45-65)."""

    name: str
    dtype: str
    shape: tuple
    shard: Path
    begin: int  # absolute file offset of the first byte
    end: int

    @property
    def nbytes(self) -> int:
        return self.end - self.begin


def read_safetensors_header(path) -> tuple[dict, int]:
    """(JSON header, absolute offset of the data section).  Reads the header only."""
    path = Path(path)
    with open(path, "rb") as f:
        raw = f.read(8)
        if len(raw) != 8:
            raise ValueError(f"{path}: not a safetensors file (short header length)")
        (n,) = struct.unpack("<Q", raw)
        if n <= 0 or n > _MAX_HEADER:
            raise ValueError(f"{path}: implausible safetensors header length {n}")
        blob = f.read(n)
        if len(blob) != n:
            raise ValueError(f"{path}: truncated header")
    return json.loads(blob), 8 + n


def shard_paths(model_dir) -> list[Path]:
    """Shards named by ``model.safetensors.index.json``, else every ``*.safetensors``."""
    model_dir = Path(model_dir)
    index = model_dir / "model.safetensors.index.json"
    if index.exists():
        weight_map = json.loads(index.read_text()).get("weight_map") or {}
        return [model_dir / n for n in sorted(set(weight_map.values()))]
    return sorted(model_dir.glob("*.safetensors"))


def checkpoint_tensors(model_dir) -> dict[str, TensorMeta]:
    """Every tensor of the checkpoint, from the shard headers; a name in two
    shards, an unknown dtype or offsets that disagree with the shape are errors."""
    out: dict[str, TensorMeta] = {}
    for shard in shard_paths(model_dir):
        header, data0 = read_safetensors_header(shard)
        size = shard.stat().st_size
        for name, e in header.items():
            if name == "__metadata__":
                continue
            if name in out:
                raise ValueError(f"tensor {name} appears in two shards")
            dt = e["dtype"]
            if dt not in _DTYPES:
                raise ValueError(f"{name}: unsupported dtype {dt}")
            b, en = (int(v) for v in e["data_offsets"])
            shape = tuple(int(d) for d in e["shape"])
            want = int(np.prod(shape, dtype=np.int64)) * _DTYPES[dt][1]
            if en - b != want or b < 0 or data0 + en > size:
                raise ValueError(f"{name}: data_offsets {b}..{en} do not fit shape {shape} {dt} in {shard.name}")
            out[name] = TensorMeta(name, dt, shape, shard, data0 + b, data0 + en)
    return out


def load_config(model_dir) -> dict:
    p = Path(model_dir) / "config.json"
    return json.loads(p.read_text()) if p.exists() else {}


def _text_config(config: dict) -> dict:
    return config.get("text_config") or config


def quant_spec(config: dict, module_path: str) -> dict:
    """``{"group_size", "bits"}`` of one module: the per-module override of the
    ``quantization`` block under any of its spellings (with or without the
    ``language_model.`` root, loader.py:125-146), else the global values
    (default 64 / 4)."""
    block = config.get("quantization") or config.get("quantization_config") or {}
    cands = [module_path]
    if module_path.startswith("language_model."):
        cands.append(module_path[len("language_model."):])
    else:
        cands.append("language_model." + module_path)
    if module_path.startswith("model.language_model."):
        cands.append("language_model.model." + module_path[len("model.language_model."):])
    for c in cands:
        v = block.get(c)
        if isinstance(v, dict) and "bits" in v:
            return {"group_size": int(v.get("group_size", block.get("group_size", 64))), "bits": int(v["bits"])}
    return {"group_size": int(block.get("group_size", 64)), "bits": int(block.get("bits", 4))}


@dataclass
class MoeLayerPlan:
    """The checkpoint tensors one MoE layer binds.

    ``gate_up`` maps suffix -> (gate name, up name) to fuse, or suffix ->
    (fused name,) when the checkpoint already holds ``gate_up_proj``;
    ``down`` suffix -> name; ``router`` / ``shared_gate`` suffix -> name
    (``weight`` only when unquantised); ``shared`` proj -> suffix -> name."""

    prefix: str
    gate_up: dict = field(default_factory=dict)
    down: dict = field(default_factory=dict)
    router: dict = field(default_factory=dict)
    shared: dict = field(default_factory=dict)
    shared_gate: dict = field(default_factory=dict)
    quant: dict = field(default_factory=dict)  # module path -> {"group_size", "bits"}

    def sources(self) -> list[str]:
        out = [n for v in self.gate_up.values() for n in v]
        out += list(self.down.values()) + list(self.router.values()) + list(self.shared_gate.values())
        out += [n for d in self.shared.values() for n in d.values()]
        return out


def _module_suffixes(tensors, module: str) -> dict:
    return {s: f"{module}.{s}" for s in QUANT_SUFFIXES if f"{module}.{s}" in tensors}


def plan_moe_layers(tensors: dict, config: dict | None = None) -> dict[str, MoeLayerPlan]:
    """Every MoE layer's tensors, keyed by the layer's ``...mlp`` prefix.
    Reads headers only.  A gate without its up half (or the reverse), a
    gate/up pair whose dtype or expert count differ, or routed experts
    without a router are errors."""
    config = config or {}
    groups: dict[str, dict] = {}
    for name in sorted(tensors):
        m = _SWITCH_RE.match(name)
        if m:
            prefix, proj, suffix = m.groups()
            groups.setdefault(prefix, {}).setdefault(proj, {})[suffix] = name
    plans: dict[str, MoeLayerPlan] = {}
    for prefix, projs in groups.items():
        p = MoeLayerPlan(prefix)
        if "gate_up_proj" in projs:
            if "gate_proj" in projs or "up_proj" in projs:
                raise ValueError(f"{prefix}: both fused gate_up_proj and separate gate/up projections")
            p.gate_up = {s: (n,) for s, n in projs["gate_up_proj"].items()}
        else:
            missing = {"gate_proj", "up_proj"} - set(projs)
            if missing:
                raise ValueError(f"{prefix}: cannot fuse, missing {sorted(missing)}")
            g, u = projs["gate_proj"], projs["up_proj"]
            if set(g) != set(u):
                raise ValueError(f"{prefix}: gate/up suffixes differ {sorted(g)} {sorted(u)}")
            for s in g:
                mg, mu = tensors[g[s]], tensors[u[s]]
                if mg.dtype != mu.dtype or mg.shape[0] != mu.shape[0] or mg.shape[2:] != mu.shape[2:]:
                    raise ValueError(f"{prefix}: gate/up mismatch {mg.shape} {mu.shape}")
                p.gate_up[s] = (g[s], u[s])
        if "down_proj" not in projs:
            raise ValueError(f"{prefix}: routed experts without down_proj")
        p.down = dict(projs["down_proj"])
        for need in ("weight", "scales"):
            if need not in p.gate_up or need not in p.down:
                raise ValueError(f"{prefix}: routed experts are not affine-quantised (no {need})")
        p.router = _module_suffixes(tensors, f"{prefix}.gate")
        if "weight" not in p.router:
            raise ValueError(f"{prefix}: routed experts without a router ({prefix}.gate.weight)")
        for proj in ("gate_proj", "up_proj", "down_proj"):
            d = _module_suffixes(tensors, f"{prefix}.shared_expert.{proj}")
            if d:
                p.shared[proj] = d
        if p.shared and set(p.shared) != {"gate_proj", "up_proj", "down_proj"}:
            raise ValueError(f"{prefix}: incomplete shared expert {sorted(p.shared)}")
        p.shared_gate = _module_suffixes(tensors, f"{prefix}.shared_expert_gate")
        if p.shared and "weight" not in p.shared_gate:
            raise ValueError(f"{prefix}: shared expert without shared_expert_gate")
        mods = [f"{prefix}.switch_mlp.gate_up_proj", f"{prefix}.switch_mlp.down_proj"]
        if "scales" in p.router:
            mods.append(f"{prefix}.gate")
        if p.shared:
            mods += [f"{prefix}.shared_expert.{proj}" for proj in ("gate_proj", "up_proj", "down_proj")]
        if "scales" in p.shared_gate:
            mods.append(f"{prefix}.shared_expert_gate")
        for mod in mods:
            spec = quant_spec(config, mod)
            if mod.endswith(".gate_up_proj") and not _has_override(config, mod):
                # the fused module has no override of its own: its halves' (loader.py:270-274)
                spec = quant_spec(config, mod[: -len("gate_up_proj")] + "gate_proj")
            p.quant[mod] = spec
        plans[prefix] = p
    return plans


def _has_override(config: dict, module_path: str) -> bool:
    block = config.get("quantization") or config.get("quantization_config") or {}
    roots = {module_path, module_path.removeprefix("language_model."), "language_model." + module_path}
    return any(isinstance(block.get(c), dict) for c in roots)


# numpy dtype a tensor is read as, and the torch dtype it is viewed as after
# (bf16 arrives as its int16 bit patterns, unsigned words as signed ones)
_HOST_VIEW = {"BF16": (np.int16, "bfloat16"), "U32": (np.int32, None), "U16": (np.int16, None),
              "U64": (np.int64, None)}


def read_tensor(meta: TensorMeta):
    """The tensor's data as a host torch tensor, read through a memory map of
    the shard.  bf16 arrives as torch.bfloat16, u32 as int32 words (the same
    bits)."""
    import torch

    npdt, hv = _HOST_VIEW.get(meta.dtype, (_DTYPES[meta.dtype][0], None))
    arr = np.memmap(meta.shard, dtype=np.uint8, mode="r", offset=meta.begin, shape=(meta.nbytes,))
    t = torch.from_numpy(np.array(arr).view(npdt).reshape(meta.shape))
    return t.view(getattr(torch, hv)) if hv else t


def _dense(tensors, d: dict, device, spec):
    """A router / gate weight as bf16 [out, in]: as stored, or dequantised
    on the device when the checkpoint quantises it."""
    import torch

    w = read_tensor(tensors[d["weight"]]).to(device)
    if "scales" not in d:
        return w.to(torch.bfloat16)
    from . import ops

    s = read_tensor(tensors[d["scales"]]).to(device)
    b = read_tensor(tensors[d["biases"]]).to(device) if "biases" in d else torch.zeros_like(s)
    return ops.dequantize(w, s, b, spec["group_size"], spec["bits"])


def load_moe_tensors(tensors: dict, plan: MoeLayerPlan, device="cpu") -> dict:
    """The layer's device tensors: ``gate_up`` / ``down`` (w, scales, biases)
    with gate_up fused gate rows first, and the shared expert's projections
    with a leading expert axis of one."""
    import torch

    def trio(d):
        return tuple(read_tensor(tensors[d[s]]).to(device) if s in d else None for s in QUANT_SUFFIXES)

    gu = []
    for s in QUANT_SUFFIXES:
        names = plan.gate_up.get(s)
        if names is None:
            gu.append(None)
        elif len(names) == 1:
            gu.append(read_tensor(tensors[names[0]]).to(device))
        else:
            gu.append(torch.cat([read_tensor(tensors[n]).to(device) for n in names], dim=1))
    out = {"gate_up": tuple(gu), "down": trio(plan.down)}
    if plan.shared:
        g, u, d = (trio(plan.shared[p]) for p in ("gate_proj", "up_proj", "down_proj"))
        out["shared_gate_up"] = tuple(None if a is None else torch.cat([a, c], dim=0)[None] for a, c in zip(g, u))
        out["shared_down"] = tuple(None if a is None else a[None] for a in d)
    return out


def load_moe_block(model_dir, prefix: str | None = None, device="cuda", *, tensors=None, config=None,
                   plans=None, wsum_mode: str = "fast", prefill_tiles: bool = True, resident: str = "tiles"):
    """Load one MoE layer (the first one, or the one at ``prefix``) into a
    :class:`~titan_amd.moe_block.SparseMoeBlock` on ``device``.  ``top_k``
    and ``norm_topk_prob`` come from the config's text section
    (``num_experts_per_tok``, default 8; ``norm_topk_prob``, default True).
    ``resident`` is the block's: "tiles" keeps one tile-layout copy of the
    expert weights, "both" keeps the MLX tensors for decode as well."""
    import torch

    from . import moe_block

    tensors = checkpoint_tensors(model_dir) if tensors is None else tensors
    config = load_config(model_dir) if config is None else config
    plans = plan_moe_layers(tensors, config) if plans is None else plans
    if not plans:
        raise ValueError("no MoE layer in the checkpoint")
    if prefix is None:
        prefix = sorted(plans, key=_layer_order)[0]
    plan = plans[prefix]
    spec = plan.quant[f"{prefix}.switch_mlp.gate_up_proj"]
    if plan.quant[f"{prefix}.switch_mlp.down_proj"] != spec:
        raise ValueError(f"{prefix}: gate_up and down quantised differently "
                         f"({spec} vs {plan.quant[f'{prefix}.switch_mlp.down_proj']})")
    t = load_moe_tensors(tensors, plan, device)
    gu, dn = _with_biases(t["gate_up"]), _with_biases(t["down"])
    rspec = plan.quant.get(f"{prefix}.gate") or spec
    if "scales" in plan.router:  # kept quantised: the decode logits come from the codes
        router = _with_biases(tuple(read_tensor(tensors[plan.router[s]]).to(device) if s in plan.router else None
                                    for s in QUANT_SUFFIXES))
    else:
        router = _dense(tensors, plan.router, device, None)
    shared = None
    if plan.shared:
        sspec = plan.quant[f"{prefix}.shared_expert.gate_proj"]
        if sspec != spec:
            raise ValueError(f"{prefix}: shared expert quantised as {sspec}, routed experts as {spec}")
        sg = _dense(tensors, plan.shared_gate, device, plan.quant.get(f"{prefix}.shared_expert_gate"))
        shared = moe_block.SharedExpert(_with_biases(t["shared_gate_up"]), _with_biases(t["shared_down"]),
                                        sg.reshape(1, -1))
    text = _text_config(config)
    top_k = int(text.get("num_experts_per_tok", 8))
    norm = bool(text.get("norm_topk_prob", True))
    return moe_block.SparseMoeBlock(router, gu, dn, top_k, norm_topk_prob=norm, wsum_mode=wsum_mode,
                                    group_size=spec["group_size"], bits=spec["bits"], shared=shared,
                                    prefill_tiles=prefill_tiles, resident=resident,
                                    router_quant=(rspec["group_size"], rspec["bits"]))


def _with_biases(trio):
    import torch

    w, s, b = trio
    return (w, s, torch.zeros_like(s) if b is None else b)


def _layer_order(prefix: str):
    m = re.search(r"layers\.(\d+)\.", prefix + ".")
    return (int(m.group(1)) if m else 1 << 30, prefix)


def write_safetensors(path, arrays: dict, metadata: dict | None = None) -> None:
    """Write ``{name: (dtype, numpy array)}`` as one safetensors shard (dtype a
    header code such as "U32" or "BF16"; BF16 arrays are uint16 bit patterns).
    Tensors are laid out back to back in name order (no holes), the header
    padded with spaces to a multiple of 8 bytes."""
    header: dict = {}
    if metadata:
        header["__metadata__"] = {str(k): str(v) for k, v in metadata.items()}
    blobs = []
    off = 0
    for name in sorted(arrays):
        dt, a = arrays[name]
        _, size = _DTYPES[dt]
        a = np.ascontiguousarray(a)
        if a.dtype.itemsize != size:
            raise ValueError(f"{name}: {a.dtype} does not hold {dt}")
        raw = a.tobytes()
        header[name] = {"dtype": dt, "shape": list(a.shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    hb = json.dumps(header, separators=(",", ":")).encode()
    hb += b" " * ((-len(hb)) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hb)))
        f.write(hb)
        for blob in blobs:
            f.write(blob)
