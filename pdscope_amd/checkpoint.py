"""Where expert weights come from: Qwen3-MoE safetensors checkpoints, loaded
transformers models, and the page-locked host pool they are staged from.

Interfaces kept from the reference so the same checkpoints and callers work:
tensor names ``model.layers.{l}.mlp.experts.{e}.{gate,up,down}_proj.weight``
and ``model.layers.{l}.mlp.gate.weight`` in a sharded checkpoint with
``model.safetensors.index.json`` (expertbench/adapters/qwen.py:48-129), the
functions ``load_expert(model_path, key, max_bytes)`` -> ExpertWeights and
``load_router(model_path, layer)`` -> (weight, config, info),
``collect_model_experts(model)`` (qwen.py:177-191), and the pooled
page-locked master storage ``pin_cpu_master_storage`` /
``pinned_master_layout`` (qwen.py:194-261) plus private copies
``copy_cpu_master_storage`` (qwen.py:264-288).

How it is built here:

* ``SafetensorsCheckpoint`` opens a checkpoint directory once: it reads the
  config and the index (bounded JSON), derives the MoE shape and which layers
  are sparse, resolves every tensor name to a shard inside the directory, and
  reads tensors with their shape and dtype verified through the safetensors
  slice API before any bytes are copied.
* Pooled pinned storage lays whole experts out in (layer, expert) order and
  cuts the sequence into page-locked blocks of at most ``block_cap_bytes``;
  within its block every expert is one contiguous gate|up|down slice
  (``ExpertWeights.flat``), so staging it into an HBM slot is one DMA of
  exactly the slot layout the kernels read.

Invalid requests raise ValueError; a copy that breaks its own layout raises
AssertionError; a pinned allocation that is not what was asked for raises
RuntimeError.
"""
from __future__ import annotations

import hashlib
import json
from dataclasses import dataclass, field
from pathlib import Path

import torch

from .cache import ExpertKey
from .executor import PROJECTIONS, ExpertWeights

EXPERT_NAME = "model.layers.{layer}.mlp.experts.{expert}.{proj}.weight"
ROUTER_NAME = "model.layers.{layer}.mlp.gate.weight"
ROUTER_READ_CAP = 8 * 1024**2


def digest(payload):
    """SHA-256 hex digest of bytes or text."""
    return hashlib.sha256(payload.encode() if isinstance(payload, str) else payload).hexdigest()


def read_json_bounded(path, cap_bytes=8 * 1024**2):
    """Parse a JSON file, refusing one above cap_bytes (the size is checked first)."""
    path = Path(path)
    size = path.stat().st_size
    if size > cap_bytes:
        raise ValueError(f"{path.name} is {size} bytes, above the {cap_bytes}-byte JSON bound")
    return json.loads(path.read_bytes())


def tensor_hash(tensor):
    """SHA-256 of a tensor's raw bytes."""
    t = tensor.detach().to("cpu").contiguous()
    return digest(t.view(torch.uint8).numpy().tobytes())


@dataclass
class MoEShape:
    hidden: int
    intermediate: int
    experts: int
    layers: int
    top_k: int
    normalize: bool
    sparse_layers: frozenset = field(default_factory=frozenset)

    def expert_shapes(self):
        H, I = self.hidden, self.intermediate
        return {"gate_proj": (I, H), "up_proj": (I, H), "down_proj": (H, I)}

    @property
    def expert_bytes(self):
        return 3 * self.intermediate * self.hidden * 2


class SafetensorsCheckpoint:
    """A Qwen3-MoE checkpoint directory: config.json, the safetensors index
    and its shards."""

    def __init__(self, model_path):
        self.root = Path(model_path).resolve()
        self.config_path = self.root / "config.json"
        self.index_path = self.root / "model.safetensors.index.json"
        self.config = read_json_bounded(self.config_path)
        index = read_json_bounded(self.index_path)
        self.weight_map = dict(index.get("weight_map", {}))
        c = self.config
        if c.get("model_type") != "qwen3_moe":
            raise ValueError(f"a Qwen3 MoE checkpoint is required, config says {c.get('model_type')!r}")
        layers, step = c["num_hidden_layers"], c.get("decoder_sparse_step", 1)
        dense = set(c.get("mlp_only_layers", []))
        # transformers' Qwen3-MoE decoder: a layer has experts unless listed as
        # MLP-only, when experts exist and (layer + 1) is a multiple of the sparse step
        sparse = frozenset(l for l in range(layers)
                           if l not in dense and c.get("num_experts", 0) > 0 and (l + 1) % step == 0)
        self.shape = MoEShape(c["hidden_size"], c["moe_intermediate_size"], c["num_experts"], layers,
                              c["num_experts_per_tok"], c["norm_topk_prob"], sparse)

    def digests(self):
        return dict(config_sha256=digest(self.config_path.read_bytes()), index_sha256=digest(self.index_path.read_bytes()))

    def shard_of(self, name):
        """The shard file holding tensor `name`: a relative .safetensors path
        that stays inside the checkpoint directory."""
        rel = self.weight_map.get(name)
        if rel is None:
            raise ValueError(f"tensor {name} is not listed in the checkpoint index")
        rel = Path(rel)
        if rel.is_absolute() or ".." in rel.parts or rel.suffix != ".safetensors":
            raise ValueError(f"refusing shard path {str(rel)!r} for {name}: it must be a relative .safetensors file")
        path = (self.root / rel).resolve()
        if self.root not in path.parents:
            raise ValueError(f"refusing shard path {str(rel)!r} for {name}: it leaves the checkpoint directory")
        return path

    def read(self, name, shape):
        """Tensor `name` as an owned contiguous CPU bf16 tensor of `shape`."""
        from safetensors import safe_open
        path = self.shard_of(name)
        with safe_open(str(path), framework="pt", device="cpu") as f:
            meta = f.get_slice(name)
            got_shape, got_dtype = tuple(meta.get_shape()), meta.get_dtype()
            if got_shape != tuple(shape) or got_dtype != "BF16":
                raise ValueError(f"tensor {name}: shape/dtype mismatch ({got_shape}, {got_dtype}); "
                                 f"expected {tuple(shape)} BF16")
            return f.get_tensor(name).clone().contiguous(), path


def load_expert(model_path, key, max_bytes=64 * 1024**2):
    """One expert's gate, up and down projections (bf16) from a checkpoint."""
    ckpt = SafetensorsCheckpoint(model_path)
    s = ckpt.shape
    if ckpt.config.get("hidden_act") != "silu" or key.representation != "bf16":
        raise ValueError("only SiLU experts stored as original BF16 are supported")
    if not (0 <= key.layer < s.layers and 0 <= key.expert < s.experts):
        raise ValueError(f"{key} lies outside the checkpoint ({s.layers} layers x {s.experts} experts)")
    if type(max_bytes) is not int or s.expert_bytes > max_bytes:
        raise ValueError(f"an expert is {s.expert_bytes} bytes, above the read budget of {max_bytes}")
    tensors, record = {}, {}
    for proj, shape in s.expert_shapes().items():
        name = EXPERT_NAME.format(layer=key.layer, expert=key.expert, proj=proj)
        tensors[proj], path = ckpt.read(name, shape)
        record[proj] = dict(name=name, shard=str(path), shape=list(shape), sha256=tensor_hash(tensors[proj]))
    return ExpertWeights(key, tensors, dict(source="safetensors checkpoint", checkpoint=str(ckpt.root),
                                            tensors=record, **ckpt.digests()))


def load_router(model_path, layer, *, max_bytes=ROUTER_READ_CAP):
    """The router weight [E, H] of one sparse layer: (weight, config, info)."""
    ckpt = SafetensorsCheckpoint(model_path)
    s = ckpt.shape
    if type(layer) is not int or layer not in s.sparse_layers:
        raise ValueError(f"layer {layer!r} is not a sparse MoE layer of this checkpoint")
    if not 0 < s.top_k <= s.experts or type(s.normalize) is not bool:
        raise ValueError("the checkpoint's routing configuration is invalid")
    shape = (s.experts, s.hidden)
    nbytes = shape[0] * shape[1] * 2
    if nbytes > max_bytes:
        raise ValueError(f"the router is {nbytes} bytes, above its read budget of {max_bytes}")
    name = ROUTER_NAME.format(layer=layer)
    weight, path = ckpt.read(name, shape)
    return weight, ckpt.config, dict(name=name, shard=str(path), shape=list(shape), bytes=nbytes,
                                     sha256=tensor_hash(weight), **ckpt.digests())


def collect_model_experts(model):
    """ExpertWeights viewing every expert of a loaded transformers Qwen3-MoE
    model in place: per-expert modules (``mlp.experts[e].{gate,up,down}_proj``)
    or fused parameters (``mlp.experts.gate_up_proj`` [E, 2I, H] with the gate
    rows first, ``mlp.experts.down_proj`` [E, H, I])."""
    if model.config.model_type != "qwen3_moe":
        raise ValueError("collect_model_experts reads Qwen3 MoE models")
    out = {}
    for layer, block in enumerate(model.model.layers):
        experts = getattr(block.mlp, "experts", None)
        if experts is None:
            raise ValueError(f"layer {layer} is dense; its MLP has no experts")
        if hasattr(experts, "gate_up_proj"):
            gate_up, down = experts.gate_up_proj.detach(), experts.down_proj.detach()
            half = gate_up.shape[1] // 2
            per_expert = [dict(gate_proj=gate_up[e, :half], up_proj=gate_up[e, half:], down_proj=down[e])
                          for e in range(gate_up.shape[0])]
        else:
            per_expert = [{p: getattr(m, p).weight.detach() for p in PROJECTIONS} for m in experts]
        for e, tensors in enumerate(per_expert):
            if not all(t.device.type == "cpu" and t.dtype == torch.bfloat16 for t in tensors.values()):
                raise ValueError("model experts must be CPU bf16 tensors")
            key = ExpertKey(layer, e, "bf16")
            out[key] = ExpertWeights(key, tensors, {"source": "transformers model (CPU storage)"})
    return out


def pinned_master_layout(sizes, *, block_cap_bytes):
    """Experts in (layer, expert) order cut into consecutive groups of at most
    block_cap_bytes each; an expert is never split and a group closes when the
    next expert would not fit.  block_cap_bytes: a power of two up to 1 GiB
    (page-locked allocations are rounded up to powers of two); expert sizes:
    even and within the cap.  Returns a tuple of key tuples, one per block."""
    cap = block_cap_bytes
    if type(cap) is not int or cap <= 0 or cap > 1024**3 or cap & (cap - 1):
        raise ValueError("block_cap_bytes must be a power of two no larger than 1 GiB")
    if not sizes:
        raise ValueError("no experts to lay out")
    bad = [k for k, n in sizes.items() if type(n) is not int or n <= 0 or n % 2 or n > cap]
    if bad:
        raise ValueError(f"expert sizes must be even, positive and fit one block ({len(bad)} do not)")
    ordered = sorted(sizes, key=lambda k: (k.layer, k.expert, k.representation))
    starts = [0]
    fill = 0
    for i, key in enumerate(ordered):
        if fill + sizes[key] > cap:
            starts.append(i)
            fill = 0
        fill += sizes[key]
    bounds = starts + [len(ordered)]
    return tuple(tuple(ordered[a:b]) for a, b in zip(bounds, bounds[1:]))


def _check_masters(masters, *, allow_pinned):
    for key, w in masters.items():
        ok = (w.key == key and set(w.tensors) == set(PROJECTIONS)
              and all(t.device.type == "cpu" and t.dtype == torch.bfloat16 and t.is_contiguous()
                      and (allow_pinned or not t.is_pinned()) for t in w.tensors.values()))
        if not ok:
            raise ValueError(f"master {key} must hold contiguous CPU bf16 gate/up/down tensors"
                             + ("" if allow_pinned else " that are not already page-locked"))


def pin_cpu_master_storage(masters, *, block_cap_bytes, check_budget=lambda: None):
    """Move every master into pooled page-locked blocks (pinned_master_layout),
    each expert one contiguous gate|up|down slice of its block.  `masters` is
    updated in place (tensors become views of the block, ``flat`` the slice).
    check_budget() runs before each allocation and after each copy.
    Returns a summary: experts and bytes copied, and one record per block."""
    _check_masters(masters, allow_pinned=False)
    sizes = {k: w.nbytes for k, w in masters.items()}
    layout = pinned_master_layout(sizes, block_cap_bytes=block_cap_bytes)
    blocks = []
    for index, keys in enumerate(layout):
        need = sum(sizes[k] for k in keys)
        check_budget()
        pool = torch.empty(need, dtype=torch.uint8, pin_memory=True)
        if not pool.is_pinned() or pool.numel() != need:
            raise RuntimeError(f"pinned block {index} is not the {need} page-locked bytes requested")
        base = 0
        for key in keys:
            src = masters[key]
            piece = pool[base:base + sizes[key]]
            views, at = {}, 0
            for proj in PROJECTIONS:
                t = src.tensors[proj]
                n = t.numel() * t.element_size()
                views[proj] = piece[at:at + n].view(t.dtype).view(t.shape)
                views[proj].copy_(t)
                at += n
            if at != sizes[key] or views["gate_proj"].data_ptr() != piece.data_ptr():
                raise AssertionError(f"pinned copy of {key} is not one gate|up|down slice")
            masters[key] = ExpertWeights(key, views, dict(src.provenance, storage="pooled page-locked block",
                                                         block=index, offset=base), flat=piece)
            base += sizes[key]
            check_budget()
        blocks.append(dict(index=index, experts=len(keys), bytes=need,
                           storage_bytes=pool.untyped_storage().nbytes(),
                           first=[keys[0].layer, keys[0].expert], last=[keys[-1].layer, keys[-1].expert]))
    copied = sum(sizes.values())
    return dict(experts_copied=len(masters), bytes_copied=copied, block_cap_bytes=block_cap_bytes, blocks=blocks)


def copy_cpu_master_storage(masters, *, check_budget=lambda: None):
    """Give every master private CPU storage (clones with the same strides),
    one expert at a time; `masters` is updated in place."""
    _check_masters(masters, allow_pinned=True)
    copied = 0
    for key in list(masters):
        src = masters[key]
        check_budget()
        own = {p: t.detach().clone(memory_format=torch.preserve_format) for p, t in src.tensors.items()}
        for p, t in own.items():
            if t.data_ptr() == src.tensors[p].data_ptr() or t.stride() != src.tensors[p].stride():
                raise AssertionError(f"private copy of {key}.{p} shares storage or changed its strides")
        masters[key] = ExpertWeights(key, own, dict(src.provenance, storage="private CPU copy"))
        copied += src.nbytes
        check_budget()
    return dict(experts_copied=len(masters), bytes_copied=copied)
