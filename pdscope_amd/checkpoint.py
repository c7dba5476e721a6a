"""On-disk and host-memory formats of the expert masters (drop-in for the loader
half of expertbench/adapters/qwen.py).

* ``load_expert(model_path, key, max_bytes)`` / ``load_router(model_path, layer)``
  read single tensors of a Qwen3-MoE safetensors checkpoint through its index,
  with the reference's names (``model.layers.{l}.mlp.experts.{e}.{proj}.weight``,
  ``model.layers.{l}.mlp.gate.weight``), shape/dtype checks, shard-path safety
  checks and read budgets (qwen.py:48-84, :101-129).
* ``collect_model_experts(model)`` takes CPU references to every expert of a
  loaded transformers Qwen3-MoE model (qwen.py:175-190); it accepts both the
  per-expert module layout (transformers 4.x) and the fused ``gate_up_proj`` /
  ``down_proj`` parameters of later versions (gate rows first).
* ``pinned_master_layout`` / ``pin_cpu_master_storage`` pack whole experts,
  gate|up|down back to back, into page-locked blocks of at most
  ``block_cap_bytes`` (qwen.py:193-261).  Each expert's bytes are one
  contiguous slice of its block, kept as ``ExpertWeights.flat``, so staging an
  expert into an HBM slot is one DMA of the slot layout the kernels read.
* ``copy_cpu_master_storage`` owns private CPU copies (qwen.py:264-289).

Invalid inputs raise ValueError; broken copy invariants AssertionError; a
pinned allocation that does not meet its contract RuntimeError.
"""
from __future__ import annotations

import hashlib
import json
from pathlib import Path

import torch

from .cache import ExpertKey
from .executor import PROJECTIONS, ExpertWeights


def digest(payload):
    """SHA-256 hex digest of bytes or text (provenance records)."""
    return hashlib.sha256(payload.encode() if isinstance(payload, str) else payload).hexdigest()


def read_json_bounded(path, cap_bytes=8 * 1024**2):
    """A small JSON document, refused above cap_bytes."""
    path = Path(path)
    if path.stat().st_size > cap_bytes:
        raise ValueError(f"{path} exceeds the {cap_bytes} byte JSON bound")
    return json.loads(path.read_text())


def tensor_hash(tensor):
    """SHA-256 of a tensor's bytes (CPU copy, contiguous)."""
    return digest(tensor.detach().cpu().contiguous().view(torch.uint8).numpy().tobytes())


def weights_hashes(weights):
    return {name: tensor_hash(t) for name, t in weights.tensors.items()}


def _checkpoint(model_path):
    root = Path(model_path).resolve()
    config_path, index_path = root / "config.json", root / "model.safetensors.index.json"
    return root, config_path, index_path, read_json_bounded(config_path), read_json_bounded(index_path)


def _shard(root, index, name):
    """Path of the shard holding tensor `name`, refusing paths that leave the checkpoint."""
    try:
        relative = Path(index["weight_map"][name])
    except KeyError as exc:
        raise ValueError(f"{name} is not in the checkpoint index") from exc
    path = (root / relative).resolve()
    if relative.is_absolute() or ".." in relative.parts or root not in path.parents or path.suffix != ".safetensors":
        raise ValueError("unsafe or unsupported checkpoint shard path")
    return path


def _read(path, name, shape):
    from safetensors import safe_open
    with safe_open(str(path), framework="pt", device="cpu") as handle:
        view = handle.get_slice(name)
        if list(view.get_shape()) != list(shape) or view.get_dtype() != "BF16":
            raise ValueError(f"checkpoint shape/dtype mismatch: {name}")
        # own the bytes once the shard's mapping is closed
        return handle.get_tensor(name).clone().contiguous()


def load_expert(model_path, key, max_bytes=64 * 1024**2):
    """One expert's three BF16 projections from a Qwen3-MoE checkpoint (qwen.py:48-84)."""
    root, config_path, index_path, cfg, index = _checkpoint(model_path)
    if cfg.get("model_type") != "qwen3_moe" or cfg.get("hidden_act") != "silu" or key.representation != "bf16":
        raise ValueError("only Qwen3 MoE SiLU with original BF16 experts is supported")
    if not 0 <= key.layer < cfg["num_hidden_layers"] or not 0 <= key.expert < cfg["num_experts"]:
        raise ValueError("expert index outside checkpoint config")
    H, I = cfg["hidden_size"], cfg["moe_intermediate_size"]
    shapes = {"gate_proj": [I, H], "up_proj": [I, H], "down_proj": [H, I]}
    if type(max_bytes) is not int or not 0 < 3 * I * H * 2 <= max_bytes:
        raise ValueError("selected expert exceeds the explicit weight read budget")
    tensors, files = {}, {}
    for proj in PROJECTIONS:
        name = f"model.layers.{key.layer}.mlp.experts.{key.expert}.{proj}.weight"
        path = _shard(root, index, name)
        tensors[proj] = _read(path, name, shapes[proj])
        st = path.stat()
        files[proj] = dict(tensor_name=name, shard=str(path), shard_bytes=st.st_size, shard_mtime_ns=st.st_mtime_ns,
                           shape=shapes[proj], dtype="bfloat16")
    weights = ExpertWeights(key, tensors, {})
    weights.provenance.update(model_path=str(root), config_sha256=digest(config_path.read_bytes()),
                              index_sha256=digest(index_path.read_bytes()), tensors=files,
                              tensor_sha256=weights_hashes(weights), selected_bytes=weights.nbytes,
                              full_checkpoint_checksums="not_computed", checkpoint_revision="unverified")
    return weights


def load_router(model_path, layer):
    """The gate weight [E, H] of one sparse layer and the routing contract (qwen.py:101-129).
    Returns (weight, config, info)."""
    root, config_path, index_path, cfg, index = _checkpoint(model_path)
    if (cfg.get("model_type") != "qwen3_moe" or type(layer) is not int
            or not 0 <= layer < cfg["num_hidden_layers"] or layer in cfg.get("mlp_only_layers", [])
            or (layer + 1) % cfg.get("decoder_sparse_step", 1) != 0):
        raise ValueError("requested layer is not a Qwen3 sparse MoE layer")
    top_k = cfg["num_experts_per_tok"]
    if not 0 < top_k <= cfg["num_experts"] or type(cfg["norm_topk_prob"]) is not bool:
        raise ValueError("invalid native routing contract")
    name = f"model.layers.{layer}.mlp.gate.weight"
    path = _shard(root, index, name)
    shape = [cfg["num_experts"], cfg["hidden_size"]]
    if shape[0] * shape[1] * 2 > 8 * 1024**2:
        raise ValueError("router exceeds 8 MiB read limit")
    weight = _read(path, name, shape)
    return weight, cfg, dict(tensor_name=name, shard=str(path), shape=shape, dtype=str(weight.dtype),
                             bytes=weight.numel() * weight.element_size(), sha256=tensor_hash(weight),
                             config_sha256=digest(config_path.read_bytes()),
                             index_sha256=digest(index_path.read_bytes()))


def collect_model_experts(model):
    """CPU references to every expert of a Qwen3-MoE model (qwen.py:175-190).

    Per-expert modules (``mlp.experts[e].{gate,up,down}_proj``) and fused
    parameters (``mlp.experts.gate_up_proj`` [E, 2I, H], gate rows first, and
    ``mlp.experts.down_proj`` [E, H, I]) are both accepted; the tensors are
    views of the model's own CPU storage."""
    if model.config.model_type != "qwen3_moe":
        raise ValueError("only Qwen3 MoE supported")
    masters = {}
    for layer, decoder in enumerate(model.model.layers):
        experts = getattr(decoder.mlp, "experts", None)
        if experts is None:
            raise ValueError("dense layers require a separate adapter")
        if hasattr(experts, "gate_up_proj"):
            gu, down = experts.gate_up_proj.detach(), experts.down_proj.detach()
            I = gu.shape[1] // 2
            views = [{"gate_proj": gu[e, :I], "up_proj": gu[e, I:], "down_proj": down[e]} for e in range(gu.shape[0])]
        else:
            views = [{name: getattr(mlp, name).weight.detach() for name in PROJECTIONS} for mlp in experts]
        for expert, tensors in enumerate(views):
            if any(t.device.type != "cpu" or t.dtype != torch.bfloat16 for t in tensors.values()):
                raise ValueError("model masters must already be CPU BF16")
            key = ExpertKey(layer, expert, "bf16")
            masters[key] = ExpertWeights(key, tensors, {"source": "loaded native checkpoint CPU storage"})
    return masters


def pinned_master_layout(sizes, *, block_cap_bytes):
    """Whole experts in (layer, expert) order packed into blocks of at most
    block_cap_bytes (a power of two up to 1 GiB); returns a tuple of key
    tuples, one per block (qwen.py:193-205)."""
    if (type(block_cap_bytes) is not int or not 0 < block_cap_bytes <= 1024**3
            or block_cap_bytes & (block_cap_bytes - 1) or not sizes
            or any(type(n) is not int or n <= 0 or n % 2 or n > block_cap_bytes for n in sizes.values())):
        raise ValueError("pinned master layout requires even expert bytes within a power-of-two block cap")
    blocks, current, used = [], [], 0
    for key in sorted(sizes, key=lambda k: (k.layer, k.expert, k.representation)):
        if used + sizes[key] > block_cap_bytes:
            blocks.append(tuple(current))
            current, used = [], 0
        current.append(key)
        used += sizes[key]
    blocks.append(tuple(current))
    return tuple(blocks)


def pin_cpu_master_storage(masters, *, block_cap_bytes, check_budget=lambda: None):
    """Copy every expert into owned page-locked blocks, gate|up|down back to back
    (qwen.py:208-261).  masters is updated in place: each entry's tensors become
    views of its block and ``flat`` its whole contiguous slice.  Returns a
    summary of the blocks.  check_budget() is called around every allocation
    and copy; on failure the registry may be partly converted."""
    for key, weights in masters.items():
        if (weights.key != key or set(weights.tensors) != set(PROJECTIONS)
                or any(t.device.type != "cpu" or t.dtype != torch.bfloat16 or not t.is_contiguous()
                       or t.is_pinned() for t in weights.tensors.values())):
            raise ValueError("pooled pinned copy requires unpinned contiguous CPU BF16 weights")
    sizes = {key: w.nbytes for key, w in masters.items()}
    groups = pinned_master_layout(sizes, block_cap_bytes=block_cap_bytes)
    records, copied = [], 0
    for block_index, keys in enumerate(groups):
        payload = sum(sizes[k] for k in keys)
        check_budget()
        block = torch.empty(payload, dtype=torch.uint8, device="cpu", pin_memory=True)
        if not block.is_pinned() or block.numel() != payload:
            raise RuntimeError("pinned block allocation did not meet the source contract")
        check_budget()
        offset = 0
        for key in keys:
            weights = masters[key]
            start = offset
            tensors = {}
            for name in PROJECTIONS:
                src = weights.tensors[name]
                n = src.numel() * src.element_size()
                dst = block[offset:offset + n].view(src.dtype).view(src.shape)
                dst.copy_(src)
                if dst.data_ptr() == src.data_ptr() or dst.data_ptr() != block.data_ptr() + offset:
                    raise AssertionError("pinned expert view aliases its source or changes the packed layout")
                tensors[name] = dst
                offset += n
            masters[key] = ExpertWeights(key, tensors, {**weights.provenance,
                                                        "storage": "owned pooled pinned CPU BF16 copy",
                                                        "pinned_pool_block": block_index,
                                                        "pinned_pool_offset_bytes": start},
                                         flat=block[start:offset])
            copied += sizes[key]
            check_budget()
        if offset != payload:
            raise AssertionError("pinned expert packing does not conserve source bytes")
        records.append(dict(block=block_index, requested_bytes=payload,
                            storage_bytes=block.untyped_storage().nbytes(), experts=len(keys),
                            first_key=[keys[0].layer, keys[0].expert, keys[0].representation],
                            last_key=[keys[-1].layer, keys[-1].expert, keys[-1].representation]))
    return dict(mode="pooled_pinned_copy", experts_copied=len(masters), copied_bytes=copied,
                pinned_payload_bytes=copied, blocks=records, block_cap_bytes=block_cap_bytes,
                pool_tensor_storage_bytes=sum(r["storage_bytes"] for r in records))


def copy_cpu_master_storage(masters, *, check_budget=lambda: None):
    """Private CPU copies of every expert, one at a time (qwen.py:264-289)."""
    copied = 0
    for key in masters:
        weights = masters[key]
        if (weights.key != key or set(weights.tensors) != set(PROJECTIONS)
                or any(t.device.type != "cpu" or t.dtype != torch.bfloat16 or not t.is_contiguous()
                       for t in weights.tensors.values())):
            raise ValueError("private master copy requires contiguous CPU BF16 weights")
        check_budget()
        tensors = {name: t.detach().clone(memory_format=torch.preserve_format) for name, t in weights.tensors.items()}
        if any(t.data_ptr() == weights.tensors[name].data_ptr() or t.stride() != weights.tensors[name].stride()
               for name, t in tensors.items()):
            raise AssertionError("private CPU copy aliases its source or changes the layout")
        masters[key] = ExpertWeights(key, tensors, {**weights.provenance,
                                                    "storage": "private CPU copy"})
        copied += weights.nbytes
        check_budget()
    return dict(experts_copied=len(masters), copied_bytes=copied, source_storage_reused=False, strides_preserved=True)
