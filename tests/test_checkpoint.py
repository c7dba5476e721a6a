"""On-disk expert/router formats and host master storage (CPU tests).

A small Qwen3-MoE checkpoint (config.json, model.safetensors.index.json and
two safetensors shards, tensor names as expertbench/adapters/qwen.py:66,117)
is written to a temporary directory; the loaders must return its tensors
bit for bit and refuse unsafe shard paths, shape or dtype mismatches,
dense layers and over-budget reads.  The pinned pool layout is checked
against its packing rule; collect_model_experts against a randomly
initialised transformers Qwen3-MoE model.
"""
import json

import pytest
import torch

from pdscope_amd.cache import ExpertKey
from pdscope_amd.checkpoint import (collect_model_experts, load_expert, load_router, pinned_master_layout,
                                    read_json_bounded, tensor_hash)

H, I, E, L = 64, 32, 4, 3


def write_checkpoint(root, *, mlp_only=(), router_dtype=torch.bfloat16, shard_map=None, H=H, I=I, E=E, L=L, top_k=2):
    from safetensors.torch import save_file
    gen = torch.Generator().manual_seed(11)
    tensors = {}
    for l in range(L):
        tensors[f"model.layers.{l}.mlp.gate.weight"] = torch.randn(E, H, generator=gen).to(router_dtype)
        for e in range(E):
            for proj, shape in (("gate_proj", (I, H)), ("up_proj", (I, H)), ("down_proj", (H, I))):
                tensors[f"model.layers.{l}.mlp.experts.{e}.{proj}.weight"] = (
                    torch.randn(*shape, generator=gen) * 0.02).to(torch.bfloat16)
    names = sorted(tensors)
    half = len(names) // 2
    shards = {"model-00001-of-00002.safetensors": names[:half], "model-00002-of-00002.safetensors": names[half:]}
    weight_map = {}
    for fname, part in shards.items():
        save_file({n: tensors[n].contiguous() for n in part}, str(root / fname))
        weight_map.update({n: fname for n in part})
    if shard_map:
        weight_map.update(shard_map)
    (root / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": weight_map}))
    cfg = dict(model_type="qwen3_moe", hidden_act="silu", num_hidden_layers=L, num_experts=E, hidden_size=H,
               moe_intermediate_size=I, num_experts_per_tok=top_k, norm_topk_prob=True, decoder_sparse_step=1,
               mlp_only_layers=list(mlp_only))
    (root / "config.json").write_text(json.dumps(cfg))
    return tensors


def test_load_expert_and_router_round_trip(tmp_path):
    tensors = write_checkpoint(tmp_path)
    w = load_expert(tmp_path, ExpertKey(2, 3, "bf16"))
    for proj in ("gate_proj", "up_proj", "down_proj"):
        assert torch.equal(w.tensors[proj], tensors[f"model.layers.2.mlp.experts.3.{proj}.weight"])
        assert w.tensors[proj].is_contiguous() and w.tensors[proj].dtype == torch.bfloat16
    assert w.nbytes == 3 * I * H * 2
    assert w.provenance["tensors"]["up_proj"]["sha256"] == tensor_hash(
        tensors["model.layers.2.mlp.experts.3.up_proj.weight"])
    gate, cfg, info = load_router(tmp_path, 1)
    assert torch.equal(gate, tensors["model.layers.1.mlp.gate.weight"])
    assert cfg["num_experts_per_tok"] == 2 and info["shape"] == [E, H] and info["bytes"] == E * H * 2


def test_loaders_refuse_bad_requests(tmp_path):
    write_checkpoint(tmp_path, mlp_only=(0,))
    with pytest.raises(ValueError, match="outside"):
        load_expert(tmp_path, ExpertKey(L, 0, "bf16"))
    with pytest.raises(ValueError, match="outside"):
        load_expert(tmp_path, ExpertKey(0, E, "bf16"))
    with pytest.raises(ValueError, match="BF16"):
        load_expert(tmp_path, ExpertKey(0, 0, "fp8"))
    with pytest.raises(ValueError, match="budget"):
        load_expert(tmp_path, ExpertKey(0, 0, "bf16"), max_bytes=3 * I * H * 2 - 1)
    with pytest.raises(ValueError, match="sparse"):
        load_router(tmp_path, 0)   # listed in mlp_only_layers
    with pytest.raises(ValueError, match="sparse"):
        load_router(tmp_path, L)


@pytest.mark.parametrize("bad", ["../outside.safetensors", "/abs/model.safetensors", "model.bin"])
def test_unsafe_shard_paths_are_refused(tmp_path, bad):
    name = "model.layers.1.mlp.experts.0.gate_proj.weight"
    write_checkpoint(tmp_path, shard_map={name: bad})
    with pytest.raises(ValueError, match="shard path"):
        load_expert(tmp_path, ExpertKey(1, 0, "bf16"))


def test_router_dtype_mismatch_is_refused(tmp_path):
    write_checkpoint(tmp_path, router_dtype=torch.float32)
    with pytest.raises(ValueError, match="mismatch"):
        load_router(tmp_path, 1)


def test_json_bound(tmp_path):
    p = tmp_path / "big.json"
    p.write_text(json.dumps({"x": "y" * 100}))
    assert read_json_bounded(p)["x"] == "y" * 100
    with pytest.raises(ValueError, match="bound"):
        read_json_bounded(p, cap_bytes=50)


def test_pinned_layout_packs_whole_experts_in_order():
    sizes = {ExpertKey(l, e, "bf16"): 6 for l in range(2) for e in range(5)}
    blocks = pinned_master_layout(sizes, block_cap_bytes=16)
    # two experts (12 bytes) per 16-byte block, in (layer, expert) order, nothing split
    flat = [k for b in blocks for k in b]
    assert flat == sorted(sizes, key=lambda k: (k.layer, k.expert))
    assert all(len(b) == 2 for b in blocks[:-1]) and len(blocks) == 5
    assert all(sum(sizes[k] for k in b) <= 16 for b in blocks)
    for cap, szs in ((24, sizes), (16, {ExpertKey(0, 0, "bf16"): 18}), (16, {ExpertKey(0, 0, "bf16"): 5}), (16, {})):
        with pytest.raises(ValueError):
            pinned_master_layout(szs, block_cap_bytes=cap)


def test_collect_model_experts_from_transformers_model():
    from transformers import Qwen3MoeConfig, Qwen3MoeForCausalLM
    cfg = Qwen3MoeConfig(vocab_size=64, hidden_size=H, intermediate_size=2 * H, moe_intermediate_size=I,
                         num_hidden_layers=2, num_attention_heads=2, num_key_value_heads=1, head_dim=32,
                         num_experts=E, num_experts_per_tok=2, decoder_sparse_step=1, mlp_only_layers=[])
    torch.manual_seed(0)
    model = Qwen3MoeForCausalLM(cfg).to(torch.bfloat16).eval()
    masters = collect_model_experts(model)
    assert len(masters) == 2 * E
    for (l, e) in ((0, 0), (1, E - 1)):
        w = masters[ExpertKey(l, e, "bf16")]
        experts = model.model.layers[l].mlp.experts
        if hasattr(experts, "gate_up_proj"):
            gu, down = experts.gate_up_proj[e], experts.down_proj[e]
            ref = {"gate_proj": gu[:I], "up_proj": gu[I:], "down_proj": down}
        else:
            ref = {p: getattr(experts[e], p).weight for p in ("gate_proj", "up_proj", "down_proj")}
        for p in ref:
            assert w.tensors[p].shape == ref[p].shape and torch.equal(w.tensors[p], ref[p])
            assert w.tensors[p].data_ptr() == ref[p].data_ptr()  # views of the model's storage
