"""A transformers Qwen3-MoE model driven through PDScopeCudaRuntime (the model
hook-up of benchmarks/pdscope_compare.py:181-212 and forward_layer :285-304).

``install_expert_blocks(model, forward_layer)`` replaces every decoder
layer's sparse MoE block by an ``ExpertBlock`` that keeps only the router
weight and calls ``forward_layer(layer, hidden, gate_weight)``.  The block
returns ``(out, router_logits)`` where the installed transformers decoder
unpacks a pair (4.x) and ``out`` where it takes a tensor (5.x).

``ModelSession(model, ...)`` is that driver: it takes the model's expert
masters (``collect_model_experts``), packs them into pooled pinned blocks,
installs the blocks, moves the rest of the model to the GPU and creates the
runtime with a static hot set; ``forward_layer`` feeds each layer call with
the caller's step (``session.step``: 0 for the prompt, then 1, 2, ... per
decoded token) and the next layer's router for the gate-fallback prefetch,
and keeps the runtime's per-layer trace rows.
"""
from __future__ import annotations

import torch

from .cache import ExpertKey
from .checkpoint import collect_model_experts, pin_cpu_master_storage
from .pdscope_runtime import PDScopeCudaRuntime


class ExpertBlock(torch.nn.Module):
    """Stand-in for a decoder layer's sparse MoE block (pdscope_compare.py:198-200)."""

    def __init__(self, gate, layer, forward_layer, return_router_logits):
        super().__init__()
        self.gate, self.layer = gate, layer
        self._forward_layer = forward_layer
        self.return_router_logits = return_router_logits

    def forward(self, hidden):
        out, logits = self._forward_layer(self.layer, hidden, self.gate.weight)
        return (out, logits) if self.return_router_logits else out


def _returns_pair():
    import transformers
    return int(transformers.__version__.split(".")[0]) < 5


def install_expert_blocks(model, forward_layer, *, return_router_logits=None):
    """Replace every sparse MoE block; returns {layer: original block}."""
    if return_router_logits is None:
        return_router_logits = _returns_pair()
    originals = {}
    for layer, decoder in enumerate(model.model.layers):
        if not hasattr(decoder.mlp, "experts") or not hasattr(decoder.mlp, "gate"):
            raise ValueError("dense layers require a separate adapter")
        originals[layer] = decoder.mlp
        decoder.mlp = ExpertBlock(decoder.mlp.gate, layer, forward_layer, return_router_logits)
    return originals


class ModelSession:
    """Qwen3-MoE model whose expert layers run on the gfx950 path.

    hot_per_layer: experts per layer placed in the static hot set (the first
    ones of ``hot_order[layer]`` when given, else ids 0, 1, ...);
    speculative_slots, demand_slots and the other keywords go to
    PDScopeCudaRuntime."""

    def __init__(self, model, *, hot_per_layer, speculative_slots, demand_slots=2, hot_order=None,
                 device=0, block_cap_bytes=256 * 1024**2, **runtime_kwargs):
        if model.config.model_type != "qwen3_moe":
            raise ValueError("only Qwen3 MoE supported")
        self.model = model
        self.device = torch.device("cuda", device) if isinstance(device, int) else torch.device(device)
        self.top_k = model.config.num_experts_per_tok
        self.normalize = bool(model.config.norm_topk_prob)
        self.masters = collect_model_experts(model)
        self.pinned = pin_cpu_master_storage(self.masters, block_cap_bytes=block_cap_bytes)
        self.gates = {}
        install_expert_blocks(model, self.forward_layer)
        for layer, decoder in enumerate(model.model.layers):
            self.gates[layer] = decoder.mlp.gate
        model.to(self.device)
        E = model.config.num_experts
        hot = []
        for layer in self.gates:
            order = list(hot_order[layer]) if hot_order is not None else list(range(E))
            hot += [ExpertKey(layer, e, "bf16") for e in order[:hot_per_layer]]
        self.runtime = PDScopeCudaRuntime(self.masters, hot_keys=hot, speculative_slots=speculative_slots,
                                          device=self.device.index, demand_slots=demand_slots, **runtime_kwargs)
        self.step = 0
        self.request = "pdscope"
        self.traces = []

    def forward_layer(self, layer, hidden, gate):
        shape = hidden.shape
        x = hidden.reshape(-1, shape[-1])
        nxt = self.gates.get(layer + 1)
        out, routing, row = self.runtime.forward(x, gate, layer=layer, step=self.step, request=self.request,
                                                 next_gate=None if nxt is None else nxt.weight,
                                                 top_k=self.top_k, normalize=self.normalize)
        if sum(row["token_counts"].values()) != x.shape[0] * self.top_k:
            raise AssertionError("missing routed assignment")
        self.traces.append(row)
        return out.reshape(shape), routing.logits

    def close(self):
        self.runtime.close()
