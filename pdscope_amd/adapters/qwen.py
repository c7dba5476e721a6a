"""Qwen3-MoE expert math on the gfx950 kernels (mirror of expertbench/adapters/qwen.py).

Same names and argument meaning as the reference adapter:
``route`` (qwen.py:140-152), ``Routing`` (:132-137), ``expert_groups``
(:155-174), ``expert_forward`` (:87-90), ``reference_fp32`` (:93-98) and
``PROJECTIONS`` (:27).  ``route`` and ``expert_forward`` run on the GPU
through the C-ABI; there is no CPU or eager-torch fallback.

Differences that are part of the contract here: ``selected`` ties break
toward the lower expert id (torch.topk leaves the order unspecified), and an
optional fp32 logit ``bias`` may be added before the softmax.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from .. import ops
from ..executor import PROJECTIONS, ExpertWeights, expert_rows  # noqa: F401


@dataclass(frozen=True)
class Routing:
    logits: object
    selected: object
    weights: object
    probabilities: object = None


def route(inputs, gate, top_k, normalize, *, capture_probabilities=False, bias=None):
    """Qwen3's gate: bf16 logits, fp32 softmax, top-k (ties -> lower id), optional renorm."""
    if inputs.ndim != 2 or inputs.shape[1] != gate.shape[1] or inputs.dtype != gate.dtype:
        raise ValueError("router input shape/dtype mismatch")
    if (type(top_k) is not int or not 0 < top_k <= gate.shape[0] or type(normalize) is not bool
            or type(capture_probabilities) is not bool):
        raise ValueError("invalid routing parameters")
    logits, ids, weights, probs = ops.route_topk(inputs.contiguous(), gate.contiguous(), top_k, normalize,
                                                 bias=bias, capture_probabilities=capture_probabilities)
    return Routing(logits, ids.long(), weights, probs)


def expert_groups(routing, *, mode="generic"):
    """[(expert, token indices, weights)] in ascending expert order.

    'generic': rows of each expert in (top-k slot, token) order; 'single_token':
    one token, experts ascending, each with its own slot weight.
    """
    if mode not in ("generic", "single_token"):
        raise ValueError("unsupported expert grouping mode")
    sel = routing.selected
    if mode == "single_token":
        if sel.ndim != 2 or sel.shape[0] != 1:
            raise ValueError("single-token grouping requires exactly one token")
        ids = sel[0].tolist()
        if not ids or len(set(ids)) != len(ids):
            raise ValueError("single-token grouping requires distinct selected expert IDs")
        tokens = torch.zeros((1,), dtype=torch.long, device=sel.device)
        return [(e, tokens, routing.weights[0, s:s + 1]) for s, e in sorted(enumerate(ids), key=lambda p: p[1])]
    T, k = sel.shape
    E = int(sel.max().item()) + 1
    packed = ops.pack(sel.to(torch.int32).contiguous(), E)
    counts = packed.counts.tolist()
    offsets = packed.offsets.tolist()
    tokens = packed.perm_token.long()
    pos = packed.perm_pos.long()
    w = routing.weights.reshape(-1)[pos]
    return [(e, tokens[offsets[e]:offsets[e + 1]], w[offsets[e]:offsets[e + 1]]) for e in range(E) if counts[e]]


def expert_forward(inputs, tensors):
    """y = down(silu(gate(x)) * up(x)) for one expert whose three projections are
    consecutive views of one gate|up|down block (the executor's slot layout)."""
    g, u, d = (tensors[n] for n in PROJECTIONS)
    I, H = g.shape
    nb = g.numel() * g.element_size()
    if (u.data_ptr() != g.data_ptr() + nb or d.data_ptr() != g.data_ptr() + 2 * nb
            or not all(t.is_contiguous() and t.is_cuda for t in (g, u, d))):
        raise ValueError("expert_forward needs the gate|up|down projections as one contiguous device block")
    return expert_rows(inputs, g.data_ptr(), H, I)


def reference_fp32(inputs, tensors):
    """Full-fp32 CPU reference with explicit matmul and sigmoid SiLU (test helper)."""
    x = inputs.float().cpu()
    gate = x @ tensors["gate_proj"].float().cpu().T
    up = x @ tensors["up_proj"].float().cpu().T
    return ((gate * torch.sigmoid(gate)) * up) @ tensors["down_proj"].float().cpu().T
