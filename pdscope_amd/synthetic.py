"""Seeded synthetic MoE layers of the benchmark shapes (random init, no checkpoint).

Qwen3-30B-A3B layer: hidden 2048, 128 experts of intermediate 768, top-8,
router ~N(0, 0.02), experts ~N(0, 0.02), activations ~N(0, 1), all bf16.
DeepSeek-V2-Lite layer: hidden 2048, 64 routed experts of 1408, top-6 without
renormalisation, plus 2 shared experts of 1408 (one 2816-wide MLP).

Draw order (one generator, seed base 20261011): router, then the experts'
gate, up and down blocks in id order, then activations.  Expert blocks are
stored in one contiguous [E, 3*I*H] tensor whose row e is the slot layout
gate|up|down (expertbench/adapters/qwen.py:27; expertbench/executor.py:344-357).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

SEED = 20261011
QWEN = dict(H=2048, I=768, E=128, k=8, normalize=True)
DSV2 = dict(H=2048, I=1408, E=64, k=6, normalize=False, shared_I=2816)


@dataclass
class SyntheticLayer:
    H: int
    I: int
    E: int
    k: int
    normalize: bool
    gate: torch.Tensor      # [E, H] bf16
    experts: torch.Tensor   # [E, 3*I*H] bf16 (gate|up|down per row)
    shared: torch.Tensor | None = None  # [3*Is*H] bf16 (one fused shared MLP) or None

    def expert_views(self, e: int):
        b = self.experts[e]
        IH = self.I * self.H
        return (b[:IH].view(self.I, self.H), b[IH:2 * IH].view(self.I, self.H), b[2 * IH:].view(self.H, self.I))


def _normal(shape, std, gen, device, chunk=1 << 26):
    """N(0, std) drawn in fp32 in fixed-size chunks, cast to bf16."""
    n = 1
    for s in shape:
        n *= s
    out = torch.empty(n, dtype=torch.bfloat16, device=device)
    for i in range(0, n, chunk):
        m = min(chunk, n - i)
        out[i:i + m] = (torch.randn(m, generator=gen, device=device, dtype=torch.float32) * std).to(torch.bfloat16)
    return out.view(*shape)


def make_layer(H=2048, I=768, E=128, k=8, normalize=True, *, seed=SEED, device="cuda", shared_I=None):
    device = torch.device(device)
    gen = torch.Generator(device=device).manual_seed(seed)
    gate = _normal((E, H), 0.02, gen, device)
    experts = _normal((E, 3 * I * H), 0.02, gen, device)
    shared = _normal((3 * shared_I * H,), 0.02, gen, device) if shared_I else None
    return SyntheticLayer(H, I, E, k, normalize, gate, experts, shared)


def make_tokens(T, H, *, seed=SEED + 1, device="cuda"):
    device = torch.device(device)
    gen = torch.Generator(device=device).manual_seed(seed)
    return _normal((T, H), 1.0, gen, device)


def zipf_bias(E=128, s=1.1, *, seed=SEED, device="cpu"):
    """Router logit bias b_e = ln p_{pi(e)}, p_r ~ r^-s over a seeded permutation."""
    g = torch.Generator().manual_seed(seed)
    ranks = torch.arange(1, E + 1, dtype=torch.float64)
    p = ranks ** -s
    p = p / p.sum()
    perm = torch.randperm(E, generator=g)
    return torch.log(p[perm]).to(torch.float32).to(device), perm
