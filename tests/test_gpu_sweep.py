"""Seeded random layers across shapes, token counts, logit bias, renormalisation
and merge mode, through layer.moe_forward, against the oracle.

Each case draws a shape inside every kernel's limits (the Qwen3-30B-A3B and
DeepSeek-V2-Lite shapes and smaller ones, E from 32 to 256, k from 2 to 8),
a token count from 1 (the single-launch decode) through the multi-block pack
(above 2048 ids) to 4096, and the other switches.  Routing must be bit-exact
against the oracle given the kernel's logits; a sample of tokens (the first,
the last and up to six more) must be within max rel err 1e-2 and mean abs
err 1e-3 of the oracle's layer output with the same merge.
"""
import random

import numpy as np
import pytest
import torch

from tests.gpu_helpers import MAX_REL, MEAN_ABS, err_metrics, oracle_tokens_given_routing, u16

pytestmark = pytest.mark.gpu
DEV = "cuda"

SHAPES = [(2048, 768, 128, 8), (2048, 1408, 64, 6), (1024, 512, 64, 4), (512, 256, 32, 4), (1536, 384, 96, 6),
          (2048, 768, 256, 8), (768, 256, 32, 2)]
TOKENS = [1, 2, 3, 7, 9, 16, 33, 100, 255, 256, 257, 511, 512, 777, 1000, 2047, 2049, 3001, 4096]


def _case(i):
    """Case i: every shape and every token count within the first 19 cases,
    the switches and the seed drawn."""
    rng = random.Random(4000 + i)
    return dict(shape=SHAPES[i % len(SHAPES)], T=TOKENS[(5 * i) % len(TOKENS)], normalize=rng.random() < 0.7,
                merge=rng.choice(["fused", "reference"]), bias=rng.random() < 0.3, seed=rng.randrange(1 << 20))


@pytest.mark.parametrize("i", range(24))
def test_random_layer_against_the_oracle(orc, i):
    from pdscope_amd import layer, ops, synthetic
    c = _case(i)
    H, I, E, k = c["shape"]
    T = c["T"]
    print(f"case {i}: {c}", flush=True)
    lay = synthetic.make_layer(H, I, E, k, c["normalize"], seed=c["seed"], device=DEV)
    slots = ops.slot_table([lay.experts[e] for e in range(E)], DEV)
    ws = layer.MoEWorkspace(T, H, I, E, k, DEV)
    x = synthetic.make_tokens(T, H, seed=c["seed"] + 1, device=DEV)
    bias = synthetic.zipf_bias(E, 1.1, seed=c["seed"] + 2, device=DEV)[0] if c["bias"] else None
    out, logits, ids, w = layer.moe_forward(x, lay.gate, slots, ws, normalize=c["normalize"], bias=bias,
                                            merge=c["merge"])
    torch.cuda.synchronize()
    ids_np = ids.cpu().numpy()
    oi, ow = orc.route_from_logits(u16(logits), k, c["normalize"],
                                   bias=None if bias is None else bias.cpu().numpy())
    assert np.array_equal(ids_np, oi) and np.array_equal(u16(w), ow), "routing differs from the oracle's"
    rng = random.Random(c["seed"])
    tokens = sorted(set(rng.sample(range(T), min(T, 6))) | {0, T - 1})
    experts = u16(lay.experts)
    ref, _ = oracle_tokens_given_routing(orc, u16(x), ids_np, u16(w), tokens, lambda e: experts[e], H, I,
                                         merge=c["merge"])
    m = err_metrics(orc.bf16_to_f32(u16(out)[tokens]), orc.bf16_to_f32(ref))
    assert m["max_rel"] <= MAX_REL and m["mean_abs"] <= MEAN_ABS, m
