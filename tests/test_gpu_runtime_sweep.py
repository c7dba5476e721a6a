"""Seeded random sequences through the drop-in runtime (PDScopeCudaRuntime).

Each case draws a shape (the Qwen3-30B-A3B shape and smaller ones), 2 or 3
layers, the share of experts in the static hot set (none to all), the
speculative and demand slots, resident decode on or off, the merge mode,
next-layer prefetch on or off and the prompt length, then runs one request:
a prefill step and three decode steps through every layer, each layer's
output (layer-normed with its input) feeding the next.  Every call serves
one of the runtime's paths (grouped with staging, the whole-layer prefill
launch, the single-launch decode or the bound decode launch); every output
is checked against the oracle given the call's routing, with the runtime's
merge, and the ledger closes at the end.
"""
import random

import pytest
import torch

from tests.test_gpu_runtime import build, check_output, closure

pytestmark = pytest.mark.gpu

SHAPES = [(512, 256, 32, 4), (1024, 512, 64, 4), (768, 256, 32, 2), (2048, 768, 128, 8)]


def _case(i):
    rng = random.Random(7000 + i)
    H, I, E, k = SHAPES[i % len(SHAPES)]
    return dict(shape=(H, I, E, k), layers=2 + i % 2, hot_frac=[0.0, 0.25, 0.5, 1.0][(i // 2) % 4],
                spec=rng.choice([0, 2, 4, 8]), demand_slots=rng.choice([2, 4, 8]) if k <= 4 else 8,
                graphs=i % 3 != 2, merge=["reference", "fused"][(i // 4) % 2], prefetch=rng.random() < 0.7,
                T0=rng.choice([2, 5, 31, 64, 200]), seed=rng.randrange(1 << 20))


@pytest.mark.parametrize("i", range(12))
def test_random_request_through_the_runtime(orc, i):
    from pdscope_amd import synthetic
    from pdscope_amd.cache import ExpertKey
    from pdscope_amd.pdscope_runtime import PDScopeCudaRuntime
    c = _case(i)
    H, I, E, k = c["shape"]
    nl = c["layers"]
    print(f"case {i}: {c}", flush=True)
    rng = random.Random(c["seed"])
    layers, masters = build(nl, H, I, E, k, seed=c["seed"])
    nh = int(round(c["hot_frac"] * E))
    hot = [ExpertKey(l, e, "bf16") for l in range(nl) for e in rng.sample(range(E), nh)]
    rt = PDScopeCudaRuntime(masters, hot_keys=hot, speculative_slots=c["spec"], demand_slots=c["demand_slots"],
                            resident_graphs=c["graphs"], merge=c["merge"])
    paths = set()
    try:
        x = synthetic.make_tokens(c["T0"], H, seed=c["seed"] + 1)
        for step in range(4):
            for l in range(nl):
                nxt = layers[l + 1].gate if (c["prefetch"] and l + 1 < nl) else None
                out, routing, row = rt.forward(x, layers[l].gate, layer=l, step=step, next_gate=nxt, top_k=k,
                                               request="r")
                torch.cuda.synchronize()
                check_output(orc, out, routing, x, layers[l], H, I, k, row=row)
                paths.add(row["decode_path"])
                x = torch.nn.functional.layer_norm(out.float() + x.float(), (H,)).to(torch.bfloat16)
            if step == 0:
                x = x[-1:].contiguous()
        closure(rt)
        print(f"case {i}: paths {sorted(paths)}", flush=True)
    finally:
        rt.close()
