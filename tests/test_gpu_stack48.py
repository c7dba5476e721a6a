"""The 48-layer stack at its full size, checked against the oracle.

48 Qwen3-30B-A3B-shaped MoE blocks (identity attention, residual and
RMSNorm between blocks) through PDScopeCudaRuntime, exactly as the bench's
stack workload builds them: 58 GB of pinned expert masters, a 24 GiB device
budget (allocator capped below it by the memory already in use outside the
allocator plus a margin, expert slots sized within the cap), 8 demand
staging slots, gate-fallback prefetch of the next layer and decode layers
served by their bound single-launch decode.  Prefill 2048 tokens,
then 64 decode steps.

At every layer of the prefill and of six seeded decode steps:
* routing bit-exact against the oracle given the kernel's logits, for every
  token;
* the layer output of sampled tokens (10 per prefill layer, the token of a
  decode layer) against the oracle with the runtime's merge (the reference's
  bf16 index_add_ in ascending expert id): max rel err <= 1e-2, mean abs
  err <= 1e-3.
At the end the ledger closes as in benchmarks/pdscope_compare.py:355-371 and
the device footprint (allocator peak plus memory outside the allocator)
fits the 24 GiB budget (:376-385); StackSession raises otherwise.
"""
import gc

import numpy as np
import pytest
import torch

from tests.gpu_helpers import MAX_REL, MEAN_ABS, err_metrics, oracle_tokens_given_routing, u16

pytestmark = pytest.mark.gpu


def _host_bf16(t):
    return t.view(torch.int16).numpy().view(np.uint16)


def test_stack48_full_size_against_the_oracle(orc):
    from pdscope_amd import stack
    dev = torch.device("cuda", 0)
    print("stack48: building 48 layers and pinning 58 GB of masters", flush=True)
    model = stack.build_stack(48, dev)
    H, I, k = model.H, model.I, model.k
    rng = np.random.default_rng(20261011)
    decode_checked = sorted({1, 64, *rng.choice(np.arange(2, 64), 4, replace=False).tolist()})
    checked = {"prefill": 0, "decode": 0, "tokens": 0}
    worst = {"max_rel": 0.0, "mean_abs": 0.0}

    def observe(call):
        torch.cuda.synchronize(dev)
        l, T = call.layer, call.x.shape[0]
        logits = u16(call.routing.logits)
        ids = call.routing.selected.cpu().numpy()
        w = u16(call.routing.weights)
        oi, ow = orc.route_from_logits(logits, k, True)
        assert np.array_equal(ids, oi) and np.array_equal(w, ow), f"step {call.step} layer {l}: routing"
        if T > 1:
            pick = np.random.default_rng(1000 * l + 7).choice(np.arange(1, T - 1), 8, replace=False)
            tokens = np.array(sorted({0, T - 1, *pick.tolist()}))
        else:
            tokens = np.array([0])
        ref, _ = oracle_tokens_given_routing(orc, u16(call.x), ids, w, tokens,
                                             lambda e: _host_bf16(model.expert_block(l, e)), H, I,
                                             merge=merge)
        got = u16(call.out)[tokens]
        m = err_metrics(orc.bf16_to_f32(got), orc.bf16_to_f32(ref))
        assert m["max_rel"] <= MAX_REL and m["mean_abs"] <= MEAN_ABS, (call.step, l, m)
        for kk in worst:
            worst[kk] = max(worst[kk], m[kk])
        checked["prefill" if call.step == 0 else "decode"] += 1
        checked["tokens"] += len(tokens)
        if l % 16 == 0:
            print(f"stack48 step {call.step} layer {l}: routing bit-exact, {len(tokens)} tokens "
                  f"max_rel={m['max_rel']:.2e} mean_abs={m['mean_abs']:.2e}", flush=True)

    session = stack.StackSession(model, dev)
    try:
        merge = session.runtime.merge
        assert merge == "reference"
        res = session.run(2048, 64, observe=observe, observe_steps={0, *decode_checked})
    finally:
        session.close()
    mem, cl = res["memory"], res["closure"]
    print(f"stack48: checked {checked}, worst {worst}; memory {mem}; closure {cl}", flush=True)
    assert checked["prefill"] == 48 and checked["decode"] == 48 * len(decode_checked)
    assert cl["layer_calls"] == 48 * 65
    assert cl["physical_demand_tokens"] == (2048 + 64) * 48 * k
    assert cl["h2d_bytes_submitted"] == cl["h2d_bytes_completed"] > 0
    assert mem["gpu_peak_reserved_plus_end_external_bytes"] <= 24 << 30
    assert res["prefill"]["demand_misses"] > 0, "the budget forced no demand misses"
    assert res["prefill"]["prefetch_issued"] > 0 and res["decode"]["prefetch_issued"] > 0
    assert res["decode"]["paths"] == ["bound_launch"]
    del session, model
    gc.collect()
    torch._C._host_emptyCache()
