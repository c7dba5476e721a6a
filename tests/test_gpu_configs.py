"""GPU parity tests at the benchmark configurations' own sizes.

* T=512 uniform Qwen3-30B-A3B-shaped layer, all 128 experts resident, on the
  64-row tile that launch selects: every token's grouped rows and merged
  output against the oracle.
* DeepSeek-V2-Lite-shaped mixed batch (48 decode tokens + 256 + 1000 prefill
  tokens in one launch, 64 routed experts top-6 without renormalisation, 2
  shared experts as one 2816-wide MLP) on the 256-row routed tile and the
  1304-row shared expert: grouping in full, and a seeded sample of tokens
  from every segment (with the segment boundaries) against the oracle.
* A chained stack of Qwen-shaped MoE blocks through PDScopeCudaRuntime
  (identity attention, residual and RMSNorm between blocks), with masters in
  pinned host memory, an HBM slot cap that forces demand misses through the
  8 staging slots, gate-fallback prefetch of the next layer and decode steps
  served by each layer's bound single-launch decode: every layer of the prefill and of
  each decode step against the oracle given the runtime's routing.

Routing is checked bit-exact against the oracle given the kernel's logits;
expert rows and layer outputs within max rel err <= 1e-2 and mean abs err
<= 1e-3.
"""
import numpy as np
import pytest
import torch

from tests.gpu_helpers import MAX_REL, MEAN_ABS, err_metrics, oracle_layer_given_routing, u16, ulp_diff_bf16

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _close(orc, got_u16, ref_u16, what):
    m = err_metrics(orc.bf16_to_f32(got_u16), orc.bf16_to_f32(ref_u16))
    assert m["max_rel"] <= MAX_REL and m["mean_abs"] <= MEAN_ABS, (what, m)
    return m


def test_prefill_t512_uniform_every_token(orc):
    from pdscope_amd import layer, ops, synthetic
    H, I, E, k, T = 2048, 768, 128, 8, 512
    lay = synthetic.make_layer(**synthetic.QWEN, device=DEV)
    x = synthetic.make_tokens(T, H, seed=20261011 + 7)
    ws = layer.MoEWorkspace(T, H, I, E, k, DEV)
    slots = ops.slot_table([lay.experts[e] for e in range(E)], DEV)
    assert ops.grouped_block_m(T * k // E) == 64
    out, logits, ids, w = layer.moe_forward(x, lay.gate, slots, ws)
    torch.cuda.synchronize()
    ik, wk, xu = ids.cpu().numpy(), u16(w), u16(x)
    oi, ow = orc.route_from_logits(u16(logits), k, True)
    assert np.array_equal(ik, oi) and np.array_equal(wk, ow), "routing differs from the oracle"
    ref, y_ref, p = oracle_layer_given_routing(orc, xu, ik, wk, u16(lay.experts), H, I)
    assert np.array_equal(ws.row_of[:T * k].cpu().numpy(), p["row_of"])
    assert np.array_equal(ws.offsets.cpu().numpy(), p["offsets"])
    assert int((p["counts"] > 0).sum()) == E, "uniform T=512 routing should touch every expert"
    y_k = u16(ws.y[:T * k * H]).reshape(T * k, H)
    _close(orc, y_k, y_ref, "grouped rows")
    _close(orc, u16(out), ref, "layer output")
    # the merge itself, on the device's own rows: at most one bf16 ulp from
    # the exactly rounded weighted sum
    d = ulp_diff_bf16(u16(out), orc.merge(y_k, p["row_of"], wk))
    assert (d <= 1).all()


def test_dsv2_mixed_batch_1304_tokens(orc):
    from pdscope_amd import layer, ops, synthetic
    cfg = dict(synthetic.DSV2)
    H, I, E, k, Is = cfg["H"], cfg["I"], cfg["E"], cfg["k"], cfg["shared_I"]
    segments = [(0, 48), (48, 304), (304, 1304)]  # 48 decode tokens, prefill chunks of 256 and 1000
    T = segments[-1][1]
    lay = synthetic.make_layer(H, I, E, k, False, seed=20261011 + 5000, device=DEV, shared_I=Is)
    x = synthetic.make_tokens(T, H, seed=20261011 + 5007)
    ws = layer.MoEWorkspace(T, H, I, E, k, DEV, shared_I=Is)
    slots = ops.slot_table([lay.experts[e] for e in range(E)], DEV)
    shared_slot = ops.slot_table([lay.shared], DEV)
    assert ops.grouped_block_m(T * k // E) == 256
    out, logits, ids, w = layer.moe_forward(x, lay.gate, slots, ws, normalize=False, shared_slot=shared_slot)
    torch.cuda.synchronize()
    ik, wk, xu = ids.cpu().numpy(), u16(w), u16(x)
    oi, ow = orc.route_from_logits(u16(logits), k, False)
    assert np.array_equal(ik, oi) and np.array_equal(wk, ow), "routing differs from the oracle"
    p = orc.pack(np.ascontiguousarray(ik, dtype=np.int32), E)
    for name in ("counts", "offsets"):
        assert np.array_equal(getattr(ws, name).cpu().numpy(), p[name]), name
    assert np.array_equal(ws.row_of[:T * k].cpu().numpy(), p["row_of"])
    assert np.array_equal(ws.perm_token[:T * k].cpu().numpy(), p["perm_token"])
    rng = np.random.default_rng(1304)
    tokens = []
    for a, b in segments:
        tokens += [a, b - 1] + rng.choice(np.arange(a + 1, b - 1), 14, replace=False).tolist()
    tokens = np.array(sorted(set(tokens)))
    experts = u16(lay.experts)
    IH = I * H
    y_all = u16(ws.y[:T * k * H]).reshape(T * k, H)
    row_of = p["row_of"].reshape(T, k)
    got_y, ref_y = [], []
    for t in tokens:
        for s in range(k):
            blk = experts[ik[t, s]]
            ref_y.append(orc.expert_forward(xu[t:t + 1], blk[:IH].reshape(I, H), blk[IH:2 * IH].reshape(I, H),
                                            blk[2 * IH:].reshape(H, I))[0])
            got_y.append(y_all[row_of[t, s]])
    got_y, ref_y = np.stack(got_y), np.stack(ref_y)
    _close(orc, got_y, ref_y, "routed rows")
    sh = u16(lay.shared)
    IsH = Is * H
    shared_ref = orc.expert_forward(np.ascontiguousarray(xu[tokens]), sh[:IsH].reshape(Is, H),
                                    sh[IsH:2 * IsH].reshape(Is, H), sh[2 * IsH:].reshape(H, Is))
    _close(orc, u16(ws.y_shared[:T])[tokens], shared_ref, "shared expert rows")
    local_row_of = np.arange(len(tokens) * k, dtype=np.int32).reshape(len(tokens), k)
    ref_out = orc.merge(ref_y, local_row_of, np.ascontiguousarray(wk[tokens]), add_in=shared_ref)
    _close(orc, u16(out)[tokens], ref_out, "layer output")


def _rms_residual(out, x, eps=1e-6):
    h = out.float() + x.float()
    return (h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + eps)).to(torch.bfloat16)


def test_chained_stack_through_runtime(orc):
    from pdscope_amd import layer as LY
    from pdscope_amd import synthetic
    from pdscope_amd.cache import ExpertKey
    from pdscope_amd.executor import masters_from_block
    from pdscope_amd.pdscope_runtime import PDScopeCudaRuntime
    H, I, E, k = 2048, 768, 128, 8
    n_layers, hot_per_layer, speculative, demand_slots = 4, 40, 24, 8
    T_prefill, decode_steps = 64, 3
    seed0 = 20261011
    gates, masters, hot, experts_host = [], {}, [], []
    calib = synthetic.make_tokens(256, H, seed=seed0 + 30001)
    cws = LY.MoEWorkspace(256, H, I, E, k, DEV, route_only=True)
    for l in range(n_layers):
        lay = synthetic.make_layer(H, I, E, k, True, seed=seed0 + 20000 + 1000 * l, device=DEV)
        masters.update(masters_from_block(l, lay.experts, E, H, I))
        experts_host.append(u16(lay.experts))
        gates.append(lay.gate)
        _, cids, _ = LY.route(calib, lay.gate, cws)
        cnt = torch.bincount(cids.reshape(-1).long(), minlength=E).cpu().tolist()
        hot += [ExpertKey(l, e, "bf16") for e in sorted(range(E), key=lambda e: (-cnt[e], e))[:hot_per_layer]]
        del lay
    torch.cuda.empty_cache()
    rt = PDScopeCudaRuntime(masters, hot_keys=hot, speculative_slots=speculative, demand_slots=demand_slots,
                            resident_graphs=True, device=DEV)
    checked, rows_all = 0, []
    try:
        def check(out, routing, x, l):
            ids = routing.selected.cpu().numpy()
            oi, ow = orc.route_from_logits(u16(routing.logits), k, True)
            assert np.array_equal(ids, oi) and np.array_equal(u16(routing.weights), ow), f"layer {l} routing"
            ref, _, _ = oracle_layer_given_routing(orc, u16(x), ids, u16(routing.weights), experts_host[l], H, I,
                                                   merge=rt.merge)
            _close(orc, u16(out), ref, f"layer {l}")

        for step in range(decode_steps + 1):
            T = T_prefill if step == 0 else 1
            x = synthetic.make_tokens(T, H, seed=seed0 + 30002 + step)
            for l in range(n_layers):
                print(f"stack step {step} layer {l} T={T}", flush=True)
                out, routing, row = rt.forward(x, gates[l], layer=l, step=step, request="stack",
                                               next_gate=gates[l + 1] if l + 1 < n_layers else None, top_k=k)
                torch.cuda.synchronize()
                check(out, routing, x, l)
                checked += 1
                rows_all.append(row)
                x = _rms_residual(out, x)
        st = rt.cache.stats()
        assert st.get("h2d_bytes_submitted", 0) == st.get("h2d_bytes_completed", 0)
        assert rt.cache.active_demand is None
    finally:
        rt.close()
    assert checked == n_layers * (decode_steps + 1)
    prefill_rows, decode_rows = rows_all[:n_layers], rows_all[n_layers:]
    assert sum(len(r["decision"]["on_demand_queue"]) for r in prefill_rows) > 0, "the slot cap forced no misses"
    assert sum(len(r["prefetch_issued"]) for r in rows_all) > 0, "the predictor prefetched nothing"
    assert all(r["decode_path"] == "bound_launch" for r in decode_rows)
    assert st.get("prefetch_loads_submitted", 0) > 0
