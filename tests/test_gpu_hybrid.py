"""GPU tests of the widened drop-in: CPU/GPU placement through plan_pdscope
with a caller's CPU backend, masters loaded from a safetensors checkpoint
into pooled pinned blocks, and a transformers Qwen3-MoE model whose MoE
blocks run through the runtime.

The CPU backend used here is test scaffolding standing in for the
reference's native CPU kernel: it computes one expert with the oracle and
counts its calls.  Layer outputs are compared with the oracle applied to the
runtime's own routing (itself checked bit-exact against the oracle on the
returned logits), within the layer tolerance.
"""
import json

import numpy as np
import pytest
import torch

from tests.gpu_helpers import u16
from tests.test_gpu_runtime import build, check_output, closure

pytestmark = pytest.mark.gpu
DEV = "cuda"


class OracleCpuBackend:
    """(key, rows) -> rows: one expert's SwiGLU on the host, by the oracle."""

    def __init__(self, orc, masters):
        self.orc, self.masters, self.calls, self.rows = orc, masters, 0, 0

    def __call__(self, key, rows):
        w = self.masters[key].tensors
        y = self.orc.expert_forward(u16(rows), u16(w["gate_proj"]), u16(w["up_proj"]), u16(w["down_proj"]))
        self.calls += 1
        self.rows += rows.shape[0]
        return torch.from_numpy(y.view(np.int16)).view(torch.bfloat16)


# the keys of the reference's per-layer trace row (expertbench/pdscope_runtime.py:492-512)
REFERENCE_ROW_KEYS = {
    "phase", "step", "layer", "token_counts", "balance", "cpu_packing", "cpu_batched_io", "dispatch",
    "decode_submission", "decision", "prefetch_issued", "prefetch_capacity_skipped", "next_prediction_counts",
    "causal_hit_counts", "predictor", "scheduler", "predictor_prior_hit_rate", "selected_sha256",
    "next_selected_sha256", "ready_at_reveal", "loading_at_reveal", "counters", "ping_pong_slots",
    "static_retention", "merge_mode", "input_pregather", "demand_slots", "graph_output_pool", "pipeline",
    "measured_performance"}


def cost_table(tmp_path, cpu_ms_per_row, gpu_ms=0.2, h2d_ms=0.5):
    points = {str(n): dict(cpu_ms=cpu_ms_per_row * n, gpu_ms=gpu_ms, h2d_ms=h2d_ms)
              for n in (1, 4, 16, 64, 128, 256, 1024, 4096)}
    p = tmp_path / "costs.json"
    p.write_text(json.dumps(dict(kind="pdscope_cost_table", points=points)))
    from pdscope_amd.costs import FileCosts
    return FileCosts(p)


def test_runtime_places_experts_on_the_cpu_backend(orc, tmp_path):
    """Cheap CPU costs: plan_pdscope sends the lightly loaded non-resident
    experts to the CPU backend; prefill and decode outputs match the oracle."""
    from pdscope_amd.cache import ExpertKey
    from pdscope_amd.pdscope_runtime import PDScopeCudaRuntime
    H, I, E, k = 256, 128, 32, 4
    layers, masters = build(2, H, I, E, k, seed=91)
    hot = [ExpertKey(l, e, "bf16") for l in range(2) for e in range(4)]
    backend = OracleCpuBackend(orc, masters)
    rt = PDScopeCudaRuntime(masters, hot_keys=hot, speculative_slots=2, demand_slots=2,
                            costs=cost_table(tmp_path, 0.02), cpu_backend=backend)
    gen = torch.Generator(device=DEV).manual_seed(5)
    cpu_total = 0
    try:
        for step, T in enumerate((24, 1, 1)):
            x = torch.randn((T, H), generator=gen, device=DEV).to(torch.bfloat16)
            for l in range(2):
                out, routing, row = rt.forward(x, layers[l].gate, layer=l, step=step,
                                               next_gate=layers[1].gate if l == 0 else None, top_k=k)
                torch.cuda.synchronize()
                check_output(orc, out, routing, x, layers[l], H, I, k, merge=rt.merge)
                d = row["decision"]
                assert row["scheduler"] == "cross_layer" and d["mode"] in (
                    "prefill", "a_load", "b_prefetch", "c_unload", "d_cross_layer")
                assert set(d["cpu_queue"]) | set(d["gpu_resident_queue"]) | set(d["on_demand_queue"]) == \
                    set(row["token_counts"])
                assert row["counters"]["cpu_completed_experts"] == len(d["cpu_queue"])
                assert row["counters"]["cpu_completed_experts"] + row["counters"]["gpu_completed_experts"] == \
                    len(row["token_counts"])
                cpu_total += len(d["cpu_queue"])
                assert REFERENCE_ROW_KEYS <= set(row), REFERENCE_ROW_KEYS - set(row)
                assert row["selected_sha256"] is not None and row["balance"] is None
        assert cpu_total > 0 and backend.calls == cpu_total
        closure(rt)
    finally:
        rt.close()


def test_runtime_with_expensive_cpu_keeps_the_load_on_the_gpu(orc, tmp_path):
    """Expensive CPU costs: the prefill plan leaves the CPU at most its first
    candidate, the least loaded non-resident expert (the local boundary of
    pdscope_policy.py starts at 1: an empty CPU prefix costs nothing), and
    every other expert runs on the GPU."""
    from pdscope_amd.cache import ExpertKey
    from pdscope_amd.pdscope_runtime import PDScopeCudaRuntime
    H, I, E, k = 256, 128, 32, 4
    layers, masters = build(1, H, I, E, k, seed=93)
    backend = OracleCpuBackend(orc, masters)
    rt = PDScopeCudaRuntime(masters, hot_keys=[ExpertKey(0, e, "bf16") for e in range(8)], speculative_slots=0,
                            costs=cost_table(tmp_path, 50.0), cpu_backend=backend)
    try:
        x = torch.randn((32, H), generator=torch.Generator(device=DEV).manual_seed(6), device=DEV).to(torch.bfloat16)
        out, routing, row = rt.forward(x, layers[0].gate, layer=0, step=0, top_k=k)
        torch.cuda.synchronize()
        check_output(orc, out, routing, x, layers[0], H, I, k, merge=rt.merge)
        d, counts = row["decision"], row["token_counts"]
        assert len(d["cpu_queue"]) <= 1 and backend.calls == len(d["cpu_queue"])
        if d["cpu_queue"]:
            assert d["cpu_queue"][0] == min(d["current_cpu_candidates"], key=lambda e: (counts[e], e))
        closure(rt)
    finally:
        rt.close()


def test_checkpoint_masters_in_pinned_pool_drive_the_runtime(orc, tmp_path):
    """Experts and routers read from a safetensors checkpoint, packed into
    pooled pinned blocks (each expert one contiguous gate|up|down slice),
    staged and computed by the runtime."""
    from pdscope_amd.cache import ExpertKey
    from pdscope_amd.checkpoint import load_expert, load_router, pin_cpu_master_storage
    from pdscope_amd.pdscope_runtime import PDScopeCudaRuntime
    from tests.test_checkpoint import write_checkpoint
    CH, CI, CE, CL, CK = 256, 128, 32, 2, 4
    write_checkpoint(tmp_path, H=CH, I=CI, E=CE, L=CL, top_k=CK)
    masters = {ExpertKey(l, e, "bf16"): load_expert(tmp_path, ExpertKey(l, e, "bf16"))
               for l in range(CL) for e in range(CE)}
    originals = {k: {p: t.clone() for p, t in w.tensors.items()} for k, w in masters.items()}
    info = pin_cpu_master_storage(masters, block_cap_bytes=1 << 22)
    assert info["experts_copied"] == CL * CE and len(info["blocks"]) > 1
    for key, w in masters.items():
        assert w.flat is not None and w.flat.is_pinned() and w.flat.numel() == w.nbytes
        for p, t in w.tensors.items():
            assert torch.equal(t, originals[key][p])
    gates = [load_router(tmp_path, l)[0].to(DEV) for l in range(CL)]
    rt = PDScopeCudaRuntime(masters, hot_keys=[ExpertKey(0, 0, "bf16")], speculative_slots=1, demand_slots=2)
    try:
        x = torch.randn((40, CH), generator=torch.Generator(device=DEV).manual_seed(8), device=DEV)
        x = x.to(torch.bfloat16)
        for l in range(CL):
            out, routing, row = rt.forward(x, gates[l], layer=l, step=0, top_k=CK,
                                           next_gate=gates[l + 1] if l + 1 < CL else None)
            torch.cuda.synchronize()
            ids = routing.selected.cpu().numpy()
            oi, ow = orc.route_from_logits(u16(routing.logits), CK, True)
            assert np.array_equal(ids, oi) and np.array_equal(u16(routing.weights), ow)
            blocks = np.stack([u16(masters[ExpertKey(l, e, "bf16")].flat.view(torch.bfloat16)) for e in range(CE)])
            from tests.gpu_helpers import assert_layer_close, oracle_layer_given_routing
            ref, _, _ = oracle_layer_given_routing(orc, u16(x), ids, u16(routing.weights), blocks, CH, CI,
                                                   merge=rt.merge)
            assert_layer_close(orc, out, ref)
        closure(rt)
    finally:
        rt.close()


def test_transformers_model_through_expert_blocks(orc):
    """A randomly initialised transformers Qwen3-MoE model (2 sparse layers)
    whose MoE blocks are replaced by ExpertBlocks running the runtime: the
    prompt (step 0) and two decoded tokens (steps 1, 2) give the same
    next-token logits as the unmodified model within bf16 tolerance."""
    from transformers import Qwen3MoeConfig, Qwen3MoeForCausalLM
    from pdscope_amd.hf import ExpertBlock, ModelSession
    cfg = Qwen3MoeConfig(vocab_size=256, hidden_size=256, intermediate_size=512, moe_intermediate_size=128,
                         num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2, head_dim=64,
                         num_experts=32, num_experts_per_tok=4, norm_topk_prob=True, decoder_sparse_step=1,
                         mlp_only_layers=[], initializer_range=0.05)
    torch.manual_seed(1)
    native = Qwen3MoeForCausalLM(cfg).to(torch.bfloat16).eval()
    with torch.no_grad():  # distinct router logits (a zero router would tie every expert)
        for d in native.model.layers:
            d.mlp.gate.weight.normal_(0.0, 0.5)
    ours = Qwen3MoeForCausalLM(cfg).to(torch.bfloat16).eval()
    ours.load_state_dict(native.state_dict())
    native.to(DEV)
    session = ModelSession(ours, hot_per_layer=6, speculative_slots=2, demand_slots=2, device=0)
    try:
        assert all(isinstance(d.mlp, ExpertBlock) for d in ours.model.layers)
        ids = torch.randint(0, cfg.vocab_size, (1, 24), generator=torch.Generator().manual_seed(2)).to(DEV)
        with torch.no_grad():
            ref = native(ids, use_cache=True)
            session.step = 0
            got = ours(ids, use_cache=True)
            pk_ref, pk_got = ref.past_key_values, got.past_key_values
            outs = [(ref.logits[0, -1].float(), got.logits[0, -1].float())]
            nxt = ref.logits[0, -1].argmax().view(1, 1)
            for step in (1, 2):
                r = native(nxt, past_key_values=pk_ref, use_cache=True)
                session.step = step
                g = ours(nxt, past_key_values=pk_got, use_cache=True)
                pk_ref, pk_got = r.past_key_values, g.past_key_values
                outs.append((r.logits[0, -1].float(), g.logits[0, -1].float()))
                nxt = r.logits[0, -1].argmax().view(1, 1)
        torch.cuda.synchronize()
        for a, b in outs:
            rel = (a - b).norm() / a.norm()
            assert rel < 3e-2, float(rel)
        assert [t["step"] for t in session.traces] == [0, 0, 1, 1, 2, 2]
        assert all(sum(t["token_counts"].values()) == (24 if t["step"] == 0 else 1) * 4 for t in session.traces)
        closure(session.runtime)
    finally:
        session.close()


# ---------------------------------------------------------------- drop-in switches of the runtime

class NativeOracleBackend(OracleCpuBackend):
    """A CPU backend that also exposes the native queue objects the decode
    tail drives (native_group_handles / note_native_dispatch) and a packed
    submit_many; every expert is computed by the oracle."""

    def __init__(self, orc, masters, layers_u16, H, I):
        super().__init__(orc, masters)
        from tests.test_gpu_runtime import _OracleLayer, _Pool
        self.pool = _Pool()
        self.native_layers = {l: _OracleLayer(orc, e, H, I) for l, e in layers_u16.items()}
        self.native_rows, self.packed_calls = 0, 0

    def native_group_handles(self, layer):
        obj = self.native_layers.get(layer)
        return None if obj is None else (self.pool, obj)

    def note_native_dispatch(self, rows):
        self.native_rows += rows

    def submit_many(self, jobs):
        from concurrent.futures import Future
        self.packed_calls += 1
        out = {}
        for key, rows in jobs.items():
            f = Future()
            f.set_result(self(key, rows))
            out[key] = f
        return out


def test_runtime_native_dispatch_runs_the_decode_cpu_group(orc, tmp_path):
    """merge='fused' with native_dispatch: decode CPU experts go through
    submit_group / finish_and_merge as one native group (pdscope_runtime.py:
    284-298, 407-426), their rows staged and added into the output before the
    GPU rows are merged on top; every output within tolerance of the oracle."""
    from pdscope_amd import pdscope_layer_dispatch
    from pdscope_amd.cache import ExpertKey
    from pdscope_amd.pdscope_runtime import PDScopeCudaRuntime
    H, I, E, k = 256, 128, 32, 4
    layers, masters = build(2, H, I, E, k, seed=61)
    backend = NativeOracleBackend(orc, masters, {l: u16(layers[l].experts) for l in range(2)}, H, I)
    hot = [ExpertKey(l, e, "bf16") for l in range(2) for e in range(6)]
    rt = PDScopeCudaRuntime(masters, hot_keys=hot, speculative_slots=2, demand_slots=2, merge="fused",
                            costs=cost_table(tmp_path, 0.02), cpu_backend=backend,
                            native_dispatch=pdscope_layer_dispatch, decode_cpu_target=2)
    native_layers = 0
    try:
        gen = torch.Generator(device=DEV).manual_seed(62)
        for step, T in enumerate((16, 1, 1, 1)):
            x = torch.randn((T, H), generator=gen, device=DEV).to(torch.bfloat16)
            for l in range(2):
                out, routing, row = rt.forward(x, layers[l].gate, layer=l, step=step, top_k=k,
                                               next_gate=layers[1].gate if l == 0 else None)
                torch.cuda.synchronize()
                check_output(orc, out, routing, x, layers[l], H, I, k, row=row)
                if row["decode_submission"] == "native_group":
                    native_layers += 1
                    assert row["counters"]["cpu_completed_experts"] == len(row["decision"]["cpu_queue"]) > 0
        assert native_layers > 0 and backend.native_rows > 0
        closure(rt)
    finally:
        rt.close()


def test_runtime_cpu_batch_packs_cpu_experts_into_one_submission(orc, tmp_path):
    from pdscope_amd.cache import ExpertKey
    from pdscope_amd.pdscope_runtime import PDScopeCudaRuntime
    H, I, E, k = 256, 128, 32, 4
    layers, masters = build(1, H, I, E, k, seed=63)
    backend = NativeOracleBackend(orc, masters, {}, H, I)
    rt = PDScopeCudaRuntime(masters, hot_keys=[ExpertKey(0, e, "bf16") for e in range(4)], speculative_slots=0,
                            costs=cost_table(tmp_path, 0.02), cpu_backend=backend, cpu_batch="both")
    try:
        x = torch.randn((24, H), generator=torch.Generator(device=DEV).manual_seed(64), device=DEV).to(torch.bfloat16)
        out, routing, row = rt.forward(x, layers[0].gate, layer=0, step=0, top_k=k)
        torch.cuda.synchronize()
        check_output(orc, out, routing, x, layers[0], H, I, k, row=row)
        assert row["decision"]["cpu_queue"] and backend.packed_calls == 1 and row["cpu_packing"] is True
        closure(rt)
    finally:
        rt.close()
    # a backend without submit_many cannot run packed CPU groups
    rt = PDScopeCudaRuntime(masters, hot_keys=[ExpertKey(0, e, "bf16") for e in range(4)], speculative_slots=0,
                            costs=cost_table(tmp_path, 0.02), cpu_backend=OracleCpuBackend(orc, masters),
                            cpu_batch="both")
    try:
        with pytest.raises(ValueError, match="submit_many"):
            rt.forward(x, layers[0].gate, layer=0, step=0, top_k=k)
    finally:
        rt.close()


def test_runtime_input_pregather_gives_the_same_bits(orc):
    """input_pregather gathers the activation rows into grouped order once and
    the grouped kernels read them in order: same tiles, same arithmetic, the
    same output bit for bit (also through the demand staging batches)."""
    from pdscope_amd.cache import ExpertKey
    from pdscope_amd.pdscope_runtime import PDScopeCudaRuntime
    H, I, E, k = 256, 128, 32, 4
    layers, masters = build(1, H, I, E, k, seed=65)
    hot = [ExpertKey(0, e, "bf16") for e in range(12)]
    x = torch.randn((200, H), generator=torch.Generator(device=DEV).manual_seed(66), device=DEV).to(torch.bfloat16)
    outs = []
    for pre in (False, True):
        rt = PDScopeCudaRuntime(masters, hot_keys=hot, speculative_slots=0, demand_slots=8, input_pregather=pre)
        try:
            out, routing, row = rt.forward(x, layers[0].gate, layer=0, step=0, top_k=k)
            torch.cuda.synchronize()
            assert row["input_pregather"] is pre and row["decision"]["on_demand_queue"]
            outs.append(out.clone())
            closure(rt)
        finally:
            rt.close()
    assert torch.equal(outs[0], outs[1])
    check_output(orc, outs[1], routing, x, layers[0], H, I, k, merge=rt.merge)


def test_runtime_graph_output_pool_is_a_two_deep_ring(orc):
    """graph_output_pool: decode layers return one of two output buffers per
    layer, alternating, which the bound launch writes directly; each output
    equals the eager single-launch layer until the call after next."""
    from pdscope_amd import layer, ops, synthetic
    from pdscope_amd.cache import ExpertKey
    from pdscope_amd.pdscope_runtime import PDScopeCudaRuntime
    q = synthetic.QWEN
    layers, masters = build(1, q["H"], q["I"], q["E"], q["k"], seed=67)
    rt = PDScopeCudaRuntime(masters, hot_keys=[ExpertKey(0, e, "bf16") for e in range(q["E"])], speculative_slots=0,
                            resident_graphs=True, graph_output_pool=True)
    slots = ops.slot_table([layers[0].experts[e] for e in range(q["E"])], DEV)
    ws = layer.MoEWorkspace(1, q["H"], q["I"], q["E"], 8, DEV)
    try:
        rt.forward(synthetic.make_tokens(4, q["H"], seed=68), layers[0].gate, layer=0, step=0)
        ptrs = []
        for step in range(1, 5):
            x = synthetic.make_tokens(1, q["H"], seed=68 + step)
            out, routing, row = rt.forward(x, layers[0].gate, layer=0, step=step)
            ref, _, _, _ = layer.moe_forward(x, layers[0].gate, slots, ws, merge=rt.merge)
            torch.cuda.synchronize()
            assert row["decode_path"] == "bound_launch" and row["graph_output_pool"] is True
            assert torch.equal(out, ref)
            ptrs.append(out.data_ptr())
        assert ptrs[0] == ptrs[2] and ptrs[1] == ptrs[3] and ptrs[0] != ptrs[1]
        closure(rt)
    finally:
        rt.close()


def test_runtime_planned_decode_takes_the_bound_launch_with_calibrated_costs(orc, tmp_path):
    """With a cost table, a CPU backend and resident_graphs, construction
    calibrates the bound resident launch (graph_cost_mode='measured' charges
    it to one-token GPU work); a decode plan that keeps every expert on the
    GPU is served by the layer's bound launch."""
    from pdscope_amd.cache import ExpertKey
    from pdscope_amd.costs import ResidentGraphCosts
    from pdscope_amd.pdscope_runtime import PDScopeCudaRuntime
    H, I, E, k = 256, 128, 32, 4
    layers, masters = build(1, H, I, E, k, seed=69)
    base = cost_table(tmp_path, 50.0)
    rt = PDScopeCudaRuntime(masters, hot_keys=[ExpertKey(0, e, "bf16") for e in range(E)], speculative_slots=0,
                            costs=base, cpu_backend=OracleCpuBackend(orc, masters), resident_graphs=True,
                            graph_cost_mode="measured", decode_cpu_target=0)
    try:
        cal = rt.graph_cost_calibration
        assert cal is not None and cal["scheduler_cost_mode"] == "measured" and cal["per_expert_ms"] > 0
        assert isinstance(rt.costs, ResidentGraphCosts) and rt.costs.for_load(1)["gpu_ms"] == cal["per_expert_ms"]
        gen = torch.Generator(device=DEV).manual_seed(70)
        rt.forward(torch.randn((8, H), generator=gen, device=DEV).to(torch.bfloat16), layers[0].gate, layer=0,
                   step=0, top_k=k)
        for step in range(1, 4):
            x = torch.randn((1, H), generator=gen, device=DEV).to(torch.bfloat16)
            out, routing, row = rt.forward(x, layers[0].gate, layer=0, step=step, top_k=k)
            torch.cuda.synchronize()
            assert row["decision"]["cpu_queue"] == [] and row["decode_path"] == "bound_launch"
            check_output(orc, out, routing, x, layers[0], H, I, k, merge=rt.merge)
        closure(rt)
    finally:
        rt.close()
    with pytest.raises(ValueError):
        PDScopeCudaRuntime(masters, hot_keys=[], speculative_slots=0, graph_cost_mode="other")


def test_runtime_reference_merge_is_the_bf16_expert_order_sum(orc):
    """merge='reference' (the default): the layer output is the reference's
    per-expert bf16 index_add_ sequence over the runtime's own expert rows,
    bit for bit (the oracle's ordered merge of ws.y)."""
    from pdscope_amd.cache import ExpertKey
    from pdscope_amd.pdscope_runtime import PDScopeCudaRuntime
    H, I, E, k = 256, 128, 32, 4
    layers, masters = build(1, H, I, E, k, seed=71)
    rt = PDScopeCudaRuntime(masters, hot_keys=[ExpertKey(0, e, "bf16") for e in range(E)], speculative_slots=0)
    try:
        assert rt.merge == "reference"
        x = torch.randn((64, H), generator=torch.Generator(device=DEV).manual_seed(72), device=DEV).to(torch.bfloat16)
        out, routing, row = rt.forward(x, layers[0].gate, layer=0, step=0, top_k=k)
        torch.cuda.synchronize()
        ws = rt._ws[k]
        y = u16(ws.y[:64 * k * H]).reshape(64 * k, H)
        p = orc.pack(routing.selected.cpu().numpy().astype(np.int32), E)
        assert np.array_equal(u16(out), orc.merge_ordered(y, p["row_of"], u16(routing.weights)))
        check_output(orc, out, routing, x, layers[0], H, I, k, merge=rt.merge)
    finally:
        rt.close()


def test_measured_requests_write_the_reference_run_files(tmp_path):
    """pdscope_amd.compare on a small random Qwen3-MoE model: two warm-up and
    one measured request, each a prefill plus decode forwards through the
    runtime, recorded as manifest / cases / requests / traces / result with
    the reference's key sets; trace rows and ledger counters close."""
    import gzip
    import json
    from pdscope_amd import compare
    from tests.test_records import MANIFEST_END_KEYS, MANIFEST_KEYS, METRIC_KEYS, REQUEST_KEYS, RESULT_KEYS
    model = compare.random_qwen3_moe(2, vocab_size=512, hidden_size=256, intermediate_size=512,
                                     moe_intermediate_size=128, num_attention_heads=4, num_key_value_heads=2,
                                     head_dim=64, num_experts=32, num_experts_per_tok=4)
    with torch.no_grad():
        for d in model.model.layers:
            d.mlp.gate.weight.normal_(0.0, 0.5)
    specs = compare.build_cases([24], repetitions=1, output_tokens=4, warmups=2, demand_slots=4,
                                resident_graphs=True, merge="reference")
    out = tmp_path / "run" / "result.json"
    result = compare.run(model, specs, output=out, argv=["test"], config=dict(test=True), model_name="tiny",
                         hot_per_layer=8, speculative_slots=4, demand_slots=4, resident_graphs=True,
                         merge="reference")
    run = out.parent
    man = json.loads((run / "manifest.json").read_text())
    assert MANIFEST_KEYS | MANIFEST_END_KEYS <= set(man) and man["status"] == "completed"
    res = json.loads(out.read_text())
    assert RESULT_KEYS <= set(res) and res["status"] == "completed" and res["measured_performance"]
    reqs = [json.loads(x) for x in (run / "requests.jsonl").read_text().splitlines()]
    assert len(reqs) == 3 and [r["case"]["role"] for r in reqs] == ["warmup", "warmup", "measure"]
    for r in reqs:
        assert REQUEST_KEYS <= set(r) and METRIC_KEYS == set(r["metrics"])
        assert len(r["generated_ids"]) == 4 and r["kv_final_length"] == 24 + 3
        with gzip.open(run / r["trace"]["path"], "rt") as f:
            rows = json.load(f)
        assert len(rows) == 4 * 2 and [x["step"] for x in rows] == [0, 0, 1, 1, 2, 2, 3, 3]
        assert all(x["decode_path"] == "bound_launch" for x in rows if x["phase"] == "decode")
        assert r["cache_stats"]["physical_demand_tokens"] == (24 + 3) * 2 * 4
    assert result["requests"][-1]["generated_ids"] == reqs[-1]["generated_ids"]
    # the three requests share the prompt and the model: the same greedy tokens
    assert len({tuple(r["generated_ids"]) for r in reqs}) == 1
    assert res["attention_cost_table"] and res["master_storage"]["experts_copied"] == 64
