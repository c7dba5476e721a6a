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
                check_output(orc, out, routing, x, layers[l], H, I, k)
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
        check_output(orc, out, routing, x, layers[0], H, I, k)
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
            ref, _, _ = oracle_layer_given_routing(orc, u16(x), ids, u16(routing.weights), blocks, CH, CI)
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
