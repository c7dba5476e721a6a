"""Measured generate requests of a Qwen3-MoE model whose MoE blocks run on the
gfx950 path, recorded in the reference's run layout (pdscope_amd.records).

It mirrors the measure mode of benchmarks/pdscope_compare.py (cases
:473-512, one request per case :320-436, run-wide result :436-470):
each case runs one prompt through a prefill and ``output_tokens - 1`` greedy
decode forwards, taking the completion time of every generated token; the
runtime's per-layer trace rows, its ledger counters and the memory figures
of the case are recorded, and the run closes with one ``result.json``.

The model comes from a Qwen3-MoE checkpoint directory (``--model``) or, with
no checkpoint at hand, is a randomly initialised Qwen3-30B-A3B-shaped model
of ``--random-layers`` decoder layers; prompts are seeded synthetic token
ids (no dataset is read).

    python -m pdscope_amd.compare --random-layers 2 --lengths 128 --output-tokens 8 \\
        --output runs/demo/result.json
"""
from __future__ import annotations

import argparse
import statistics
import sys
import time
from collections import Counter
from pathlib import Path

import torch

from . import records

ENTRY = "pdscope_amd/compare.py"


def build_cases(lengths, *, repetitions=1, output_tokens=64, warmups=2, **runtime_options):
    """Case specifications: `warmups` warm-up plus `repetitions` measured
    requests per prompt length (pdscope_compare.py:473-512)."""
    if not 1 <= repetitions <= 10:
        raise ValueError(f"repetitions must be 1..10, got {repetitions}")
    if not lengths or any(type(n) is not int or n < 2 for n in lengths):
        raise ValueError(f"prompt lengths must be integers >= 2, got {lengths!r}")
    if type(output_tokens) is not int or output_tokens < 2:
        raise ValueError("at least two output tokens are needed (one prefill, one decode)")
    suffix = "graph" if runtime_options.get("resident_graphs") else "eager"
    specs = []
    for n in lengths:
        for r in range(warmups + repetitions):
            specs.append(dict(case_id=f"pdscope_{suffix}_{n}_{r:02d}", method="pdscope", input_tokens=n,
                              output_tokens=output_tokens, prompt_index=0,
                              role="warmup" if r < warmups else "measure", diagnostics=False,
                              capture_attention=True, **runtime_options))
    return specs


def synthetic_prompt(n, vocab, seed):
    g = torch.Generator().manual_seed(seed + n)
    ids = torch.randint(0, vocab, (n,), generator=g).tolist()
    return dict(source="synthetic seeded token ids", seed=seed + n, requested_input_tokens=n,
                actual_input_tokens=n, ids=ids)


class MeasureSession:
    """A ModelSession plus per-layer attention timing and per-case accounting."""

    def __init__(self, model, *, hot_per_layer, speculative_slots, demand_slots=2, device=0, **runtime_options):
        from .hf import ModelSession
        t0 = time.perf_counter()
        self.session = ModelSession(model, hot_per_layer=hot_per_layer, speculative_slots=speculative_slots,
                                    demand_slots=demand_slots, device=device, **runtime_options)
        self.setup_seconds = time.perf_counter() - t0
        self.model = model
        self.device = self.session.device
        self.options = dict(hot_per_layer=hot_per_layer, speculative_slots=speculative_slots,
                            demand_slots=demand_slots, **runtime_options)
        self.attention = {}
        self.hooks = []
        for layer, decoder in enumerate(model.model.layers):
            attn = decoder.self_attn
            self.hooks.append(attn.register_forward_pre_hook(self._attn_start(layer)))
            self.hooks.append(attn.register_forward_hook(self._attn_end(layer)))
        self.completed = []

    def _attn_start(self, layer):
        def hook(module, args):
            ev = torch.cuda.Event(enable_timing=True)
            ev.record(torch.cuda.current_stream(self.device))
            self.attention[(self.session.step, layer)] = [ev]
        return hook

    def _attn_end(self, layer):
        def hook(module, args, out):
            ev = torch.cuda.Event(enable_timing=True)
            ev.record(torch.cuda.current_stream(self.device))
            self.attention[(self.session.step, layer)].append(ev)
        return hook

    def execute_case(self, spec, prompt, recorder):
        rt = self.session.runtime
        self.session.request = spec["case_id"]
        self.session.traces = []
        self.attention = {}
        stats_before = Counter(rt.cache.stats())
        torch.cuda.reset_peak_memory_stats(self.device)
        ids = torch.tensor([prompt["ids"]], device=self.device, dtype=torch.long)
        past, generated, ready = None, [], []
        n_in = len(prompt["ids"])
        with torch.inference_mode():
            torch.cuda.current_stream(self.device).synchronize()
            began = time.perf_counter()
            for step in range(spec["output_tokens"]):
                self.session.step = step
                mask = torch.ones((1, n_in + step), device=self.device, dtype=torch.long)
                out = self.model(input_ids=ids, attention_mask=mask, past_key_values=past, use_cache=True,
                                 return_dict=True, logits_to_keep=1)
                ids = out.logits[:, -1:].argmax(dim=-1)
                past = out.past_key_values
                generated.append(int(ids.item()))
                ready.append(time.perf_counter() - began)
            output_end = time.perf_counter()
        rt.poll(wait=True)
        ex = rt.executor
        if rt.pending or rt.transient or ex.loads or ex.computes or rt.cache.active_demand is not None:
            raise AssertionError("the runtime did not drain after the request")
        complete_end = time.perf_counter()
        stats = Counter(rt.cache.stats())
        stats.subtract(stats_before)
        layers = len(self.model.model.layers)
        k = self.session.top_k
        expected = (n_in + spec["output_tokens"] - 1) * layers * k
        traces = self.session.traces
        if (len(traces) != spec["output_tokens"] * layers or stats["physical_demand_tokens"] != expected
                or stats["h2d_bytes_completed"] != stats["h2d_bytes_submitted"]
                or stats["physical_expert_demands"] != stats["cpu_completed_experts"] + stats["gpu_completed_experts"]
                or past.get_seq_length() != n_in + spec["output_tokens"] - 1):
            raise AssertionError("request work, KV length or transfer accounting does not close")
        attention = [dict(step=s, layer=l, ms=ev[0].elapsed_time(ev[1]))
                     for (s, l), ev in sorted(self.attention.items()) if len(ev) == 2]
        free, total = torch.cuda.mem_get_info(self.device)
        reserved = torch.cuda.memory_reserved(self.device)
        peak = torch.cuda.max_memory_reserved(self.device)
        used = total - free
        external = max(0, used - reserved)
        trace = recorder.trace(spec["case_id"], [records.trace_row_json(r) for r in traces])
        first = traces[0]
        if (first.get("demand_slots") != self.options["demand_slots"]
                or first.get("merge_mode") != rt.merge
                or bool(first.get("input_pregather")) != bool(rt.input_pregather)
                or bool(first.get("graph_output_pool")) != bool(rt.graph_output_pool)):
            raise AssertionError("the configured host path did not reach the runtime")
        result = dict(
            case=dict(spec), prompt={k: v for k, v in prompt.items() if k != "ids"} | dict(input_tokens=n_in),
            metrics=records.phase_metrics(n_in, ready),
            measured_performance=spec["role"] == "measure" and not spec["diagnostics"],
            token_ready_seconds=ready, generated_ids=generated, kv_final_length=past.get_seq_length(),
            strategy_initialization_seconds=self.setup_seconds if not self.completed else 0.0,
            background_drain_seconds=complete_end - output_end, request_complete_seconds=complete_end - began,
            cache_stats={kk: v for kk, v in stats.items() if v}, hot_profile=None,
            native_completed_chunks=0,
            cache_payload_allowance_bytes=rt.cache.cache_bytes,
            source_metrics_delta={}, resident_graphs=(dict(calibration=rt.graph_cost_calibration,
                                                           replays=rt.bound_launches,
                                                           bindings=len(rt._bindings)) if rt.resident_graphs else None),
            cache_pool_reserved_bytes=ex.storage()["cache_reserved_tensor_bytes"],
            demand_staging_bytes=sum(rt.cache.staging_slot_bytes),
            demand_staging_aliases="declared demand slots; one expert payload per slot",
            gpu_peak_allocated_bytes=torch.cuda.max_memory_allocated(self.device), gpu_peak_reserved_bytes=peak,
            gpu_process_end_bytes=used, gpu_process_end_external_bytes=external,
            gpu_peak_reserved_plus_end_external_bytes=peak + external,
            gpu_peak_scope="allocator peak plus device bytes in use beyond the allocator at the end (whole device)",
            host_peak_rss_bytes=records.peak_rss_bytes(), trace=trace, attention_cuda_ms=attention,
            timing_scope="host clock per generated token (scalar delivery); attention by HIP events; drain separate")
        recorder.request(result)
        self.completed.append(result)
        return result

    def finalize(self, *, model_name, model_identity, calibration_sources):
        rt = self.session.runtime
        att = {}
        for r in self.completed:
            if r["case"]["role"] == "measure":
                continue
            for a in r["attention_cuda_ms"]:
                phase = "prefill" if a["step"] == 0 else "decode"
                att.setdefault((r["case"]["input_tokens"], phase, a["layer"]), []).append(a["ms"])
        return dict(schema_version=2, status="completed", kind="single_request_measure",
                    measured_performance=any(r["measured_performance"] for r in self.completed),
                    requests=self.completed, model=model_name, model_initialization_stages=[],
                    native_attention_and_kv=True, attention_implementation=getattr(
                        self.model.config, "_attn_implementation", None),
                    native_backend=None, master_storage=self.session.pinned, device_buffer_pool=None,
                    original_weight_samples_unchanged=True, all_master_storage_versions_unchanged=True,
                    calibration_sources=calibration_sources,
                    attention_cost_table=[dict(input_tokens=n, phase=p, layer=l, median_ms=statistics.median(v),
                                               samples=len(v)) for (n, p, l), v in sorted(att.items())],
                    model_identity=model_identity,
                    torch_environment=dict(version=torch.__version__, file=torch.__file__, hip=torch.version.hip,
                                           cuda=torch.version.cuda, control_threads=torch.get_num_threads(),
                                           allow_tf32=torch.backends.cuda.matmul.allow_tf32,
                                           allow_bf16_reduced_precision_reduction=(
                                               torch.backends.cuda.matmul.allow_bf16_reduced_precision_reduction)),
                    total_device_budget_bytes=None, allocator_cap_bytes=None,
                    control_affinity=sorted(__import__("os").sched_getaffinity(0)),
                    host_peak_rss_bytes=records.peak_rss_bytes(), runtime=dict(merge=rt.merge, E=rt.E, H=rt.H, I=rt.I))

    def close(self):
        for h in self.hooks:
            h.remove()
        self.hooks.clear()
        self.session.close()


def random_qwen3_moe(layers, *, seed=20261011, **shape):
    """A randomly initialised Qwen3-MoE model of the Qwen3-30B-A3B shape (or
    `shape` overrides) with `layers` decoder layers, bf16 on the CPU."""
    from transformers import Qwen3MoeConfig, Qwen3MoeForCausalLM
    cfg = dict(vocab_size=151936, hidden_size=2048, intermediate_size=6144, moe_intermediate_size=768,
               num_hidden_layers=layers, num_attention_heads=32, num_key_value_heads=4, head_dim=128,
               num_experts=128, num_experts_per_tok=8, norm_topk_prob=True, decoder_sparse_step=1,
               mlp_only_layers=[], max_position_embeddings=8192, rms_norm_eps=1e-6)
    cfg.update(shape)
    torch.manual_seed(seed)
    return Qwen3MoeForCausalLM(Qwen3MoeConfig(**cfg)).to(torch.bfloat16).eval()


def run(model, specs, *, output, argv, config, model_name, model_identity=None, calibration_sources=(),
        hot_per_layer, speculative_slots, demand_slots=2, seed=20261011, device=0, **runtime_options):
    """Run every case through `model` and record the run under output's directory."""
    recorder = records.RunRecorder(output, entry=ENTRY, argv=argv, config=config)
    session = None
    try:
        recorder.cases(specs)
        torch.backends.cuda.matmul.allow_tf32 = False
        torch.backends.cuda.matmul.allow_bf16_reduced_precision_reduction = False
        session = MeasureSession(model, hot_per_layer=hot_per_layer, speculative_slots=speculative_slots,
                                 demand_slots=demand_slots, device=device, **runtime_options)
        vocab = model.config.vocab_size
        for spec in specs:
            session.execute_case(spec, synthetic_prompt(spec["input_tokens"], vocab, seed), recorder)
        result = session.finalize(model_name=model_name, model_identity=model_identity,
                                  calibration_sources=list(calibration_sources))
        recorder.finish(result)
        return result
    except BaseException as exc:
        recorder.fail(exc)
        raise
    finally:
        if session is not None:
            session.close()


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    src = ap.add_mutually_exclusive_group(required=True)
    src.add_argument("--model", type=Path, help="Qwen3-MoE checkpoint directory (safetensors)")
    src.add_argument("--random-layers", type=int, help="random-init Qwen3-30B-A3B-shaped model of N layers")
    ap.add_argument("--lengths", type=int, nargs="+", default=[128])
    ap.add_argument("--output-tokens", type=int, default=64)
    ap.add_argument("--repetitions", type=int, default=1)
    ap.add_argument("--warmups", type=int, default=2)
    ap.add_argument("--hot-per-layer", type=int, default=40)
    ap.add_argument("--speculative-slots", type=int, default=16)
    ap.add_argument("--demand-slots", type=int, default=8)
    ap.add_argument("--graphs", action="store_true", help="resident_graphs: decode layers through their bound single launch")
    ap.add_argument("--merge", choices=["reference", "fused"], default="reference")
    ap.add_argument("--input-pregather", action="store_true")
    ap.add_argument("--graph-output-pool", action="store_true")
    ap.add_argument("--seed", type=int, default=20261011)
    ap.add_argument("--output", type=Path, required=True, help="result.json path (its directory holds the run)")
    args = ap.parse_args(argv)
    opts = dict(resident_graphs=args.graphs, merge=args.merge, input_pregather=args.input_pregather,
                graph_output_pool=args.graph_output_pool)
    specs = build_cases(args.lengths, repetitions=args.repetitions, output_tokens=args.output_tokens,
                        warmups=args.warmups, demand_slots=args.demand_slots, **opts)
    identity = None
    if args.model is not None:
        from transformers import Qwen3MoeForCausalLM
        model = Qwen3MoeForCausalLM.from_pretrained(args.model, torch_dtype=torch.bfloat16).eval()
        identity = dict(config_sha256=records.sha256_file(args.model / "config.json"),
                        index_sha256=records.sha256_file(args.model / "model.safetensors.index.json"))
        name = str(args.model)
    else:
        model = random_qwen3_moe(args.random_layers, seed=args.seed)
        name = f"random-init Qwen3-30B-A3B-shaped, {args.random_layers} layers, seed {args.seed}"
    result = run(model, specs, output=args.output, argv=sys.argv if argv is None else argv, config=vars(args),
                 model_name=name, model_identity=identity, hot_per_layer=args.hot_per_layer,
                 speculative_slots=args.speculative_slots, demand_slots=args.demand_slots, seed=args.seed, **opts)
    print(records.json.dumps(dict(status=result["status"], output=str(args.output.resolve()))), flush=True)


if __name__ == "__main__":
    main()
