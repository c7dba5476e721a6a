"""Run records (pdscope_amd.records) in the reference's layout, on the CPU:
request metrics, and the manifest / cases / requests / traces / result files
with the reference's key sets (benchmarks/harness.py:168-183,
benchmarks/pdscope_compare.py:129-141, 390-408, 436-470, 840-850)."""
import gzip
import json
import math

import pytest

from pdscope_amd import records

# keys the reference writes (restated from the cited lines)
MANIFEST_KEYS = {"schema_version", "entry", "argv", "config", "started_at", "pid", "cwd", "python", "executable",
                 "host", "platform", "package_versions", "process_argv", "affinity", "env", "git_commit",
                 "git_status", "nvidia_smi", "lscpu", "source_archive", "native_prefetch_build", "status"}
MANIFEST_END_KEYS = {"finished_at", "runner_seconds", "host_peak_rss_bytes"}
METRIC_KEYS = {"input_tokens", "output_tokens", "decode_forwards", "prefill_seconds", "decode_seconds",
               "request_output_seconds", "prefill_tokens_per_second", "decode_tokens_per_second",
               "end_to_end_output_tokens_per_second", "decode_tpot_seconds", "scope"}
REQUEST_KEYS = {"case", "prompt", "metrics", "measured_performance", "token_ready_seconds", "generated_ids",
                "kv_final_length", "strategy_initialization_seconds", "background_drain_seconds",
                "request_complete_seconds", "cache_stats", "hot_profile", "native_completed_chunks",
                "cache_payload_allowance_bytes", "source_metrics_delta", "resident_graphs",
                "cache_pool_reserved_bytes", "demand_staging_bytes", "demand_staging_aliases",
                "gpu_peak_allocated_bytes", "gpu_peak_reserved_bytes", "gpu_process_end_bytes",
                "gpu_process_end_external_bytes", "gpu_peak_reserved_plus_end_external_bytes", "gpu_peak_scope",
                "host_peak_rss_bytes", "trace", "attention_cuda_ms", "timing_scope"}
RESULT_KEYS = {"schema_version", "status", "kind", "measured_performance", "requests", "model",
               "model_initialization_stages", "native_attention_and_kv", "attention_implementation",
               "native_backend", "master_storage", "device_buffer_pool", "original_weight_samples_unchanged",
               "all_master_storage_versions_unchanged", "calibration_sources", "attention_cost_table",
               "model_identity", "torch_environment", "total_device_budget_bytes", "allocator_cap_bytes",
               "control_affinity", "host_peak_rss_bytes"}


def test_phase_metrics_closed_form():
    m = records.phase_metrics(100, [0.5, 0.6, 0.8, 1.0])
    assert set(m) == METRIC_KEYS
    assert m["prefill_seconds"] == 0.5 and math.isclose(m["decode_seconds"], 0.5)
    assert m["decode_forwards"] == 3 and m["output_tokens"] == 4
    assert m["prefill_tokens_per_second"] == 200.0 and math.isclose(m["decode_tokens_per_second"], 6.0)
    assert math.isclose(m["decode_tpot_seconds"], 0.5 / 3) and m["end_to_end_output_tokens_per_second"] == 4.0
    for bad in ([0.5], [0.5, 0.5], [0.0, 1.0], [0.5, float("nan")]):
        with pytest.raises(ValueError):
            records.phase_metrics(100, bad)
    with pytest.raises(ValueError):
        records.phase_metrics(0, [0.5, 1.0])


def test_recorder_writes_the_reference_layout(tmp_path):
    out = tmp_path / "run" / "result.json"
    rec = records.RunRecorder(out, entry="tests", argv=["x"], config=dict(lengths=[8], output=out))
    man = json.loads((out.parent / "manifest.json").read_text())
    assert MANIFEST_KEYS <= set(man) and man["status"] == "running"
    assert man["source_archive"]["members"] and (out.parent / "source.zip").is_file()
    assert "pdscope_amd/cache.py" in man["source_archive"]["members"]
    assert records.sha256_file(out.parent / "source.zip") == man["source_archive"]["sha256"]
    rec.cases([dict(case_id="c0", role="measure")])
    rows = [dict(phase="prefill", step=0, layer=0, token_counts={3: 2, 7: 1})]
    trace = rec.trace("c0", [records.trace_row_json(r) for r in rows])
    with gzip.open(out.parent / trace["path"], "rt") as f:
        assert json.load(f)[0]["token_counts"] == {"3": 2, "7": 1}
    assert trace["sha256"] == records.sha256_file(out.parent / trace["path"])
    rec.request(dict(case=dict(case_id="c0"), metrics=records.phase_metrics(8, [0.1, 0.2])))
    rec.request(dict(case=dict(case_id="c1"), metrics=records.phase_metrics(8, [0.1, 0.3])))
    lines = (out.parent / "requests.jsonl").read_text().splitlines()
    assert [json.loads(x)["case"]["case_id"] for x in lines] == ["c0", "c1"]
    rec.finish(dict(schema_version=2, status="completed", requests=rec.requests))
    man = json.loads((out.parent / "manifest.json").read_text())
    assert man["status"] == "completed" and MANIFEST_END_KEYS <= set(man)
    assert man["result_sha256"] == records.sha256_file(out)
    with pytest.raises(FileExistsError):       # a result is never overwritten
        records.RunRecorder(out, entry="tests", argv=[], config={})


def test_recorder_marks_a_failed_run(tmp_path):
    out = tmp_path / "r2" / "result.json"
    rec = records.RunRecorder(out, entry="tests", argv=[], config={})
    try:
        raise RuntimeError("boom")
    except RuntimeError as err:
        rec.fail(err)
    man = json.loads((out.parent / "manifest.json").read_text())
    assert man["status"] == "failed" and man["error_type"] == "RuntimeError" and man["error"] == "boom"
    assert "RuntimeError: boom" in (out.parent / "failure.txt").read_text() and not out.exists()


def test_build_cases_warmups_then_measured():
    from pdscope_amd.compare import build_cases
    specs = build_cases([128, 256], repetitions=2, output_tokens=8, warmups=2, demand_slots=8, merge="reference")
    assert [s["role"] for s in specs] == ["warmup", "warmup", "measure", "measure"] * 2
    assert len({s["case_id"] for s in specs}) == 8 and all(s["demand_slots"] == 8 for s in specs)
    for bad in (dict(lengths=[], repetitions=1), dict(lengths=[128], repetitions=0),
                dict(lengths=[128], repetitions=1, output_tokens=1)):
        with pytest.raises(ValueError):
            build_cases(**bad)
