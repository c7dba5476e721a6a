"""Write the placement-planner vectors (tests/golden/policy_vectors.json.gz).

``plan_pdscope`` is a decision procedure with no closed form, and the
reference ships no plans, traces or tests for it, so its input/output pairs
come from the reference's own pure-Python module
expertbench/pdscope_policy.py (imports only ``math`` and ``operator``),
loaded from its file in the source tree.  Inputs are seeded random layer
calls over both phases, every decode mode, overrides, the joint-next ablation
and invalid arguments, costed by four tables: the reference's shipped
costs/cost_table.json points (A100 + Xeon) and three seeded synthetic tables
whose CPU and GPU costs cross so that prefill splits land mid-list.  Costs go through
pdscope_amd.costs.FileCosts, whose interpolation is pinned separately.

Run here, where the reference tree exists:
    python tests/golden/make_policy_vectors.py
"""
from __future__ import annotations

import gzip
import importlib.util
import json
import random
import sys
import tempfile
from pathlib import Path

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))
from pdscope_amd.costs import FileCosts  # noqa: E402

REF_POLICY = Path("/root/reference/expertbench/pdscope_policy.py")
REF_COSTS = Path("/root/reference/costs/cost_table.json")
OUT = HERE / "policy_vectors.json.gz"
SEED = 20261201
LOADS = (1, 4, 16, 64, 128, 256, 1024, 4096)


def load_reference():
    spec = importlib.util.spec_from_file_location("ref_pdscope_policy", REF_POLICY)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def synthetic_points(rng):
    """CPU cost linear in tokens, GPU cost flat then linear, copy cost flat:
    the CPU wins small loads, the GPU large ones."""
    cpu0, cpu1 = rng.uniform(0.05, 0.4), rng.uniform(0.005, 0.05)
    gpu0, gpu1 = rng.uniform(0.05, 0.3), rng.uniform(1e-5, 2e-4)
    h2d = rng.uniform(0.2, 1.5)
    return {str(n): dict(cpu_ms=cpu0 + cpu1 * (n - 1), gpu_ms=gpu0 + gpu1 * n, h2d_ms=h2d + gpu1 * n)
            for n in LOADS}


def table_payload(points, name):
    return dict(schema_version=1, kind="pdscope_cost_table", model="Qwen3-30B-A3B BF16", platform=name,
                loads=list(LOADS), points=points)


def jsonable(x):
    if isinstance(x, dict):
        return {str(k): jsonable(v) for k, v in x.items()}
    if isinstance(x, (list, tuple)):
        return [jsonable(v) for v in x]
    return x


def prefill_counts(rng, tokens, top_k, experts=128, skew=1.0):
    weights = [1.0 / (i + 1) ** skew for i in range(experts)]
    order = list(range(experts))
    rng.shuffle(order)
    counts = {}
    for _ in range(tokens):
        chosen = set()
        while len(chosen) < top_k:
            chosen.add(order[rng.choices(range(experts), weights)[0]])
        for e in chosen:
            counts[e] = counts.get(e, 0) + 1
    return counts


def decode_counts(rng, top_k):
    return {e: 1 for e in rng.sample(range(128), top_k)}


def make_case(rng, phase, table):
    top_k = 8 if rng.random() < 0.8 else rng.choice((2, 4, 6))
    layer = rng.randrange(48)
    if phase == "prefill":
        tokens = rng.choice((1, 3, 16, 64, 200, 512))
        cur = prefill_counts(rng, tokens, top_k, skew=rng.choice((0.0, 0.8, 1.2)))
        nxt = prefill_counts(rng, tokens, top_k, skew=rng.choice((0.0, 0.8, 1.2))) if layer < 47 else {}
    else:
        cur = decode_counts(rng, top_k)
        nxt = decode_counts(rng, top_k) if layer < 47 else {}
    def gpu_ids(demand):
        # a share of the demanded experts (every share from none to all) plus unrelated ids
        ids = rng.sample(sorted(demand), rng.randrange(len(demand) + 1)) if demand else []
        ids += rng.sample(range(128), rng.randrange(4))
        return list(dict.fromkeys(ids))
    cur_gpu, nxt_gpu = gpu_ids(cur), gpu_ids(nxt)
    kw = dict(current_layer=layer, phase=phase, current_gpu_ids=cur_gpu, next_gpu_ids=nxt_gpu,
              attention_ms=rng.choice((0.0, rng.uniform(0, 0.5), rng.uniform(0.5, 4.0))),
              hit_rate=rng.choice((0.0, 1.0, 0.5, rng.random())),
              prefetch_slots=rng.choice((0, 1, 2, 4, 8, 16)),
              io_startup_ms=rng.choice((0.0, 0.0, rng.uniform(0, 0.2))), top_k=top_k)
    if rng.random() < 0.2:
        kw["cpu_balance_target_override"] = rng.randrange(top_k + 1)
    if rng.random() < 0.2:
        kw["joint_next"] = False
    if rng.random() < 0.2:
        kw["record_checks"] = False
    if rng.random() < 0.1:
        kw["compute_formula_target"] = False
    if rng.random() < 0.1:
        kw["trusted"] = True
    return dict(table=table, current_counts=sorted(cur.items()), next_counts=sorted(nxt.items()), kwargs=kw)


def invalid_cases(table):
    base = dict(table=table, current_counts=[[3, 1], [9, 2]], next_counts=[[4, 1]],
                kwargs=dict(current_layer=5, phase="prefill", current_gpu_ids=[], next_gpu_ids=[],
                            attention_ms=0.1, hit_rate=0.5, prefetch_slots=2))
    edits = [
        ("current_counts", []), ("current_counts", [[128, 1]]), ("current_counts", [[3, 0]]),
        ("next_counts", [[-1, 1]]), ("phase", "train"), ("current_layer", 48), ("current_layer", 47),
        ("top_k", 0), ("top_k", 129), ("prefetch_slots", -1), ("attention_ms", -1.0),
        ("attention_ms", float("inf")), ("io_startup_ms", float("nan")), ("hit_rate", 1.5), ("hit_rate", -0.1),
        ("cpu_balance_target_override", 9), ("joint_next", 1), ("current_gpu_ids", [3, 3]),
        ("next_gpu_ids", [200]), ("phase", "decode"), ("attention_ms", True),
    ]
    out = []
    for key, value in edits:
        case = json.loads(json.dumps(base))
        if key in ("current_counts", "next_counts"):
            case[key] = value
        else:
            case["kwargs"][key] = value
        out.append(case)
    return out


def run_case(ref, case, tables):
    costs = tables[case["table"]]
    kw = dict(case["kwargs"])
    try:
        result = ref.plan_pdscope(dict(map(tuple, case["current_counts"])), dict(map(tuple, case["next_counts"])),
                                  costs=costs, **kw)
        return dict(result=jsonable(result))
    except ref.PDScopePolicyError as exc:
        return dict(error=str(exc))


def main():
    ref = load_reference()
    rng = random.Random(SEED)
    ref_points = json.loads(REF_COSTS.read_text())["points"]
    tables_payload = {"a100_xeon": table_payload(ref_points, "reference shipped table (A100 + Xeon)")}
    for i in range(3):
        tables_payload[f"synthetic{i}"] = table_payload(synthetic_points(rng), "synthetic crossing costs")
    tmp = Path(tempfile.mkdtemp())
    tables = {}
    for name, payload in tables_payload.items():
        (tmp / f"{name}.json").write_text(json.dumps(payload))
        tables[name] = FileCosts(tmp / f"{name}.json")

    cases = []
    names = list(tables_payload)
    for i in range(240):
        phase = "decode" if i % 2 else "prefill"
        cases.append(make_case(rng, phase, names[i % len(names)]))
    cases += invalid_cases("a100_xeon")
    for case in cases:
        case.update(run_case(ref, case, tables))

    prefetch = [dict(window=w, hit_rate=h, limit=lim,
                     result=jsonable(ref.confidence_prefetch_count(w, h, lim)))
                for w in (0.0, 0.3, 0.5, 1.0, 1.7, 2.0, 2.25, 3.9, 7.5)
                for h in (0.0, 0.25, 0.5, 0.9, 1.0) for lim in (0, 2, 8)]
    targets = [dict(table=name, top_k=k, result=ref.decode_cpu_target(k, tables[name]))
               for name in names for k in (1, 2, 4, 6, 8, 16, 128)]
    modes = {}
    for case in cases:
        if "result" in case:
            modes[case["result"]["mode"]] = modes.get(case["result"]["mode"], 0) + 1
    payload = dict(source=str(REF_POLICY.relative_to("/root/reference")), seed=SEED, tables=tables_payload,
                   cases=cases, prefetch=prefetch, decode_targets=targets)
    with gzip.open(OUT, "wt") as f:
        json.dump(payload, f, separators=(",", ":"))
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes): {len(cases)} cases, modes {modes}, "
          f"errors {sum('error' in c for c in cases)}")


if __name__ == "__main__":
    main()
