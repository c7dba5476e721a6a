"""Placement planner (pdscope_amd.policy) and cost tables (pdscope_amd.costs).

Pinned three ways:
* vectors written by the reference's own expertbench/pdscope_policy.py
  (tests/golden/make_policy_vectors.py): every result key, every error;
* known answers derived by hand below, chosen so that the usual slips (the
  CPU prefix inclusive where it is exclusive, copies and compute summed
  instead of overlapped, the a_load shift) change the answer;
* FileCosts interpolation against the closed form.
"""
from __future__ import annotations

import gzip
import json
import math
from pathlib import Path

import pytest

from pdscope_amd.costs import FileCosts
from pdscope_amd.policy import PDScopePolicyError, confidence_prefetch_count, decode_cpu_target, plan_pdscope

GOLDEN = Path(__file__).resolve().parent / "golden" / "policy_vectors.json.gz"
LOADS = (1, 4, 16, 64, 128, 256, 1024, 4096)


@pytest.fixture(scope="module")
def vectors(tmp_path_factory):
    payload = json.load(gzip.open(GOLDEN, "rt"))
    tmp = tmp_path_factory.mktemp("tables")
    tables = {}
    for name, table in payload["tables"].items():
        (tmp / f"{name}.json").write_text(json.dumps(table))
        tables[name] = FileCosts(tmp / f"{name}.json")
    return payload, tables


def _jsonable(x):
    if isinstance(x, dict):
        return {str(k): _jsonable(v) for k, v in x.items()}
    if isinstance(x, (list, tuple)):
        return [_jsonable(v) for v in x]
    return x


def _same(a, b, path=""):
    """Equal structure, equal ids and strings; floats to 1e-12 relative."""
    if isinstance(b, float) or isinstance(a, float):
        assert math.isclose(a, b, rel_tol=1e-12, abs_tol=1e-15), path
    elif isinstance(b, dict):
        assert set(a) == set(b), path
        for k in b:
            _same(a[k], b[k], f"{path}.{k}")
    elif isinstance(b, list):
        assert len(a) == len(b), path
        for i, (x, y) in enumerate(zip(a, b)):
            _same(x, y, f"{path}[{i}]")
    else:
        assert a == b, path


def test_plan_matches_reference_vectors(vectors):
    payload, tables = vectors
    checked = errors = 0
    for i, case in enumerate(payload["cases"]):
        args = (dict(map(tuple, case["current_counts"])), dict(map(tuple, case["next_counts"])))
        kwargs = dict(case["kwargs"], costs=tables[case["table"]])
        if "error" in case:
            with pytest.raises(PDScopePolicyError) as info:
                plan_pdscope(*args, **kwargs)
            assert str(info.value) == case["error"], i
            errors += 1
            continue
        got = _jsonable(plan_pdscope(*args, **kwargs))
        want = case["result"]
        got.pop("scope"), want.pop("scope")
        _same(got, want, f"case{i}")
        checked += 1
    assert checked >= 200 and errors >= 20


def test_prefetch_count_and_decode_target_match_reference_vectors(vectors):
    payload, tables = vectors
    for v in payload["prefetch"]:
        _same(_jsonable(confidence_prefetch_count(v["window"], v["hit_rate"], v["limit"])), v["result"])
    for v in payload["decode_targets"]:
        assert decode_cpu_target(v["top_k"], tables[v["table"]]) == v["result"]


class _Costs:
    """A cost table given per load as (cpu_ms, gpu_ms, h2d_ms)."""

    def __init__(self, rows):
        self.rows = rows

    def for_load(self, n):
        cpu, gpu, h2d = self.rows[n]
        return dict(tokens=n, cpu_ms=cpu, gpu_ms=gpu, h2d_ms=h2d)


def test_decode_target_closed_form():
    # n_c = argmin_n max((k-n) g, n c), smallest n on ties
    for g, c, k in [(1.0, 1.0, 8), (1.0, 3.0, 8), (3.0, 1.0, 8), (0.24, 0.265, 8), (1.0, 1.0, 1), (2.0, 1.0, 3)]:
        brute = min(range(k + 1), key=lambda n: (max((k - n) * g, n * c), n))
        assert decode_cpu_target(k, _Costs({1: (c, g, 1.0)})) == brute
    assert decode_cpu_target(8, _Costs({1: (1.0, 1.0, 1.0)})) == 4   # even split
    assert decode_cpu_target(8, _Costs({1: (3.0, 1.0, 1.0)})) == 2   # max(6, 6)
    assert decode_cpu_target(2, _Costs({1: (1.0, 1.0, 1.0)})) == 1


def test_confidence_prefetch_closed_form():
    assert confidence_prefetch_count(2.0, 0.0, 8)[0] == 2             # whole copies are free
    assert confidence_prefetch_count(2.25, 0.5, 8)[0] == 2            # .5*.25 - .5*.75 < 0
    assert confidence_prefetch_count(2.25, 0.9, 8)[0] == 3            # .9*.25 - .1*.75 > 0
    assert confidence_prefetch_count(2.75, 0.25, 8)[0] == 2           # .25*.75 - .75*.25 == 0: not taken
    assert confidence_prefetch_count(0.4, 1.0, 8)[0] == 1
    assert confidence_prefetch_count(0.4, 1.0, 0)[0] == 0              # capacity
    with pytest.raises(PDScopePolicyError):
        confidence_prefetch_count(1.0, 1.5, 2)


def test_prefill_known_answer_exclusive_local_boundary():
    # loads 1, 4, 16 on experts 10, 20, 30; copies 2 ms each, one at a time
    costs = _Costs({1: (1.0, 1.0, 2.0), 4: (4.0, 0.5, 2.0), 16: (16.0, 1.0, 2.0)})
    plan = plan_pdscope({10: 1, 20: 4, 30: 16}, {}, current_layer=47, phase="prefill", current_gpu_ids=[],
                        next_gpu_ids=[], costs=costs, attention_ms=0.5, hit_rate=1.0, prefetch_slots=4)
    # GPU suffix (copies from the largest end, compute after its copy):
    #   [30]: dma 2, done 3;  [20,30]: dma 4, done max(3,4)+.5 = 4.5;  [10,20,30]: dma 6, done 7
    # CPU prefix: 0, 1, 5, 21.  Joint boundary (inclusive CPU + attention):
    #   i=0: 7 < 1.5 no;  i=1: 4.5 < 5.5 yes -> experts 20, 30 eligible
    # local boundary (exclusive CPU): i=1: 4.5 < 1 no;  i=2: 3 < 5 yes
    assert plan["mode"] == "prefill"
    assert plan["global_queue"] == [[47, 20, 4], [47, 30, 16]]
    assert plan["boundary"] == 2
    assert plan["on_demand_queue"] == [30] and plan["cpu_queue"] == [20, 10]
    assert plan["placements"] == {10: "cpu", 20: "cpu", 30: "gpu"}
    assert plan["estimate"]["cpu_ms"] == 5.0 and plan["estimate"]["gpu_ms"] == 3.0
    assert plan["prefetch_queue"] == [] and plan["unload_queue"] == []


def test_decode_a_load_known_answer_inclusive_boundary():
    # k=2, cpu 3 / gpu 1 per token: n_c = argmin(max(2,0), max(1,3), max(0,6)) = 0
    costs = _Costs({1: (3.0, 1.0, 2.0)})
    plan = plan_pdscope({5: 1, 7: 1}, {1: 1, 2: 1}, current_layer=3, phase="decode", current_gpu_ids=[],
                        next_gpu_ids=[1, 2], costs=costs, attention_ms=0.0, hit_rate=1.0, prefetch_slots=4, top_k=2)
    # current high (2 > 0), next all resident -> a_load; local boundary with
    # the inclusive CPU prefix [0, 3, 6] against GPU suffix [5, 3]:
    #   i=0: 5 < 3 no;  i=1: 3 < 6 yes -> expert 7 staged, expert 5 on the CPU
    assert plan["cpu_balance_target"] == 0 and plan["mode"] == "a_load"
    assert plan["boundary"] == 1 and plan["on_demand_queue"] == [7] and plan["cpu_queue"] == [5]
    assert plan["local_checks"] == [dict(boundary=0, expert=5, gpu_ms=5.0, cpu_ms=3.0),
                                    dict(boundary=1, expert=7, gpu_ms=3.0, cpu_ms=6.0)]
    assert plan["prefetch_queue"] == [] and plan["unload_queue"] == []


def test_decode_unload_and_prefetch_known_answers():
    # k=2, cpu 1.5 / gpu 1: n_c = argmin(2, 1.5, 3) = 1
    costs = _Costs({1: (1.5, 1.0, 2.0)})
    common = dict(current_layer=3, phase="decode", current_gpu_ids=[5, 7], costs=costs, top_k=2)
    # both current experts resident, next all resident -> c_unload, hand back
    # n_c - 0 = 1 resident expert, the lowest (load, id): 5
    plan = plan_pdscope({5: 1, 7: 1}, {1: 1, 2: 1}, next_gpu_ids=[1, 2], attention_ms=4.0, hit_rate=1.0,
                        prefetch_slots=8, **common)
    assert plan["mode"] == "c_unload" and plan["unload_queue"] == [5]
    assert plan["placements"] == {5: "cpu", 7: "gpu"} and plan["prefetch_queue"] == []
    # next not resident -> b_prefetch.  cpu 1.5 - gpu 1 = gap .5;  window
    # (.5 + 4) / 2 = 2.25 copies, hit rate 1 takes the ceiling 3, capacity
    # 2 next candidates, decode cap 2 - n_c = 1;  Eq.6 check for 1 copy:
    # exposed max(0, 1 - 2.25) * 2 + max gpu 1 = 1 < remaining cpu 1.5 -> keep
    plan = plan_pdscope({5: 1, 7: 1}, {1: 1, 2: 1}, next_gpu_ids=[], attention_ms=4.0, hit_rate=1.0,
                        prefetch_slots=8, **common)
    assert plan["mode"] == "b_prefetch" and plan["unload_queue"] == [5]
    assert plan["estimate"]["gap_ms"] == 0.5 and plan["estimate"]["confidence"]["continuous_window"] == 2.25
    assert plan["decode_prefetch_constraints"] == [dict(count=1, exposed_gpu_ms=1.0, remaining_cpu_ms=1.5)]
    assert plan["prefetch_queue"] == [2]


def test_plan_invariants_random():
    import random
    rng = random.Random(7)
    costs = _Costs({n: (0.1 + 0.02 * n, 0.2 + 1e-4 * n, 0.6) for n in range(1, 4097)})
    for _ in range(200):
        decode = rng.random() < 0.5
        k = 8
        if decode:
            cur = {e: 1 for e in rng.sample(range(128), k)}
            nxt = {e: 1 for e in rng.sample(range(128), k)}
        else:
            cur = {e: rng.randint(1, 300) for e in rng.sample(range(128), rng.randint(1, 60))}
            nxt = {e: rng.randint(1, 300) for e in rng.sample(range(128), rng.randint(1, 60))}
        res = rng.sample(sorted(cur), rng.randint(0, len(cur)))
        plan = plan_pdscope(cur, nxt, current_layer=rng.randrange(47), phase="decode" if decode else "prefill",
                            current_gpu_ids=res, next_gpu_ids=[], costs=costs, attention_ms=rng.uniform(0, 2),
                            hit_rate=rng.random(), prefetch_slots=rng.randint(0, 8), top_k=k)
        gpu = set(plan["gpu_resident_queue"]) | set(plan["on_demand_queue"])
        assert gpu.isdisjoint(plan["cpu_queue"]) and gpu | set(plan["cpu_queue"]) == set(cur)
        assert set(plan["gpu_resident_queue"]) <= set(res) and set(plan["unload_queue"]) <= set(res)
        assert set(plan["on_demand_queue"]).isdisjoint(res)
        assert plan["cpu_queue"] == sorted(plan["cpu_queue"], key=lambda e: (-cur[e], e))
        loads = [cur[e] for e in plan["on_demand_queue"]]
        assert loads == sorted(loads, reverse=True)              # largest staged first
        assert set(plan["prefetch_queue"]) <= set(nxt) and len(plan["prefetch_queue"]) <= 8
        if plan["mode"] in ("a_load", "c_unload"):
            assert plan["prefetch_queue"] == []


def _table(tmp_path, points, kind="pdscope_cost_table"):
    path = tmp_path / "t.json"
    path.write_text(json.dumps(dict(kind=kind, points={str(n): p for n, p in points.items()})))
    return path


def test_file_costs_interpolation_closed_form(tmp_path):
    pts = {n: dict(cpu_ms=0.5 * n, gpu_ms=1.0 + 0.01 * n, h2d_ms=2.0) for n in LOADS}
    pts[16]["cpu_ms"] = 100.0                                     # a kink: interpolation is piecewise
    costs = FileCosts(_table(tmp_path, pts))
    assert costs.for_load(4) == dict(tokens=4, **pts[4])
    got = costs.for_load(10)                                      # 4 .. 16, t = 0.5
    assert got["tokens"] == 10 and math.isclose(got["cpu_ms"], (2.0 + 100.0) / 2)
    assert math.isclose(got["gpu_ms"], 1.10) and got["h2d_ms"] == 2.0
    got = costs.for_load(2)                                       # 1 .. 4, t = 1/3
    assert math.isclose(got["cpu_ms"], 0.5 + (2.0 - 0.5) / 3)
    for bad in (0, 4097):
        with pytest.raises(ValueError):
            costs.for_load(bad)
    assert costs.sources[0]["kind"] == "shipped_cost_table" and len(costs.sources[0]["sha256"]) == 64


def test_file_costs_rejects_bad_tables(tmp_path):
    pts = {n: dict(cpu_ms=1.0, gpu_ms=1.0, h2d_ms=1.0) for n in LOADS}
    with pytest.raises(ValueError):
        FileCosts(_table(tmp_path, pts, kind="other"))
    with pytest.raises(ValueError):
        FileCosts(_table(tmp_path, {n: p for n, p in pts.items() if n != 4096}))


def test_shipped_mi355x_cost_table():
    """The table measured on MI355X loads, covers the measured domain and
    interpolates linearly between its points."""
    from pdscope_amd.costs import mi355x_costs
    c = mi355x_costs()
    assert c.loads == [1, 4, 16, 64, 128, 256, 1024, 4096]
    lo, hi = c.for_load(64), c.for_load(128)
    mid = c.for_load(96)
    for k in ("cpu_ms", "gpu_ms", "h2d_ms"):
        assert lo[k] > 0 and abs(mid[k] - (lo[k] + hi[k]) / 2) <= 1e-12 * max(1.0, hi[k])
    assert c.for_load(4096)["cpu_ms"] > c.for_load(1)["cpu_ms"]
