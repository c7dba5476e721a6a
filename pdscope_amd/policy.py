"""CPU/GPU placement planner of the PDScope runtime (drop-in for
expertbench/pdscope_policy.py:39-223), a host-side decision from measured costs.

For one layer call it splits the routed experts between the CPU backend and
the GPU (resident copies or demand staging), picks the next-layer experts to
prefetch and, in decode, the resident experts to hand back to the CPU, with
the same inputs, rules and result keys as ``plan_pdscope`` in the reference:

* candidates not on the GPU are ordered by (tokens, layer, expert), ascending;
  the CPU takes a prefix of that order, the GPU the remaining suffix;
* the CPU time of a prefix is the left-to-right sum of per-expert CPU costs;
  the GPU time of a suffix follows copies issued from the largest end
  (``dma`` grows by the copy cost, compute starts when both the previous
  compute and this expert's copy are done, then adds the GPU cost);
* prefill (and decode with both layers above the CPU balance target) first
  picks a joint boundary over current + next-layer candidates (the first
  boundary where GPU suffix < CPU prefix + attention), then the current-layer
  boundary among the jointly eligible experts;
* decode modes follow the counts of non-resident current / next candidates
  against n_c = argmin_n max((k - n) t_gpu, n t_cpu) at load 1;
* the prefetch count is the number of copies hidden in the CPU/GPU gap plus
  attention, with the partially hidden boundary copy taken when its
  hit-rate-weighted benefit is positive, then (decode) reduced until the
  exposed GPU tail is shorter than the remaining CPU work.

Pure Python: no clocks, tensors or device calls.
"""
from __future__ import annotations

import math
from typing import NamedTuple


class PDScopePolicyError(ValueError):
    pass


MODES = {(True, False): "a_load", (False, True): "b_prefetch", (False, False): "c_unload",
         (True, True): "d_cross_layer"}


def _finite(value, name, *, positive=False):
    if type(value) not in (int, float) or not math.isfinite(value) or value < 0 or (positive and value == 0):
        raise PDScopePolicyError("invalid " + name)
    return float(value)


def _demand(values, name, num_experts):
    d = dict(values)
    for e, n in d.items():
        if type(e) is not int or not 0 <= e < num_experts or type(n) is not int or n < 1:
            raise PDScopePolicyError("invalid " + name)
    return d


def _expert_ids(values, num_experts):
    ids = tuple(values)
    if len(ids) != len(set(ids)) or any(type(e) is not int or not 0 <= e < num_experts for e in ids):
        raise PDScopePolicyError("invalid resident IDs")
    return set(ids)


class Job(NamedTuple):
    """One expert execution candidate: (layer, expert, routed tokens)."""
    layer: int
    expert: int
    tokens: int


def _job_order(job):
    return (job.tokens, job.layer, job.expert)


def confidence_prefetch_count(window, hit_rate, limit):
    """Copies to prefetch in a hidden window of `window` copy times.

    Whole copies inside the window are free; the copy across the window's
    edge is taken when hit_rate * (hidden part) exceeds (1 - hit_rate) *
    (exposed part).  An integral window takes exactly its whole copies.
    """
    _finite(window, "prefetch window")
    _finite(hit_rate, "hit rate")
    if hit_rate > 1 or type(limit) is not int or limit < 0:
        raise PDScopePolicyError("invalid prefetch confidence or capacity")
    edge = math.ceil(window)
    benefit = hit_rate * (window - edge + 1) - (1 - hit_rate) * (edge - window)
    chosen = edge if benefit > 0 else edge - 1
    chosen = max(0, chosen)
    if window == math.floor(window):
        chosen = int(window)
    return min(limit, chosen), dict(continuous_window=window, ceil_boundary=edge,
                                    normalized_boundary_benefit=benefit, hit_rate=hit_rate)


def decode_cpu_target(top_k, costs):
    """n_c = argmin over n in 0..k of max((k - n) * gpu_ms, n * cpu_ms) at one
    token per expert, the smaller n on ties."""
    if type(top_k) is not int or not 1 <= top_k <= 128:
        raise PDScopePolicyError("invalid top-k for the CPU balance target")
    point = costs.for_load(1)
    t_gpu = _finite(point["gpu_ms"], "gpu cost", positive=True)
    t_cpu = _finite(point["cpu_ms"], "cpu cost", positive=True)
    best, best_key = 0, None
    for n in range(top_k + 1):
        key = (max((top_k - n) * t_gpu, n * t_cpu), n)
        if best_key is None or key < best_key:
            best, best_key = n, key
    return best


class _CostModel:
    """Per-load cost rows and the prefix / suffix recurrences over job lists."""

    def __init__(self, costs, loads, io_startup_ms):
        self.io_startup_ms = io_startup_ms
        self.rows = {}
        for n in loads:
            row = costs.for_load(n)
            if row.get("tokens") != n:
                raise PDScopePolicyError("cost token load mismatch")
            self.rows[n] = {k: _finite(row[k], k, positive=True) for k in ("cpu_ms", "gpu_ms", "h2d_ms")}

    def cost(self, job, what):
        return self.rows[job.tokens][what]

    def cpu_prefix(self, jobs):
        """out[m] = CPU time of jobs[:m], summed left to right."""
        out = [0.0]
        for job in jobs:
            out.append(out[-1] + self.cost(job, "cpu_ms"))
        return out

    def gpu_suffix(self, jobs, initial=0.0):
        """out[i] = completion time of jobs[i:] on the GPU: copies issued from
        the last job backwards, compute waiting for its copy; out[len] is
        `initial` (compute already queued ahead)."""
        out = [0.0] * (len(jobs) + 1)
        dma, compute = self.io_startup_ms, initial
        for i in range(len(jobs) - 1, -1, -1):
            dma += self.cost(jobs[i], "h2d_ms")
            compute = max(compute, dma) + self.cost(jobs[i], "gpu_ms")
            out[i] = compute
        out[len(jobs)] = initial if initial else 0.0
        return out

    def max_suffix(self, jobs, what):
        out = [0.0] * (len(jobs) + 1)
        for i in range(len(jobs) - 1, -1, -1):
            out[i] = max(out[i + 1], self.cost(jobs[i], what))
        return out


def plan_pdscope(current_counts, next_counts, *, current_layer, phase, current_gpu_ids, next_gpu_ids, costs,
                 attention_ms, hit_rate, prefetch_slots, io_startup_ms=0., top_k=8, cpu_balance_target_override=None,
                 joint_next=True, record_checks=True, compute_formula_target=True, trusted=False, num_experts=128,
                 num_layers=48):
    """Placement of one layer's routed experts (same arguments and result keys
    as expertbench/pdscope_policy.py:71-223; num_experts / num_layers bound
    the expert and layer ids, 128 and 48 for Qwen3-30B-A3B)."""
    if trusted:
        cur, nxt = dict(current_counts), dict(next_counts)
    else:
        cur = _demand(current_counts, "current demand", num_experts)
        nxt = _demand(next_counts, "next prediction", num_experts)
    if (not cur or phase not in ("prefill", "decode") or type(current_layer) is not int
            or not 0 <= current_layer < num_layers or (current_layer == num_layers - 1 and nxt)
            or type(top_k) is not int or not 1 <= top_k <= 128
            or type(prefetch_slots) is not int or prefetch_slots < 0):
        raise PDScopePolicyError("invalid phase, layer, demand or capacity")
    if phase == "decode":
        one_each = lambda d: len(d) == top_k and all(n == 1 for n in d.values())  # noqa: E731
        if not one_each(cur) or (nxt and not one_each(nxt)):
            raise PDScopePolicyError("decode needs one top-k assignment per expert")
    attention_ms = _finite(attention_ms, "attention cost")
    io_startup_ms = _finite(io_startup_ms, "IO startup")
    _finite(hit_rate, "hit rate")
    if hit_rate > 1:
        raise PDScopePolicyError("hit rate exceeds one")
    if cpu_balance_target_override is not None and (type(cpu_balance_target_override) is not int
                                                    or not 0 <= cpu_balance_target_override <= top_k):
        raise PDScopePolicyError("invalid CPU balance target override")
    if any(type(flag) is not bool for flag in (joint_next, record_checks, compute_formula_target, trusted)):
        raise PDScopePolicyError("invalid next-layer coordination mode or check recording")

    resident = _expert_ids(current_gpu_ids, num_experts) & cur.keys()
    next_resident = _expert_ids(next_gpu_ids, num_experts) & nxt.keys()
    model = _CostModel(costs, set(cur.values()) | set(nxt.values()) | {1}, io_startup_ms)
    current = sorted((Job(current_layer, e, n) for e, n in cur.items() if e not in resident), key=_job_order)
    following = sorted((Job(current_layer + 1, e, n) for e, n in nxt.items() if e not in next_resident),
                       key=_job_order)

    formula_nc = decode_cpu_target(top_k, costs) if compute_formula_target else None
    if cpu_balance_target_override is not None:
        nc = cpu_balance_target_override
    else:
        nc = formula_nc if formula_nc is not None else decode_cpu_target(top_k, costs)
    mode = "prefill" if phase == "prefill" else MODES[(len(current) > nc, len(following) > nc)]

    # joint boundary over this layer and the next (prefill, cross-layer decode)
    global_queue, global_checks, local_checks = [], [], []
    if mode in ("prefill", "d_cross_layer"):
        merged = sorted(current + (following if joint_next else []), key=_job_order)
        gpu_t, cpu_t = model.gpu_suffix(merged), model.cpu_prefix(merged)
        for i in range(len(merged)):
            tg, tc = gpu_t[i], cpu_t[i + 1] + attention_ms
            if record_checks:
                global_checks.append(dict(boundary=i, gpu_ms=tg, cpu_ms=tc))
            if tg < tc:
                global_queue = merged[i:]
                break
        eligible = {(j.layer, j.expert) for j in global_queue}
    elif mode == "a_load":
        eligible = {(j.layer, j.expert) for j in current}
    else:
        eligible = set()

    # this layer's boundary among the eligible candidates
    boundary = len(current)
    if mode in ("prefill", "d_cross_layer", "a_load"):
        gpu_t, cpu_t = model.gpu_suffix(current), model.cpu_prefix(current)
        shift = 1 if mode == "a_load" else 0
        for i, job in enumerate(current):
            if (job.layer, job.expert) not in eligible:
                continue
            tc, tg = cpu_t[i + shift], gpu_t[i]
            if record_checks:
                local_checks.append(dict(boundary=i, expert=job.expert, gpu_ms=tg, cpu_ms=tc))
            if tg < tc:
                boundary = i
                break
    on_demand = current[boundary:]

    unload = []
    if mode in ("b_prefetch", "c_unload"):
        unload = sorted(resident, key=lambda e: (cur[e], e))[:max(0, nc - len(current))]
    gpu_ids = (resident - set(unload)) | {j.expert for j in on_demand}
    cpu_ids = set(cur) - gpu_ids
    cpu_ms = sum(model.rows[cur[e]]["cpu_ms"] for e in cpu_ids)
    resident_gpu_ms = sum(model.rows[cur[e]]["gpu_ms"] for e in resident - set(unload))
    gpu_ms = model.gpu_suffix(on_demand, resident_gpu_ms)[0] if on_demand else resident_gpu_ms
    gap = cpu_ms - gpu_ms

    # prefetch: copies hidden in the CPU/GPU gap plus attention
    tio = max((model.cost(j, "h2d_ms") for j in following), default=model.rows[1]["h2d_ms"])
    window = max(0., (gap + attention_ms) / tio)
    count, confidence = confidence_prefetch_count(window, hit_rate, min(prefetch_slots, len(following)))
    if mode in ("a_load", "c_unload") or not following:
        count = 0
    constraints = []
    if phase == "decode":
        count = min(count, max(0, len(following) - nc))
        if count:
            f_cpu, f_gpu_max = model.cpu_prefix(following), model.max_suffix(following, "gpu_ms")
            n = len(following)
            while count:
                exposed = max(0., count - window) * tio + f_gpu_max[n - count]
                remaining = f_cpu[n - count]
                constraints.append(dict(count=count, exposed_gpu_ms=exposed, remaining_cpu_ms=remaining))
                if exposed < remaining:
                    break
                count -= 1
    prefetch = list(reversed(following[-count:])) if count else []

    if gpu_ids & cpu_ids or gpu_ids | cpu_ids != set(cur):
        raise AssertionError("demand partition failed")
    by_load = lambda e: (-cur[e], e)  # noqa: E731
    return dict(
        phase=phase, mode=mode, cpu_balance_target=nc, cpu_balance_formula_target=formula_nc,
        cpu_balance_target_override=cpu_balance_target_override,
        cpu_queue=sorted(cpu_ids, key=by_load),
        gpu_resident_queue=sorted(resident - set(unload), key=by_load),
        on_demand_queue=[j.expert for j in reversed(on_demand)],
        prefetch_queue=[j.expert for j in prefetch], unload_queue=unload,
        placements={e: "gpu" if e in gpu_ids else "cpu" for e in sorted(cur)},
        current_cpu_candidates=[j.expert for j in current], next_cpu_candidates=[j.expert for j in following],
        global_queue=[list(j) for j in global_queue], global_checks=global_checks, local_checks=local_checks,
        boundary=boundary, decode_prefetch_constraints=constraints,
        estimate=dict(cpu_ms=cpu_ms, gpu_ms=gpu_ms, gap_ms=gap, attention_ms=attention_ms, io_ms=tio,
                      io_startup_ms=io_startup_ms, confidence=confidence),
        joint_next=joint_next, record_checks=record_checks,
        scope="PDScope Algorithm 1 placement (joint and local boundaries, decode modes, confidence prefetch); "
              "measured costs supplied by the caller")
