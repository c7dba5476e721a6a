"""A stack of Qwen3-30B-A3B-shaped MoE blocks served through PDScopeCudaRuntime
under a whole-device memory budget.

This is the end-to-end workload of the reference's capped-GPU runs
(benchmarks/pdscope_compare.py: model session and budget :144-179, runtime
per case :259-283, layer hook :285-304, per-case closure and memory checks
:340-389), with the decoder's attention replaced by the identity: block l
computes h = x + moe_l(x) and RMSNorm(h) (weight 1, eps 1e-6) feeds block
l + 1.  Expert weights are seeded random bf16 (no checkpoint is read) and
live as pinned host masters; the device holds a static hot set, speculative
prefetch slots and demand staging slots, all sized so that the process's
device memory stays within the budget:

* the torch allocator is capped below the budget, as the reference does
  (pdscope_compare.py:178-179), by at least 1 GiB and at least the device
  memory already in use outside the allocator plus a margin for its growth;
  the cap is checked at every layer call;
* the expert slots are sized from the allocator cap minus the bytes already
  reserved and a reserve for the layer workspaces;
* at the end of a run the allocator's peak plus the device memory in use
  outside the allocator must fit the budget (pdscope_compare.py:376-385);
* the ledger must close: every submitted copy completed, no open demand,
  every routed expert computed (pdscope_compare.py:355-371).

A violation raises (MemoryError, AssertionError) instead of being reported.
"""
from __future__ import annotations

import time
from collections import Counter
from dataclasses import dataclass, field

import torch

from . import layer as LY
from . import synthetic
from .cache import ExpertKey
from .executor import masters_from_block
from .pdscope_runtime import PDScopeCudaRuntime

GIB = 1 << 30


def rms_residual(out, x, eps=1e-6):
    """Next block's input: attention is the identity, so h = x + moe(x),
    then RMSNorm with weight 1, in fp32, rounded to bf16."""
    h = out.float() + x.float()
    return (h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + eps)).to(torch.bfloat16)


@dataclass
class StackModel:
    """Seeded router gates (on the device), pinned expert masters and the
    static hot profile of every layer."""
    gates: list
    masters: dict
    hot: list
    H: int
    I: int
    E: int
    k: int
    seed0: int
    build_s: float = 0.0

    @property
    def n_layers(self):
        return len(self.gates)

    def expert_block(self, layer, expert):
        """The pinned host master of one expert as its flat bf16 block."""
        return self.masters[ExpertKey(layer, expert, "bf16")].flat


def build_stack(n_layers, device, *, seed0=20261011, hot_per_layer=40, calib_tokens=512, H=2048, I=768, E=128,
                k=8):
    """Layer l is synthetic.make_layer(seed=seed0 + 20000 + 1000 l); its hot
    profile is the hot_per_layer experts a seeded calibration batch routes to
    most (ties to the lower id), in the reference's hot-file order."""
    t0 = time.perf_counter()
    gates, masters, hot = [], {}, []
    calib = synthetic.make_tokens(calib_tokens, H, seed=seed0 + 30001, device=device)
    cws = LY.MoEWorkspace(calib_tokens, H, I, E, k, device, route_only=True)
    for l in range(n_layers):
        lay = synthetic.make_layer(H, I, E, k, True, seed=seed0 + 20000 + 1000 * l, device=device)
        masters.update(masters_from_block(l, lay.experts, E, H, I))
        gates.append(lay.gate)
        _, ids, _ = LY.route(calib, lay.gate, cws)
        cnt = torch.bincount(ids.reshape(-1).long(), minlength=E).cpu().tolist()
        hot += [ExpertKey(l, e, "bf16") for e in sorted(range(E), key=lambda e: (-cnt[e], e))[:hot_per_layer]]
        del lay
    del cws, calib
    torch.cuda.synchronize(device)
    torch.cuda.empty_cache()
    return StackModel(gates, masters, hot, H, I, E, k, seed0, time.perf_counter() - t0)


@dataclass
class LayerCall:
    """What a per-layer observer sees: the block's input, the layer output and
    the runtime's routing and trace row (device tensors, not yet synchronised)."""
    step: int
    layer: int
    x: torch.Tensor
    out: torch.Tensor
    routing: object
    row: dict


@dataclass
class StackBudget:
    """Device-memory budget of a stack session (bytes).

    The reference caps the allocator 1 GiB below the budget, leaving that
    GiB to device memory outside the allocator (pdscope_compare.py:178-179).
    Here that headroom is at least min_headroom and at least the memory
    already in use outside the allocator when the session starts plus
    external_growth (code objects and runtime buffers loaded later);
    the expert slots get what the allocator cap leaves after the bytes
    already reserved and workspace_reserve for the layer workspaces."""
    device_total: int = 24 * GIB
    min_headroom: int = 1 * GIB
    external_growth: int = GIB // 2
    workspace_reserve: int = GIB // 2
    demand_slots: int = 8

    def plan(self, external_now, reserved_now, expert_bytes):
        """(allocator cap, expert slots incl. demand slots) for a device whose
        memory outside the allocator is external_now and whose allocator holds
        reserved_now bytes."""
        cap = self.device_total - max(self.min_headroom, external_now + self.external_growth)
        return cap, max(0, (cap - reserved_now - self.workspace_reserve) // expert_bytes)


@dataclass
class StackSession:
    """One runtime over a StackModel under a StackBudget."""
    model: StackModel
    device: torch.device
    budget: StackBudget = field(default_factory=StackBudget)
    resident_graphs: bool = True
    diagnostics: bool = False

    def __post_init__(self):
        m = self.model
        self.expert_bytes = 3 * m.I * m.H * 2
        total = torch.cuda.get_device_properties(self.device).total_memory
        if self.budget.device_total > total:
            raise ValueError("the device budget exceeds the device")
        torch.cuda.synchronize(self.device)
        torch.cuda.empty_cache()
        free, _ = torch.cuda.mem_get_info(self.device)
        reserved = torch.cuda.memory_reserved(self.device)
        self.external_at_start = max(0, total - free - reserved)
        self.reserved_at_start = reserved
        self.allocator_cap, slots = self.budget.plan(self.external_at_start, reserved, self.expert_bytes)
        self.speculative = slots - self.budget.demand_slots - len(m.hot)
        if self.speculative < 0:
            raise ValueError("hot set and staging slots exceed the device budget")
        # the reference caps the allocator below the device budget
        # (pdscope_compare.py:178-179); restored by close()
        torch.cuda.set_per_process_memory_fraction(self.allocator_cap / total, self.device)
        torch.cuda.reset_peak_memory_stats(self.device)
        t0 = time.perf_counter()
        try:
            self.runtime = PDScopeCudaRuntime(m.masters, hot_keys=m.hot, speculative_slots=self.speculative,
                                              demand_slots=self.budget.demand_slots,
                                              resident_graphs=self.resident_graphs, device=self.device,
                                              diagnostics=self.diagnostics)
        except BaseException:
            torch.cuda.set_per_process_memory_fraction(1.0, self.device)
            raise
        self.setup_s = time.perf_counter() - t0

    def close(self):
        rt = getattr(self, "runtime", None)
        if rt is not None:
            rt.close()
            self.runtime = None
        torch.cuda.synchronize(self.device)
        torch.cuda.empty_cache()
        torch.cuda.set_per_process_memory_fraction(1.0, self.device)

    def _check_allocator(self):
        if torch.cuda.memory_reserved(self.device) > self.allocator_cap:
            raise MemoryError("GPU allocator cap exceeded")

    def run_pass(self, x, step, observe=None):
        """One token position through every block: returns the last block's
        output activation and the trace rows."""
        m, rt = self.model, self.runtime
        rows = []
        for l in range(m.n_layers):
            out, routing, row = rt.forward(x, m.gates[l], layer=l, step=step, request="stack",
                                           next_gate=m.gates[l + 1] if l + 1 < m.n_layers else None, top_k=m.k)
            self._check_allocator()
            if observe is not None:
                observe(LayerCall(step, l, x, out, routing, row))
            rows.append(row)
            x = rms_residual(out, x)
        return x, rows

    def run(self, T_prefill=2048, n_decode=64, observe=None, observe_steps=None):
        """Prefill T_prefill tokens, then n_decode single-token steps.

        observe(LayerCall) runs after every layer of the steps in
        observe_steps (all steps when None).  Returns phase statistics and
        the memory record; raises if the ledger or the budget does not close.
        """
        m, rt, dev = self.model, self.runtime, self.device
        watch = (lambda s: observe) if observe_steps is None else (
            lambda s: observe if s in observe_steps else None)
        x = synthetic.make_tokens(T_prefill, m.H, seed=m.seed0 + 30002, device=dev)
        # the residual block's torch kernels load on their first call: call
        # it once outside the timed passes
        rms_residual(x, x)
        torch.cuda.synchronize(dev)
        st0 = Counter(rt.cache.stats())
        t0 = time.perf_counter()
        _, rows_p = self.run_pass(x, 0, watch(0))
        torch.cuda.synchronize(dev)
        wall_p = time.perf_counter() - t0
        st1 = Counter(rt.cache.stats())
        rows_d = []
        t0 = time.perf_counter()
        for step in range(1, n_decode + 1):
            tok = synthetic.make_tokens(1, m.H, seed=m.seed0 + 30100 + step, device=dev)
            _, rows = self.run_pass(tok, step, watch(step))
            rows_d += rows
        torch.cuda.synchronize(dev)
        wall_d = time.perf_counter() - t0
        st2 = Counter(rt.cache.stats())
        closure = self.check_closure(st0, st2, (T_prefill + n_decode) * m.n_layers * m.k,
                                     len(rows_p) + len(rows_d), (1 + n_decode) * m.n_layers)
        memory = self.check_memory()
        prefill = _phase(rows_p, wall_p, T_prefill, st0, st1)
        decode = _phase(rows_d, wall_d, n_decode, st1, st2)
        pred = {p: dict(v) for p, v in rt.prediction_counts.items()}
        return dict(prefill=prefill, decode=decode, predictor=pred, memory=memory, closure=closure,
                    layers=m.n_layers, tokens_prefill=T_prefill, decode_steps=n_decode, setup_s=self.setup_s)

    def check_closure(self, before, after, expected_tokens, rows, expected_rows):
        """The reference's per-case closure (pdscope_compare.py:355-371)."""
        rt = self.runtime
        rt.poll(wait=True)
        ex = rt.executor
        if rt.pending or rt.transient or ex.loads or ex.computes or rt.cache.active_demand is not None:
            raise AssertionError("the runtime did not drain after the run")
        fresh = Counter(rt.cache.stats())
        fresh.subtract(before)
        if (rows != expected_rows or fresh["physical_demand_tokens"] != expected_tokens
                or fresh["h2d_bytes_completed"] != fresh["h2d_bytes_submitted"]
                or fresh["physical_expert_demands"] != fresh["cpu_completed_experts"] + fresh["gpu_completed_experts"]):
            raise AssertionError("stack work or transfer accounting does not close")
        return dict(layer_calls=rows, physical_demand_tokens=fresh["physical_demand_tokens"],
                    physical_expert_demands=fresh["physical_expert_demands"],
                    gpu_completed_experts=fresh["gpu_completed_experts"],
                    cpu_completed_experts=fresh["cpu_completed_experts"],
                    h2d_bytes_submitted=fresh["h2d_bytes_submitted"],
                    h2d_bytes_completed=fresh["h2d_bytes_completed"])

    def check_memory(self):
        """Peak allocator bytes plus the device bytes in use outside the
        allocator must fit the budget (pdscope_compare.py:376-385).  The
        device's used bytes are taken as this process's (one process per
        device)."""
        dev, b = self.device, self.budget
        free, total = torch.cuda.mem_get_info(dev)
        used = total - free
        reserved = torch.cuda.memory_reserved(dev)
        peak = torch.cuda.max_memory_reserved(dev)
        external = max(0, used - reserved)
        slots = len(self.model.hot) + self.speculative
        rec = dict(device_budget_bytes=b.device_total, allocator_cap_bytes=self.allocator_cap,
                   external_at_start_bytes=self.external_at_start, reserved_at_start_bytes=self.reserved_at_start,
                   cache_slots=slots, hot_slots=len(self.model.hot), speculative_slots=self.speculative,
                   demand_slots=b.demand_slots, expert_slot_bytes=(slots + b.demand_slots) * self.expert_bytes,
                   gpu_peak_allocated_bytes=torch.cuda.max_memory_allocated(dev), gpu_peak_reserved_bytes=peak,
                   gpu_end_used_bytes=used, gpu_end_external_bytes=external,
                   gpu_peak_reserved_plus_end_external_bytes=peak + external,
                   non_slot_peak_reserved_bytes=peak - (slots + b.demand_slots) * self.expert_bytes,
                   pinned_master_bytes=len(self.model.masters) * self.expert_bytes,
                   scope="allocator peak plus device bytes in use beyond the allocator at the end (whole device)")
        if used > b.device_total or peak + external > b.device_total:
            raise MemoryError(f"GPU total or peak estimate exceeds the {b.device_total / GIB:.0f} GiB budget: {rec}")
        return rec


def _phase(rows, wall, tokens, before, after):
    """Phase totals from the ledger counters (a copy that lands between two
    layer calls is completed by the next call's poll, outside any row)."""
    h2d = after.get("h2d_bytes_submitted", 0) - before.get("h2d_bytes_submitted", 0)
    demand = sum(len(r["decision"]["on_demand_queue"]) for r in rows)
    routed = sum(len(r["token_counts"]) for r in rows)
    return dict(tok_s=tokens / wall, wall_s=wall, h2d_bytes=h2d, h2d_gbs=h2d / wall / 1e9,
                routed_experts=routed, demand_misses=demand, resident_hit_rate=1 - demand / max(1, routed),
                prefetch_issued=sum(len(r["prefetch_issued"]) for r in rows),
                **{kk: after.get(kk, 0) - before.get(kk, 0) for kk in
                   ("demand_loads_submitted", "prefetch_loads_submitted", "unused_prefetch_evictions",
                    "fresh_prefetch_hits", "loading_misses", "absent_misses")},
                paths=sorted({r.get("decode_path", "grouped") for r in rows}))
