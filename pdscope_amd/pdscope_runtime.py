"""Per-layer MoE runtime on the gfx950 kernels (drop-in for expertbench/pdscope_runtime.py).

``PDScopeCudaRuntime(masters, *, hot_keys, speculative_slots, ...)`` and
``.forward(inputs, gate, *, layer, step, request, next_gate, top_k, normalize,
attention_ms, prefetch) -> (out, Routing, trace_row)`` keep the reference
signature (pdscope_runtime.py:76-82, :208-209) and return triple
(:492-512); invalid arguments raise ValueError, broken invariants
AssertionError.

One layer call:
 1. route on the GPU (K1); the gate-fallback predictor routes the same
    activation with the next layer's gate and histograms it (K1 + hist);
 2. grouping (K2) on the GPU; one device->host copy of the per-expert counts
    (and the predictor histogram) reveals the true demand to the ledger;
 3. every routed expert with a cache copy runs in ONE grouped launch (K3; K4
    for a fully resident decode token) on the compute stream;
 4. experts without a copy stream through the demand staging slots: copy on
    the load stream, grouped launch over the staged batch when its copy
    events completed, slots released after the compute event (ping-pong as
    pdscope_runtime.py:361 with one expert per launch, or two halves of the
    slot budget from 6 slots on, see _demand_pipeline);
 5. predicted next-layer experts are prefetched into the cache pool
    (speculative_slots bound, LRU eviction, never evicting the static hot set);
 6. the merge (K5) writes the layer output in token order.
With ``resident_graphs=True`` a decode layer is served by its bound
single-launch decode (K1 + K4 in one kernel, ops.DecodeBinding: arguments
checked and planned once per layer, then one C call per token that also
reads the routed ids back into pinned host memory).  On this device that
direct launch costs the host far less than replaying a captured hipGraph of
the same kernel, which is what the reference's per-expert resident graphs
are for.  Its ledger accounting follows the launch (nothing can evict while
the control thread waits).

Placement.  Given a cost table (``costs``, e.g. costs.FileCosts) AND a
``cpu_backend``, each call plans with ``plan_pdscope``
(expertbench/pdscope_policy.py:72-223, restated in policy.py): the CPU queue
runs on the backend (``cpu_backend(key, rows) -> rows`` or its ``submit``),
overlapped with the GPU launches, and its outputs fill their rows of the
grouped output before the merge; resident, demand and prefetch queues follow
the plan, and a decode layer whose plan keeps every routed expert on the GPU
takes the bound launch after routing.  Without either, every expert runs on
the GPU.  There is no built-in CPU expert path.
"""
from __future__ import annotations

import collections
import contextlib
import ctypes
import hashlib
import itertools
import operator
import statistics
import time
from pathlib import Path

import torch

from . import layer as L
from . import ops
from .adapters.qwen import Routing
from .cache import DemandID, ExpertCache, ExpertKey
from .executor import ExpertExecutor
from .policy import plan_pdscope

# the current stream's raw handle without building a Stream object
_raw_current_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)

# how long the host polls a bound launch's read-back word before it blocks on
# an event instead (a decode layer takes tens of microseconds)
_READBACK_POLL_S = 0.002

# bound decode layers kept at once: every layer of a deep stack with a few
# gate / predictor variants each; a caller that passes new gate tensors call
# after call evicts the least recently used binding instead of growing
_MAX_BINDINGS = 512


class _HostWordTagged:
    """Completion test of a bound launch numbered `value`: its read-back
    stored the error word tagged with that number into words[at] after the
    launch completed (query() as an event's)."""
    __slots__ = ("words", "at", "value")

    def __init__(self, words, at):
        self.words, self.at, self.value = words, at, None

    def query(self):
        return self.value is not None and int(self.words[self.at]) >> 16 == self.value


def load_hot_profile(path, masters, slots):
    """The static hot set from a profile file (the hot/qwen.txt format read by
    expertbench/pdscope_runtime.py:62-72): one ``layer,expert`` pair per
    non-blank line.  Returns the first `slots` listed experts that have a
    master, in file order, and a provenance record (path, sha256, entry
    counts).  A malformed or duplicated line, a negative index, a bad
    capacity, or too few listed experts with masters raise ValueError."""
    blob = Path(path).read_bytes()
    if type(slots) is not int or slots < 0:
        raise ValueError("invalid static hot profile or capacity")
    listed, seen = [], set()
    for number, line in enumerate(blob.decode().splitlines(), 1):
        if not line.strip():
            continue
        fields = line.split(",")
        try:
            pair = tuple(int(f) for f in fields)
        except ValueError:
            raise ValueError(f"invalid static hot profile or capacity (line {number}: {line!r})") from None
        if len(pair) != 2 or min(pair) < 0 or pair in seen:
            raise ValueError(f"invalid static hot profile or capacity (line {number}: {line!r})")
        seen.add(pair)
        listed.append(ExpertKey(pair[0], pair[1], "bf16"))
    eligible = [key for key in listed if key in masters]
    if len(eligible) < slots:
        raise ValueError("hot table cannot fill the declared static capacity")
    return eligible[:slots], dict(path=str(Path(path).resolve()), sha256=hashlib.sha256(blob).hexdigest(),
                                  entries=len(listed), eligible_entries=len(eligible), selected=slots)


class PDScopeCudaRuntime:
    def __init__(self, masters, *, hot_keys, speculative_slots, costs=None, cpu_backend=None, device=0,
                 streams=None, capture_events=False, diagnostics=True, cache_storage=None, staging_storage=None,
                 source_mode="all_masters", resident_graphs=False, graph_cost_mode="eager_bound", cpu_batch="off",
                 balance_profile=False, dispatch="reference", decode_cpu_target=None, merge="reference",
                 input_pregather=False, graph_output_pool=False, demand_slots=2, native_dispatch=None):
        if (type(speculative_slots) is not int or speculative_slots < 0
                or len(set(hot_keys)) != len(hot_keys) or not set(hot_keys) <= masters.keys()):
            raise ValueError("invalid PDScope cache contract")
        sizes = {k: w.nbytes for k, w in masters.items()}
        if len(set(sizes.values())) != 1:
            raise ValueError("equal-size original BF16 experts required")
        if cpu_batch not in ("off", "decode", "both") or dispatch not in ("reference", "compact"):
            raise ValueError("invalid CPU packing or dispatch mode")
        if merge not in ("reference", "fused") or type(input_pregather) is not bool:
            raise ValueError("invalid merge mode or pre-gather switch")
        if type(graph_output_pool) is not bool or type(resident_graphs) is not bool:
            raise ValueError("graph switches must be boolean")
        if graph_cost_mode not in ("eager_bound", "measured"):
            raise ValueError("invalid resident graph cost mode")
        if native_dispatch is not None and not all(
                callable(getattr(native_dispatch, f, None)) for f in ("submit_group", "finish_and_merge")):
            raise ValueError("native dispatch must provide submit_group and finish_and_merge")
        # the reference allows 2..4 staging slots (pdscope_runtime.py:108-109); this
        # path also serves configurations with 8
        if type(demand_slots) is not int or not 2 <= demand_slots <= 8:
            raise ValueError("invalid demand staging depth")
        if decode_cpu_target is not None and (type(decode_cpu_target) is not int or not 0 <= decode_cpu_target <= 8):
            raise ValueError("invalid decode CPU balance target")
        self.size = next(iter(sizes.values()))
        self.hot = set(hot_keys)
        self._hot_by_layer = {}
        for hk in hot_keys:
            self._hot_by_layer.setdefault(hk.layer, []).append(hk)
        self.layers = {k.layer for k in masters}
        any_w = next(iter(masters.values()))
        self.I, self.H = any_w.tensors["gate_proj"].shape
        self.E = 1 + max(k.expert for k in masters)
        self.speculative_slots = speculative_slots
        self.costs, self.cpu_backend, self.native_dispatch = costs, cpu_backend, native_dispatch
        self.demand_slots, self.diagnostics = demand_slots, diagnostics
        self.merge, self.dispatch, self.cpu_batch = merge, dispatch, cpu_batch
        self.input_pregather, self.graph_output_pool = input_pregather, graph_output_pool
        self.graph_cost_mode, self.graph_cost_calibration = graph_cost_mode, None
        self.balance_profile, self.decode_cpu_target = balance_profile, decode_cpu_target
        self.resident_graphs = resident_graphs
        self.cache = ExpertCache(sizes, (len(hot_keys) + speculative_slots) * self.size, [self.size] * demand_slots,
                                 policy="LRU", initial_hotset=hot_keys)
        self.executor = ExpertExecutor(self.cache, masters, device, pinned_source_mode=source_mode,
                                       cpu_backend=cpu_backend, streams=streams, capture_events=capture_events,
                                       cache_storage=cache_storage, staging_storage=staging_storage)
        self.device = self.executor.device
        self.pending = {}
        self.transient = set()
        # the masters' own key objects: the ledger's tables are keyed by them,
        # so lookups with these hit on identity
        self._keys = {}
        for mk in masters:
            if mk.representation == "bf16":
                self._keys.setdefault(mk.layer, [None] * self.E)[mk.expert] = mk
        self.forecasts = {}
        self.prediction_counts = {p: dict(hits=0, total=0) for p in ("prefill", "decode")}
        self._ws = {}
        self._pws = {}
        # bound decode launches, by (layer, k, normalize, gate, next gate),
        # least recently used first (a binding keeps its tensors alive)
        self._bindings = collections.OrderedDict()
        self.bound_launches = 0  # tokens served through them (the reference counts its graph replays)
        self._out_ring = {}     # graph_output_pool: two output buffers per layer
        self._graph_turn = {}
        self._dispatch_buffers = {}
        self._pinned_counts = torch.zeros(2 * self.E + 64, dtype=torch.int32, pin_memory=True)
        self._pinned_np = self._pinned_counts.numpy()   # host reads without tensor indexing
        self._streams = {}   # raw hipStream_t -> its torch Stream object
        self._err_at = 2 * self.E + 8    # the decode error word's place in _pinned_counts
        self._seq = 0                    # number of the last bound launch (1 .. 32767, the read-back tag)
        self._readback = _HostWordTagged(self._pinned_np, self._err_at)
        self._decode_ok = {}             # k -> (single launch fits, with the fused predictor)
        self._out_stash = None           # (raw stream, k, outputs) of the next bound decode call
        self._keys_full = set()          # layers whose key list holds every expert
        self._copy_done = torch.cuda.Event()
        self._layer_done = torch.cuda.Event()    # end of a prelaunched prefill layer
        try:
            for key in hot_keys:
                self.executor.finish_load(self.executor.load(key, origin="initial"), wait=True)
            self.initial_stats = self.cache.stats()
            if resident_graphs and costs is not None and hot_keys:
                self._calibrate_graph_costs(hot_keys)
        except BaseException:
            self.close()
            raise

    # ------------------------------------------------------------ helpers

    def _workspace(self, T, k):
        ws = self._ws.get(k)
        if ws is None or ws.max_tokens < T:
            cap = max(T, 1 if ws is None else 2 * ws.max_tokens)
            ws = L.MoEWorkspace(cap, self.H, self.I, self.E, k, self.device)
            self._ws[k] = ws
        return ws

    def _pred_workspace(self, T, k):
        ws = self._pws.get(k)
        if ws is None or ws.max_tokens < T:
            cap = max(T, 1 if ws is None else 2 * ws.max_tokens)
            ws = L.MoEWorkspace(cap, self.H, self.I, self.E, k, self.device, route_only=True)
            self._pws[k] = ws
        return ws

    def _key(self, layer, e):
        # one key object per expert, built once (a key is an immutable record)
        keys = self._keys.get(layer)
        if keys is None:
            keys = self._keys[layer] = [None] * self.E
        if not 0 <= e < self.E:
            return ExpertKey(layer, e, "bf16")
        k = keys[e]
        if k is None:
            k = keys[e] = ExpertKey(layer, e, "bf16")
        return k

    def poll(self, wait=False):
        for key, ticket in list(self.pending.items()):
            if self.executor.finish_load(ticket, wait=wait):
                del self.pending[key]

    def _retire_current(self, layer, *, wait):
        if not self.transient:   # no speculative copy to retire
            self.executor.reclaim()
            return
        unfinished = set(self.cache.unfinished_demand_keys)
        for key in list(self.transient):
            if key.layer != layer or key in unfinished:
                continue
            if key in self.pending:
                if not self.executor.finish_load(self.pending[key], wait=wait):
                    continue
                del self.pending[key]
            view = self.cache.lookup(key)
            if view is not None and view.state == "ready" and view.pool == "cache":
                self.cache.evict(key)
            self.transient.discard(key)
        self.executor.reclaim()

    def _current_stream(self):
        """The current stream of the runtime's device, one torch Stream object
        per raw stream (built on first sight instead of once per call)."""
        raw = _raw_current_stream(self.device.index) if _raw_current_stream is not None else None
        s = self._streams.get(raw) if raw is not None else None
        if s is None:
            s = torch.cuda.current_stream(self.device)
            if raw is not None:
                self._streams[raw] = s
        return s

    def _layer_keys(self, layer):
        """The key objects of `layer`'s experts 0..E-1, as a list."""
        if layer not in self._keys_full:
            for e in range(self.E):
                self._key(layer, e)   # fills self._keys[layer]
            self._keys_full.add(layer)
        return self._keys[layer]

    def _decode_support(self, k):
        """(the single-launch decode fits k, and also with the fused next-layer predictor)."""
        got = self._decode_ok.get(k)
        if got is None:
            fits = ops.decode_layer_supported(self.H, self.I, self.E, k, self.device)
            got = (fits, fits and ops.decode_chained_supported(self.H, self.I, self.E, k, self.device))
            self._decode_ok[k] = got
        return got

    def _new_decode_outputs(self, k):
        """Fresh (out [1,H], logits [1,E], weights [1,k] bf16, selected [1,k]
        int64) for one bound decode call, on the current stream."""
        dev, bf16 = self.device, torch.bfloat16
        return (torch.empty((1, self.H), dtype=bf16, device=dev), torch.empty((1, self.E), dtype=bf16, device=dev),
                torch.empty((1, k), dtype=bf16, device=dev), torch.empty((1, k), dtype=torch.int64, device=dev))

    def _decode_outputs(self, stream, k):
        """The output tensors of this bound decode call: the ones allocated
        during the previous call's wait when they were allocated on this
        stream for this k (the caching allocator ties a block to the stream
        it was allocated on), else fresh ones.  Each set is handed out once."""
        st, self._out_stash = self._out_stash, None
        if st is not None and st[0] == stream.cuda_stream and st[1] == k:
            return st[2]
        return self._new_decode_outputs(k)

    def _tagged_or_raise(self, at, n, seq):
        """Values of the n read-back words at `at` stored by the bound launch
        numbered seq; the launch is known to have completed, so each word must
        carry seq."""
        vals = ops.DecodeBinding.tagged_words(self._pinned_np[at:at + n].tolist(), seq)
        if vals is None:
            raise RuntimeError("a bound decode launch completed without its read-back words")
        return vals

    def _await_tagged(self, at, n, seq, stream):
        """Values of the n read-back words at `at` once each carries seq: the
        bound launch numbered seq stores them (the routed ids before it
        completes, the error word after).  Polls; after _READBACK_POLL_S it
        blocks on an event recorded on `stream` instead."""
        words, last = self._pinned_np, at + n - 1
        deadline = None
        while True:
            if int(words[last]) >> 16 == seq:
                vals = ops.DecodeBinding.tagged_words(words[at:at + n].tolist(), seq)
                if vals is not None:
                    return vals
            now = time.perf_counter()
            if deadline is None:
                deadline = now + _READBACK_POLL_S
            elif now > deadline:
                self._copy_done.record(stream)
                self._copy_done.synchronize()
                return self._tagged_or_raise(at, n, seq)

    def _next_counts(self, predict, pred_ids, n0, k, E, seq):
        """The next-layer forecast {expert: predicted tokens}: the fused
        prediction's k tagged words (seq) of a bound launch, else the
        predictor histogram copied into the read-back buffer."""
        if not predict:
            return {}
        if pred_ids is None:
            return {e: c for e, c in enumerate(self._pinned_np[n0:n0 + E].tolist()) if c}
        # one token: each predicted expert once
        vals = self._tagged_or_raise(n0, k, seq if seq is not None else self._seq)
        next_counts = {e: 1 for e in vals}
        if len(next_counts) != k:
            raise AssertionError("decode prediction selected duplicate experts")
        if min(next_counts) < 0 or max(next_counts) >= E:
            raise AssertionError("decode prediction selected an expert id outside [0, E)")
        return next_counts

    def _layer_fully_resident(self, layer):
        ready = self.cache.ready_in_cache
        return all(ready(self._key(layer, e)) for e in range(self.E))

    # ------------------------------------------------------------ forward

    def forward(self, inputs, gate, *, layer, step, request="pdscope", next_gate=None, top_k=8, normalize=True,
                attention_ms=0., prefetch=True, bias=None):
        if (inputs.ndim != 2 or (step > 0 and inputs.shape[0] != 1) or (step == 0 and inputs.shape[0] < 2)
                or layer not in self.layers):
            raise ValueError("invalid prefill/decode activation or layer")
        if inputs.device != self.device or inputs.dtype != torch.bfloat16 or inputs.shape[1] != self.H:
            raise ValueError("inputs must be bf16 [T, H] on the runtime device")
        if gate.shape != (self.E, self.H):
            raise ValueError("gate must be [E, H]")
        phase = "prefill" if step == 0 else "decode"
        started = time.perf_counter()
        T, H = inputs.shape
        E, k = self.E, top_k
        x = inputs.contiguous()
        ws = self._workspace(T, k)
        cur = self._current_stream()
        key = self._layer_keys(layer).__getitem__   # routed ids are range-checked below
        nkey = (self._layer_keys(layer + 1).__getitem__ if (layer + 1) in self.layers
                else lambda e: self._key(layer + 1, e))  # noqa: E731
        self.poll()
        before = self.cache.stats()
        # decode runs the bound single-launch layer over the slot table
        # (experts without a device copy have a null entry and contribute 0);
        # misses, at most k <= demand_slots of them, are staged in one batch
        # and the same launch runs once more over the completed table
        # (with fewer slots than k only a fully resident layer takes it)
        planned = self.costs is not None and self.cpu_backend is not None
        fits, fits_pred = self._decode_support(k)
        graph_ok = (self.resident_graphs and phase == "decode" and bias is None and fits
                    and (k <= self.demand_slots or self._layer_fully_resident(layer)))
        # unplanned: the first launch also routes; planned: routing comes
        # first, and the bound launch serves the layer when the plan keeps
        # every routed expert on the GPU (decided below)
        graph_path = graph_ok and not planned
        # a prefill layer whose every expert has a ready device copy is
        # launched whole before its counts come back, and its demand is
        # revealed while it runs (nothing evicts between the launch and the
        # reveal: no ledger call comes in between)
        prelaunch = T > 1 and not planned and not self.input_pregather and self.executor.table_full(layer, E)
        ring_out = None
        if graph_ok and self.graph_output_pool:
            ring = self._graph_turn.get(layer, 0)
            self._graph_turn[layer] = ring ^ 1
            ring_out = self._ring_output(layer, ring)
        launch_table, late_replays = None, 0

        # ---- 1-2: route (+ predictor), grouping, one D2H of the demand
        if graph_ok:
            # the bound launch writes the output and the routing straight into
            # the tensors the call returns (allocated during the previous
            # call's wait where it ran on this stream)
            d_out, r_logits, r_weights, r_selected = self._decode_outputs(cur, k)
        else:
            d_out = torch.empty((T, H), dtype=torch.bfloat16, device=self.device)
        out = ring_out if graph_path and ring_out is not None else d_out
        predict = prefetch and next_gate is not None
        # the bound launch also predicts the next layer where its grid allows
        graph_pred = next_gate if (graph_path and predict and fits_pred) else None
        pred_ids = None
        bound_routing = graph_path
        if graph_path:
            # the table version the first launch saw (a copy still in flight
            # reads as null; a copy that lands moves the version on)
            launch_table = self.executor.table_version(layer)
            binding, seq = self._bound_decode(layer, x, gate, normalize, k, out, r_logits, r_weights, r_selected,
                                              next_gate=graph_pred, stream=cur)
            logits, ids, weights = r_logits, r_selected, r_weights
            pred_ids = binding.pred if graph_pred is not None else None
            # the next call's outputs, allocated while this launch runs
            self._out_stash = (cur.cuda_stream, k, self._new_decode_outputs(k))
        else:
            logits, ids, weights = L.route(x, gate, ws, normalize=normalize, bias=bias)
        nws = None
        pred_sel = pred_ids.view(1, k) if pred_ids is not None else None
        if predict and pred_ids is None:
            nws = self._pred_workspace(T, k)
            _, pred_sel, _ = L.route(x, next_gate, nws, normalize=normalize)
            ops.route_hist(pred_sel, E, out=nws.hist)
        if graph_path:
            packed, n0 = None, k   # the bound launch needs no grouping
        else:
            _, _, _, packed = ws.views(T)
            if prelaunch:
                pre_bm = self._pack_scheduled(ids, packed, ws)
                counts_dev = packed.counts
            elif T > 1:
                ops.pack(ids, E, out=packed, workspace=ws.pack_ws)
                counts_dev = packed.counts
            else:
                counts_dev = ids.reshape(-1)
            n0 = counts_dev.numel()
        host, hn = self._pinned_counts, self._pinned_np
        err_at = self._err_at
        if graph_path:
            # the bound launch stores the routed ids, its prediction and the
            # fused kernel's sticky error word into `host` itself (tagged seq)
            if pred_ids is None and predict:
                host[n0:n0 + E].copy_(nws.hist, non_blocking=True)
        else:
            host[:n0].copy_(counts_dev, non_blocking=True)
            if predict:
                host[n0:n0 + E].copy_(nws.hist, non_blocking=True)
        # with nothing else to read back, the bound launch's routed ids are
        # taken as soon as the kernel stored them, and the demand is revealed
        # while the kernel still runs; its completion is awaited after that
        early = graph_path and not (predict and pred_ids is None)
        completed = self._copy_done
        decode_failed = False
        if early:
            sel = self._await_tagged(0, k, seq, cur)
        else:
            self._copy_done.record(cur)
            if prelaunch:
                self._launch_resident_layer(x, packed, weights, out, ws, layer, pre_bm, cur)
            self._copy_done.synchronize()
            if graph_path:
                sel = self._tagged_or_raise(0, k, seq)
                decode_failed = self._tagged_or_raise(err_at, 1, seq)[0] != 0
            elif T == 1:
                sel = hn[:k].tolist()
        if T > 1:
            counts = {e: c for e, c in enumerate(hn[:E].tolist()) if c}
        else:
            if len(set(sel)) != k:
                raise AssertionError("decode routing selected duplicate experts")
            if min(sel) < 0 or max(sel) >= E:
                raise AssertionError("decode routing selected an expert id outside [0, E)")
            counts = {e: 1 for e in sel}
        if not early:
            next_counts = self._next_counts(predict, pred_ids, n0, k, E, None)
        if sum(counts.values()) != T * k:
            raise AssertionError("lost or duplicated routed assignment")

        identity = DemandID(request, step, layer)
        observations = self.cache.on_demand(identity, {key(e): n for e, n in counts.items()})
        prior = self.forecasts.pop((request, step, layer), None)
        if prior:
            self.prediction_counts[phase]["hits"] += len(set(prior) & set(counts))
            self.prediction_counts[phase]["total"] += len(prior)
        observed = dict(self.prediction_counts[phase])
        if early:
            # the launch has completed once its error word carries seq; a set
            # word fails the call after the ledger has closed its demand
            decode_failed = self._await_tagged(err_at, 1, seq, cur)[0] != 0
            completed = self._readback
            self._readback.value = seq
            next_counts = self._next_counts(predict, pred_ids, n0, k, E, seq)

        # ---- plan: with a cost table and a CPU backend, plan_pdscope splits the
        # experts between the CPU backend, resident copies and demand staging
        # and picks the prefetch (pdscope_runtime.py:268-279); else every
        # expert runs on the GPU, resident first, misses through staging
        # (state, ticket) of each routed expert's copy, or None (no views built)
        has_next = predict and (layer + 1) in self.layers
        views = None
        if not planned and all(o[4] == "ready" for o in observations):
            # every routed copy was ready at the reveal (the observations come
            # in expert order): all resident, none loading, no demand
            decision = None
            cpu_list, demand = [], []
            resident = ([o[0].expert for o in observations] if T == 1
                        else sorted(counts, key=lambda e: (-counts[e], e)))
        elif planned:
            views = {e: self.cache.residency(key(e)) for e in counts}
            hit_rate = observed["hits"] / observed["total"] if observed["total"] else 0.0
            next_resident = [e for e in next_counts if self.cache.residency(nkey(e)) is not None] if has_next else []
            decision = plan_pdscope(counts, next_counts if has_next else {}, current_layer=layer, phase=phase,
                                    current_gpu_ids=[e for e in counts if views[e] is not None],
                                    next_gpu_ids=next_resident, costs=self.costs, attention_ms=attention_ms,
                                    hit_rate=hit_rate, prefetch_slots=self.speculative_slots, top_k=k,
                                    cpu_balance_target_override=self.decode_cpu_target if phase == "decode" else None,
                                    record_checks=False, trusted=True,
                                    compute_formula_target=self.decode_cpu_target is None,
                                    num_experts=E, num_layers=max(self.layers) + 1)
            cpu_list = list(decision["cpu_queue"])
            resident = list(decision["gpu_resident_queue"])
            demand = list(decision["on_demand_queue"])
            if graph_ok and not cpu_list:
                graph_path = True  # launched below over the (completed) slot table
                if ring_out is not None:
                    out = ring_out
        else:
            views = {e: self.cache.residency(key(e)) for e in counts}
            decision = None
            cpu_list = []
            resident = sorted((e for e in counts if views[e] is not None), key=lambda e: (-counts[e], e))
            demand = sorted((e for e in counts if views[e] is None), key=lambda e: (-counts[e], e))
        for e in (resident if views is not None else ()):
            if views[e][0] == "loading":
                self.executor.finish_load(views[e][1], wait=True)
                self.pending.pop(key(e), None)

        ex = self.executor
        # first demand copies go out before the resident launch is prepared
        batches, inflight, nxt = [], [], 0
        if demand:
            group, held = (len(demand), 1) if graph_path else self._demand_pipeline(phase)
            batches = [demand[i:i + group] for i in range(0, len(demand), group)]
            while nxt < min(held, len(batches)):
                inflight.append([ex.load(key(e), admit=False) for e in batches[nxt]])
                nxt += 1
        slots_dev = None
        tasks = []

        def require_copies(experts):
            missing = [e for e in experts if ex.table_entry(layer, e) == 0]
            if missing:
                raise AssertionError(f"experts {missing} of layer {layer} have no ready device copy")
        decode_fast = (T == 1 and not demand and not cpu_list and not graph_path)
        if T == 1 and (demand or cpu_list) and not graph_path:
            ops.pack(ids, E, out=packed, workspace=ws.pack_ws)  # decode misses take the grouped path
        # grouped launches read the activation rows through perm_token; with
        # input_pregather the rows are first gathered into grouped order by
        # one gather launch and the grouped kernels read them in order
        x_src, perm_src = x, None
        if self.input_pregather and T > 1 and not graph_path:
            n = T * k
            x_src, perm_src = ws.pregathered(n), ws.identity_rows(n)
            with torch.cuda.stream(ex.compute_stream):
                ex.compute_stream.wait_stream(cur)
                torch.index_select(x, 0, packed.perm_token, out=x_src)
        # ---- CPU experts start before the GPU launches (pdscope_runtime.py:284-336):
        # a decode group through the native dispatch module (merge='fused'),
        # else per expert, or packed into one backend submission (cpu_batch);
        # each expert gets its routed rows in grouped order, and its output
        # later fills the same rows of the grouped output
        cpu_tasks, cpu_group, native_cpu = {}, None, None
        packed_cpu = self.cpu_batch == "both" or (self.cpu_batch == "decode" and phase == "decode")
        if (cpu_list and self.native_dispatch is not None and self.merge == "fused" and phase == "decode"):
            handles = self.cpu_backend.native_group_handles(layer) if callable(
                getattr(self.cpu_backend, "native_group_handles", None)) else None
            if handles is not None:
                native_cpu = sorted(cpu_list)
                pool, layer_obj = handles
                dws = self._dispatch_workspace(len(native_cpu), H)
                row = x.cpu().contiguous()
                self.native_dispatch.submit_group(
                    pool, layer_obj, row.data_ptr(), len(native_cpu), H * 2, dws["packed"].data_ptr(),
                    dws["block"].data_ptr(), ctypes.addressof(dws["count"]), ctypes.addressof(dws["selected"]),
                    ctypes.addressof(dws["coeff"]), list(native_cpu))
                del handles, pool, layer_obj, row
        late_cpu = [] if native_cpu is not None else cpu_list
        if late_cpu:
            x_host = x.cpu()
            if T > 1:
                offs = packed.offsets.cpu().tolist()
                perm = packed.perm_token.cpu()
            jobs = {e: (x_host if T == 1 else x_host.index_select(0, perm[offs[e]:offs[e + 1]].long())).contiguous()
                    for e in late_cpu}
            if packed_cpu:
                cpu_group = ex.submit_cpu_many({key(e): r for e, r in jobs.items()})
            else:
                for e, r in jobs.items():
                    cpu_tasks[e] = ex.submit_cpu(key(e), r)
        if graph_path:
            if not demand:  # with misses the demand batch below launches over the completed table
                table = self.executor.table(layer, E)[1]
                if (launch_table is None or launch_table != self.executor.table_version(layer)
                        or any(table[e] == 0 for e in counts)):
                    # not launched yet (planned path), or a routed copy landed
                    # after the first launch: launch over the completed table
                    late_replays += 1

                    def launch():
                        self._bound_decode(layer, x, gate, normalize, k, out, r_logits, r_weights, r_selected,
                                           next_gate=graph_pred)
                else:
                    # the launch on `cur` already produced `out` (the host waited
                    # for it through _copy_done): account the uses it made
                    launch = None
                tasks.append(ex.gpu_group([key(e) for e in resident], launch, input_ref=x, wait_for=cur,
                                          completed=completed))
        elif resident and prelaunch:
            # the whole layer runs on `cur` since before the reveal: hold its
            # copies from now on, while it still runs; finishing waits for it
            tasks.append(ex.gpu_group([key(e) for e in resident], None, input_ref=x, wait_for=cur,
                                      running=self._layer_done))
        elif resident:
            ex.table(layer, E)
            require_copies(resident if not decode_fast else sorted(counts))
            slots_dev = ex.upload_table(layer, E, ex.compute_stream)
            if decode_fast:
                def launch():
                    ops.swiglu_decode(x, ids, weights, slots_dev, H, self.I, ws.h_ws, out, merge=self.merge)
            else:
                sel_dev = ex.upload_ints(resident, ex.compute_stream)

                def launch():
                    self._grouped(x_src, packed, sel_dev, [counts[e] for e in resident], slots_dev, ws, perm_src)
            tasks.append(ex.gpu_group([key(e) for e in resident], launch, input_ref=x, wait_for=cur))

        # ---- demand misses through the staging slots
        ping_pong = []
        if demand:
            for batch in batches:
                tickets = inflight.pop(0)
                for ticket in tickets:
                    ex.finish_load(ticket, wait=True)
                ex.table(layer, E)
                require_copies(batch)
                if graph_path:
                    late_replays += 1

                    def launch():
                        self._bound_decode(layer, x, gate, normalize, k, out, r_logits, r_weights, r_selected,
                                           next_gate=graph_pred)
                    comp = ex.gpu_group([key(e) for e in resident + batch], launch, input_ref=x, wait_for=cur)
                else:
                    tab = ex.upload_table(layer, E, ex.compute_stream)
                    sel_dev = ex.upload_ints(batch, ex.compute_stream)

                    def launch(sel_dev=sel_dev, tab=tab, rows=[counts[e] for e in batch]):
                        self._grouped(x_src, packed, sel_dev, rows, tab, ws, perm_src)
                    comp = ex.gpu_group([key(e) for e in batch], launch, input_ref=x, wait_for=cur)
                ping_pong += [dict(expert=e, slot=t.slot, generation=t.generation) for e, t in zip(batch, tickets)]
                live = [t.slot for b in inflight for t in b]
                if len(set(live)) != len(live) or set(live) & {t.slot for t in tickets}:
                    raise AssertionError("an in-flight copy reuses a live consumer slot")
                ex.finish_gpu(comp, wait=True)
                if nxt < len(batches):
                    inflight.append([ex.load(key(e), admit=False) for e in batches[nxt]])
                    nxt += 1

        # ---- retire this layer's speculation, prefetch the next layer's forecast
        self._retire_current(layer, wait=True)
        issued, skipped = [], []
        if has_next and not planned and ex.table_full(layer + 1, E):
            pass   # every forecast expert already has a ready copy: nothing to prefetch
        elif has_next:
            forecast = (list(decision["prefetch_queue"]) if planned
                        else sorted(next_counts) if pred_ids is not None   # one token: every count is 1
                        else sorted(next_counts, key=lambda e: (-next_counts[e], e)))
            for e in forecast:
                target = nkey(e)
                if self.cache.residency(target) is not None:
                    continue
                if len(self.transient) >= self.speculative_slots:
                    skipped.append(e)
                    continue
                try:
                    ticket = ex.load(target, origin="prefetch")
                except Exception as err:  # CapacityBlocked: no evictable bytes
                    if type(err).__name__ != "CapacityBlocked":
                        raise
                    skipped.append(e)
                    continue
                self.pending[target] = ticket
                self.transient.add(target)
                issued.append(e)
            if issued:
                self.forecasts[(request, step, layer + 1)] = tuple(issued)

        # ---- finish GPU work, place the CPU experts' rows, merge in token order
        for task in tasks:
            ex.finish_gpu(task, wait=True)
        cpu_rows = dict((e, ex.finish_cpu(p, wait=True)) for e, p in cpu_tasks.items())
        if cpu_group is not None:
            cpu_rows.update(ex.finish_cpu_group(cpu_group.values()))
        add_in = None
        if cpu_rows or native_cpu:
            offs = packed.offsets.cpu().tolist() if T == 1 else offs
        # a layer served by its bound launch or prelaunched, with no CPU rows, has nothing
        # left to enqueue here (its merge ran with the launch)
        finish_ctx = (contextlib.nullcontext() if (graph_path or prelaunch) and not cpu_rows and not native_cpu
                      else torch.cuda.stream(ex.compute_stream))
        with finish_ctx:
            for e, rows in cpu_rows.items():
                ws.y[offs[e] * H:offs[e + 1] * H].view(-1, H).copy_(rows)
            if native_cpu:
                # join the native queue, stage its block and add it (bf16 index_add)
                # into a zero output; the GPU rows are then merged on top of it
                # and the CPU experts' own rows contribute nothing there
                # (pdscope_runtime.py:407-426, then the fused merge :455-464)
                sel_host = ids.reshape(-1).tolist()
                slot_idx = torch.tensor([sel_host.index(e) for e in native_cpu], dtype=torch.long,
                                        device=self.device)
                w_cpu = weights.reshape(-1).index_select(0, slot_idx)
                dws = self._dispatch_workspace(len(native_cpu), H)
                handles = self.cpu_backend.native_group_handles(layer)
                if handles is None:
                    raise AssertionError("native CPU group lost its handles")
                add_in = torch.zeros((1, H), dtype=torch.bfloat16, device=self.device)
                add_in = self.native_dispatch.finish_and_merge(handles[0], dws["block"].data_ptr(), len(native_cpu),
                                                               H * 2, dws["scratch"], add_in, dws["tokens"], w_cpu)
                del handles
                for e in native_cpu:
                    ws.y[offs[e] * H:offs[e + 1] * H].zero_()
            if not (decode_fast or graph_path or prelaunch):
                ops.merge(ws.y, packed.row_of, weights, out, add_in=add_in, mode=self.merge)
        if native_cpu:
            for e in native_cpu:
                self.cache.finish_cpu(key(e))
            note = getattr(self.cpu_backend, "note_native_dispatch", None)
            if note is not None:
                note(len(native_cpu))
        if not ((graph_path and not late_replays) or prelaunch):
            # (a launch served before the reveal enqueued nothing on the compute stream)
            done = torch.cuda.Event()
            done.record(ex.compute_stream)
            cur.wait_event(done)
        if graph_path and late_replays:
            # launches after the demand reveal wrote their error word into
            # `host` themselves: read it once they completed
            self._copy_done.record(cur)
            self._copy_done.synchronize()
            decode_failed |= self._tagged_or_raise(err_at, 1, self._seq)[0] != 0
        self.cache.end_demand(identity)
        self._retire_current(layer, wait=True)
        self.poll()
        if decode_failed:
            self._raise_if_decode_gave_up(True)
        # the ledger never chooses a static copy as a victim; checking the
        # layer just served keeps the guard without a scan of every layer
        if self.diagnostics and any(self.cache.lookup(h) is None for h in self._hot_by_layer.get(layer, ())):
            raise AssertionError("speculation evicted a charged static hot copy")
        after = self.cache.stats()
        delta = dict(zip(after, map(operator.sub, after.values(), map(before.get, after, itertools.repeat(0)))))
        if delta.get("cpu_completed_experts", 0) + delta.get("gpu_completed_experts", 0) != len(counts):
            raise AssertionError("lost or duplicated routed expert")
        # the bound launch wrote fresh tensors; the other paths' routing lives
        # in reused workspaces
        routing = (Routing(logits, ids, weights) if bound_routing
                   else Routing(logits.clone(), ids.long(), weights.clone()))
        if decision is None:
            decision = dict(phase=phase, mode="gpu_all", cpu_queue=[], gpu_resident_queue=resident,
                            on_demand_queue=demand, prefetch_queue=issued, unload_queue=[],
                            placements={e: "gpu" for e in sorted(counts)})
        cpu_tokens = sum(counts[e] for e in cpu_list)
        balance = (dict(cpu_experts=len(cpu_list), gpu_experts=len(counts) - len(cpu_list),
                        cpu_token_assignments=cpu_tokens, gpu_token_assignments=sum(counts.values()) - cpu_tokens,
                        host_ms=dict(layer_host_ms=(time.perf_counter() - started) * 1e3),
                        timing_scope="host wall time of the layer call, completion waits included")
                   if self.balance_profile else None)
        digest = lambda t: hashlib.sha256(t.detach().cpu().contiguous().numpy().tobytes()).hexdigest()  # noqa: E731
        row = dict(phase=phase, step=step, layer=layer, token_counts=counts, balance=balance,
                   cpu_packing=bool(packed_cpu and cpu_list), cpu_batched_io=bool(packed_cpu and cpu_list),
                   dispatch=self.dispatch,
                   decode_submission=("native_group" if native_cpu else "single_launch"
                                      if phase == "decode" and (decode_fast or graph_path) else "grouped_launch"),
                   decision=decision, prefetch_issued=issued, prefetch_capacity_skipped=skipped,
                   next_prediction_counts=next_counts, causal_hit_counts=observed,
                   predictor="next_layer_gate_on_current_activation",
                   scheduler="cross_layer" if planned else "gpu_all", predictor_prior_hit_rate=0.0,
                   selected_sha256=digest(routing.selected) if self.diagnostics else None,
                   next_selected_sha256=digest(pred_sel.long()) if self.diagnostics and predict else None,
                   ready_at_reveal=sum(o[6] is not None for o in observations),    # hit_source: a ready hit
                   loading_at_reveal=sum(o[4] == "loading" for o in observations),  # state_at_reveal
                   counters=delta, ping_pong_slots=ping_pong,
                   static_retention="CPU placement keeps the charged device copy of a static hot expert",
                   merge_mode=self.merge, input_pregather=self.input_pregather, demand_slots=self.demand_slots,
                   graph_output_pool=self.graph_output_pool,
                   pipeline="CPU queue on the backend beside the GPU launches; demand copies in staging-slot "
                            "batches before next-layer speculation",
                   decode_path=("bound_launch" if graph_path else "fused_gemv" if decode_fast else "grouped")
                   if phase == "decode" else "prelaunched" if prelaunch else "grouped",
                   measured_performance=False)
        return out, routing, row

    def _calibrate_graph_costs(self, hot_keys, reps=48, warm=16):
        """Cost of the bound resident decode launch for the planner
        (pdscope_runtime.py:143-175 calibrates its per-expert graphs the same
        way): the bound launch of the first hot layer, routed by a calibration
        gate onto k of its resident experts, runs `reps` times; the median
        over the last reps-warm, divided by k, is one expert's resident-launch
        cost.  'measured' charges it to one-row GPU work in the cost table,
        'eager_bound' keeps the table's eager cost (the cost model of the
        reference's ResidentGraphCosts)."""
        from .costs import ResidentGraphCosts
        layer = min(k.layer for k in hot_keys)
        resident = sorted(k.expert for k in hot_keys if k.layer == layer)
        kk = min(8, len(resident))
        if kk < 1 or not ops.decode_layer_supported(self.H, self.I, self.E, kk, self.device):
            return
        x = torch.linspace(-.5, .5, self.H, device=self.device).to(torch.bfloat16).reshape(1, -1)
        gate = torch.zeros((self.E, self.H), dtype=torch.bfloat16, device=self.device)
        for j, e in enumerate(resident[:kk]):
            gate[e] = (x[0].float() * (0.01 * (kk - j))).to(torch.bfloat16)
        out = torch.empty_like(x)
        logits = torch.empty((1, self.E), dtype=torch.bfloat16, device=self.device)
        weights = torch.empty((1, kk), dtype=torch.bfloat16, device=self.device)
        selected = torch.empty((1, kk), dtype=torch.int64, device=self.device)
        samples = []
        for i in range(reps):
            t0 = time.perf_counter()
            self._bound_decode(layer, x, gate, True, kk, out, logits, weights, selected,
                               key=("calibration", layer, kk))
            torch.cuda.synchronize(self.device)
            if i >= warm:
                samples.append((time.perf_counter() - t0) * 1e3)
        self._bindings.pop(("calibration", layer, kk)).close()
        gpu_ms = statistics.median(samples) / kk
        base = self.costs.for_load(1)
        self.graph_cost_calibration = dict(samples_ms=samples, median_ms=statistics.median(samples),
                                           per_expert_ms=gpu_ms, experts_per_replay=kk, previous_gpu_ms=base["gpu_ms"],
                                           scheduler_cost_mode=self.graph_cost_mode,
                                           scheduler_gpu_ms=base["gpu_ms"] if self.graph_cost_mode == "eager_bound"
                                           else gpu_ms,
                                           scope="host wall time of one bound decode-layer launch over resident "
                                                 "experts, per routed expert")
        self.costs = ResidentGraphCosts(self.costs, gpu_ms, self.graph_cost_mode)

    def _dispatch_workspace(self, rows, hidden):
        """Borrowed buffers of the native decode tail (pdscope_runtime.py:177-192):
        host packed/block rows, count/selected/coeff words, device token index
        and scratch."""
        ws = self._dispatch_buffers.get((rows, hidden))
        if ws is None:
            ws = dict(packed=torch.empty((rows, hidden), dtype=torch.bfloat16),
                      block=torch.empty((rows, hidden), dtype=torch.bfloat16),
                      count=ctypes.c_int32(rows), selected=(ctypes.c_int64 * rows)(),
                      coeff=(ctypes.c_float * rows)(*([1.0] * rows)),
                      tokens=torch.zeros(rows, dtype=torch.long, device=self.device),
                      scratch=torch.empty((rows, hidden), dtype=torch.bfloat16, device=self.device))
            self._dispatch_buffers[(rows, hidden)] = ws
        return ws

    def _decode_error_word(self):
        """The fused decode kernel's sticky error word (int32 [1] device view)."""
        w = ops.DECODE_WS_ERROR_WORD
        return ops.decode_workspace(self.device, self.H)[w:w + 1]

    def _raise_if_decode_gave_up(self, flag):
        """A bounded wait of the fused decode kernel gave up (its grid was not
        co-resident, e.g. while other work held CUs): the layer output is
        invalid.  The word is cleared so later calls report only their own."""
        if flag:
            self._decode_error_word().zero_()
            raise RuntimeError("fused decode layer: a bounded internal wait gave up, so this layer's output is "
                               "invalid (its blocks were not all resident at once)")

    def _demand_pipeline(self, phase):
        """(experts per grouped launch, batches whose staging slots are held at once).

        The reference stages one expert per compute call with demand_slots-1
        copies in flight beside it for prefill and 1 for decode
        (pdscope_runtime.py:361), i.e. it holds demand_slots or 2 slots.  The
        slot budget here is the same, but from 6 slots on a prefill layer
        splits it into two halves: one half computes as ONE grouped launch
        while the other half's copies stream.  The per-expert host work
        (ledger, table upload, launches) then shrinks by the batch size and
        stays below the copy time of a 9 MiB expert, so the copy engine does
        not wait for the control thread.
        """
        if phase != "prefill":
            return 1, 2
        if self.demand_slots >= 6:
            return self.demand_slots // 2, 2
        return 1, self.demand_slots

    def _pack_scheduled(self, ids, packed, ws):
        """Grouping of a prelaunched layer with the balanced schedule of all
        experts written by the pack launch itself; returns the row tile (from
        the mean rows per expert, which needs no counts on the host)."""
        T, k = ids.shape
        bm = ops.grouped_block_m((T * k) // self.E)
        bmd = L.down_block_m(bm, self.H, self.I)
        sched = (ws.sel_all, bm, ws.sel_order, ws.tile_start) + ((bmd, ws.tile_start_down) if bmd != bm else ())
        ops.pack(ids, self.E, out=packed, workspace=ws.pack_ws, schedule=sched)
        return bm

    def _launch_resident_layer(self, x, packed, weights, out, ws, layer, bm, stream):
        """Grouped SwiGLU over every expert of a fully resident layer and the
        merge into `out`, on `stream`, on tile counts bounded without the
        host counts (the schedule came out of the pack launch); records
        _layer_done after them."""
        T, k = weights.shape
        bmd = L.down_block_m(bm, self.H, self.I)
        slots_dev = self.executor.upload_table(layer, self.E, stream)
        with torch.cuda.stream(stream):
            L.grouped_ffn(x, packed, ws.sel_all, bm, (T * k + bm - 1) // bm + self.E, slots_dev, ws,
                          max_tiles_down=(T * k + bmd - 1) // bmd + self.E, scheduled=True)
            ops.merge(ws.y, packed.row_of, weights, out, mode=self.merge)
        self._layer_done.record(stream)

    def _grouped(self, x, packed, sel_dev, rows, slots_dev, ws, perm=None):
        """One grouped SwiGLU launch over the experts in sel_dev, whose routed
        row counts (known on the host since the demand reveal) are `rows`:
        the row-tile height follows their mean, the grid their exact tile count.
        perm overrides packed.perm_token (pre-gathered rows read in order)."""
        bm = ops.grouped_block_m(sum(rows) // len(rows), max(rows))
        bmd = L.down_block_m(bm, self.H, self.I)
        L.grouped_ffn(x, packed, sel_dev, bm, sum((r + bm - 1) // bm for r in rows), slots_dev, ws,
                      max_tiles_down=sum((r + bmd - 1) // bmd for r in rows), perm=perm)

    # ------------------------------------------------------------ bound resident decode

    def _ring_output(self, layer, turn):
        """graph_output_pool: output buffer `turn` (0 or 1) of `layer`'s
        two-deep ring (the reference's per-key output ring, executor.py:129-133)."""
        ring = self._out_ring.get(layer)
        if ring is None:
            ring = self._out_ring[layer] = tuple(torch.empty((1, self.H), dtype=torch.bfloat16, device=self.device)
                                                 for _ in range(2))
        return ring[turn]

    def _bound_decode(self, layer, x, gate, normalize, k, out, logits, weights, selected, *, next_gate=None,
                      stream=None, key=None):
        """One token of `layer` through its bound single-launch decode over the
        layer's current slot table (bound on first use): route + SwiGLU +
        merge write out [1,H], logits [1,E], weights [1,k] and selected [1,k]
        int64; with next_gate the same launch predicts the next layer.  The
        routed ids, the prediction and the fused kernel's sticky error word
        land in the pinned read-back buffer (ids at 0, prediction at k, error
        word at _err_at, each tagged with the launch's number, the routed ids
        before the kernel completes).  Returns (the binding, that number)."""
        if key is None:
            key = (layer, k, normalize, gate.data_ptr(), 0 if next_gate is None else next_gate.data_ptr())
        cur = torch.cuda.current_stream(self.device) if stream is None else stream
        # the table is bound by address; refresh its contents (copies may have
        # moved between calls) on the launch stream
        slots_dev = self.executor.upload_table(layer, self.E, cur)
        b = self._bindings.get(key)
        if b is not None:
            self._bindings.move_to_end(key)
        else:
            if len(self._bindings) >= _MAX_BINDINGS:
                self._bindings.popitem(last=False)[1].close()
            b = ops.DecodeBinding(gate, slots_dev, self.I, k, normalize, host=self._pinned_counts,
                                  error_at=self._err_at, merge=self.merge, next_gate=next_gate)
            self._bindings[key] = b
        self._seq = self._seq % 0x7FFF + 1
        b.run_ptrs(x.data_ptr(), out.data_ptr(), logits.data_ptr(), weights.data_ptr(), selected.data_ptr(),
                   self._seq, cur.cuda_stream)
        self.bound_launches += 1
        return b, self._seq

    def close(self):
        self._out_stash = None
        for b in self._bindings.values():
            b.close()
        self._bindings.clear()
        self.executor.shutdown()
