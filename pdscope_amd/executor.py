"""Device executor: pinned-source staging into HBM slots and grouped expert launches.

Mirrors ExpertExecutor (expertbench/executor.py:165-680) for the GPU path:

* ``load`` reserves a copy in the ledger and stages the expert's whole
  gate|up|down block (one pinned host block, one ``hipMemcpyAsync``) into a
  cache-pool slot or a demand staging slot on the load stream, recording one
  event (executor.py:333-372);
* ``finish_load`` reports completion to the ledger only after that event
  completed (executor.py:374-390);
* ``gpu_group`` acquires every expert of a launch, runs ONE grouped launch on
  the compute stream and records one event; ``finish_gpu`` releases them after
  the event completed (executor.py:430-511 keep one event per expert; here a
  layer's experts share one launch and one event);
* ``gpu(key, inputs)`` keeps the per-expert operator hook of executor.py:454-488
  (rows of one expert through the same grouped kernel);
* each layer has a device slot table (int64 base address per expert, 0 when
  no ready copy), so kernels address cache and staging slots uniformly.

Single control thread; streams keep the default priority.
"""
from __future__ import annotations

import contextlib
import ctypes
import os
import threading
import time
from dataclasses import dataclass, field

import torch

from . import ops
from .cache import ExpertKey

PROJECTIONS = ("gate_proj", "up_proj", "down_proj")


@dataclass
class ExpertWeights:
    """One expert's three projections; ``flat`` is the gate|up|down block when contiguous."""
    key: ExpertKey
    tensors: dict
    provenance: dict = field(default_factory=dict)
    flat: torch.Tensor | None = None

    @property
    def nbytes(self):
        return sum(t.numel() * t.element_size() for t in self.tensors.values())


def masters_from_block(layer, block, E, H, I, *, pin=True, chunk_bytes=1 << 28):
    """ExpertWeights for one layer whose experts are rows of a [E, 3*I*H] bf16 tensor.

    The host copy is page-locked (pinned) so staging is one DMA per expert.
    It is allocated in chunks of whole experts of at most chunk_bytes: the
    pinned-memory allocator rounds every allocation up to a power of two, so
    one [E, 3*I*H] buffer of 1.18 GB would hold 2 GiB of locked pages.
    """
    block = block.detach()
    per = max(1, chunk_bytes // (block.shape[1] * block.element_size())) if pin else E
    rows = []
    for e0 in range(0, E, per):
        n = min(per, E - e0)
        if pin:
            host = torch.empty((n, block.shape[1]), dtype=block.dtype, pin_memory=True)
            host.copy_(block[e0:e0 + n])
        else:
            host = block[e0:e0 + n].to("cpu")
        rows += [host[j] for j in range(n)]
    IH = I * H
    out = {}
    for e in range(E):
        row = rows[e]
        tensors = {"gate_proj": row[:IH].view(I, H), "up_proj": row[IH:2 * IH].view(I, H),
                   "down_proj": row[2 * IH:].view(H, I)}
        key = ExpertKey(layer, e, "bf16")
        out[key] = ExpertWeights(key, tensors, {"source": "synthetic seeded layer"}, flat=row)
    return out


@dataclass
class PendingCpu:
    """A CPU-backend expert call in flight (key, future, input rows)."""
    key: ExpertKey
    future: object
    input_ref: object


@dataclass
class PendingCompute:
    handles: tuple
    output: object
    event: object                 # completion event (or the caller's proof); None: accounted after it completed
    input_ref: object
    keys: tuple = ()
    timing_start: object = None   # start event of the launch when stages are profiled
    event_owned: bool = True      # the event came from this executor's pool


class _PinnedRing:
    """Small page-locked upload buffers reused after their last copy completed."""

    def __init__(self, nbytes, depth=16):
        self.bufs = [torch.empty(nbytes, dtype=torch.uint8, pin_memory=True) for _ in range(depth)]
        self.events = [None] * depth
        self.i = 0

    def take(self):
        i = self.i
        self.i = (i + 1) % len(self.bufs)
        if self.events[i] is not None:
            self.events[i].synchronize()
        return i, self.bufs[i]

    def mark(self, i, stream):
        ev = torch.cuda.Event()
        ev.record(stream)
        self.events[i] = ev


class ExpertExecutor:
    """Expert copies, launches and CPU calls under the ledger (expertbench/executor.py:165-596).

    profile_stages records per-stage times in ``stage_timings`` as the
    reference does (executor.py:352-355, 384-385, 472-481, 518-528): the device
    span of each expert copy (``weight_dma_gpu_span_ms``), the host time to
    submit a grouped launch (``gpu_forward_host_submit_ms``) and its device
    span (``gpu_forward_device_span_ms``), the host time of pinning a master
    on first use (``source_copy_ms``) and a CPU expert call's time on the
    worker (``cpu_forward_ms``); each key holds the latest value.
    initialize_cpu_worker: the worker thread that runs a callable CPU backend
    first sets torch's thread count to the control thread's (its result is
    ``cpu_worker_init``).  cpu_staging_copy: how a master that is not already
    one pinned block is copied into one ("torch": tensor copies, "memcpy":
    byte copies of contiguous tensors)."""

    def __init__(self, cache, masters, device=0, *, pinned_source_mode="all_masters", profile_stages=False,
                 capture_events=True, streams=None, initialize_cpu_worker=True, cpu_backend=None,
                 cpu_staging_copy="torch", cache_storage=None, staging_storage=None):
        if pinned_source_mode not in ("all_masters", "lazy_pinned"):
            raise ValueError("unknown pinned source mode")
        if cpu_staging_copy not in ("torch", "memcpy"):
            raise ValueError("unknown CPU staging copy implementation")
        if type(initialize_cpu_worker) is not bool:
            raise ValueError("CPU worker initialization must be explicitly boolean")
        if type(profile_stages) is not bool:
            raise ValueError("stage profiling must be explicitly boolean")
        self.cpu_staging_copy, self.initialize_cpu_worker = cpu_staging_copy, initialize_cpu_worker
        self.cpu_worker_init = None
        self.stage_timings, self._load_starts = {}, {}
        if cpu_backend is not None and not callable(cpu_backend):
            raise ValueError("CPU backend must be an explicit callable")
        self.cache, self.masters = cache, dict(masters)
        if set(cache.expert_bytes) != set(self.masters):
            raise ValueError("cache and master weight registries differ")
        for key, w in self.masters.items():
            if w.nbytes != cache.expert_bytes[key] or any(
                    t.device.type != "cpu" or t.dtype != torch.bfloat16 for t in w.tensors.values()):
                raise ValueError("master bytes/device/dtype do not match the cache contract")
        sizes = set(cache.expert_bytes.values())
        if len(sizes) != 1:
            raise ValueError("equal-size bf16 experts required")
        self.expert_bytes = next(iter(sizes))
        self.device = torch.device("cuda", device) if isinstance(device, int) else torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("the executor runs on a GPU device")
        if self.device.index is None:  # "cuda" names the current device; keep its index so placement checks compare
            self.device = torch.device("cuda", torch.cuda.current_device())
        self.cpu_backend = cpu_backend
        self.gpu_backend = None
        self.capture_events = capture_events
        self.profile_stages = profile_stages
        self.pinned_source_mode = pinned_source_mode
        self.events: list = []
        if streams is None:
            self.load_stream = torch.cuda.Stream(device=self.device)
            self.compute_stream = torch.cuda.Stream(device=self.device)
        else:
            if (not isinstance(streams, tuple) or len(streams) != 2 or streams[0] == streams[1]
                    or any(s.device != self.device for s in streams)):
                raise ValueError("shared executor streams must be a distinct pair on the same device")
            self.load_stream, self.compute_stream = streams
        # ---- device storage: one contiguous cache pool of equal slots, plus staging slots
        nslots = cache.cache_bytes // self.expert_bytes
        if cache_storage is None:
            cache_storage = torch.empty(nslots * self.expert_bytes, dtype=torch.uint8, device=self.device)
        if (cache_storage.device != self.device or cache_storage.dtype != torch.uint8 or cache_storage.ndim != 1
                or not cache_storage.is_contiguous() or cache_storage.numel() < nslots * self.expert_bytes):
            raise ValueError("cache storage must be a contiguous uint8 device tensor covering every cache slot")
        self.cache_storage = cache_storage
        self._free_cache_slots = list(reversed(range(nslots)))
        if staging_storage is None:
            staging_storage = tuple(torch.empty(n, dtype=torch.uint8, device=self.device)
                                    for n in cache.staging_slot_bytes)
        if (len(staging_storage) != len(cache.staging_slot_bytes)
                or any(t.device != self.device or t.dtype != torch.uint8 or not t.is_contiguous() or t.numel() < n
                       for t, n in zip(staging_storage, cache.staging_slot_bytes))):
            raise ValueError("staging storage must match every declared staging slot")
        spans = sorted((t.data_ptr(), t.data_ptr() + t.numel()) for t in staging_storage)
        spans.append((cache_storage.data_ptr(), cache_storage.data_ptr() + cache_storage.numel()))
        spans.sort()
        if any(a[1] > b[0] for a, b in zip(spans, spans[1:])):
            raise ValueError("cache and staging buffers must not overlap")
        self.staging = list(staging_storage)
        # ---- pinned sources (one flat block per expert)
        self.pinned = {}
        if pinned_source_mode == "all_masters":
            for key in self.masters:
                self.pinned[key] = self._pinned_block(key)
        # ---- bookkeeping
        self.copies = {}     # ticket -> flat device uint8 view
        self._cache_slot_of = {}
        self.loads = {}      # ticket -> event
        self.computes = {}   # id(pending) -> pending
        self._free_events = []
        self.closed = False
        self._host_tables = {}  # layer -> host list of base addresses (0 = no ready copy)
        self._dev_tables = {}   # layer -> device int64 [E]
        self._table_version = {}  # layer -> count of host table changes
        self._uploaded = {}       # layer -> (version, stream, event) of the last upload
        self._ring = _PinnedRing(8 * 256)
        # the slot storage was allocated on the current stream, whose queued
        # work may still touch the blocks' previous owners: order both
        # executor streams after it before they write or read a slot
        cur = torch.cuda.current_stream(self.device)
        self.load_stream.wait_stream(cur)
        self.compute_stream.wait_stream(cur)
        self._group_stream_ctx = None
        self._cpu_pool = None
        self._cpu_tasks = {}  # key -> PendingCpu
        self._landed = {}     # ticket -> completed load event not yet waited on by a consumer
        # optional check hook: consume_hook(key, flat) runs on the compute
        # stream right before each grouped launch, once per device copy it reads
        self.consume_hook = None

    # ------------------------------------------------------------ sources

    def _pinned_block(self, key):
        w = self.masters[key]
        flat = w.flat
        if flat is not None and flat.is_pinned() and flat.is_contiguous():
            return flat.view(torch.uint8) if flat.dtype != torch.uint8 else flat
        started = time.perf_counter_ns() if self.profile_stages else None
        block = torch.empty(self.expert_bytes, dtype=torch.uint8, pin_memory=True)
        off = 0
        for name in PROJECTIONS:
            t = w.tensors[name]
            n = t.numel() * t.element_size()
            if self.cpu_staging_copy == "memcpy":
                if not t.is_contiguous():
                    raise ValueError("byte staging requires contiguous BF16 master tensors")
                ctypes.memmove(block.data_ptr() + off, t.data_ptr(), n)
            else:
                block[off:off + n].copy_(t.contiguous().view(torch.uint8).reshape(-1))
            off += n
        if started is not None:
            self.stage_timings["source_copy_ms"] = (time.perf_counter_ns() - started) / 1e6
        return block

    def prepare_source(self, key):
        self._open()
        if key not in self.pinned:
            self.pinned[key] = self._pinned_block(key)
        return self.pinned[key]

    # ------------------------------------------------------------ helpers

    def _open(self):
        if self.closed:
            raise RuntimeError("executor has been shut down; its ledger cannot be reused")

    def _event(self):
        return self._free_events.pop() if self._free_events else torch.cuda.Event(enable_timing=self.profile_stages)

    def _log(self, **kw):
        if self.capture_events:
            self.events.append(kw)

    def _host_table(self, layer, E):
        """Host mirror of a layer's slot table, seeded from the ready copies in the ledger."""
        host = self._host_tables.get(layer)
        if host is None:
            host = [0] * E
            for e in range(E):
                key = ExpertKey(layer, e, "bf16")
                if key not in self.masters:
                    continue
                view = self.cache.lookup(key)
                if view is not None and view.state != "loading" and view.ticket in self.copies:
                    host[e] = self.copies[view.ticket].data_ptr()
            self._host_tables[layer] = host
        return host

    def table(self, layer, E):
        """Device slot table of `layer` (int64 [E]) and its host mirror; 0 = no ready copy."""
        host = self._host_table(layer, E)
        dev = self._dev_tables.get(layer)
        if dev is None:
            # the zero fill runs on the current stream while uploads and
            # launches use other streams: let it finish before any of them
            # can write or read the table
            dev = torch.zeros(E, dtype=torch.int64, device=self.device)
            torch.cuda.current_stream(self.device).synchronize()
            self._dev_tables[layer] = dev
        return dev, host

    def _set_entry(self, key, addr):
        host = self._host_tables.get(key.layer)
        if host is not None and key.expert < len(host) and host[key.expert] != addr:
            host[key.expert] = addr
            self._table_version[key.layer] = self._table_version.get(key.layer, 0) + 1

    def table_full(self, layer, E):
        """Whether every one of `layer`'s E experts has a ready device copy in its slot table."""
        return 0 not in self._host_table(layer, E)

    def table_version(self, layer):
        """A number that changes whenever an entry of `layer`'s slot table changes."""
        return self._table_version.get(layer, 0)

    def table_entry(self, layer, e):
        host = self._host_tables.get(layer)
        return 0 if host is None or e >= len(host) else host[e]

    def upload_table(self, layer, E, stream):
        """Copy the host mirror of a layer's slot table to the device on `stream`.

        A table whose host mirror has not changed since its last upload is not
        copied again; a reader on another stream is ordered after that copy."""
        dev, host = self.table(layer, E)
        ver = self._table_version.get(layer, 0)
        last = self._uploaded.get(layer)
        if last is not None and last[0] == ver:
            if last[1] is not stream and last[1] != stream:
                stream.wait_event(last[2])
            return dev
        i, buf = self._ring.take()
        view = buf[:8 * E].view(torch.int64)
        view.copy_(torch.tensor(host, dtype=torch.int64))
        with torch.cuda.stream(stream):
            dev.copy_(view, non_blocking=True)
        self._ring.mark(i, stream)
        self._uploaded[layer] = (ver, stream, self._ring.events[i])
        return dev

    def upload_ints(self, values, stream):
        """A fresh int32 device tensor holding `values`, copied on `stream` via the pinned ring."""
        n = len(values)
        if 4 * n > self._ring.bufs[0].numel():
            raise ValueError("too many values for one upload")
        i, buf = self._ring.take()
        view = buf[:4 * n].view(torch.int32)
        view.copy_(torch.tensor(values, dtype=torch.int32))
        with torch.cuda.stream(stream):
            # allocated on the stream that writes and reads it, so the caching
            # allocator reuses its block only in that stream's order
            dev = torch.empty(n, dtype=torch.int32, device=self.device)
            dev.copy_(view, non_blocking=True)
        self._ring.mark(i, stream)
        return dev

    def base_address(self, key):
        view = self.cache.lookup(key)
        if view is None:
            return 0
        flat = self.copies.get(view.ticket)
        return 0 if flat is None else flat.data_ptr()

    def reclaim(self):
        self._open()
        retired = self.cache.take_retired()
        if not retired:
            return
        for ticket in retired:
            if ticket in self.loads:
                raise RuntimeError("the ledger retired a copy with a transfer in flight")
            self.copies.pop(ticket, None)
            ev = self._landed.pop(ticket, None)
            if ev is not None:
                self._free_events.append(ev)
            slot = self._cache_slot_of.pop(ticket, None)
            if slot is not None:
                self._free_cache_slots.append(slot)
            self._set_entry(ticket.key, 0)
            self._log(event="retired", generation=ticket.generation, pool=ticket.pool)

    # ------------------------------------------------------------ loads

    def load(self, key, *, origin="demand", admit=True):
        self._open()
        ticket = self.cache.begin_load(key, origin=origin, admit=admit)
        self.reclaim()
        if ticket in self.copies:
            return ticket
        src = self.prepare_source(key)
        if ticket.pool == "demand_staging":
            flat = self.staging[ticket.slot][:self.expert_bytes]
        else:
            if not self._free_cache_slots:
                raise RuntimeError("cache pool slot accounting differs from the ledger")
            slot = self._free_cache_slots.pop()
            self._cache_slot_of[ticket] = slot
            flat = self.cache_storage[slot * self.expert_bytes:(slot + 1) * self.expert_bytes]
        self.copies[ticket] = flat
        self.cache.submit(ticket)
        if self.profile_stages:
            start = torch.cuda.Event(enable_timing=True)
            start.record(self.load_stream)
            self._load_starts[ticket] = start
        ev = self._event()
        ops.stage_expert(flat, src, event=ev, stream=self.load_stream)
        self.loads[ticket] = ev
        self._log(event="load_submitted", generation=ticket.generation, pool=ticket.pool,
                  expert_bytes=self.expert_bytes, source_pinned=bool(src.is_pinned()))
        return ticket

    def finish_load(self, ticket, *, wait=False):
        self._open()
        ev = self.loads[ticket]
        if wait:
            ev.synchronize()
        if not ev.query():
            return False
        self.cache.complete_load(ticket)
        del self.loads[ticket]
        start = self._load_starts.pop(ticket, None)
        if start is not None:
            self.stage_timings["weight_dma_gpu_span_ms"] = start.elapsed_time(ev)
        # kept until the copy's first consumer is launched, which waits on it
        # on the compute stream (gpu_group)
        self._landed[ticket] = ev
        self._set_entry(ticket.key, self.copies[ticket].data_ptr())
        self._log(event="load_completed", generation=ticket.generation)
        return True

    # ------------------------------------------------------------ compute

    def begin_gpu_group(self):
        """Join the current stream once for a span of already materialised inputs."""
        self._open()
        self.compute_stream.wait_stream(torch.cuda.current_stream(self.device))
        self._group_stream_ctx = torch.cuda.stream(self.compute_stream)
        self._group_stream_ctx.__enter__()

    def end_gpu_group(self):
        if self._group_stream_ctx is not None:
            self._group_stream_ctx.__exit__(None, None, None)
            self._group_stream_ctx = None

    def gpu_group(self, keys, launch, *, input_ref=None, wait_for=None, completed=None, running=None):
        """Acquire `keys`, run `launch()` (one grouped launch) on the compute stream, record one event.

        With launch=None the work that read these copies was enqueued on
        `wait_for` before the ledger revealed them (a launch issued ahead of
        the reveal): the uses are accounted with no compute-stream join and
        no event of their own.  Either that work has finished -- `completed`
        proves it through query() (an event recorded after the work, or a
        host word the work writes last) and must report completion, or the
        call raises -- or it may still run: `running` is such a proof (with
        synchronize()) that need not report completion yet, and finish_gpu
        waits on it.  A running use is held from this call on, so the caller
        must make sure that nothing could evict these copies between the
        work's launch and this call (the runtime reveals them first, with no
        ledger call in between: an expert of the open demand is never
        evicted)."""
        self._open()
        if launch is None:
            if (completed is None) == (running is None):
                raise RuntimeError("an already enqueued use of expert copies needs exactly one of completed= "
                                   "(the work has finished) and running= (a proof to wait on)")
            if completed is not None and not completed.query():
                raise RuntimeError("an already enqueued use of expert copies is accounted only after it has "
                                   "completed: pass the completed event recorded after it")
        handles = self.cache.acquire_many(keys)
        copies, loads = self.copies, self.loads
        for h in handles:
            if h.ticket not in copies or h.ticket in loads:
                raise RuntimeError("acquired a copy whose transfer has not been confirmed")
        if launch is None:
            for h in handles:
                ev = self._landed.pop(h.ticket, None)
                if ev is not None:
                    self._free_events.append(ev)
            # no event of its own: finish_gpu finds the work complete, or
            # waits on the caller's proof
            p = PendingCompute(handles, None, running, input_ref, tuple(keys), event_owned=False)
            self.computes[id(p)] = p
            if self.capture_events:
                self._log(event="compute_submitted", experts=len(keys))
            return p
        span = self._group_stream_ctx is not None
        ctx = contextlib.nullcontext() if span else torch.cuda.stream(self.compute_stream)
        with ctx:
            if not span:
                self.compute_stream.wait_stream(torch.cuda.current_stream(self.device)
                                                if wait_for is None else wait_for)
            # order each copy's transfer (load stream) before its first consumer
            # on the device as well: the host already saw the transfer complete,
            # so the wait costs nothing, and the dependency is explicit to the
            # runtime, which applies its cache visibility rules to it
            for h in handles:
                ev = self._landed.pop(h.ticket, None)
                if ev is not None:
                    self.compute_stream.wait_event(ev)
                    self._free_events.append(ev)
            if self.consume_hook is not None:
                for h in handles:
                    self.consume_hook(h.ticket.key, self.copies[h.ticket])
            start = None
            if self.profile_stages:
                start = torch.cuda.Event(enable_timing=True)
                start.record(self.compute_stream)
                submit_start = time.perf_counter_ns()
            output = launch()
            if start is not None:
                self.stage_timings["gpu_forward_host_submit_ms"] = (time.perf_counter_ns() - submit_start) / 1e6
            ev = self._event()
            ev.record(self.compute_stream)
        p = PendingCompute(handles, output, ev, input_ref, tuple(keys), start)
        self.computes[id(p)] = p
        self._log(event="compute_submitted", experts=len(keys))
        return p

    def finish_gpu(self, pending, *, wait=False):
        self._open()
        if self.computes.get(id(pending)) is not pending:
            raise ValueError("unknown or already completed GPU computation")
        ev = pending.event
        if ev is not None:   # None: accounted after it had completed
            if wait:
                ev.synchronize()
            if not ev.query():
                return None
        self.cache.release_many(pending.handles)
        del self.computes[id(pending)]
        if pending.timing_start is not None:
            self.stage_timings["gpu_forward_device_span_ms"] = pending.timing_start.elapsed_time(ev)
            pending.timing_start = None
        if ev is not None and pending.event_owned:
            self._free_events.append(ev)
        pending.event, pending.input_ref = None, None
        self.reclaim()
        if self.capture_events:
            self._log(event="compute_completed", experts=len(pending.handles))
        return pending.output

    def gpu(self, key, inputs):
        """Per-expert operator hook: rows of one expert -> unweighted bf16 outputs."""
        self._open()
        if inputs.device != self.device or inputs.dtype != torch.bfloat16:
            raise ValueError("GPU input must already be bf16 on the configured device")
        w = self.masters[key]
        I, H = w.tensors["gate_proj"].shape
        if inputs.ndim != 2 or inputs.shape[1] != H:
            raise ValueError("invalid expert input shape")
        view = self.cache.lookup(key)
        if view is None or view.ticket not in self.copies:
            raise ValueError("expert has no device copy")
        flat = self.copies[view.ticket]

        def launch():
            if self.gpu_backend is not None:
                return self.gpu_backend(key, inputs, flat)
            return expert_rows(inputs, flat, H, I)

        return self.gpu_group([key], launch, input_ref=inputs)

    # ------------------------------------------------------------ CPU experts

    def submit_cpu(self, key, inputs):
        """Run one expert on the caller's CPU backend (executor.py:528-560):
        ``cpu_backend.submit(key, inputs)`` when the backend has it, else the
        callable ``cpu_backend(key, inputs)`` on one worker thread, so the CPU
        work overlaps the GPU launches.  inputs: CPU bf16 [rows, H].  There is
        no built-in CPU expert: without a backend this raises."""
        self._open()
        backend = self.cpu_backend
        if backend is None:
            raise ValueError("CPU placement needs an explicit CPU backend")
        if (key in self._cpu_tasks or key not in self.cache.unfinished_demand_keys or inputs.device.type != "cpu"
                or inputs.dtype != torch.bfloat16 or inputs.ndim != 2
                or inputs.shape[1] != self.masters[key].tensors["gate_proj"].shape[1]):
            raise ValueError("CPU submission requires unique active demand and CPU BF16 input")
        if callable(getattr(backend, "submit", None)):
            future = backend.submit(key, inputs)
        else:
            if self._cpu_pool is None:
                from concurrent.futures import ThreadPoolExecutor
                expected = torch.get_num_threads()

                def initialize():
                    torch.set_num_threads(expected)
                    self.cpu_worker_init = dict(expected_threads=expected, torch_threads=torch.get_num_threads(),
                                                native_thread_id=threading.get_native_id(),
                                                affinity=sorted(os.sched_getaffinity(0)))
                self._cpu_pool = ThreadPoolExecutor(max_workers=1, thread_name_prefix="pdscope-cpu",
                                                    initializer=initialize if self.initialize_cpu_worker else None)

            def work():
                started = time.perf_counter_ns()
                out = backend(key, inputs)
                if isinstance(out, tuple):  # (output, timing) as the reference's pool returns
                    out = out[0]
                return out, (time.perf_counter_ns() - started) / 1e6
            future = self._cpu_pool.submit(work)
        pending = PendingCpu(key, future, inputs)
        self._cpu_tasks[key] = pending
        return pending

    def finish_cpu(self, pending, *, wait=False):
        """The expert's unweighted CPU bf16 output [rows, H] (None while it runs
        and wait is False); completes its demand in the ledger."""
        self._open()
        if self._cpu_tasks.get(pending.key) is not pending:
            raise ValueError("CPU completion does not own an active task")
        if not wait and not pending.future.done():
            return None
        out = pending.future.result()
        if isinstance(out, tuple):  # (output, timing) as the reference's pool returns
            out, timing = out[0], out[1] if len(out) > 1 else None
            if self.profile_stages and isinstance(timing, (int, float)):
                self.stage_timings["cpu_forward_ms"] = float(timing)
        if (not isinstance(out, torch.Tensor) or out.device.type != "cpu" or out.dtype != torch.bfloat16
                or tuple(out.shape) != tuple(pending.input_ref.shape)):
            raise ValueError("CPU backend must return completed unweighted CPU BF16 input-shaped output")
        self.cache.finish_cpu(pending.key)
        del self._cpu_tasks[pending.key]
        pending.input_ref = None
        return out

    def submit_cpu_many(self, jobs):
        """Several experts of one layer in one packed backend submission
        (executor.py:580-596): ``cpu_backend.submit_many({key: rows})`` returns
        one future per expert; each expert keeps its own ledger demand."""
        self._open()
        backend = self.cpu_backend
        if not jobs or not callable(getattr(backend, "submit_many", None)):
            raise ValueError("packed CPU execution needs a backend with submit_many")
        active = self.cache.unfinished_demand_keys
        for key, inputs in jobs.items():
            if (key in self._cpu_tasks or key not in active or inputs.device.type != "cpu"
                    or inputs.dtype != torch.bfloat16 or inputs.ndim != 2
                    or inputs.shape[1] != self.masters[key].tensors["gate_proj"].shape[1]):
                raise ValueError("packed CPU submission requires unique active BF16 demands")
        futures = backend.submit_many(dict(jobs))
        if set(futures) != set(jobs):
            raise AssertionError("packed CPU backend lost expert ownership")
        pending = {key: PendingCpu(key, futures[key], inputs) for key, inputs in jobs.items()}
        self._cpu_tasks.update(pending)
        return pending

    def finish_cpu_group(self, pendings):
        """Outputs {expert id: rows} of a packed submission, each expert's
        demand completed in the ledger (waits for every future)."""
        return {p.key.expert: self.finish_cpu(p, wait=True) for p in pendings}

    def shutdown(self):
        if self._cpu_pool is not None:
            self._cpu_pool.shutdown(wait=True)
            self._cpu_pool = None
        if not self.closed:
            self.load_stream.synchronize()
            self.compute_stream.synchronize()
            self.copies.clear()
            self.loads.clear()
            self._landed.clear()
            self.computes.clear()
            self.staging.clear()
            self.pinned.clear()
            self._host_tables.clear()
            self._dev_tables.clear()
            self._table_version.clear()
            self._uploaded.clear()
            self.cache_storage = None
            self.closed = True

    def storage(self):
        return dict(cache_tensor_bytes=sum(f.numel() for t, f in self.copies.items() if t.pool == "cache"),
                    cache_reserved_tensor_bytes=self.cache_storage.numel() if self.cache_storage is not None else 0,
                    staging_tensor_bytes=sum(t.numel() for t in self.staging),
                    pinned_source_bytes=sum(t.numel() * t.element_size() for t in self.pinned.values()))


def expert_rows(x, base, H, I, *, h_ws=None, y=None):
    """y = expert(x) for rows x [m, H] of one expert whose gate|up|down block starts
    at `base` (a device tensor or an integer device address)."""
    m = x.shape[0]
    dev = x.device
    addr = base if isinstance(base, int) else base.data_ptr()
    slots = torch.tensor([addr], dtype=torch.int64, device=dev)
    i32 = dict(dtype=torch.int32, device=dev)
    perm = torch.arange(m, **i32)
    offsets = torch.tensor([0, m], **i32)
    sel = torch.zeros(1, **i32)
    bm = ops.grouped_block_m(m)
    tile_start = torch.tensor([0, (m + bm - 1) // bm], **i32)
    h_ws = torch.empty(m * I, dtype=torch.bfloat16, device=dev) if h_ws is None else h_ws
    y = torch.empty((m, H), dtype=torch.bfloat16, device=dev) if y is None else y
    ops.swiglu_grouped(x.contiguous(), perm, offsets, sel, tile_start, (m + bm - 1) // bm, bm, slots, H, I, h_ws, y)
    return y
