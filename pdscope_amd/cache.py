"""Expert residency ledger: one byte-budgeted cache pool plus demand staging slots.

Host-side bookkeeping only (no tensors, no clocks), owned by one control
thread.  It keeps the contract of expertbench/cache.py:136-662
(``ExpertCache``) that the executor and runtime depend on:

* a load is reserved (``begin_load``), then its transfer is ``submit``-ted, then
  ``complete_load`` is reported only after the copy's event has completed;
* a copy that is computing is held by ``acquire`` until ``release`` (again only
  after the compute event completed), so it can be neither evicted nor reused;
* demand misses that cannot be admitted into the cache fall back to the
  smallest free staging slot that fits (cache.py:531-537) and leave the ledger
  when their single use is released (cache.py:621-624);
* the true demand of one (request, step, layer) is declared first
  (``on_demand``) and closed by ``end_demand`` once every expert completed on
  the GPU (``release``) or the CPU (``finish_cpu``);
* illegal transitions raise ``CacheError`` (``CapacityBlocked`` when a caller
  must wait for work in flight or decline speculation).

Eviction order: LRU over demand ticks (ties by ExpertKey), or LFU
(frequency, then tick, then key); copies protected by a retention hint
sort after unprotected ones; ``static`` never evicts.
"""
from __future__ import annotations

import heapq
from collections import Counter
from collections.abc import Mapping
from dataclasses import dataclass, field
from types import MappingProxyType
from uuid import uuid4


class CacheError(ValueError):
    """Illegal configuration, identity or lifecycle transition."""


class CapacityBlocked(CacheError):
    """Wait for transfers/uses in flight, or decline speculative work."""


def _nonneg_int(value, name, minimum=0):
    if type(value) is not int or value < minimum:
        raise CacheError(f"{name} must be an integer >= {minimum}")


@dataclass(frozen=True, order=True)
class ExpertKey:
    layer: int
    expert: int
    representation: str

    def __post_init__(self):
        _nonneg_int(self.layer, "layer")
        _nonneg_int(self.expert, "expert")
        if not isinstance(self.representation, str) or not self.representation:
            raise CacheError("representation must be explicit")


@dataclass(frozen=True)
class DemandID:
    request: str
    step: int
    layer: int

    def __post_init__(self):
        if not isinstance(self.request, str) or not self.request:
            raise CacheError("request must be a nonempty string")
        _nonneg_int(self.step, "step")
        _nonneg_int(self.layer, "layer")


@dataclass(frozen=True)
class LoadTicket:
    owner: str
    generation: int
    key: ExpertKey
    pool: str          # "cache" or "demand_staging"
    slot: int | None   # staging slot index, None for the cache pool


@dataclass(frozen=True)
class UseHandle:
    ticket: LoadTicket
    serial: int


@dataclass(frozen=True)
class EntryView:
    key: ExpertKey
    nbytes: int
    pool: str
    state: str
    ticket: LoadTicket
    submitted: bool
    users: int
    origin: str
    used: bool
    expired: bool


@dataclass(frozen=True)
class DemandObservation:
    key: ExpertKey
    tokens: int
    valid_tokens: int
    nbytes: int
    state_at_reveal: str
    pool_at_reveal: str | None
    hit_source: str | None

    @property
    def ready_hit(self):
        return self.hit_source is not None


@dataclass
class _Copy:
    ticket: LoadTicket
    nbytes: int
    origin: str
    submitted: bool = False
    ready: bool = False
    used: bool = False
    expired: bool = False
    users: set = field(default_factory=set)
    rev: int = 0

    @property
    def state(self):
        if self.users:
            return "in_use"
        return "ready" if self.ready else "loading"


@dataclass
class _Demand:
    identity: DemandID
    counts: tuple
    valid: dict
    observations: tuple
    remaining: set


class ExpertCache:
    EVICTING = ("LRU", "LFU")

    def __init__(self, expert_bytes, cache_bytes, staging_slot_bytes, *, policy="LRU", initial_hotset=()):
        _nonneg_int(cache_bytes, "cache_bytes")
        sizes = dict(expert_bytes)
        if not sizes or not all(isinstance(k, ExpertKey) for k in sizes):
            raise CacheError("expert_bytes must map ExpertKey to representation bytes")
        for n in sizes.values():
            _nonneg_int(n, "expert bytes", 1)
        slots = tuple(staging_slot_bytes)
        if not slots:
            raise CacheError("at least one demand staging slot is required")
        for n in slots:
            _nonneg_int(n, "staging slot bytes", 1)
        if max(slots) < max(sizes.values()):
            raise CacheError("demand staging cannot hold the largest expert; no forward progress")
        hot = tuple(initial_hotset)
        if len(set(hot)) != len(hot) or any(k not in sizes for k in hot):
            raise CacheError("initial hotset must contain unique registered keys")
        if sum(sizes[k] for k in hot) > cache_bytes:
            raise CacheError("initial hotset exceeds the cache byte budget")
        if policy not in ("static", "LRU", "LFU"):
            raise CacheError("policy must be static, LRU or LFU")
        self.expert_bytes = MappingProxyType(sizes)
        self.cache_bytes = cache_bytes
        self.staging_slot_bytes = slots
        self.policy = policy
        self.initial_hotset = frozenset(hot)
        self._owner = uuid4().hex
        self._serial = 0
        self._copies: dict[ExpertKey, _Copy] = {}
        self._staging_busy: set[int] = set()
        self._cache_used = 0
        self._active: _Demand | None = None
        self._last_event: dict[str, tuple] = {}
        self._tick: dict[ExpertKey, int] = {}
        self._freq: Counter = Counter()
        self._stats: Counter = Counter()
        self._retired: list[LoadTicket] = []
        self._heap: list = []
        self._protected: frozenset = frozenset()

    # ------------------------------------------------------------ queries

    def _known(self, key):
        if key not in self.expert_bytes:
            raise CacheError(f"unknown expert: {key!r}")

    def _copy_of(self, ticket):
        c = self._copies.get(ticket.key)
        if c is None or c.ticket != ticket:
            raise CacheError("stale or foreign load ticket")
        return c

    def _remaining(self, key):
        return self._active is not None and key in self._active.remaining

    def lookup(self, key):
        """Side-effect-free view of the current copy of `key` (or None)."""
        self._known(key)
        c = self._copies.get(key)
        if c is None:
            return None
        return EntryView(key, c.nbytes, c.ticket.pool, c.state, c.ticket, c.submitted, len(c.users), c.origin,
                         c.used, c.expired)

    @property
    def resident_payload_bytes(self):
        return self._cache_used

    @property
    def active_demand(self):
        return None if self._active is None else self._active.identity

    @property
    def unfinished_demand_keys(self):
        return tuple(sorted(self._active.remaining)) if self._active is not None else ()

    def stats(self):
        return dict(self._stats)

    def memory(self):
        staged = [c for c in self._copies.values() if c.ticket.pool == "demand_staging"]
        return dict(cache_capacity_bytes=self.cache_bytes, cache_payload_bytes=self._cache_used,
                    staging_reserved_bytes=sum(self.staging_slot_bytes),
                    staging_payload_bytes=sum(c.nbytes for c in staged), staging_occupied_slots=len(staged),
                    expert_reserved_bytes=self.cache_bytes + sum(self.staging_slot_bytes))

    def demand_frequency(self, key):
        self._known(key)
        return self._freq[key]

    def take_retired(self):
        """Copies whose device memory may now be reused (consumed once)."""
        out = tuple(self._retired)
        self._retired.clear()
        return out

    # ------------------------------------------------------------ eviction

    def _evictable(self, c):
        return (self.policy in self.EVICTING and c.ticket.pool == "cache" and c.ready and not c.users
                and not self._remaining(c.ticket.key))

    def _priority(self, c):
        key = c.ticket.key
        tick = self._tick.get(key, 0)
        base = (self._freq[key], tick, key) if self.policy == "LFU" else (tick, key)
        return (key in self._protected,) + base

    def _push(self, key):
        c = self._copies.get(key)
        if c is not None and self._evictable(c):
            c.rev += 1
            heapq.heappush(self._heap, (self._priority(c), c.ticket.generation, c.rev, key))
            if len(self._heap) > max(64, 4 * len(self._copies)):
                self._heap = [(self._priority(x), x.ticket.generation, x.rev, x.ticket.key)
                              for x in self._copies.values() if self._evictable(x)]
                heapq.heapify(self._heap)

    def _plan_victims(self, size):
        """Evictable copies freeing enough bytes, or None.  Changes nothing."""
        need = self._cache_used + size - self.cache_bytes
        if need <= 0:
            return []
        popped, chosen = [], []
        while self._heap and need > 0:
            node = heapq.heappop(self._heap)
            popped.append(node)
            prio, gen, rev, key = node
            c = self._copies.get(key)
            if c is None or c.ticket.generation != gen or c.rev != rev or not self._evictable(c):
                continue
            if prio != self._priority(c):
                # priority changed since the node was queued: requeue it
                c.rev += 1
                heapq.heappush(self._heap, (self._priority(c), gen, c.rev, key))
                continue
            chosen.append(key)
            need -= c.nbytes
        for node in popped:
            heapq.heappush(self._heap, node)
        return chosen if need <= 0 else None

    def _drop(self, key):
        c = self._copies.pop(key)
        if c.ticket.pool == "cache":
            self._cache_used -= c.nbytes
        else:
            self._staging_busy.discard(c.ticket.slot)
        self._retired.append(c.ticket)
        return c

    def _evict(self, key):
        c = self._drop(key)
        self._stats["evictions"] += 1
        self._stats["evicted_bytes"] += c.nbytes
        if c.origin == "prefetch" and not c.used:
            self._stats["unused_prefetch_evictions"] += 1

    def evict(self, key):
        self._known(key)
        c = self._copies.get(key)
        if c is None or not self._evictable(c):
            raise CacheError("cannot evict an absent, static, loading, referenced or demanded copy")
        self._evict(key)

    def set_protected(self, keys):
        """Soft eviction preference: these copies are evicted last (next-layer forecast)."""
        self._protected = frozenset(keys)
        for k in self._protected:
            self._push(k)

    # ------------------------------------------------------------ demand

    def on_demand(self, identity, token_counts, *, valid_token_counts=None):
        """Declare the true demand of one (request, step, layer) before any work."""
        if not isinstance(identity, DemandID):
            raise CacheError("only true routing can declare a demand")
        if not isinstance(token_counts, Mapping):
            raise CacheError("token_counts must map ExpertKey to token count")
        counts = tuple(sorted(dict(token_counts).items()))
        if not counts:
            raise CacheError("empty demands are not recorded")
        for key, n in counts:
            self._known(key)
            if key.layer != identity.layer:
                raise CacheError("demand keys must belong to the revealed layer")
            _nonneg_int(n, "tokens per expert", 1)
        phys = dict(counts)
        valid = dict(phys if valid_token_counts is None else valid_token_counts)
        for key, n in valid.items():
            if key not in phys:
                raise CacheError("valid demand has no physical execution")
            _nonneg_int(n, "valid tokens", 1)
            if n > phys[key]:
                raise CacheError("valid tokens exceed physical tokens")
        if self._active is not None:
            if self._active.identity == identity and self._active.counts == counts and self._active.valid == valid:
                return self._active.observations
            raise CacheError("another or conflicting layer-step demand is active")
        prev = self._last_event.get(identity.request)
        if prev is not None and (identity.step, identity.layer) <= prev:
            raise CacheError("duplicate or out-of-order demand event")
        if not self._stats["physical_layer_events"] and any(
                k not in self._copies or not self._copies[k].ready for k in self.initial_hotset):
            raise CacheError("initial hotset must finish loading before the first demand")
        old_protected, self._protected = self._protected, frozenset()
        for k in old_protected:
            self._push(k)
        self._stats["physical_layer_events"] += 1
        tick = self._stats["physical_layer_events"]
        obs = []
        for key, n in counts:
            c = self._copies.get(key)
            src = None
            if c is not None and c.ready:
                src = "fresh_prefetch" if (c.origin == "prefetch" and not c.used) else "history"
            o = DemandObservation(key, n, valid.get(key, 0), self.expert_bytes[key],
                                  c.state if c else "absent", c.ticket.pool if c else None, src)
            obs.append(o)
            self._stats["physical_expert_demands"] += 1
            self._stats["physical_demand_tokens"] += n
            if not o.valid_tokens:
                continue
            self._freq[key] += 1
            self._tick[key] = tick
            self._stats["expert_demands"] += 1
            self._stats["demand_tokens"] += o.valid_tokens
            self._stats["demand_bytes"] += o.nbytes
            if o.ready_hit:
                self._stats["ready_hits"] += 1
                self._stats["history_ready_hits" if src == "history" else "fresh_prefetch_hits"] += 1
                self._stats["cache_resident_hits" if o.pool_at_reveal == "cache" else "staging_ready_hits"] += 1
            else:
                self._stats["loading_misses" if o.state_at_reveal == "loading" else "absent_misses"] += 1
        self._active = _Demand(identity, counts, valid, tuple(obs), {k for k, _ in counts})
        return self._active.observations

    def end_demand(self, identity):
        if self._active is None or self._active.identity != identity:
            raise CacheError("no matching active demand")
        if self._active.remaining:
            raise CacheError("cannot finish the layer: some demanded experts have not completed")
        self._last_event[identity.request] = (identity.step, identity.layer)
        done = self._active.counts
        self._active = None
        for key, _ in done:
            self._push(key)

    # ------------------------------------------------------------ loads

    def begin_load(self, key, *, origin="demand", admit=True):
        """Reserve one copy (cache pool, or a staging slot for demand misses)."""
        self._known(key)
        if origin not in ("initial", "demand", "prefetch"):
            raise CacheError("unknown load origin")
        if type(admit) is not bool or (not admit and origin != "demand"):
            raise CacheError("non-admission is a demand-only option")
        if origin == "demand":
            if not self._remaining(key):
                raise CacheError("demand load for an expert outside the active demand")
        elif origin == "initial":
            if self._stats["physical_layer_events"] or self._active is not None or key not in self.initial_hotset:
                raise CacheError("initial loads are limited to the declared hotset before the first demand")
        elif self.policy == "static" or self._remaining(key):
            raise CacheError("prefetch is not allowed for a static cache or an already revealed demand")
        existing = self._copies.get(key)
        if existing is not None:
            return existing.ticket
        size = self.expert_bytes[key]
        victims = None
        if admit and (self.policy in self.EVICTING or origin == "initial"):
            victims = self._plan_victims(size)
        if victims is not None:
            pool, slot = "cache", None
        elif origin == "demand":
            free = [(cap, i) for i, cap in enumerate(self.staging_slot_bytes)
                    if i not in self._staging_busy and cap >= size]
            if not free:
                raise CapacityBlocked("demand staging busy: finish transfers/uses in flight first")
            pool, slot = "demand_staging", min(free)[1]
        else:
            raise CapacityBlocked("no evictable cache bytes; speculation cannot use demand staging")
        for v in victims or ():
            self._evict(v)
        self._serial += 1
        ticket = LoadTicket(self._owner, self._serial, key, pool, slot)
        self._copies[key] = _Copy(ticket, size, origin)
        if pool == "cache":
            self._cache_used += size
        else:
            self._staging_busy.add(slot)
        return ticket

    def submit(self, ticket):
        c = self._copy_of(ticket)
        if c.submitted or c.ready:
            raise CacheError("transfer already submitted")
        if c.origin == "prefetch" and self._remaining(ticket.key):
            c.origin, c.expired = "demand", True
        c.submitted = True
        self._stats[f"{c.origin}_loads_submitted"] += 1
        self._stats["h2d_bytes_submitted"] += c.nbytes

    def complete_load(self, ticket):
        """Report that this generation's copy has landed (event completed)."""
        c = self._copy_of(ticket)
        if not c.submitted or c.ready:
            raise CacheError("completion needs one submitted, incomplete transfer")
        c.ready = True
        self._stats["h2d_bytes_completed"] += c.nbytes
        self._push(ticket.key)

    # ------------------------------------------------------------ uses

    def acquire(self, key):
        """Hold a ready copy for GPU compute; pairs with release()."""
        if not self._remaining(key):
            raise CacheError("expert is not an unfinished member of the active demand")
        c = self._copies.get(key)
        if c is None or not c.ready:
            raise CacheError("weights are not ready; a loading copy is not a hit")
        self._serial += 1
        c.users.add(self._serial)
        return UseHandle(c.ticket, self._serial)

    def release(self, handle):
        """Report completed GPU compute; the last release completes the expert."""
        c = self._copy_of(handle.ticket)
        if handle.serial not in c.users:
            raise CacheError("stale, foreign or already released use handle")
        c.users.remove(handle.serial)
        key = handle.ticket.key
        c.used = c.used or key in self._active.valid
        if c.users:
            return
        self._active.remaining.discard(key)
        self._stats["gpu_completed_experts"] += 1
        self._stats["gpu_completed_valid_experts"] += int(key in self._active.valid)
        if handle.ticket.pool == "demand_staging":
            self._drop(key)  # a staged miss never stays resident
        else:
            self._push(key)

    def finish_cpu(self, key):
        """The CPU consumed the master copy of `key`; no GPU copy is admitted."""
        if not self._remaining(key):
            raise CacheError("expert is not an unfinished member of the active demand")
        c = self._copies.get(key)
        if c is not None and (c.users or (c.origin == "demand" and not c.ready)):
            raise CacheError("cannot switch an active GPU use/load to CPU completion")
        if c is not None and c.ticket.pool == "demand_staging":
            raise CacheError("a staged copy must complete through the GPU")
        self._active.remaining.discard(key)
        self._stats["cpu_completed_experts"] += 1
        self._stats["cpu_completed_valid_experts"] += int(key in self._active.valid)
        self._push(key)

    def reset(self):
        if self._active is not None or any(not c.ready or c.users for c in self._copies.values()):
            raise CacheError("cannot reset with active demands, loads or uses")
        self._retired.extend(c.ticket for c in self._copies.values())
        self._copies.clear()
        self._cache_used = 0
        self._staging_busy.clear()
        self._heap.clear()
        self._last_event.clear()
        self._tick.clear()
        self._freq.clear()
        self._stats.clear()
        self._protected = frozenset()
