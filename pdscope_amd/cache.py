"""Expert residency ledger: which expert copies live in HBM, and where.

Host-side bookkeeping for one control thread (no tensors, clocks or device
calls).  It honours the ExpertCache contract of expertbench/cache.py:136-662,
on which the executor and runtime rely:

* one byte-budgeted cache pool plus a few demand-only staging slots, disjoint;
* a copy is reserved (``begin_load``), its transfer submitted (``submit``),
  and made usable by ``complete_load`` -- reported only after the copy's
  event completed;
* a copy feeding a computation is held (``acquire``) until ``release``, again
  reported only once that computation completed; held copies are never
  evicted or reused;
* a demand miss that the cache cannot admit takes the smallest free staging
  slot that fits (``min((capacity, index))``, cache.py:531-537) and leaves the
  ledger when its single use is released;
* the true demand of one (request, step, layer) is revealed first
  (``on_demand``) and closed (``end_demand``) once each of its experts has
  completed on the GPU (``release``) or the CPU (``finish_cpu``);
* illegal transitions raise ``CacheError``; ``CapacityBlocked`` means the
  caller must wait for work in flight or decline speculation, and a blocked
  reservation changes nothing.

Victim order when the cache pool must make room: LRU evicts the copy whose
expert was demanded least recently (demand ticks; ties by ExpertKey), LFU
the least frequently demanded (then least recently, then by key); copies
under protection (an explicit set, or a next-layer retention hint) go only
after every unprotected one; ``static`` never evicts.

Design: every copy carries an explicit lifecycle phase; the evictable copies
are kept in rankings -- buckets keyed by their rank (tick, or frequency and
tick), each holding its keys sorted, plus the sorted list of live ranks --
that are updated whenever a copy's eligibility or rank changes, so choosing
victims walks the cheapest copies in order without scanning the pool.
"""
from __future__ import annotations

import bisect
import itertools
from collections import Counter
from collections.abc import Mapping
from dataclasses import dataclass, field
from functools import partial
from types import MappingProxyType
from typing import NamedTuple
from uuid import uuid4

try:
    # hash and ==/!= of the key records in C (built by pdscope_amd.build)
    from ._records import HashedRecord as _RecordBase
except ImportError:     # not built: the same semantics in Python
    class _RecordBase:
        """Record with a cached field tuple (_t) and hash (_h): equal only to a
        record of the same class with equal fields."""
        __slots__ = ()

        def __eq__(self, other):
            if self is other:
                return True
            if other.__class__ is self.__class__:
                return self._h == other._h and self._t == other._t
            return NotImplemented

        def __ne__(self, other):
            eq = self.__eq__(other)
            return eq if eq is NotImplemented else not eq

        def __hash__(self):
            return self._h


class CacheError(ValueError):
    """An illegal configuration, identity or lifecycle transition."""


class CapacityBlocked(CacheError):
    """No room now: wait for transfers or uses in flight, or decline speculation."""


def _require_int(value, what, low=0):
    if type(value) is not int or value < low:
        raise CacheError(f"{what} must be an int >= {low}, got {value!r}")


# ---------------------------------------------------------------- public records

@dataclass(frozen=True, order=True)
class ExpertKey(_RecordBase):
    layer: int
    expert: int
    representation: str

    def __post_init__(self):
        _require_int(self.layer, "layer")
        _require_int(self.expert, "expert")
        if not isinstance(self.representation, str) or not self.representation:
            raise CacheError("an expert key names its representation")
        # the ledger hashes and compares keys on every transition: the field
        # tuple and its hash are computed once (the record is immutable) and
        # the base answers hash() and == from them
        t = (self.layer, self.expert, self.representation)
        object.__setattr__(self, "_t", t)
        object.__setattr__(self, "_h", hash(t))

    __eq__ = _RecordBase.__eq__
    __ne__ = _RecordBase.__ne__
    __hash__ = _RecordBase.__hash__

    def __reduce__(self):
        # rebuilt through __init__, so the cached hash is recomputed where the
        # key is loaded (string hashes differ between processes)
        return (ExpertKey, (self.layer, self.expert, self.representation))


@dataclass(frozen=True)
class DemandID:
    """One revealed layer demand: (step, layer) increases within a request."""
    request: str
    step: int
    layer: int

    def __post_init__(self):
        if not isinstance(self.request, str) or not self.request:
            raise CacheError("a demand names its request")
        _require_int(self.step, "step")
        _require_int(self.layer, "layer")


@dataclass(frozen=True)
class LoadTicket(_RecordBase):
    owner: str
    generation: int
    key: ExpertKey
    pool: str            # "cache" or "demand_staging"
    slot: int | None     # staging slot index

    def __post_init__(self):
        # tickets key the executor's copy and transfer tables: fields and
        # hash once, hash() and == from the base
        t = (self.owner, self.generation, self.key, self.pool, self.slot)
        object.__setattr__(self, "_t", t)
        object.__setattr__(self, "_h", hash(t))

    __eq__ = _RecordBase.__eq__
    __ne__ = _RecordBase.__ne__
    __hash__ = _RecordBase.__hash__

    def __reduce__(self):
        return (LoadTicket, (self.owner, self.generation, self.key, self.pool, self.slot))


# The records below are built on every layer call (several per routed
# expert): immutable named tuples, which construct in a fraction of a frozen
# dataclass's time.

class UseHandle(NamedTuple):
    ticket: LoadTicket
    serial: int


class EntryView(NamedTuple):
    key: ExpertKey
    nbytes: int
    pool: str
    state: str           # "loading", "ready" or "in_use"
    ticket: LoadTicket
    submitted: bool
    users: int
    origin: str
    used: bool
    expired: bool


class DemandObservation(NamedTuple):
    key: ExpertKey
    tokens: int
    valid_tokens: int
    nbytes: int
    state_at_reveal: str
    pool_at_reveal: str | None
    hit_source: str | None   # "history", "fresh_prefetch", "fresh_refresh" or None

    @property
    def ready_hit(self):
        return self.hit_source is not None


# the hot loops build these from a field tuple in one C call, without the
# Python-level __new__ a NamedTuple class generates
_new_use_handle = partial(tuple.__new__, UseHandle)
_new_observation = partial(tuple.__new__, DemandObservation)


@dataclass(frozen=True)
class RetentionHint:
    source: DemandID
    target: DemandID
    keys: frozenset


# ---------------------------------------------------------------- internals

RESERVED, IN_FLIGHT, READY = "reserved", "in_flight", "ready"

# counter of a ready hit by the source of the copy it hit
_HIT_KIND = {"history": "history_ready_hits", "fresh_prefetch": "fresh_prefetch_hits",
             "fresh_refresh": "fresh_refresh_hits"}


@dataclass
class _Residency:
    """One device copy: its ticket, lifecycle phase and current holders."""
    ticket: LoadTicket
    nbytes: int
    origin: str
    phase: str = RESERVED
    holders: set = field(default_factory=set)
    used: bool = False
    expired: bool = False

    @property
    def state(self):
        if self.holders:
            return "in_use"
        return "ready" if self.phase == READY else "loading"


@dataclass
class _Reveal:
    identity: DemandID
    counts: tuple
    valid: dict
    observations: tuple
    open_keys: set


def _order(key):
    """ExpertKey order as a plain tuple (the dataclass orders by these fields
    in this order): sorting and bisecting on it compares in C."""
    return key._t


def _order_item(item):
    return _order(item[0])


class _Ranking:
    """Keys ordered by (rank, key): one sorted bucket per rank value (holding
    the keys' field tuples) and the sorted list of ranks that have a
    non-empty bucket."""

    def __init__(self):
        self._rank_of = {}
        self._buckets = {}
        self._ranks = []
        self._key_of = {}

    def __contains__(self, key):
        return key in self._rank_of

    def __len__(self):
        return len(self._rank_of)

    def put(self, key, rank):
        rank_of = self._rank_of
        old = rank_of.get(key)
        if old == rank:
            return
        if old is not None:
            self.discard(key)
        bucket = self._buckets.get(rank)
        if bucket is None:
            bucket = self._buckets[rank] = []
            bisect.insort(self._ranks, rank)
        t = key._t   # _order(key), inline on this path
        bisect.insort(bucket, t)
        self._key_of[t] = key
        rank_of[key] = rank

    def put_new(self, keys, rank):
        """put(key, rank) of each key, none of them in this ranking yet, in
        one pass over the rank's bucket."""
        bucket = self._buckets.get(rank)
        if bucket is None:
            bucket = self._buckets[rank] = []
            bisect.insort(self._ranks, rank)
        key_of, rank_of = self._key_of, self._rank_of
        for key in keys:
            t = key._t
            key_of[t] = key
            rank_of[key] = rank
            bucket.append(t)
        bucket.sort()

    def discard(self, key):
        rank = self._rank_of.pop(key, None)
        if rank is None:
            return
        bucket = self._buckets[rank]
        t = key._t
        del bucket[bisect.bisect_left(bucket, t)]
        del self._key_of[t]
        if not bucket:
            del self._buckets[rank]
            del self._ranks[bisect.bisect_left(self._ranks, rank)]

    def ascending(self):
        for rank in list(self._ranks):
            for t in list(self._buckets.get(rank, ())):
                yield self._key_of[t]

    def clear(self):
        self._rank_of.clear()
        self._buckets.clear()
        self._ranks.clear()
        self._key_of.clear()


class ExpertCache:
    """Residency ledger with LRU, LFU or static replacement and staging fallback."""

    POLICIES = ("static", "LRU", "LFU")
    ORIGINS = ("initial", "demand", "prefetch")

    def __init__(self, expert_bytes, cache_bytes, staging_slot_bytes, *, policy="LRU", initial_hotset=()):
        _require_int(cache_bytes, "cache_bytes")
        registry = dict(expert_bytes)
        if not registry or not all(isinstance(k, ExpertKey) for k in registry):
            raise CacheError("expert_bytes must map every ExpertKey to its byte size")
        for n in registry.values():
            _require_int(n, "expert bytes", 1)
        slots = tuple(staging_slot_bytes)
        if not slots:
            raise CacheError("the ledger needs at least one demand staging slot")
        for n in slots:
            _require_int(n, "staging slot bytes", 1)
        if max(slots) < max(registry.values()):
            raise CacheError("no staging slot holds the largest expert, so a miss could never be served")
        hot = tuple(initial_hotset)
        if len(set(hot)) != len(hot) or not set(hot) <= registry.keys():
            raise CacheError("the initial hot set must list distinct registered experts")
        if sum(registry[k] for k in hot) > cache_bytes:
            raise CacheError("the initial hot set does not fit the cache budget")
        if policy not in self.POLICIES:
            raise CacheError(f"policy must be one of {self.POLICIES}")
        self.expert_bytes = MappingProxyType(registry)
        self.cache_bytes = cache_bytes
        self.staging_slot_bytes = slots
        self.policy = policy
        self.initial_hotset = frozenset(hot)
        self._owner = uuid4().hex
        self._serials = itertools.count(1)      # tickets and use handles; never restarts
        self._copies = {}
        self._staging_busy = set()
        self._cache_charged = 0
        self._retired = []
        self._reveal = None
        self._closed = {}                       # request -> last closed (step, layer)
        self._tick = 0                          # one per revealed layer demand
        self._last_tick = {}
        self._times_demanded = Counter()
        self._counters = Counter()
        self._unprotected = _Ranking()
        self._protected_rank = _Ranking()
        self._ranked = {}                       # key -> the ranking that holds it
        self._protected = frozenset()
        self._hint = None

    # ------------------------------------------------------------ lookups

    def _registered(self, key):
        if key not in self.expert_bytes:
            raise CacheError(f"unregistered expert {key!r}")

    def _copy_for(self, ticket):
        copy = self._copies.get(ticket.key)
        if copy is None or (copy.ticket is not ticket and copy.ticket != ticket):
            raise CacheError("the ticket belongs to no live copy of this ledger")
        return copy

    def _open(self, key):
        return self._reveal is not None and key in self._reveal.open_keys

    def _require_open(self, key):
        self._registered(key)
        if not self._open(key):
            raise CacheError(f"{key!r} is not an unfinished expert of the active demand")

    def lookup(self, key):
        """The copy of `key` as it is now (None if absent); observing is not a demand."""
        self._registered(key)
        c = self._copies.get(key)
        if c is None:
            return None
        return EntryView(key, c.nbytes, c.ticket.pool, c.state, c.ticket, c.phase != RESERVED, len(c.holders),
                         c.origin, c.used, c.expired)

    def residency(self, key):
        """(state, ticket) of the copy of `key` as lookup() would show them,
        or None if it has no copy; builds no view."""
        c = self._copies.get(key)
        if c is None:
            self._registered(key)
            return None
        return ("in_use" if c.holders else "ready" if c.phase == READY else "loading"), c.ticket

    def ready_in_cache(self, key):
        """Whether lookup(key) would show state 'ready' (landed, not held) in
        pool 'cache', without building the view."""
        c = self._copies.get(key)
        if c is None:
            self._registered(key)
            return False
        return not c.holders and c.phase == READY and c.ticket.pool == "cache"

    @property
    def resident_payload_bytes(self):
        return self._cache_charged

    @property
    def active_demand(self):
        return None if self._reveal is None else self._reveal.identity

    @property
    def unfinished_demand_keys(self):
        return () if self._reveal is None else tuple(sorted(self._reveal.open_keys, key=_order))

    @property
    def retention_hint(self):
        return self._hint

    def stats(self):
        """Event counters (counts and bytes of ledger events, never times)."""
        return dict(self._counters)

    def memory(self):
        staged = [c for c in self._copies.values() if c.ticket.pool == "demand_staging"]
        return dict(cache_capacity_bytes=self.cache_bytes, cache_payload_bytes=self._cache_charged,
                    staging_reserved_bytes=sum(self.staging_slot_bytes),
                    staging_payload_bytes=sum(c.nbytes for c in staged), staging_occupied_slots=len(staged),
                    expert_reserved_bytes=self.cache_bytes + sum(self.staging_slot_bytes),
                    physical_allocation="executor_responsibility_not_measured_here")

    def prefetch_inventory(self):
        """Speculative copies by outcome: counts and bytes."""
        spec = [c for c in self._copies.values() if c.origin == "prefetch"]
        groups = dict(unused_ready=[c for c in spec if c.phase == READY and not c.used],
                      unused_loading=[c for c in spec if c.phase != READY and not c.used],
                      unused_expired=[c for c in spec if c.expired and not c.used],
                      used_resident=[c for c in spec if c.used])
        out = {}
        for name, members in groups.items():
            out[f"{name}_copies"] = len(members)
            out[f"{name}_bytes"] = sum(c.nbytes for c in members)
        return out

    def demand_frequency(self, key):
        self._registered(key)
        return self._times_demanded[key]

    def take_retired(self):
        """Tickets whose device storage the executor may now free or reuse."""
        out, self._retired = tuple(self._retired), []
        return out

    # ------------------------------------------------------------ replacement

    def _evictable(self, key, c):
        return (self.policy in ("LRU", "LFU") and c.ticket.pool == "cache" and c.phase == READY
                and not c.holders and not self._open(key))

    def _rank(self, key):
        tick = self._last_tick.get(key, 0)
        return (self._times_demanded[key], tick) if self.policy == "LFU" else (tick,)

    def _is_protected(self, key):
        return key in self._protected or (self._hint is not None and key in self._hint.keys)

    def _unrank(self, key):
        home = self._ranked.pop(key, None)
        if home is not None:
            home.discard(key)

    def _reindex(self, key):
        """Place `key` in the ranking its copy belongs to now (or in none).
        (_evictable, _is_protected and _rank, inline: every release and
        retention change passes here.)"""
        c = self._copies.get(key)
        target = None
        r = self._reveal
        if (c is not None and self.policy != "static" and c.ticket.pool == "cache" and c.phase == READY
                and not c.holders and (r is None or key not in r.open_keys)):
            hint = self._hint
            target = (self._protected_rank if key in self._protected or (hint is not None and key in hint.keys)
                      else self._unprotected)
        ranked = self._ranked
        home = ranked.get(key)
        if home is not None and home is not target:
            home.discard(key)
            del ranked[key]
        if target is not None:
            tick = self._last_tick.get(key, 0)
            target.put(key, (self._times_demanded[key], tick) if self.policy == "LFU" else (tick,))
            ranked[key] = target

    def _reindex_many(self, keys):
        """_reindex of each key (distinct keys, none in a ranking yet unless
        noted there): the keys that join a ranking at one rank go into its
        bucket in one pass instead of one insertion each."""
        ranked, copies, r, hint = self._ranked, self._copies, self._reveal, self._hint
        replacing, lfu = self.policy != "static", self.policy == "LFU"
        groups = {}
        for key in keys:
            if key in ranked:
                self._reindex(key)
                continue
            c = copies.get(key)
            if (c is None or not replacing or c.ticket.pool != "cache" or c.phase != READY or c.holders
                    or (r is not None and key in r.open_keys)):
                continue
            target = (self._protected_rank if key in self._protected or (hint is not None and key in hint.keys)
                      else self._unprotected)
            tick = self._last_tick.get(key, 0)
            rank = (self._times_demanded[key], tick) if lfu else (tick,)
            group = groups.get((id(target), rank))
            if group is None:
                group = groups[(id(target), rank)] = (target, rank, [])
            group[2].append(key)
            ranked[key] = target
        for target, rank, members in groups.values():
            target.put_new(members, rank)

    def _choose_victims(self, size):
        """Cheapest evictable copies freeing room for `size` more bytes, or
        None if even all of them would not suffice (nothing is changed)."""
        short = self._cache_charged + size - self.cache_bytes
        if short <= 0:
            return []
        chosen = []
        for ranking in (self._unprotected, self._protected_rank):
            for key in ranking.ascending():
                chosen.append(key)
                short -= self._copies[key].nbytes
                if short <= 0:
                    return chosen
        return None

    def _drop(self, key):
        c = self._copies.pop(key)
        self._unrank(key)
        if c.ticket.pool == "cache":
            self._cache_charged -= c.nbytes
        else:
            self._staging_busy.discard(c.ticket.slot)
        self._retired.append(c.ticket)
        return c

    def _evict_now(self, key):
        c = self._drop(key)
        self._counters["evictions"] += 1
        self._counters["evicted_bytes"] += c.nbytes
        if c.origin == "prefetch" and not c.used:
            self._counters["unused_prefetch_evictions"] += 1

    def evict(self, key):
        self._registered(key)
        c = self._copies.get(key)
        if c is None or not self._evictable(key, c):
            raise CacheError("only a ready, unheld, cached copy outside the active demand can be evicted")
        self._evict_now(key)

    def set_protected(self, keys):
        """Soft preference: these copies are evicted only after every other
        one (e.g. a next-layer forecast); replaces the previous set."""
        keys = frozenset(keys)
        for key in keys:
            self._registered(key)
        before, self._protected = self._protected, keys
        for key in before | keys:
            self._reindex(key)

    def set_retention_hint(self, source, target, keys):
        """Protect forecast copies of the next layer of the active demand until
        the next reveal (LRU only; cache.py:286-313 sets the same horizon).
        Returns False when the same hint is already set."""
        if (self.policy != "LRU" or self._reveal is None or self._reveal.identity != source
                or not isinstance(target, DemandID)
                or target != DemandID(source.request, source.step, source.layer + 1)):
            raise CacheError("a retention hint needs an LRU ledger, the active demand as source and its next layer "
                             "as target")
        keys = tuple(keys)
        if len(set(keys)) != len(keys):
            raise CacheError("retention keys must be distinct")
        for key in keys:
            self._registered(key)
            if key.layer != target.layer:
                raise CacheError("a retention key must belong to the target layer")
        hint = RetentionHint(source, target, frozenset(keys))
        if self._hint is not None:
            if self._hint == hint:
                return False
            raise CacheError("a different retention hint is already set")
        self._hint = hint
        for key in hint.keys:
            self._reindex(key)
        self._counters["retention_hint_updates"] += 1
        self._counters["retention_hint_candidates"] += len(keys)
        return True

    def _drop_hint(self):
        if self._hint is None:
            return False
        keys, self._hint = self._hint.keys, None
        for key in keys:
            self._reindex(key)
        self._counters["retention_hint_expirations"] += 1
        return True

    def clear_retention_hint(self, request):
        if self._reveal is not None or request not in self._closed:
            raise CacheError("a hint is cleared only after its request's demand closed")
        if self._hint is not None and self._hint.source.request != request:
            raise CacheError("the retention hint belongs to another request")
        return self._drop_hint()

    # ------------------------------------------------------------ demand

    def on_demand(self, identity, token_counts, *, role="true", valid_token_counts=None):
        """Reveal the experts one (request, step, layer) routes to and how many
        tokens each serves; returns one observation per expert (sorted by key).
        Repeating the active reveal with identical counts returns it again."""
        if role != "true" or not isinstance(identity, DemandID):
            raise CacheError("only a true routing reveals demand")
        if not isinstance(token_counts, Mapping):
            raise CacheError("token counts must be a mapping expert -> tokens")
        counts = tuple(sorted(dict(token_counts).items(), key=_order_item))
        if not counts:
            raise CacheError("an empty demand cannot be revealed")
        registry, layer = self.expert_bytes, identity.layer
        for key, n in counts:
            if key not in registry:
                self._registered(key)
            if key.layer != layer:
                raise CacheError("every demanded expert belongs to the revealed layer")
            if type(n) is not int or n < 1:
                _require_int(n, "tokens per expert", 1)
        physical = dict(counts)
        if valid_token_counts is not None and not isinstance(valid_token_counts, Mapping):
            raise CacheError("valid token counts must be a mapping")
        valid = dict(physical) if valid_token_counts is None else dict(valid_token_counts)
        if valid_token_counts is not None:   # the physical counts were checked above
            for key, n in valid.items():
                if key not in physical:
                    raise CacheError("a valid count names an expert outside the demand")
                _require_int(n, "valid tokens per expert", 1)
                if n > physical[key]:
                    raise CacheError("valid tokens exceed routed tokens")
        if self._reveal is not None:
            r = self._reveal
            if r.identity == identity and r.counts == counts and r.valid == valid:
                return r.observations
            raise CacheError("another layer demand is still open")
        last = self._closed.get(identity.request)
        if last is not None and (identity.step, identity.layer) <= last:
            raise CacheError("demands of a request must arrive in increasing (step, layer) order")
        if not self._counters["physical_layer_events"]:
            missing = [k for k in self.initial_hotset
                       if k not in self._copies or self._copies[k].phase != READY]
            if missing:
                raise CacheError("the initial hot set must be loaded before the first demand")
        self._drop_hint()   # a hint covers one layer ahead only
        copies, valid_get = self._copies, valid.get
        obs = []
        for key, n in counts:   # _observe_copy, inline
            c = copies.get(key)
            if c is None:
                obs.append(_new_observation((key, n, valid_get(key, 0), registry[key], "absent", None, None)))
                continue
            phase = c.phase
            source = None
            if phase == READY:
                source = (f"fresh_{c.origin}" if c.origin in ("prefetch", "refresh") and not c.used
                          else "history")
            obs.append(_new_observation((key, n, valid_get(key, 0), registry[key],
                                         "in_use" if c.holders else "ready" if phase == READY else "loading",
                                         c.ticket.pool, source)))
        observations = tuple(obs)
        self._tick += 1
        self._account_reveal(observations, self._tick)
        self._reveal = _Reveal(identity, counts, valid, observations, set(physical))
        # open experts cannot be evicted: they leave the rankings (what
        # _reindex does for a key that is not evictable)
        ranked = self._ranked
        for key in physical:
            home = ranked.pop(key, None)
            if home is not None:
                home.discard(key)
        return observations

    def _observe(self, key, tokens, valid_tokens):
        return self._observe_copy(key, tokens, valid_tokens, self._copies.get(key), self.expert_bytes[key])

    @staticmethod
    def _observe_copy(key, tokens, valid_tokens, c, nbytes):
        """The observation of `key` at its reveal, given its copy `c` (or None)."""
        if c is None:
            return DemandObservation(key, tokens, valid_tokens, nbytes, "absent", None, None)
        source = None
        if c.phase == READY:
            fresh = c.origin in ("prefetch", "refresh") and not c.used
            source = f"fresh_{c.origin}" if fresh else "history"
        state = "in_use" if c.holders else "ready" if c.phase == READY else "loading"
        return DemandObservation(key, tokens, valid_tokens, nbytes, state, c.ticket.pool, source)

    def _account_reveal(self, observations, tick):
        """Counters, demand frequencies and last-demand ticks of one reveal.
        Sums per counter first, each counter then updated once; a counter is
        touched (and so listed in stats()) under the same conditions, and in
        the same order, as when it is counted per observation."""
        n = self._counters
        n["physical_layer_events"] += 1
        n["demand_events"] += int(any(o[2] for o in observations))
        demanded, last_tick = self._times_demanded, self._last_tick
        tokens = padding = ready = 0
        pad_only = demands = d_tokens = d_bytes = 0
        hits = hit_tokens = hit_bytes = 0
        kinds = {}
        for key, t, valid, nbytes, state, pool, source in observations:
            tokens += t
            padding += t - valid
            hit = source is not None
            ready += hit
            if not valid:
                pad_only += 1
                continue
            demanded[key] += 1
            last_tick[key] = tick
            demands += 1
            d_tokens += valid
            d_bytes += nbytes
            if hit:
                hits += 1
                hit_tokens += valid
                hit_bytes += nbytes
                for name in (_HIT_KIND[source], "cache_resident_hits" if pool == "cache" else "staging_ready_hits"):
                    kinds[name] = kinds.get(name, 0) + 1
            else:
                name = "loading_misses" if state in ("loading", "in_use") else "absent_misses"
                kinds[name] = kinds.get(name, 0) + 1
        n["physical_expert_demands"] += len(observations)
        n["physical_demand_tokens"] += tokens
        n["padding_token_assignments"] += padding
        n["physical_ready_hits"] += ready
        if pad_only:
            n["padding_only_expert_demands"] += pad_only
        if demands:
            n["expert_demands"] += demands
            n["demand_tokens"] += d_tokens
            n["demand_bytes"] += d_bytes
        if hits:
            n["ready_hits"] += hits
            n["ready_hit_tokens"] += hit_tokens
            n["ready_hit_bytes"] += hit_bytes
        for name, v in kinds.items():
            n[name] += v

    def end_demand(self, identity):
        r = self._reveal
        if r is None or r.identity != identity:
            raise CacheError("that demand is not the open one")
        if r.open_keys:
            raise CacheError("the demand still has unfinished experts")
        self._closed[identity.request] = (identity.step, identity.layer)
        self._reveal = None

    # ------------------------------------------------------------ transfers

    def _free_staging_slot(self, size):
        fits = [(cap, i) for i, cap in enumerate(self.staging_slot_bytes)
                if cap >= size and i not in self._staging_busy]
        return min(fits)[1] if fits else None

    def begin_load(self, key, *, origin="demand", admit=True):
        """Reserve one device copy of `key` (the existing ticket if it has one).
        initial: the pre-run hot set; demand: an open expert, into the cache or
        (admit=False, or no room) a staging slot; prefetch: a cache copy of an
        expert outside the open demand."""
        self._registered(key)
        if origin not in self.ORIGINS:
            raise CacheError(f"load origin must be one of {self.ORIGINS}")
        if type(admit) is not bool or (not admit and origin != "demand"):
            raise CacheError("admit=False applies to demand loads only")
        if origin == "demand":
            self._require_open(key)
        elif origin == "initial":
            if self._counters["physical_layer_events"] or self._reveal is not None or key not in self.initial_hotset:
                raise CacheError("initial loads are the declared hot set, before any demand")
        elif self.policy == "static" or self._open(key):
            raise CacheError("prefetch needs a replacing policy and an expert outside the open demand")
        if key in self._copies:
            return self._copies[key].ticket
        size = self.expert_bytes[key]
        victims = None
        if admit and (self.policy != "static" or origin == "initial"):
            victims = self._choose_victims(size)
        slot = None
        if victims is not None:
            pool = "cache"
        elif origin == "demand":
            slot = self._free_staging_slot(size)
            if slot is None:
                raise CapacityBlocked("every fitting staging slot is busy; finish a transfer or use first")
            pool = "demand_staging"
        else:
            raise CapacityBlocked("the cache has no evictable room and speculation may not use staging")
        for victim in victims or ():
            self._evict_now(victim)
        ticket = LoadTicket(self._owner, next(self._serials), key, pool, slot)
        self._copies[key] = _Residency(ticket, size, origin)
        if pool == "cache":
            self._cache_charged += size
        else:
            self._staging_busy.add(slot)
        return ticket

    def submit(self, ticket):
        """The transfer of this reservation has been issued."""
        c = self._copy_for(ticket)
        if c.phase != RESERVED:
            raise CacheError("this transfer was already submitted")
        if c.origin == "prefetch" and self._open(ticket.key):
            # the forecast was overtaken by the true demand: its copy is demand work
            c.origin, c.expired = "demand", True
        c.phase = IN_FLIGHT
        self._counters[f"{c.origin}_loads_submitted"] += 1
        self._counters["h2d_bytes_submitted"] += c.nbytes
        if c.origin == "demand" and self._reveal is not None and ticket.key not in self._reveal.valid:
            self._counters["padding_only_h2d_bytes_submitted"] += c.nbytes

    def complete_load(self, ticket):
        """The transfer of this exact copy has landed."""
        c = self._copy_for(ticket)
        if c.phase != IN_FLIGHT:
            raise CacheError("only a submitted, unfinished transfer can complete")
        c.phase = READY
        self._counters["h2d_bytes_completed"] += c.nbytes
        self._reindex(ticket.key)

    def expire_prefetch(self, ticket):
        """Give up a forecast copy: an unsubmitted one outside the open demand
        is dropped; one the demand adopted becomes demand work."""
        c = self._copy_for(ticket)
        if c.expired:
            return False
        if c.origin != "prefetch":
            raise CacheError("only speculative copies expire")
        c.expired = True
        self._counters["prefetch_expirations"] += 1
        if c.phase == RESERVED:
            if not self._open(ticket.key):
                self._drop(ticket.key)
                return True
            c.origin = "demand"
        return False

    # ------------------------------------------------------------ uses

    def acquire(self, key):
        """Hold a ready copy of an open expert for a computation."""
        return self.acquire_many((key,))[0]

    def acquire_many(self, keys):
        """acquire() of each key in order, in one call: the same checks, the
        same use serials (a failing key leaves the earlier ones held, as a
        sequence of acquire() calls would)."""
        registry, copies, serials = self.expert_bytes, self._copies, self._serials
        r = self._reveal
        handles = []
        for key in keys:
            if key not in registry:
                self._registered(key)
            if r is None or key not in r.open_keys:
                raise CacheError(f"{key!r} is not an unfinished expert of the active demand")
            c = copies.get(key)
            if c is None or c.phase != READY:
                raise CacheError("no ready copy to compute with (a loading copy is not a hit)")
            handle = _new_use_handle((c.ticket, next(serials)))
            c.holders.add(handle.serial)
            # an open expert is in no ranking (the reveal took it out and only
            # a closed one goes back), so holding it changes no ranking
            handles.append(handle)
        return tuple(handles)

    def release(self, handle):
        """The computation holding this copy has completed; the last release of
        an expert completes it for the open demand (a staged copy then leaves)."""
        self.release_many((handle,))

    def release_many(self, handles):
        """release() of each handle in order, in one call (same checks and
        transitions; a failing handle leaves the earlier ones released)."""
        r, counters, copies = self._reveal, self._counters, self._copies
        completed = []   # cache-pool experts completed here, re-ranked together
        try:
            for handle in handles:
                ticket = handle.ticket
                key = ticket.key
                c = copies.get(key)   # _copy_for, inline
                if c is None or (c.ticket is not ticket and c.ticket != ticket):
                    raise CacheError("the ticket belongs to no live copy of this ledger")
                serial, holders = handle.serial, c.holders
                if serial not in holders:
                    raise CacheError("the use handle is stale, foreign or already released")
                holders.discard(serial)
                valid = key in r.valid
                c.used = c.used or valid
                if holders:
                    continue
                r.open_keys.discard(key)
                counters["gpu_completed_experts"] += 1
                counters["gpu_completed_valid_experts"] += int(valid)
                if c.ticket.pool == "demand_staging":
                    self._drop(key)
                else:
                    completed.append(key)
        finally:
            if completed:
                self._reindex_many(completed)

    def finish_cpu(self, key):
        """The expert of the open demand was computed on the CPU from its master."""
        self._require_open(key)
        c = self._copies.get(key)
        if c is not None:
            if c.holders or (c.origin == "demand" and c.phase != READY):
                raise CacheError("a held copy or a demand transfer in flight cannot turn into CPU work")
            if c.ticket.pool == "demand_staging":
                raise CacheError("a staged copy is consumed by its GPU release")
        self._reveal.open_keys.discard(key)
        self._counters["cpu_completed_experts"] += 1
        self._counters["cpu_completed_valid_experts"] += int(key in self._reveal.valid)
        self._reindex(key)

    def reset(self):
        """Forget residency, history and counters once nothing is in flight or held."""
        if self._reveal is not None or any(c.phase != READY or c.holders for c in self._copies.values()):
            raise CacheError("reset needs no open demand, transfer or use")
        self._retired.extend(c.ticket for c in self._copies.values())
        self._copies.clear()
        self._staging_busy.clear()
        self._cache_charged = 0
        self._closed.clear()
        self._last_tick.clear()
        self._times_demanded.clear()
        self._counters.clear()
        self._unprotected.clear()
        self._protected_rank.clear()
        self._ranked.clear()
        self._hint = None
