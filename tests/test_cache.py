"""Residency ledger (pdscope_amd.cache) lifecycle rules, on the CPU.

The rules follow expertbench/cache.py:136-662: staging fallback to the
smallest free fitting slot (:531-537), CapacityBlocked without side effects,
release-frees-staging (:621-624), LRU/LFU eviction, and CacheError on every
illegal transition.
"""
import random

import pytest

from pdscope_amd.cache import CacheError, CapacityBlocked, DemandID, ExpertCache, ExpertKey

K = lambda l, e: ExpertKey(l, e, "bf16")  # noqa: E731


def make(n_layers=2, E=8, size=10, cache_slots=3, staging=(10, 10), hot=(), policy="LRU"):
    sizes = {K(l, e): size for l in range(n_layers) for e in range(E)}
    return ExpertCache(sizes, cache_slots * size, list(staging), policy=policy, initial_hotset=hot)


def load_ready(c, key, **kw):
    t = c.begin_load(key, **kw)
    c.submit(t)
    c.complete_load(t)
    return t


def test_initial_hotset_then_demand_hits():
    c = make(hot=(K(0, 0), K(0, 1)))
    with pytest.raises(CacheError):  # hotset must be loaded first
        c.on_demand(DemandID("r", 0, 0), {K(0, 0): 3})
    for k in (K(0, 0), K(0, 1)):
        load_ready(c, k, origin="initial")
    obs = c.on_demand(DemandID("r", 0, 0), {K(0, 0): 3, K(0, 5): 1})
    assert [o.ready_hit for o in obs] == [True, False]
    h = c.acquire(K(0, 0))
    c.release(h)
    assert c.unfinished_demand_keys == (K(0, 5),)
    with pytest.raises(CacheError):
        c.end_demand(DemandID("r", 0, 0))
    c.finish_cpu(K(0, 5))
    c.end_demand(DemandID("r", 0, 0))
    st = c.stats()
    assert st["gpu_completed_experts"] == 1 and st["cpu_completed_experts"] == 1


def test_staging_fallback_picks_smallest_free_slot_and_frees_on_release():
    c = make(cache_slots=0, staging=(30, 10, 10))
    c.on_demand(DemandID("r", 0, 0), {K(0, 1): 1, K(0, 2): 1, K(0, 3): 1, K(0, 4): 1})
    t1 = c.begin_load(K(0, 1))
    t2 = c.begin_load(K(0, 2))
    t3 = c.begin_load(K(0, 3))
    assert (t1.pool, t1.slot) == ("demand_staging", 1)   # min((capacity, index))
    assert (t2.slot, t3.slot) == (2, 0)
    with pytest.raises(CapacityBlocked):
        c.begin_load(K(0, 4))
    assert c.lookup(K(0, 4)) is None                       # no side effect
    c.submit(t1)
    c.complete_load(t1)
    h = c.acquire(K(0, 1))
    c.release(h)
    assert c.lookup(K(0, 1)) is None                       # staged misses never stay
    assert t1 in c.take_retired()
    t4 = c.begin_load(K(0, 4))
    assert t4.slot == 1


def test_lru_eviction_order_and_protection():
    c = make(cache_slots=2, staging=(10,))
    c.on_demand(DemandID("r", 0, 0), {K(0, 0): 1})
    load_ready(c, K(0, 0))
    c.release(c.acquire(K(0, 0)))
    c.end_demand(DemandID("r", 0, 0))
    c.on_demand(DemandID("r", 0, 1), {K(1, 0): 1})
    load_ready(c, K(1, 0))
    c.release(c.acquire(K(1, 0)))
    c.end_demand(DemandID("r", 0, 1))
    # cache full (2 slots): a prefetch evicts the least recently demanded copy
    load_ready(c, K(1, 5), origin="prefetch")
    assert c.lookup(K(0, 0)) is None and c.lookup(K(1, 0)) is not None
    assert c.stats()["evictions"] == 1
    # protected copies go last
    c.set_protected([K(1, 0)])
    load_ready(c, K(1, 6), origin="prefetch")
    assert c.lookup(K(1, 0)) is not None and c.lookup(K(1, 5)) is None


def test_lfu_prefers_rarely_used():
    c = make(cache_slots=2, staging=(10,), policy="LFU")
    for step, key in enumerate([K(0, 0), K(0, 0), K(0, 1)]):
        c.on_demand(DemandID("r", step, 0), {key: 1})
        if c.lookup(key) is None:
            load_ready(c, key)
        c.release(c.acquire(key))
        c.end_demand(DemandID("r", step, 0))
    # K(0,0) was demanded twice, K(0,1) once but more recently: LFU evicts K(0,1)
    c.on_demand(DemandID("r", 3, 0), {K(0, 7): 1})
    t = c.begin_load(K(0, 7))
    assert t.pool == "cache" and c.lookup(K(0, 1)) is None and c.lookup(K(0, 0)) is not None


def test_static_policy_never_evicts_and_misses_use_staging():
    c = make(cache_slots=1, staging=(10,), hot=(K(0, 0),), policy="static")
    load_ready(c, K(0, 0), origin="initial")
    c.on_demand(DemandID("r", 0, 0), {K(0, 3): 1})
    t = c.begin_load(K(0, 3))
    assert t.pool == "demand_staging"
    with pytest.raises(CacheError):
        c.begin_load(K(1, 2), origin="prefetch")


@pytest.mark.parametrize("bad", ["acquire_loading", "complete_unsubmitted", "double_submit", "foreign_ticket",
                                 "prefetch_revealed", "late_initial", "out_of_order", "conflicting_demand",
                                 "release_twice", "evict_in_use"])
def test_illegal_transitions_raise(bad):
    c = make()
    c.on_demand(DemandID("r", 1, 0), {K(0, 1): 1, K(0, 2): 2})
    t = c.begin_load(K(0, 1))
    with pytest.raises(CacheError):
        if bad == "acquire_loading":
            c.acquire(K(0, 1))
        elif bad == "complete_unsubmitted":
            c.complete_load(t)
        elif bad == "double_submit":
            c.submit(t)
            c.submit(t)
        elif bad == "foreign_ticket":
            other = make()
            other.on_demand(DemandID("r", 1, 0), {K(0, 1): 1})
            c.submit(other.begin_load(K(0, 1)))
        elif bad == "prefetch_revealed":
            c.begin_load(K(0, 2), origin="prefetch")
        elif bad == "late_initial":
            c.begin_load(K(1, 1), origin="initial")
        elif bad == "out_of_order":
            c.submit(t)
            c.complete_load(t)
            c.release(c.acquire(K(0, 1)))
            c.finish_cpu(K(0, 2))
            c.end_demand(DemandID("r", 1, 0))
            c.on_demand(DemandID("r", 0, 1), {K(1, 1): 1})
        elif bad == "conflicting_demand":
            c.on_demand(DemandID("r", 1, 0), {K(0, 1): 5})
        elif bad == "release_twice":
            c.submit(t)
            c.complete_load(t)
            h = c.acquire(K(0, 1))
            c.release(h)
            c.release(h)
        elif bad == "evict_in_use":
            c.submit(t)
            c.complete_load(t)
            c.acquire(K(0, 1))
            c.evict(K(0, 1))


def test_random_lifecycles_keep_invariants():
    rng = random.Random(5)
    for trial in range(30):
        E, size, slots = 12, 10, rng.randint(1, 5)
        c = make(E=E, cache_slots=slots, staging=(10,) * rng.randint(1, 4), policy=rng.choice(["LRU", "LFU"]))
        for step in range(12):
            layer = step % 2
            demand = {K(layer, e): rng.randint(1, 4) for e in rng.sample(range(E), rng.randint(1, 5))}
            c.on_demand(DemandID("q", step, layer), demand)
            for key in sorted(demand):
                view = c.lookup(key)
                if view is None:
                    try:
                        t = c.begin_load(key, admit=rng.random() < 0.7)
                    except CapacityBlocked:
                        c.finish_cpu(key)
                        continue
                    c.submit(t)
                    c.complete_load(t)
                elif view.state == "loading":
                    c.complete_load(view.ticket)
                c.release(c.acquire(key))
            c.end_demand(DemandID("q", step, layer))
            mem = c.memory()
            assert mem["cache_payload_bytes"] <= mem["cache_capacity_bytes"]
            assert mem["staging_occupied_slots"] == 0
            if rng.random() < 0.5:
                nxt = K(1 - layer, rng.randrange(E))
                if c.lookup(nxt) is None:
                    try:
                        t = c.begin_load(nxt, origin="prefetch")
                        c.submit(t)
                        c.complete_load(t)
                    except CapacityBlocked:
                        pass
        st = c.stats()
        assert st["h2d_bytes_submitted"] == st["h2d_bytes_completed"]
        assert (st.get("gpu_completed_experts", 0) + st.get("cpu_completed_experts", 0)
                == st["physical_expert_demands"])


def _brute_force_victims(c, size, protected):
    """Victims by the policy's definition, recomputed from scratch: every
    ready, unheld cache copy outside the open demand, ordered by (protected,
    LRU tick | LFU (frequency, tick), key), taken until the new copy fits."""
    short = c.memory()["cache_payload_bytes"] + size - c.cache_bytes
    if short <= 0:
        return []
    open_keys = set(c.unfinished_demand_keys)
    cands = []
    for key in c.expert_bytes:
        v = c.lookup(key)
        if v is None or v.pool != "cache" or v.state != "ready" or key in open_keys:
            continue
        tick = c._last_tick.get(key, 0)
        rank = (c.demand_frequency(key), tick) if c.policy == "LFU" else (tick,)
        cands.append(((key in protected,) + rank + (key,), key))
    out = []
    for _, key in sorted(cands):
        out.append(key)
        short -= c.expert_bytes[key]
        if short <= 0:
            return out
    return None


@pytest.mark.parametrize("policy", ["LRU", "LFU"])
def test_victims_match_brute_force_priority_order(policy):
    rng = random.Random(11 if policy == "LRU" else 12)
    for trial in range(40):
        E, size = 10, 10
        c = make(E=E, cache_slots=rng.randint(1, 5), staging=(10, 10), policy=policy)
        protected = set()
        for step in range(10):
            layer = step % 2
            keys = {K(layer, e): 1 for e in rng.sample(range(E), rng.randint(1, 4))}
            c.on_demand(DemandID("v", step, layer), keys)
            for key in sorted(keys):
                if c.lookup(key) is None:
                    before = {k for k in c.expert_bytes if c.lookup(k) is not None}
                    want = _brute_force_victims(c, size, protected)
                    try:
                        t = c.begin_load(key)
                    except CapacityBlocked:
                        raise AssertionError("a demand load always has a staging fallback here")
                    if t.pool == "cache":
                        gone = before - {k for k in c.expert_bytes if c.lookup(k) is not None}
                        assert want is not None and gone == set(want)
                    else:
                        assert want is None
                    c.submit(t)
                    c.complete_load(t)
                c.release(c.acquire(key))
            c.end_demand(DemandID("v", step, layer))
            if rng.random() < 0.4:
                protected = {K(1 - layer, e) for e in rng.sample(range(E), 2)}
                c.set_protected(protected)
            for _ in range(rng.randint(0, 2)):
                key = K(1 - layer, rng.randrange(E))
                if c.lookup(key) is not None:
                    continue
                before = {k for k in c.expert_bytes if c.lookup(k) is not None}
                want = _brute_force_victims(c, size, protected)
                try:
                    t = c.begin_load(key, origin="prefetch")
                except CapacityBlocked:
                    assert want is None
                    continue
                gone = before - {k for k in c.expert_bytes if c.lookup(k) is not None}
                assert gone == set(want)
                c.submit(t)
                c.complete_load(t)


def test_retention_hint_lasts_one_reveal_and_expire_prefetch():
    c = make(cache_slots=2, staging=(10,))
    c.on_demand(DemandID("r", 0, 0), {K(0, 0): 1})
    load_ready(c, K(0, 0))
    c.release(c.acquire(K(0, 0)))
    # a forecast for layer 1: protected until the next reveal
    t = load_ready(c, K(1, 3), origin="prefetch")
    assert c.set_retention_hint(DemandID("r", 0, 0), DemandID("r", 0, 1), [K(1, 3)])
    assert not c.set_retention_hint(DemandID("r", 0, 0), DemandID("r", 0, 1), [K(1, 3)])
    with pytest.raises(CacheError):   # target must be the next layer of the active demand
        c.set_retention_hint(DemandID("r", 0, 0), DemandID("r", 0, 2), [K(1, 3)])
    c.end_demand(DemandID("r", 0, 0))
    load_ready(c, K(1, 4), origin="prefetch")   # full: evicts K(0,0), not the protected forecast
    assert c.lookup(K(0, 0)) is None and c.lookup(K(1, 3)) is not None
    c.on_demand(DemandID("r", 0, 1), {K(1, 3): 2})
    assert c.retention_hint is None and c.stats()["retention_hint_expirations"] == 1
    assert c.stats()["fresh_prefetch_hits"] == 1
    c.release(c.acquire(K(1, 3)))
    c.end_demand(DemandID("r", 0, 1))
    inv = c.prefetch_inventory()
    assert inv["used_resident_copies"] == 1 and inv["unused_ready_copies"] == 1
    # an unsubmitted forecast outside the open demand is dropped on expiry
    c.on_demand(DemandID("r", 1, 0), {K(0, 1): 1})
    c.finish_cpu(K(0, 1))
    c.end_demand(DemandID("r", 1, 0))
    t5 = c.begin_load(K(1, 5), origin="prefetch")
    assert c.expire_prefetch(t5) and c.lookup(K(1, 5)) is None and t5 in c.take_retired()
    assert t not in c.take_retired()


def test_expert_key_record_contract():
    """ExpertKey stays a frozen, ordered dataclass record: field equality and
    hash, order by (layer, expert, representation), replace/asdict, and a
    pickle round trip that rebuilds its hash in the loading process."""
    import dataclasses
    import pickle
    a, b, c = ExpertKey(1, 2, "bf16"), ExpertKey(1, 2, "bf16"), ExpertKey(1, 10, "bf16")
    assert a == b and a is not b and hash(a) == hash(b) and len({a, b, c}) == 2
    assert a != c and a < c and sorted([c, ExpertKey(0, 99, "bf16"), a])[0] == ExpertKey(0, 99, "bf16")
    assert ExpertKey(1, 2, "a") < ExpertKey(1, 2, "b") and a != (1, 2, "bf16")
    assert dataclasses.replace(a, expert=10) == c
    assert dataclasses.asdict(a) == dict(layer=1, expert=2, representation="bf16")
    r = pickle.loads(pickle.dumps(a))
    assert r == a and hash(r) == hash(a) and {a: 1}[r] == 1
    with pytest.raises(dataclasses.FrozenInstanceError):
        a.layer = 3
    with pytest.raises(CacheError):
        ExpertKey(1, -1, "bf16")


def test_key_records_hash_in_the_native_base():
    """With the package built, ExpertKey and LoadTicket take hash() and ==
    from the C base type pdscope_amd._records.HashedRecord."""
    from pdscope_amd import cache
    from pdscope_amd._records import HashedRecord
    assert cache._RecordBase is HashedRecord
    for cls in (cache.ExpertKey, cache.LoadTicket):
        assert issubclass(cls, HashedRecord) and cls.__hash__ is HashedRecord.__hash__


def test_key_records_keep_their_contract_without_the_native_base():
    """cache.py loaded where pdscope_amd._records cannot be imported falls
    back to a Python base with the same semantics: the record contracts
    hold and a short ledger lifecycle runs."""
    import dataclasses
    import importlib.util
    import pickle
    import sys
    from pathlib import Path

    import pdscope_amd.cache as native
    name = "pdscope_amd._cache_without_records"
    saved = sys.modules.get("pdscope_amd._records")
    sys.modules["pdscope_amd._records"] = None   # the import raises ImportError
    try:
        spec = importlib.util.spec_from_file_location(name, Path(native.__file__))
        mod = importlib.util.module_from_spec(spec)
        sys.modules[name] = mod
        spec.loader.exec_module(mod)
    finally:
        if saved is None:
            del sys.modules["pdscope_amd._records"]
        else:
            sys.modules["pdscope_amd._records"] = saved
    try:
        assert mod._RecordBase.__module__ == name
        K = mod.ExpertKey
        a, b, c = K(1, 2, "bf16"), K(1, 2, "bf16"), K(1, 10, "bf16")
        assert a == b and not (a != b) and hash(a) == hash(b) and len({a, b, c}) == 2
        assert a != c and a < c and a != (1, 2, "bf16") and not (a == (1, 2, "bf16"))
        assert dataclasses.replace(a, expert=10) == c
        r = pickle.loads(pickle.dumps(a))
        assert r == a and hash(r) == hash(a)
        t1 = mod.LoadTicket("o", 3, a, "cache", None)
        t2 = mod.LoadTicket("o", 3, b, "cache", None)
        assert t1 == t2 and hash(t1) == hash(t2) and dataclasses.replace(t1, slot=0) != t1
        # a short lifecycle on the fallback records
        keys = [K(0, e, "bf16") for e in range(4)]
        ledger = mod.ExpertCache({k: 10 for k in keys}, 40, [10], initial_hotset=keys[:2])
        for k in keys[:2]:
            t = ledger.begin_load(k, origin="initial")
            ledger.submit(t)
            ledger.complete_load(t)
        ident = mod.DemandID("r", 1, 0)
        obs = ledger.on_demand(ident, {keys[0]: 2, keys[1]: 1})
        assert [o.state_at_reveal for o in obs] == ["ready", "ready"]
        ledger.release_many(ledger.acquire_many(keys[:2]))
        ledger.end_demand(ident)
        assert ledger.stats()["gpu_completed_experts"] == 2
    finally:
        del sys.modules[name]


def test_load_ticket_record_contract():
    """LoadTicket equality and hash follow its fields, also across a pickle
    round trip and for distinct but equal key objects."""
    import dataclasses
    import pickle
    from pdscope_amd.cache import LoadTicket
    a = LoadTicket("owner", 3, ExpertKey(1, 2, "bf16"), "cache", None)
    b = LoadTicket("owner", 3, ExpertKey(1, 2, "bf16"), "cache", None)
    assert a == b and hash(a) == hash(b) and {a: 1}[b] == 1
    for field, value in (("owner", "x"), ("generation", 4), ("key", ExpertKey(1, 3, "bf16")),
                         ("pool", "demand_staging"), ("slot", 0)):
        assert dataclasses.replace(a, **{field: value}) != a, field
    r = pickle.loads(pickle.dumps(a))
    assert r == a and hash(r) == hash(a)


def test_ready_in_cache_agrees_with_lookup():
    """ready_in_cache(key) is lookup's (state == 'ready' and pool == 'cache')
    through a lifecycle: hot copies, a held copy, a staged miss."""
    sizes = {ExpertKey(0, e, "bf16"): 10 for e in range(4)}
    cache = ExpertCache(sizes, 20, [10], policy="LRU", initial_hotset=[ExpertKey(0, 0, "bf16"), ExpertKey(0, 1, "bf16")])
    for k in cache.initial_hotset:
        t = cache.begin_load(k, origin="initial")
        cache.submit(t)
        cache.complete_load(t)

    def agree():
        for k in sizes:
            v = cache.lookup(k)
            assert cache.ready_in_cache(k) == (v is not None and v.state == "ready" and v.pool == "cache"), k
    agree()
    cache.on_demand(DemandID("r", 0, 0), {ExpertKey(0, 0, "bf16"): 1, ExpertKey(0, 2, "bf16"): 1})
    h = cache.acquire(ExpertKey(0, 0, "bf16"))
    agree()
    t = cache.begin_load(ExpertKey(0, 2, "bf16"), origin="demand", admit=False)
    cache.submit(t)
    agree()
    cache.complete_load(t)
    agree()
    cache.release(h)
    agree()
    with pytest.raises(CacheError):
        cache.ready_in_cache(ExpertKey(0, 9, "bf16"))
