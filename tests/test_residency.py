"""The HBM expert-residency policy against the reference's own LayerLruCache tests
(src/runtime/cache.rs:528-1174), restated over the C ABI (include/urb_residency.h).  Host code
only: no GPU."""
import ctypes
import os
import re

import pytest

from urbilateria_amd import native as N
from urbilateria_amd import residency as R
from urbilateria_amd.residency import LayerLruCache, Telemetry

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
U64_MAX = 2 ** 64 - 1


def test_library_exports_every_declared_residency_symbol():
    text = open(os.path.join(ROOT, "include", "urb_residency.h")).read()
    declared = sorted(set(re.findall(r"\b(urb_lru_[a-z0-9_]+)\s*\(", text)))
    lib = ctypes.CDLL(N.MOE_LIB)
    for name in declared:
        assert hasattr(lib, name), name
    assert set(R.EXPORTS) == set(declared)


def ok(value, nbytes, read):
    return lambda: (value, nbytes, read)


def test_cache_policy_is_independent_of_cached_value_type():
    # cache.rs:531-569
    cache = LayerLruCache(1, 1)
    t = Telemetry()
    first = cache.access(t, 0, 7, ok(10, 4, 3))
    hit = cache.access(t, 0, 7, ok(20, 4, 3))
    second = cache.access(t, 0, 8, ok(30, 8, 6))
    assert (first, hit, second) == (10, 10, 30)
    assert (t.hits, t.misses, t.evictions) == (1, 2, 1)
    assert t.resident_bytes == 8
    assert t.bytes_read == 9


def test_displaced_value_is_returned_without_changing_lru_accounting():
    # cache.rs:571-600
    cache = LayerLruCache(1, 1)
    t = Telemetry()
    cache.access(t, 0, 7, ok(123, 3, 3))
    value, evicted = cache.access_with_evicted(t, 0, 8, ok(45, 2, 2))
    assert value == 45
    assert evicted == 123
    assert t.misses == 2
    assert t.evictions == 1
    assert t.resident_experts == 1
    assert t.resident_bytes == 2
    assert t.bytes_read == 5


def test_concurrent_preload_is_allowed_only_without_eviction():
    # cache.rs:602-619
    cache = LayerLruCache(1, 1)
    t = Telemetry()
    assert cache.can_insert_without_eviction(0, [7, 7])
    assert not cache.can_insert_without_eviction(0, [7, 8])
    cache.access(t, 0, 7, ok(10, 4, 3))
    assert cache.can_insert_without_eviction(0, [7])
    assert not cache.can_insert_without_eviction(0, [8])


def _apply(cache, t, keys):
    for key in keys:
        cache.access(t, 0, key, ok(key, key + 1, 7))


def _snapshot(cache):
    return sorted((e.key, e.last_used, e.value) for e in cache.entries(0))


def _recency(cache):
    return [e.key for e in sorted(cache.entries(0), key=lambda e: (e.last_used, e.key))]


SEEDS = ([], [0, 1], [2, 0, 1, 2], [3, 1, 0, 2])


def _sequences(step=1):
    for encoded in range(0, 4096, step):
        yield [(encoded >> (i * 2)) & 3 for i in range(6)]


def test_protected_grouping_reaches_minimum_reads_and_preserves_future_lru():
    # cache.rs:621-745 (every 6-access sequence over 4 keys, capacities 1-4, four seeds)
    for capacity in range(1, 5):
        for seed in SEEDS:
            for keys in _sequences():
                serial, grouped = LayerLruCache(1, capacity), LayerLruCache(1, capacity)
                a, b = Telemetry(), Telemetry()
                _apply(serial, a, seed)
                _apply(grouped, b, seed)
                initial, initial_clock = _snapshot(grouped), grouped.clock
                missing = sorted({k for k in keys if not grouped.contains(0, k)})
                plan = grouped.grouped_access_plan(0, keys)
                assert _snapshot(grouped) == initial and grouped.clock == initial_clock
                _apply(serial, a, keys)
                if plan is None:
                    continue
                before = b.copy()
                for key in plan.order():
                    value, _retired = grouped.access_grouped_with_evicted(b, plan, key,
                                                                          ok(key, key + 1, 7))
                    assert value == key
                    assert b.resident_experts <= capacity
                grouped.finish_grouped_plan(plan)
                assert b.misses - before.misses == len(missing)
                assert b.bytes_read - before.bytes_read == len(missing) * 7
                assert b.accesses() - before.accesses() == len(plan.order())
                assert b.misses <= a.misses
                assert a.resident_bytes == b.resident_bytes
                assert a.resident_experts == b.resident_experts
                assert _snapshot(serial) == _snapshot(grouped)
                assert serial.clock == grouped.clock
                old_a, old_b = a.copy(), b.copy()
                _apply(serial, a, [4, 1, 0, 4, 3])
                _apply(grouped, b, [4, 1, 0, 4, 3])
                assert a.misses - old_a.misses == b.misses - old_b.misses
                assert a.hits - old_a.hits == b.hits - old_b.hits
                assert _snapshot(serial) == _snapshot(grouped)
    serial, grouped = LayerLruCache(1, 2), LayerLruCache(1, 2)
    a, b = Telemetry(), Telemetry()
    _apply(serial, a, [0, 1])
    _apply(grouped, b, [0, 1])
    keys = [0, 2, 0]
    assert grouped.grouped_access_order(0, keys) is None
    assert grouped.grouped_access_plan(0, keys).order() == [0, 2]
    grouped.clock = U64_MAX - 2
    assert grouped.grouped_access_plan(0, keys) is None
    serial.clock = U64_MAX - 3
    grouped.clock = U64_MAX - 3
    plan = grouped.grouped_access_plan(0, keys)
    _apply(serial, a, keys)
    for key in plan.order():
        grouped.access_grouped_with_evicted(b, plan, key, ok(key, key + 1, 7))
    grouped.finish_grouped_plan(plan)
    assert grouped.clock == U64_MAX
    assert _snapshot(serial) == _snapshot(grouped)
    _apply(serial, a, [3, 0, 3, 2, 1])
    _apply(grouped, b, [3, 0, 3, 2, 1])
    assert _snapshot(serial) == _snapshot(grouped)
    assert grouped.grouped_access_plan(0, keys) is None
    assert LayerLruCache(1, 0).grouped_access_plan(0, keys) is None


def test_protected_grouping_keeps_one_transient_value_and_preserves_cache_on_failure():
    # cache.rs:747-845: handles stand for owned values; `live` counts the handles loaded and
    # not yet released (the reference's Rc drop counter)
    live = set()
    counter = [0]

    def make(key):
        counter[0] += 1
        h = (key << 32) | counter[0]
        live.add(h)
        return h

    cache = LayerLruCache(1, 2)
    t = Telemetry()
    for key in (0, 1):
        cache.access(t, 0, key, lambda key=key: (make(key), 11, 7))
    # resident 0 survives; 2 and 3 stream without admission; final miss 4 replaces 1
    keys = [0, 2, 3, 4, 0]
    plan = cache.grouped_access_plan(0, keys)
    assert plan.order() == [0, 2, 3, 4]

    def fail():
        raise OSError("read failed")

    for key in (2, 4):
        clock, before = cache.clock, t.copy()
        entries = [(e.key, e.last_used) for e in cache.entries(0)]
        with pytest.raises(R.LoadError):
            cache.access_grouped_with_evicted(t, plan, key, fail)
        assert t == before
        assert cache.clock == clock
        assert [(e.key, e.last_used) for e in cache.entries(0)] == entries
        assert len(live) == 2
    recycled = None
    for key in plan.order():
        if not cache.contains(0, key) and recycled is not None:
            live.discard(recycled)
            recycled = None

        def load(key=key):
            value = make(key)
            assert len(live) <= 3
            return value, 11, 7

        selected, displaced = cache.access_grouped_with_evicted(t, plan, key, load)
        assert selected >> 32 == key
        assert len(live) <= 3
        if displaced is not None:
            recycled = displaced
    cache.finish_grouped_plan(plan)
    assert cache.contains(0, 0) and cache.contains(0, 4)
    assert t.resident_experts == 2
    assert t.misses == 5  # two seed loads and three distinct misses
    if recycled is not None:
        live.discard(recycled)
    for h in cache.drain_layer(t, 0):
        live.discard(h)
    assert not live


def test_grouped_accesses_preserve_lru_and_never_add_projected_misses():
    # cache.rs:847-953 (capacities 0-4)
    for capacity in range(0, 5):
        for seed in SEEDS:
            for keys in _sequences():
                serial, grouped = LayerLruCache(1, capacity), LayerLruCache(1, capacity)
                a, b = Telemetry(), Telemetry()
                _apply(serial, a, seed)
                _apply(grouped, b, seed)
                initial, clock = _recency(grouped), grouped.clock
                expected_misses = serial.projected_misses(0, keys)
                order = grouped.grouped_access_order(0, keys)
                assert _recency(grouped) == initial and grouped.clock == clock
                before = a.misses
                _apply(serial, a, keys)
                assert a.misses - before == expected_misses
                if order is None:
                    continue
                _apply(grouped, b, order)
                grouped.finish_grouped_accesses(0, keys, len(order))
                assert b.misses <= a.misses
                assert serial.clock == grouped.clock
                g = {e.key: e.last_used for e in grouped.entries(0)}
                for e in serial.entries(0):
                    assert g[e.key] == e.last_used
                assert _recency(serial) == _recency(grouped)
                assert a.resident_bytes == b.resident_bytes
                old_a, old_b = a.copy(), b.copy()
                _apply(serial, a, [4, 1, 0, 4, 3])
                _apply(grouped, b, [4, 1, 0, 4, 3])
                assert a.misses - old_a.misses == b.misses - old_b.misses
                assert a.hits - old_a.hits == b.hits - old_b.hits
                assert _recency(serial) == _recency(grouped)
    cache, t = LayerLruCache(1, 2), Telemetry()
    _apply(cache, t, [0, 1])
    # touching 0 early protects it: [0,2,0] has one miss, but [2,0] has two
    assert cache.projected_misses(0, [0, 2, 0]) == 1
    assert cache.projected_misses(0, [2, 0]) == 2
    assert cache.grouped_access_order(0, [0, 2, 0]) is None
    assert cache.grouped_access_order(0, [0, 1]) is None
    cache.clock = U64_MAX - 1
    assert cache.grouped_access_order(0, [0, 0]) is None
    cache.clock = U64_MAX - 3
    keys = [0, 1, 0]
    grouped = cache.grouped_access_order(0, keys)
    _apply(cache, t, grouped)
    cache.finish_grouped_accesses(0, keys, len(grouped))
    assert cache.clock == U64_MAX
    last = {e.key: e.last_used for e in cache.entries(0)}
    assert last[0] == U64_MAX and last[1] == U64_MAX - 1
    _apply(cache, t, [2])
    assert cache.contains(0, 0)
    assert not cache.contains(0, 1)


def test_ordered_batch_preparation_matches_serial_lru_and_telemetry():
    # cache.rs:955-1010
    def seeded():
        cache, t = LayerLruCache(1, 4), Telemetry()
        for key in (1, 2, 3, 4):
            cache.access(t, 0, key, ok(key * 10, 4, 3))
        return cache, t

    accesses = [5, 1, 6]
    serial, st = seeded()
    for key in accesses:
        serial.access(st, 0, key, ok(key * 10, 4, 3))
    prepared, pt = seeded()
    assert prepared.prepare_ordered_batch(pt, 0, accesses) == [10, 20, 30]
    assert prepared.can_insert_without_eviction(0, accesses)
    for key in accesses:
        prepared.access(pt, 0, key, ok(key * 10, 4, 3))
    assert pt == st
    for key in range(1, 7):
        assert prepared.contains(0, key) == serial.contains(0, key)
    # a batch with a repeated key, or larger than the layer, is not prepared
    other, ot = seeded()
    assert other.prepare_ordered_batch(ot, 0, [5, 5]) is None
    assert other.prepare_ordered_batch(ot, 0, [5, 6, 7, 8, 9]) is None
    assert ot == seeded()[1]


def test_peek_does_not_change_recency_or_telemetry():
    # cache.rs:1012-1034
    cache, t = LayerLruCache(1, 2), Telemetry()
    for key in (1, 2):
        cache.access(t, 0, key, ok(key * 10, 4, 3))
    before = t.copy()
    assert cache.peek(0, 1) == 10
    assert t == before
    cache.access(t, 0, 3, ok(30, 4, 3))
    assert not cache.contains(0, 1)


def test_layer_empty_state_tracks_residency():
    # cache.rs:1036-1074
    cache, t = LayerLruCache(2, 1), Telemetry()
    assert cache.layer_is_empty(0) and cache.layer_is_empty(1)
    cache.access(t, 1, 7, ok(70, 4, 3))
    assert cache.layer_is_empty(0) and not cache.layer_is_empty(1)
    before = t.copy()
    assert cache.residency() == [(0, 0, 1, 0), (1, 1, 1, 4)]
    assert t == before
    cache.access(t, 1, 8, ok(80, 9, 8))
    assert cache.residency()[1][3] == 9 and cache.residency()[1][1] == 1
    cache.drain_layer(t, 1)
    assert cache.residency()[1][3] == 0 and cache.residency()[1][2] == 1


def test_draining_a_layer_preserves_capacity_and_updates_residency():
    # cache.rs:1076-1098
    cache, t = LayerLruCache(1, 2), Telemetry()
    for key in (7, 8):
        cache.access(t, 0, key, ok(key * 10, 4, 3))
    assert cache.layer_capacity(0) == 2
    assert cache.drain_layer(t, 0) == [70, 80]
    assert cache.layer_is_empty(0)
    assert cache.layer_capacity(0) == 2
    assert (t.evictions, t.resident_experts, t.resident_bytes) == (2, 0, 0)


def test_per_layer_capacities_use_spare_slots_without_weakening_other_layers():
    # cache.rs:1100-1119
    cache, t = LayerLruCache.with_layer_capacities([1, 2]), Telemetry()
    for layer, key in ((0, 1), (1, 1), (1, 2)):
        cache.access(t, layer, key, ok(key, 4, 3))
    assert t.resident_experts == 3
    assert cache.contains(0, 1) and cache.contains(1, 1) and cache.contains(1, 2)


def test_unused_global_capacity_can_be_lent_then_trimmed_back_to_recent_entries():
    # cache.rs:1121-1161
    cache, t = LayerLruCache.with_layer_capacities([2, 2]), Telemetry()
    steady = cache.lend_unused_capacity(0, 10)
    assert steady == 2
    for key in (1, 2, 3, 4):
        cache.access(t, 0, key, ok(key * 10, 4, 3))
    assert t.resident_experts == 4
    assert cache.restore_layer_capacity(t, 0, steady) == [10, 20]
    assert not cache.contains(0, 1) and not cache.contains(0, 2)
    assert cache.contains(0, 3) and cache.contains(0, 4)
    assert (t.resident_experts, t.evictions) == (2, 2)
    for key in (5, 6):
        cache.access(t, 1, key, ok(key * 10, 4, 3))
    steady = cache.lend_unused_capacity(0, 10)
    assert steady == 2
    assert cache.layer_capacity(0) == 2  # the other layer now occupies its two slots
    cache.restore_layer_capacity(t, 0, steady)


def test_hit_rate_distinguishes_no_accesses_from_no_hits():
    # cache.rs:1163-1173
    assert Telemetry().hit_rate() is None
    t = Telemetry(hits=3, misses=1)
    assert t.accesses() == 4
    assert t.hit_rate() == 0.75


def test_failed_plain_load_hands_back_the_evicted_value():
    # LayerLruCache::access evicts before it loads (cache.rs:141-158): a failing load still
    # displaces the victim, whose handle the caller gets back to release
    cache, t = LayerLruCache(1, 1), Telemetry()
    cache.access(t, 0, 1, ok(11, 4, 3))

    def fail():
        raise OSError("read failed")

    with pytest.raises(R.LoadError) as e:
        cache.access_with_evicted(t, 0, 2, fail)
    assert e.value.evicted == 11
    assert not cache.contains(0, 1) and cache.layer_is_empty(0)
    assert (t.misses, t.evictions, t.resident_experts) == (2, 1, 0)
