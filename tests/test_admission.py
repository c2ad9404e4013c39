"""Physical admission and lookahead precommit (elastic_kv/admission.py).

Known answers are the reference's own admission tests
(tests/test_adapter_compat.py:698-867), restated over plain arena objects.
A token-by-token brute force pins the chunk-skipping walk on random inputs.
"""

import random
from types import SimpleNamespace

import pytest

from elastic_kv.admission import PhysicalAdmission, available_tokens, precommit_candidates


def admission(arenas, free, headroom=0, policy="physical", reclaimed=None):
    calls = []

    def reclaim():
        calls.append(1)

    free_values = [free] if reclaimed is None else [free, reclaimed]
    state = {"i": 0}

    def free_bytes():
        value = free_values[min(state["i"], len(free_values) - 1)]
        state["i"] += 1
        return value

    ctrl = PhysicalAdmission(arenas, 100, 1_000, policy=policy, prefill_headroom_bytes=headroom,
                             free_bytes=free_bytes, reclaim=reclaim)
    return ctrl, calls


def test_headroom_is_reserved_before_the_token_budget():
    # tests/test_adapter_compat.py:698-724: chunks 0-2 mapped or precommitted, budget 2 more chunks.
    ctrl, _ = admission([SimpleNamespace(planes=2, mapped_chunks={0, 1})], 5_500, headroom=500)
    ctrl.precommitted = {2}
    assert ctrl.physical_available_tokens(100, [(1, 101)]) == 49
    assert ctrl.counters["physical_chunk_cost_bytes"] == 2_000
    assert ctrl.counters["physical_headroom_bytes"] == 500
    assert ctrl.counters["physical_limited_calls"] == 1


def test_logical_policy_does_not_query_memory():
    # :828-833
    def fail():
        raise AssertionError("queried device memory")

    ctrl = PhysicalAdmission([], 100, 1_000, policy="logical", free_bytes=fail)
    assert ctrl.physical_available_tokens(7, None) == 7


def test_mapped_holes_are_credited_before_new_chunks():
    # :835-857: no free memory at all, but every admitted slot lies in mapped chunks.
    ctrl, reclaims = admission([SimpleNamespace(planes=1, mapped_chunks={0, 1, 2})], 0)
    assert ctrl.physical_available_tokens(10, [(1, 6), (11, 16)]) == 10
    assert "physical_limited_calls" not in ctrl.counters
    assert reclaims == [1] and ctrl.counters["physical_empty_cache_calls"] == 1


def test_reclaim_is_used_when_memory_is_short():
    ctrl, reclaims = admission([SimpleNamespace(planes=1, mapped_chunks={0})], 500, reclaimed=3_000)
    assert ctrl.physical_available_tokens(50, [(1, 51)]) == 39   # 9 sink-chunk slots + 3 new chunks
    assert reclaims == [1]
    assert ctrl.counters["physical_empty_cache_freed_bytes"] == 2_500


def brute_force(logical, ranges, slot_bytes, chunk_bytes, backed, budget):
    backed = set(backed)
    admitted = 0
    for start, stop in ranges:
        for slot in range(start, stop):
            chunks = range(slot * slot_bytes // chunk_bytes, ((slot + 1) * slot_bytes - 1) // chunk_bytes + 1)
            missing = [c for c in chunks if c not in backed]
            if len(missing) > budget:
                return admitted
            budget -= len(missing)
            backed.update(missing)
            admitted += 1
    return admitted


@pytest.mark.parametrize("seed", range(40))
def test_chunk_skipping_walk_matches_token_by_token(seed):
    rng = random.Random(seed)
    chunk_bytes = rng.choice([64, 100, 1_000, 4_096])
    slot_bytes = rng.randint(1, chunk_bytes)
    cuts = sorted(rng.sample(range(1, 400), rng.randint(2, 12)))
    ranges = [(a, b) for a, b in zip(cuts[::2], cuts[1::2]) if a < b]
    if not ranges:
        ranges = [(1, 2)]
    logical = sum(b - a for a, b in ranges)
    top = 400 * slot_bytes // chunk_bytes + 2
    backed = set(rng.sample(range(top), rng.randint(0, top)))
    budget = rng.randint(0, top)
    assert (available_tokens(logical, ranges, slot_bytes, chunk_bytes, backed, budget)
            == brute_force(logical, ranges, slot_bytes, chunk_bytes, backed, budget))


def test_invalid_ranges_are_rejected():
    with pytest.raises(ValueError, match="nonnegative"):
        available_tokens(-1, [], 100, 1_000, set(), 1)
    with pytest.raises(ValueError, match="length"):
        available_tokens(5, [(1, 4)], 100, 1_000, set(), 1)
    with pytest.raises(ValueError, match="sorted"):
        available_tokens(4, [(5, 7), (1, 3)], 100, 1_000, set(), 1)
    with pytest.raises(ValueError, match="positive"):
        available_tokens(2, [(0, 2)], 100, 1_000, set(), 1)
    with pytest.raises(ValueError, match="slot_bytes"):
        available_tokens(2, [(1, 3)], 2_000, 1_000, set(), 1)


def test_request_affine_preflight():
    ctrl, _ = admission([SimpleNamespace(planes=1, mapped_chunks={0, 1})], 2_000)
    assert ctrl.can_commit_chunks([1, 2, 3])
    assert not ctrl.can_commit_chunks([2, 3, 4])
    assert ctrl.counters["request_affine_physical_preflight_calls"] == 2
    assert ctrl.counters["request_affine_physical_fallbacks"] == 1


def test_lookahead_precommit_after_admitted_ranges():
    committed = []

    class Arena:
        planes = 1
        mapped_chunks = {0}

        def precommit(self, ids):
            committed.extend(ids)
            return len(ids)

    ctrl = PhysicalAdmission([Arena()], 100, 1_000, precommit_lookahead=3, precommit_limit=4,
                             free_bytes=lambda: 10**9)
    busy = {5}
    # Range (1, 25) ends in chunk 2; range (40, 52) ends in chunk 5.
    assert precommit_candidates([(1, 25), (40, 52)], 100, 1_000, 100, 3, lambda c: c not in busy) == [2, 3, 4, 6, 7]
    added = ctrl.precommit_after([(1, 25), (40, 52)], 100, lambda c: c not in busy)
    assert added == [2, 3, 4, 6] and committed == [2, 3, 4, 6]
    assert ctrl.counters["precommit_chunks"] == 4
    ctrl.admitted([2, 3])
    assert ctrl.precommitted == {4, 6}
    assert ctrl.backed_chunks() == {0, 4, 6}
