"""Group release accounting (CPU only).

Known answers from the reference's tests/test_scheduler_budget.py:365-625
(three requests sharing one chunk, the bounded search's examined / truncated /
rejected tallies, rotation, the owner index, the overlapping-page fallback),
a brute force of the release rule written from its definition, and the
closure search checked against exhaustive enumeration.
"""

from collections import Counter
from itertools import combinations
from random import Random
from types import SimpleNamespace

import pytest

from adaptive_sparse.minimax_vmm import PhysicalPages
from adaptive_sparse.release_groups import (PhysicalDemandIndex, bounded_demotion_groups, chunk_release_counts,
                                            demand_index_demotion_groups, indexed_demotion_groups, releasable,
                                            releasable_counts, releasable_group, releasable_pair)


def _tracker(refs, mapped, chunk_bytes=10, chunks=None):
    return SimpleNamespace(refs=refs, backing=SimpleNamespace(mapped_chunks=set(mapped)), chunk_bytes=chunk_bytes,
                           chunks=chunks)


def _entry(pages, counts):
    # The reference scheduler's request entry: item 1 pages, item 2 chunk counts.
    return (None, set(pages), Counter(counts), set())


def _three_sharing_one_chunk():
    tracker = _tracker({9: 3}, {9})
    requests = {"a": _entry({1}, {9: 1}), "b": _entry({2}, {9: 1}), "c": _entry({3}, {9: 1})}
    return tracker, requests, {"a": 4, "b": 5, "c": 6}.__getitem__


def _freed_by_definition(layout, mapped, released):
    # A mapped chunk is freed when some released page touches it and no live
    # page outside the released set does.
    return {chunk for chunk in mapped
            if any(chunk in layout[p] for p in released)
            and not any(chunk in chunks for p, chunks in enumerate(layout) if p not in released)}


def test_release_rule_matches_its_definition_on_random_layouts():
    rng = Random(137)
    for trial in range(120):
        layout = [set(rng.sample(range(9), rng.randint(1, 3))) for _ in range(16)]
        refs = Counter(chunk for chunks in layout for chunk in chunks)
        mapped = set(rng.sample(range(9), 8))
        tracker = _tracker(refs, mapped, chunks=layout.__getitem__)
        if trial % 2:
            candidates = [set(range(start, start + 3)) for start in range(1, 16, 3)]     # disjoint pages
        else:
            candidates = [set(rng.sample(range(1, 16), 7)) for _ in range(5)]           # overlapping pages
        counts = [chunk_release_counts(tracker, pages) for pages in candidates]
        for pages, count in zip(candidates, counts):
            assert releasable_counts(tracker, count) == _freed_by_definition(layout, mapped, pages)
            assert releasable(tracker, list(pages) * 2) == _freed_by_definition(layout, mapped, pages)
        for i, j in combinations(range(len(candidates)), 2):
            expected = _freed_by_definition(layout, mapped, candidates[i] | candidates[j])
            assert releasable_pair(tracker, candidates[i], counts[i], candidates[j], counts[j]) == expected
        expected = _freed_by_definition(layout, mapped, set().union(*candidates[:3]))
        assert releasable_group(tracker, zip(candidates[:3], counts[:3])) == expected


def test_group_release_needs_every_owner_of_a_shared_chunk():
    tracker, requests, _ = _three_sharing_one_chunk()
    entries = [(e[1], e[2]) for e in requests.values()]
    assert releasable_group(tracker, entries[:2]) == set()
    assert releasable_group(tracker, entries) == {9}
    tracker.backing.mapped_chunks = set()
    assert releasable_group(tracker, entries) == set()                   # unmapped chunks free nothing


def test_bounded_search_tallies_budget_cap_and_rotation():
    tracker, requests, cost = _three_sharing_one_chunk()
    groups, chunks, examined, truncated, rejected = bounded_demotion_groups(
        tracker, requests, cost, max_group=3, byte_cap=20, search_limit=8)
    assert groups == {("a", "b", "c"): (10, 15)} and chunks == {("a", "b", "c"): {9}}
    assert (examined, truncated, rejected) == (4, False, 0)

    # search_limit 3 over sizes (2, 3): shares 2 and 1, so the third pair is cut.
    groups, _, examined, truncated, rejected = bounded_demotion_groups(
        tracker, requests, cost, max_group=3, byte_cap=20, search_limit=3, rotation=0)
    assert groups == {("a", "b", "c"): (10, 15)} and (examined, truncated, rejected) == (3, True, 0)

    seen = []
    groups, _, examined, truncated, rejected = bounded_demotion_groups(
        tracker, requests, cost, max_group=3, byte_cap=12, search_limit=8, cap_observer=seen.append)
    assert groups == {} and (examined, truncated, rejected) == (4, False, 1) and seen == [15]

    pair_tracker = _tracker({9: 2}, {9})
    pairs = {"a": _entry({1}, {}), "b": _entry({2}, {}), "c": _entry({3}, {9: 1}), "d": _entry({4}, {9: 1})}
    first, _, _, truncated, _ = bounded_demotion_groups(
        pair_tracker, pairs, lambda _: 1, max_group=2, byte_cap=10, search_limit=1, rotation=0)
    assert first == {} and truncated
    later, chunks, _, _, _ = bounded_demotion_groups(
        pair_tracker, pairs, lambda _: 1, max_group=2, byte_cap=10, search_limit=1, rotation=2)
    assert later == {("c", "d"): (10, 2)} and chunks == {("c", "d"): {9}}

    for search in (bounded_demotion_groups, lambda *a, **k: indexed_demotion_groups(PhysicalDemandIndex(), *a, **k)):
        with pytest.raises(ValueError, match="search_limit"):
            search(tracker, requests, cost, max_group=3, byte_cap=20, search_limit=0)


def test_demand_index_updates_only_changed_requests():
    index = PhysicalDemandIndex()
    requests = {"a": _entry({1}, {9: 1}), "b": _entry({2}, {9: 1, 4: 0})}
    assert index.sync(requests) == 2
    assert index.page_owners == {1: {"a"}, 2: {"b"}}
    assert index.chunk_owners == {9: {"a": 1, "b": 1}}                   # zero counts are not indexed
    assert not index.has_page_overlap
    assert index.sync(requests) == 0
    requests["b"] = _entry({1}, {9: 1})
    assert index.sync(requests) == 1
    assert index.has_page_overlap and index.page_owners[1] == {"a", "b"}
    assert index.sync({}) == 2
    assert index.records == {} and index.chunk_owners == {} and index.page_owners == {}


def test_closure_search_follows_shared_chunk_owners():
    tracker, requests, cost = _three_sharing_one_chunk()
    index = PhysicalDemandIndex()
    assert index.sync(requests) == 3
    groups, chunks, examined, truncated, rejected = indexed_demotion_groups(
        index, tracker, requests, cost, max_group=3, byte_cap=20, search_limit=8)
    assert groups == {("a", "b", "c"): (10, 15)} and chunks == {("a", "b", "c"): {9}}
    assert (examined, truncated, rejected) == (1, False, 0)
    # A chain a-b, b-c, c-d of shared chunks gives three pair candidates, in
    # rotated request order; a budget of two scores the first two.
    chain = _tracker({10: 2, 11: 2, 12: 2}, {10, 11, 12})
    links = {"a": _entry({1}, {10: 1}), "b": _entry({2}, {10: 1, 11: 1}), "c": _entry({3}, {11: 1, 12: 1}),
             "d": _entry({4}, {12: 1})}
    chain_index = PhysicalDemandIndex()
    chain_index.sync(links)
    assert chain_index.candidate_groups(chain, max_group=2, candidate_limit=32, rotation=1)[0] == [
        ("b", "c"), ("c", "d"), ("a", "b")]
    groups, chunks, examined, truncated, _ = indexed_demotion_groups(
        chain_index, chain, links, lambda _: 1, max_group=2, byte_cap=10, search_limit=2)
    assert chunks == {("a", "b"): {10}, ("b", "c"): {11}} and (examined, truncated) == (2, True)
    # A chunk held by a page outside the indexed requests is never followed.
    tracker.refs[9] = 4
    groups, _, examined, _, _ = indexed_demotion_groups(
        index, tracker, requests, cost, max_group=3, byte_cap=20, search_limit=8)
    assert groups == {} and examined == 0


def test_overlapping_pages_fall_back_to_exhaustive_search():
    tracker = _tracker({9: 1}, {9}, chunks=lambda _: {9})
    requests = {"a": _entry({1}, {9: 1}), "b": _entry({1}, {9: 1})}
    index = PhysicalDemandIndex()
    index.sync(requests)
    result = demand_index_demotion_groups(index, tracker, requests, lambda _: 1, max_group=2, byte_cap=10,
                                          search_limit=4)
    groups, chunks, indexed, fallback, index_cut, fallback_cut, rejected, used_fallback = result
    assert groups == {("a", "b"): (10, 2)} and chunks == {("a", "b"): {9}}
    assert (indexed, fallback, index_cut, fallback_cut, rejected, used_fallback) == (0, 1, False, False, 0, True)


def test_closure_search_finds_every_owner_set_the_exhaustive_search_scores():
    rng = Random(911)
    for trial in range(40):
        ids = [f"r{i}" for i in range(8)]
        held = {r: Counter() for r in ids}
        refs = Counter()
        for chunk in range(12):
            for r in rng.sample(ids, rng.randint(2, 4)):
                held[r][chunk] += 1
                refs[chunk] += 1
        if trial % 3 == 0:
            refs[rng.randrange(12)] += 1                                 # a page outside every request
        requests = {r: _entry({int(r[1:]) + 1}, held[r]) for r in ids}
        tracker = _tracker(refs, set(refs) - {trial % 12}, chunk_bytes=1)
        exhaustive, exhaustive_chunks, _, cut, _ = bounded_demotion_groups(
            tracker, requests, lambda _: 1, max_group=4, byte_cap=1 << 30, search_limit=10_000)
        assert not cut
        index = PhysicalDemandIndex()
        index.sync(requests)
        groups, chunks, _, fallback, truncated, _, _, used_fallback = demand_index_demotion_groups(
            index, tracker, requests, lambda _: 1, max_group=4, byte_cap=1 << 30, search_limit=256)
        assert not truncated and fallback == 0 and not used_fallback
        for group, value in groups.items():
            assert exhaustive[group] == value and exhaustive_chunks[group] == chunks[group]
        # Every chunk that some group of at most 4 requests frees is freed by
        # the closure search's group made of exactly its owners.
        for chunk in set(refs) - {trial % 12}:
            owners = tuple(sorted(r for r in ids if held[r][chunk]))
            if sum(held[r][chunk] for r in owners) == refs[chunk] and len(owners) <= 4:
                assert chunk in chunks[owners], (trial, chunk)


class _Backing:
    def __init__(self):
        self.mapped_chunks = set()

    def ensure(self, indices):
        self.mapped_chunks.update(indices)

    def reclaim(self, indices, *, synchronize):
        self.mapped_chunks.difference_update(indices)
        return len(indices)


def test_physical_pages_tracker_predicts_what_a_trim_frees():
    # Two planes (chunks 0.. and 8..) of one 4 B row per page over 8 B chunks:
    # pages 2k and 2k+1 share chunk k of each plane, and page 1 shares chunk 0
    # with the sink page 0.
    backing = _Backing()
    pages = PhysicalPages(backing, 1, 8, [(0, 4), (8, 4)], lambda: None, chunk_bytes=8)
    pages.acquire(range(1, 8))
    requests = {"x": {1, 2}, "y": {3}, "z": {4, 5}}
    entries = {r: _entry(p, chunk_release_counts(pages, p)) for r, p in requests.items()}
    assert releasable(pages, requests["x"]) == releasable(pages, requests["y"]) == set()
    assert releasable(pages, requests["z"]) == {2, 10}
    groups, chunks, examined, _, _ = bounded_demotion_groups(pages, entries, lambda r: len(requests[r]),
                                                             max_group=2, byte_cap=100, search_limit=10)
    assert examined == 3
    assert chunks == {("x", "y"): {1, 9}, ("x", "z"): {2, 10}, ("y", "z"): {2, 10}}
    assert groups[("x", "y")] == (16, 3)
    pages.release({1, 2, 3})
    assert pages.trim_quiescent() == 16
    assert backing.mapped_chunks == {0, 2, 3, 8, 10, 11}                 # the sink keeps chunks 0 and 8
