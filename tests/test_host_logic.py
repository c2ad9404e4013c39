"""Host-side bookkeeping of the path (CPU only), ported from the reference's tests.

Sources: tests/test_slots.py, tests/test_virtual_layout.py,
tests/test_minimax_vmm.py, tests/test_backing.py:21-128 (fake native
library), the recorded chunk-aware demotion plans, and the migration
bandwidth estimator's closed form.
"""

import gc
import json
import math
import random
from types import SimpleNamespace
from unittest.mock import Mock, call, patch

import pytest

from adaptive_sparse.kv_pool import BlockMajorLayout, PlanePoolLayout
from adaptive_sparse.migration import plan_demote_pages
from adaptive_sparse.migration_budget import MigrationBandwidthEstimator
from adaptive_sparse.minimax_vmm import PageFootprints, PhysicalPages
from conftest import GOLDEN
from elastic_kv.backing import Backing, _load_library
from elastic_kv.slots import FreeSlots
from experimental.resident_arena import VmmResidentArena
from experimental.virtual_layout import VirtualKVLayout

# ------------------------------------------------------------------ FreeSlots


def test_slots_fragmented_claim_and_bridge_merge():
    slots = FreeSlots(8)
    slots.claim(slots.peek(8))
    slots.release([1, 2, 4, 5, 7, 8])
    ranges = slots.peek(3)
    assert ranges == [(1, 3), (4, 5)]
    slots.claim(ranges)
    assert slots.ranges == [(5, 6), (7, 9)]
    slots.release([6])
    assert slots.ranges == [(5, 9)]
    assert slots.count == 4


def test_slots_peek_bounds_leave_state_intact():
    slots = FreeSlots(2)
    assert slots.peek(0) == []
    assert slots.peek(3) is None
    with pytest.raises(ValueError):
        slots.peek(-1)
    assert slots.ranges == [(1, 3)] and slots.count == 2


def test_slots_remove_arbitrary_ranges():
    slots = FreeSlots(16)
    slots.remove([(5, 8)])
    assert slots.ranges == [(1, 5), (8, 17)] and slots.count == 13
    slots.remove([(1, 2), (9, 11)])
    assert slots.ranges == [(2, 5), (8, 9), (11, 17)] and slots.count == 10
    with pytest.raises(ValueError, match="crosses a non-free slot"):
        slots.remove([(1, 2)])
    with pytest.raises(ValueError, match="crosses a non-free slot"):
        slots.remove([(4, 9)])


def _as_ranges(values):
    values = sorted(values)
    ranges = []
    start = previous = values[0]
    for value in values[1:]:
        if value != previous + 1:
            ranges.append((start, previous + 1))
            start = value
        previous = value
    ranges.append((start, previous + 1))
    return ranges


def test_slots_randomized_remove_against_set_model():
    rng = random.Random(713)
    capacity = 97
    slots = FreeSlots(capacity)
    free = set(range(1, capacity + 1))
    for _ in range(1000):
        if len(free) > 12 and rng.randrange(2):
            chosen = sorted(rng.sample(sorted(free), rng.randint(1, 8)))
            slots.remove(_as_ranges(chosen))
            free.difference_update(chosen)
        else:
            live = set(range(1, capacity + 1)) - free
            if not live:
                continue
            released = rng.sample(sorted(live), rng.randint(1, min(8, len(live))))
            slots.release(sorted(released))
            free.update(released)
        assert slots.count == len(free)
        assert [s for a, b in slots.ranges for s in range(a, b)] == sorted(free)


def test_slots_randomized_conservation():
    rng = random.Random(504)
    capacity = 97
    slots = FreeSlots(capacity)
    free = set(range(1, capacity + 1))
    for _ in range(3000):
        live = sorted(set(range(1, capacity + 1)) - free)
        if live and rng.randrange(2):
            ids = sorted(rng.sample(live, rng.randint(1, min(9, len(live)))))
            slots.release(ids)
            free.update(ids)
        else:
            count = rng.randint(0, 10)
            before = slots.ranges.copy()
            ranges = slots.peek(count)
            assert slots.ranges == before
            if count > len(free):
                assert ranges is None
            else:
                chosen = [s for a, b in ranges for s in range(a, b)]
                assert chosen == sorted(free)[:count]
                slots.claim(ranges)
                free.difference_update(chosen)
        assert slots.count == len(free)
        assert [s for a, b in slots.ranges for s in range(a, b)] == sorted(free)
        assert all(a[1] < b[0] for a, b in zip(slots.ranges, slots.ranges[1:]))


# ------------------------------------------------------------------ layouts / arena


def test_layout_alignment_and_crossing_rows():
    layout = VirtualKVLayout(2, 3, 3, chunk_bytes=8)
    assert layout.capacity_bytes == 56
    assert layout.request_offset(1) == 32
    assert layout.token_offset(0, 1) == 14
    assert layout.prefix_chunks(0, 0) == set()
    assert layout.selected_chunks(0, []) == set()
    assert layout.selected_chunks(0, [1, 1]) == {1, 2}
    assert layout.prefix_chunks(0, 3) == {1, 2, 3}
    assert layout.prefix_chunks(1, 3) == {4, 5, 6}


def test_layout_rejects_invalid_fields_and_indices():
    fields = dict(max_requests=2, max_tokens=3, row_elements=3, itemsize=2, chunk_bytes=8)
    for field in fields:
        with pytest.raises(ValueError):
            VirtualKVLayout(**(fields | {field: 0}))
        with pytest.raises(TypeError):
            VirtualKVLayout(**(fields | {field: True}))
    layout = VirtualKVLayout(**fields)
    for index in (-1, 2):
        with pytest.raises(ValueError):
            layout.selected_chunks(index, [])
    for position in (-1, 3):
        with pytest.raises(ValueError):
            layout.selected_chunks(0, [position])
    for length in (-1, 4):
        with pytest.raises(ValueError):
            layout.prefix_chunks(0, length)


@pytest.fixture
def arena_calls():
    calls = Mock()
    layout = VirtualKVLayout(2, 5, 3, chunk_bytes=8)
    arena = VmmResidentArena(layout, backing_factory=calls.factory, synchronize=calls.sync)
    return calls, calls.factory.return_value, arena


def test_arena_lifecycle_preserves_live_tail_chunk(arena_calls):
    calls, _, arena = arena_calls
    arena.reserve(0, 3)
    arena.reserve(0, 1)
    arena.reserve(1, 1)
    arena.resize_quiescent(0, 2)
    arena.close()
    arena.close()
    assert calls.mock_calls == [
        call.factory(72, chunk_bytes=8, device=0), call.factory().ensure({0}),
        call.factory().ensure({1, 2, 3}), call.factory().ensure({5}),
        call.sync(), call.factory().reclaim({3}, synchronize=False),
        call.sync(), call.factory().close(),
    ]
    with pytest.raises(RuntimeError):
        arena.reserve(0, 1)


def test_arena_view_checks_extent_and_dtype(arena_calls):
    _, backing, arena = arena_calls
    dtype = SimpleNamespace(itemsize=2)
    arena.reserve(1, 2)
    arena.row_view(1, 2, dtype)
    backing.raw.narrow.assert_called_once_with(0, 40, 12)
    backing.raw.narrow.return_value.view.assert_called_once_with(dtype)
    backing.raw.narrow.return_value.view.return_value.reshape.assert_called_once_with(2, 3)
    with pytest.raises(ValueError):
        arena.row_view(1, 3, dtype)
    with pytest.raises(ValueError):
        arena.row_view(1, 2, SimpleNamespace(itemsize=4))


def test_arena_backing_failure_stops_use_and_close_still_syncs(arena_calls):
    calls, backing, arena = arena_calls
    backing.ensure.side_effect = RuntimeError("allocation failed")
    with pytest.raises(RuntimeError, match="allocation failed"):
        arena.reserve(0, 2)
    assert arena.length(0) == 0
    with pytest.raises(RuntimeError):
        arena.row_view(0, 0, SimpleNamespace(itemsize=2))
    arena.close()
    calls.sync.assert_called_once()
    backing.close.assert_called_once()


def test_plane_pool_layout_chunk_math():
    layout = PlanePoolLayout(layers=2, kv=2, rows=5, row_bytes=3, chunk_bytes=8)
    assert layout.plane_chunks == 2 and layout.plane_stride == 16 and layout.capacity_bytes == 64
    assert layout.plane_offset(1, 1) == 48
    # slot 2 covers bytes [6, 9) of each plane -> chunks 0 and 1 of every plane
    assert layout.chunks_for_slots([2]) == {0, 1, 2, 3, 4, 5, 6, 7}
    assert layout.chunks_for_slots([0]) == {0, 2, 4, 6}
    assert layout.chunks_for_slot_range(3, 5) == {1, 3, 5, 7}
    planes = layout.kv_planes(1000, 0)
    assert planes.row_offset(1, 1, 4) == 48 + 12
    block = BlockMajorLayout(blocks=4, layers=3, kv=2, row_bytes=5, chunk_bytes=16)
    assert block.block_bytes == 30 and block.capacity_bytes == 128
    assert block.chunks_for_blocks([1]) == {1, 2, 3}
    assert block.kv_planes(0, 0).row_offset(2, 1, 3) == 90 + 25


# ------------------------------------------------------------------ PhysicalPages


class _ChunkBacking:
    def __init__(self):
        self.mapped_chunks = set()
        self.fail = False

    @property
    def backed_bytes(self):
        return len(self.mapped_chunks) * 8

    def ensure(self, indices):
        if self.fail:
            raise RuntimeError("map failed")
        self.mapped_chunks.update(indices)

    def reclaim(self, indices, *, synchronize):
        assert not synchronize
        self.mapped_chunks.difference_update(indices)
        return len(indices)


def test_pages_crossing_shared_chunks_tail_reuse_and_sink():
    backing = _ChunkBacking()
    syncs = []
    pages = PhysicalPages(backing, 2, 4, [(0, 3), (8, 2)], lambda: syncs.append(True), chunk_bytes=8)
    assert pages.chunks(1) == {0, 1, 8}
    pages.acquire([1, 2, 2])
    pages.acquire([2])
    pages.release({1})
    assert pages.stats()["reclaimable_bytes"] == 0
    pages.release({2})
    assert pages.trim_quiescent() == 24
    assert backing.mapped_chunks == {0, 8}
    assert syncs == [True]
    with pytest.raises(RuntimeError):
        pages.release({0})


def test_pages_failed_map_does_not_change_ownership():
    backing = _ChunkBacking()
    pages = PhysicalPages(backing, 1, 3, [(0, 8)], lambda: None, chunk_bytes=8)
    backing.fail = True
    with pytest.raises(RuntimeError, match="map failed"):
        pages.acquire([1])
    assert pages.pages == {0}
    assert pages.refs == {0: 1}


# ------------------------------------------------------------------ demotion plans


def _tracker_from_snapshot(snapshot):
    """The planner's view of a recorded tracker: page footprints and chunk reference counts."""
    footprints = PageFootprints(snapshot["page_size"], snapshot["planes"], snapshot["chunk_bytes"])
    return SimpleNamespace(chunks=footprints, refs={int(k): v for k, v in snapshot["refs"].items()})


@pytest.mark.parametrize("rank", range(4))
def test_chunk_aware_plans_reproduce_recorded_snapshots(rank):
    snapshot = json.loads((GOLDEN / f"demotion_plans_rank{rank}.json").read_text())[0]
    tracker = _tracker_from_snapshot(snapshot)
    assert snapshot["requests"]
    for row, request in snapshot["requests"].items():
        retained, released = plan_demote_pages(tracker, request["page_ids"], len(request["retained"]),
                                               chunk_aware=True)
        assert list(retained) == request["retained"], row
        assert list(released) == request["released"], row


def test_default_plan_keeps_the_first_pages_and_validates():
    assert plan_demote_pages(None, [5, 3, 9], 2, chunk_aware=False) == ((5, 3), (9,))
    for pages, keep in (([1, 2], 0), ([1, 2], 3), ([1, 1], 1)):
        with pytest.raises(ValueError):
            plan_demote_pages(None, pages, keep, chunk_aware=False)
    with pytest.raises(RuntimeError):
        plan_demote_pages(None, [1, 2], 1, chunk_aware=True)


def test_chunk_aware_plan_keeps_pages_sharing_chunks():
    # pages 1..4 with 2 pages per chunk; chunk 0 also held by the sink
    tracker = SimpleNamespace(chunks=lambda p: {p // 2}, refs={0: 2, 1: 2, 2: 1})
    retained, released = plan_demote_pages(tracker, [4, 3, 2, 1], 2, chunk_aware=True)
    # page 1 shares chunk 0 with the sink (no exclusive chunk) -> free to keep;
    # then page 4's chunk 2 is exclusive to it alone, page 2/3 share chunk 1 (supply 2)
    assert retained == (1, 2) and released == (4, 3)


# ------------------------------------------------------------------ transactions
#
# The prepare / commit / abort split of the reference's
# adaptive_sparse/migration.py:67-288 over HiSparseCoordinator, with a fake
# pool, host cache and row mover on the CPU: the order of side effects (a
# demotion unpublishes the mapping before any page is released and trims
# before it publishes the request as host-backed; a promotion frees the host
# rows and the hot pages, publishes the new mapping, trims, then publishes the
# request as resident), the hot-buffer state a demotion leaves, the host_len
# rule of a promotion, and the clean-up of failed moves.

PAGE, HOT = 4, 6            # padded hot buffer: ceil((6 + 1) / 4) * 4 = 8 slots = 2 pages


class _FakePool:
    def __init__(self, log, backed=1000):
        self.log = log
        self.page_size = PAGE
        self.device = "cpu"
        self.layout = SimpleNamespace(layers=3, kv=2, row_bytes=16)
        self.pages = None
        self.backing = SimpleNamespace(backed_bytes=backed)

    def take(self, count):
        pages = list(range(50, 50 + count))
        self.allocate(pages)
        return pages

    def allocate(self, pages):
        self.log.append(("allocate", tuple(pages)))
        self.backing.backed_bytes += 10 * len(pages)

    def release(self, pages):
        self.log.append(("release", tuple(pages)))

    def slots(self, pages):
        import torch

        return (torch.tensor(pages).view(-1, 1) * PAGE + torch.arange(PAGE)).flatten()

    def trim(self):
        self.log.append(("trim",))
        return 0


class _FakeHost:
    def __init__(self, log, rows=64):
        self.log, self.next, self.rows = log, 200, rows

    def alloc(self, count):
        import torch

        if count > self.rows:
            return None
        self.rows -= count
        self.next += count
        return torch.arange(self.next - count, self.next)

    def free(self, rows):
        self.log.append(("free_host", tuple(rows)))
        self.rows += len(rows)


class _FakeMover:
    def __init__(self, log, fail=None):
        self.log, self.fail = log, fail

    def _log(self, kind, src, dst):
        from adaptive_sparse.migration import Transfer

        if self.fail == kind:
            raise OSError("copy failed")
        self.log.append((kind, tuple(src.tolist()), tuple(dst.tolist())))
        return Transfer(len(src) * 96)

    def pool_to_host(self, slots, rows):
        return self._log("d2h", slots, rows)

    def host_to_pool(self, rows, slots):
        return self._log("h2d", rows, slots)

    def pool_to_pool(self, src, dst):
        return self._log("d2d", src, dst)


PAGES = [7, 3, 9, 12, 5]    # the request's pages, in logical order


def _coordinator(log, fail=None, length=20):
    import torch

    from adaptive_sparse.migration import HiSparseCoordinator, MigrationRequest

    coordinator = HiSparseCoordinator(_FakePool(log), _FakeHost(log), rows=4, max_len=64, logical_size=256,
                                      hot_capacity=HOT, mover=_FakeMover(log, fail))
    logical = torch.arange(100, 100 + length)
    coordinator.req_to_token[1, :length] = logical
    coordinator.mapping[logical] = (torch.tensor(PAGES).view(-1, 1) * PAGE + torch.arange(PAGE)).flatten()[:length]
    return coordinator, MigrationRequest(row=1, length=length), logical


def _slots(pages):
    return tuple(p * PAGE + i for p in pages for i in range(PAGE))


def test_demotion_leaves_the_hisparse_hot_buffer_state(monkeypatch):
    from adaptive_sparse.migration import commit_demote, prepare_demote

    monkeypatch.delenv("EKV_CHUNK_AWARE_RETENTION", raising=False)
    log = []
    coordinator, request, logical = _coordinator(log)
    sync = lambda: log.append(("sync",))

    def publish(kind):
        # Each publish sees the mapping as the commit left it.
        return lambda row: log.append((kind, row, tuple(coordinator.mapping[logical].tolist())))

    prepared = prepare_demote(coordinator, request, sync)
    assert coordinator.padded_buffer_size == 8
    assert log == [("sync",), ("d2h", _slots(PAGES), tuple(range(200, 220))), ("sync",)]
    assert prepared.retained_rows == (0, 1) and prepared.released_rows == (2, 3, 4)
    assert coordinator.mapping[logical].tolist() == list(_slots(PAGES))         # ownership unchanged by prepare
    assert coordinator.req_to_host_pool[1, :20].tolist() == list(range(200, 220))
    log.clear()
    assert commit_demote(prepared, publish("host"), sync, trim_quiescent=lambda: log.append(("trim",)) or 30) == 30
    assert log == [("sync",), ("release", (9, 12, 5)), ("sync",), ("trim",), ("host", 1, (0,) * 20)]
    # the hot buffer: the retained pages' token slots, index HOT the reserved newest-token slot
    assert coordinator.req_to_device_buffer[1].tolist() == list(_slots([7, 3]))
    assert coordinator.newest_slot(1) == _slots([7, 3])[HOT]
    assert coordinator.req_device_buffer_size[1] == 8 and coordinator.hot_pages[1] == (7, 3)
    assert (coordinator.req_device_buffer_tokens[:, 1] == -1).all()
    assert (coordinator.lru_slots[:, 1] == coordinator._lru_init).all()
    assert coordinator.skip_first_backup[1]                                      # the host image is authoritative
    with pytest.raises(RuntimeError, match="already been resolved"):
        commit_demote(prepared, publish("host"), sync)
    with pytest.raises(RuntimeError, match="unexpectedly owns"):
        prepare_demote(coordinator, request, sync)


def _demoted(log, length=20):
    from adaptive_sparse.migration import commit_demote, prepare_demote

    coordinator, request, logical = _coordinator(log, length=length)
    commit_demote(prepare_demote(coordinator, request, lambda: None), lambda row: None, lambda: None)
    log.clear()
    return coordinator, request, logical


def test_promotion_of_an_authoritative_host_image_copies_every_token_from_host(monkeypatch):
    from adaptive_sparse.migration import abort_promote, commit_promote, prepare_promote

    monkeypatch.delenv("EKV_CHUNK_AWARE_RETENTION", raising=False)
    log = []
    coordinator, request, logical = _demoted(log)
    sync = lambda: log.append(("sync",))
    promotion = prepare_promote(coordinator, request, sync)
    # host_len == length: 20 host rows into the 5 new pages, nothing from the reserved slot
    assert log == [("sync",), ("allocate", (50, 51, 52, 53, 54)),
                   ("h2d", tuple(range(200, 220)), _slots(range(50, 55))), ("sync",)]
    assert coordinator.mapping[logical].tolist() == [0] * 20                      # unpublished until commit
    log.clear()
    abort_promote(promotion)
    assert log == [("release", (50, 51, 52, 53, 54)), ("trim",)] and promotion.status == "aborted"
    with pytest.raises(RuntimeError, match="prepared promotion"):
        abort_promote(promotion)
    promotion = prepare_promote(coordinator, request, lambda: None, destinations=[9, 8, 7, 6, 5])
    log.clear()
    published = []
    assert commit_promote(promotion, lambda row: published.append(
        (row, tuple(coordinator.mapping[logical].tolist()))), sync) == 50          # growth: 5 pages
    assert log == [("free_host", tuple(range(200, 220))), ("release", (7, 3)), ("sync",), ("trim",)]
    assert published == [(1, _slots([9, 8, 7, 6, 5]))]
    assert 1 not in coordinator.hot_pages and coordinator.req_device_buffer_size[1] == 0
    assert coordinator.req_to_host_pool_allocated_len[1] == 0 and (coordinator.req_to_host_pool[1] == -1).all()
    with pytest.raises(RuntimeError, match="already been resolved"):
        commit_promote(promotion, lambda row: None, sync)


def test_promotion_after_decode_takes_the_newest_token_from_the_reserved_slot(monkeypatch):
    from adaptive_sparse.migration import prepare_promote

    monkeypatch.delenv("EKV_CHUNK_AWARE_RETENTION", raising=False)
    log = []
    coordinator, request, logical = _demoted(log, length=20)
    reserved = coordinator.newest_slot(1)
    # decode step 1 (length 20 -> 21): the host already holds token 19, nothing to back up
    assert coordinator.backup_previous_token(1, 20) is None and log == []
    assert not coordinator.skip_first_backup[1]
    # decode step 2 (21 -> 22): token 20, in the reserved slot, goes to a new host row
    coordinator.backup_previous_token(1, 21)
    assert log == [("d2h", (reserved,), (220,))]
    assert coordinator.req_to_host_pool[1, 20] == 220 and coordinator.req_to_host_pool_allocated_len[1] == 21
    log.clear()
    request.length = 22
    extended = list(range(100, 122))
    coordinator.req_to_token[1, :22] = __import__("torch").tensor(extended)
    prepare_promote(coordinator, request, lambda: None, destinations=[30, 31, 32, 33, 34, 35])
    # host_len == length - 1 == 21: tokens 0..20 from host, token 21 from the reserved slot
    destination = _slots(range(30, 36))
    assert log == [("allocate", tuple(range(30, 36))), ("h2d", tuple(range(200, 221)), destination[:21]),
                   ("d2d", (reserved,), destination[21:22])]


def test_transactions_reject_bad_state_and_undo_failed_moves(monkeypatch):
    import torch

    from adaptive_sparse.migration import MigrationRequest, prepare_demote, prepare_promote

    monkeypatch.delenv("EKV_CHUNK_AWARE_RETENTION", raising=False)
    sync = lambda: None
    log = []
    coordinator, request, logical = _coordinator(log)
    with pytest.raises(ValueError, match="fully committed long resident"):
        prepare_demote(coordinator, MigrationRequest(row=1, length=7), sync)
    coordinator.mapping[logical[5]] = 0
    with pytest.raises(RuntimeError, match="missing physical locations"):
        prepare_demote(coordinator, request, sync)
    coordinator.mapping[logical[5]] = 3 * PAGE + 1
    coordinator.mapping[logical[4]] = 3 * PAGE + 1
    with pytest.raises(RuntimeError, match="misaligned"):
        prepare_demote(coordinator, request, sync)
    coordinator.mapping[logical[4:8]] = torch.arange(4) + 7 * PAGE               # page 7 twice
    with pytest.raises(RuntimeError, match="reuses a physical page"):
        prepare_demote(coordinator, request, sync)
    with pytest.raises(RuntimeError, match="hot-buffer capacity"):
        prepare_promote(coordinator, request, sync)

    log = []
    coordinator, request, logical = _coordinator(log, fail="d2h")
    with pytest.raises(OSError):
        prepare_demote(coordinator, request, sync)
    assert log == [("free_host", tuple(range(200, 220)))]                       # the host rows come back
    assert coordinator.req_to_host_pool_allocated_len[1] == 0 and coordinator.mapping[logical].min() > 0

    log = []
    coordinator, request, logical = _demoted(log)
    coordinator.req_to_host_pool[1, 7] = -1
    with pytest.raises(RuntimeError, match="missing committed host KV"):
        prepare_promote(coordinator, request, sync)
    coordinator.req_to_host_pool[1, 7] = 207
    coordinator.skip_first_backup[1] = False                                   # a decode step happened ...
    coordinator.req_to_device_buffer[1, HOT] = 0                               # ... but no newest token is held
    with pytest.raises(RuntimeError, match="latest device token"):
        prepare_promote(coordinator, request, sync)
    coordinator.skip_first_backup[1] = True
    coordinator.mover.fail = "h2d"
    with pytest.raises(OSError):
        prepare_promote(coordinator, request, sync)
    assert log == [("allocate", (50, 51, 52, 53, 54)), ("release", (50, 51, 52, 53, 54)), ("trim",)]
    assert coordinator.req_to_host_pool_allocated_len[1] == 20                 # the host copy survives
    with pytest.raises(ValueError, match="needs 5 destination pages"):
        prepare_promote(coordinator, request, sync, destinations=[1, 2])


def test_transactions_feed_the_bandwidth_estimator(monkeypatch):
    from adaptive_sparse.migration import (abort_promote, commit_demote, commit_promote, prepare_demote,
                                           prepare_promote)
    from adaptive_sparse.migration_budget import MigrationBandwidthEstimator

    monkeypatch.delenv("EKV_CHUNK_AWARE_RETENTION", raising=False)
    log = []
    coordinator, request, _ = _coordinator(log)
    coordinator.bandwidth = MigrationBandwidthEstimator(1 << 30, 0.5)
    seconds = iter([0.002, 0.004])                                 # the committed demotion, then promotion
    from adaptive_sparse import migration

    monkeypatch.setattr(migration.Transfer, "seconds", lambda self: next(seconds))
    prepared = prepare_demote(coordinator, request, lambda: None)
    assert coordinator.bandwidth.samples("demotion") == 0          # only committed migrations count
    commit_demote(prepared, lambda row: None, lambda: None)
    assert coordinator.bandwidth.bandwidth("demotion") == 20 * 96 / 0.002
    abort_promote(prepare_promote(coordinator, request, lambda: None))
    assert coordinator.bandwidth.samples("promotion") == 0
    commit_promote(prepare_promote(coordinator, request, lambda: None), lambda row: None, lambda: None)
    assert coordinator.bandwidth.samples("promotion") == 1
    assert coordinator.bandwidth.bandwidth("promotion") == 20 * 96 / 0.004


# ------------------------------------------------------------------ estimator


def test_estimator_ewma_closed_form_and_caps():
    est = MigrationBandwidthEstimator(1 << 30, 0.25)
    assert est.bandwidth("demotion") == float(1 << 30)
    assert est.observe("demotion", 0, 1.0) is None and est.samples("demotion") == 0
    assert est.observe("demotion", 4000, 2.0) == 2000.0
    assert est.bandwidth("demotion") == 2000.0
    assert est.observe("demotion", 8000, 1.0) == 8000.0
    assert est.bandwidth("demotion") == 0.25 * 8000 + 0.75 * 2000
    assert est.samples("demotion") == 2 and est.samples("promotion") == 0
    assert est.effective_byte_cap(10_000, 0) == 10_000
    assert est.effective_byte_cap(10_000, 1000) == math.floor(3500.0)
    assert est.snapshot() == {"demotion": 3500.0, "promotion": float(1 << 30)}
    for bad in ((True, 0.5), (0, 0.5), (1, 0.0), (1, 1.5), (1, float("nan"))):
        with pytest.raises(ValueError):
            MigrationBandwidthEstimator(*bad)
    with pytest.raises(ValueError):
        est.observe("sideways", 1, 1.0)
    with pytest.raises(ValueError):
        est.effective_byte_cap(0, 1)


# ------------------------------------------------------------------ Backing over a fake library


class _FakeLibrary:
    def __init__(self, reserved_units=2, *, partial_failure=False, rollback_on_failure=False,
                 close_failure=False):
        self.mapped = 0
        self.calls = []
        self.reserved_units = reserved_units
        self.partial_failure = partial_failure
        self.rollback_on_failure = rollback_on_failure
        self.close_failure = close_failure
        self.failure = None
        self.poisoned = False

    def ev_create(self, *_):
        return 1

    def ev_base(self, _):
        return 1 << 40

    def ev_backed(self, _):
        return self.mapped

    def ev_reserved(self, _):
        return self.reserved_units

    def ev_granularity(self, _):
        return 1

    def _commit(self, kind, count):
        if self.partial_failure:
            self.calls.append((kind + "-partial", count))
            self.failure = b"injected partial map failure"
            if not self.rollback_on_failure:
                self.mapped += max(0, count - 1)
                self.poisoned = True
            return 1
        self.mapped += count
        self.calls.append((kind, count))
        return 0

    def ev_ensure(self, _, ids, count):
        return self._commit("ensure", count)

    def ev_precommit(self, _, ids, count):
        return self._commit("precommit", count)

    def ev_drop(self, _, ids, count):
        self.mapped -= count
        self.calls.append(("drop", count))
        return 0

    def ev_poisoned(self, _):
        return int(self.poisoned)

    def ev_close(self, _):
        if self.close_failure:
            self.failure = b"injected close failure"
            return 1
        self.mapped = 0
        return 0

    def ev_error(self):
        return self.failure or b""


def _backing(library, chunk=1 << 20, units=2):
    with patch("elastic_kv.backing._load_library", return_value=library):
        return Backing(units * chunk, chunk, 0, library="fake.so")


def test_missing_library_has_actionable_build_error():
    _load_library.cache_clear()
    with patch("elastic_kv.backing.ct.CDLL", side_effect=OSError("missing native library")):
        with pytest.raises(RuntimeError, match="build_native.py"):
            _load_library("missing-libelastic-vmm.so")
    _load_library.cache_clear()


def test_outdated_library_requests_a_rebuild():
    _load_library.cache_clear()
    names = ("ev_create", "ev_ensure", "ev_precommit", "ev_drop", "ev_base", "ev_backed",
             "ev_reserved", "ev_granularity", "ev_close", "ev_error")
    library = SimpleNamespace(**{name: Mock() for name in names})
    with patch("elastic_kv.backing.ct.CDLL", return_value=library):
        with pytest.raises(RuntimeError, match="ABI is outdated"):
            _load_library("old-libelastic-vmm.so")
    _load_library.cache_clear()


def test_broker_environment_is_rejected(monkeypatch):
    monkeypatch.setenv("EKV_GLOBAL_BROKER_PATH", "/tmp/broker")
    with pytest.raises(ValueError, match="broker"):
        _backing(_FakeLibrary(2 << 20))


def test_backing_bookkeeping_over_fake_library():
    chunk = 1 << 20
    library = _FakeLibrary(4 * chunk)
    backing = _backing(library, chunk, 4)
    assert backing.ensure([0, 1]) == 2
    assert backing.ensure([1]) == 0
    assert backing.precommit([2, 1]) == 1
    assert backing.mapped_chunks == {0, 1}
    assert backing.ensure([2]) == 0            # precommitted: only waits
    assert backing.mapped_chunks == {0, 1, 2}
    assert backing.reclaim([1, 3], synchronize=False) == 1
    with pytest.raises(ValueError):
        backing.ensure([4])
    assert library.calls == [("ensure", 2), ("precommit", 1), ("ensure", 0), ("drop", 1)]
    metrics = backing.metrics
    assert metrics["ensure_calls"] == 2 and metrics["precommit_chunks"] == 1
    assert metrics["reclaim_chunks"] == 1 and metrics["backed_bytes"] == 2
    assert backing.broker_snapshot is None and backing.claim_broker_capacity("r", 1) is None
    backing.close()
    with pytest.raises(RuntimeError):
        backing.ensure([0])


def test_partial_failure_poisons_and_clean_rollback_allows_retry():
    library = _FakeLibrary(2 << 20, partial_failure=True)
    backing = _backing(library)
    with pytest.raises(RuntimeError, match="partial map failure"):
        backing.ensure([0, 1])
    assert backing._poisoned
    with pytest.raises(RuntimeError):
        backing.ensure([0])
    library = _FakeLibrary(2 << 20, partial_failure=True, rollback_on_failure=True)
    backing = _backing(library)
    with pytest.raises(RuntimeError, match="partial map failure"):
        backing.ensure([0, 1])
    assert backing.mapped_chunks == frozenset() and not backing._poisoned
    library.partial_failure = False
    assert backing.ensure([0, 1]) == 2
    backing.close()


def test_failed_close_can_be_retried_and_gc_closes():
    library = _FakeLibrary(2 << 20, close_failure=True)
    backing = _backing(library)
    backing.ensure([0])
    with pytest.raises(RuntimeError, match="close failure"):
        backing.close()
    library.close_failure = False
    backing.close()
    assert library.mapped == 0
    library = _FakeLibrary(2 << 20)

    def allocate_and_drop():
        _backing(library).ensure([0])

    allocate_and_drop()
    gc.collect()
    assert library.mapped == 0


def test_hot_buffer_rebase_keeps_the_lru_order():
    import torch

    from adaptive_sparse.swap_in import INT32_MIN, HotBuffers

    buffers = HotBuffers(2, 3, 100, 8, "cpu", with_bits=False)
    gen = torch.Generator().manual_seed(4)
    stamps = torch.randint(-50, (1 << 31) - 1, (2, 3, 8), generator=gen, dtype=torch.int64).to(torch.int32)
    stamps[0, 1, [2, 5]] = INT32_MIN                    # empty slots
    stamps[1, 2, 3] = stamps[1, 2, 6]                   # a tie: broken by slot index
    buffers.stamps.copy_(stamps)
    buffers.step = 123

    def lru_order(values):
        return [sorted(range(8), key=lambda s: (int(row[s]), s)) for row in values.reshape(-1, 8)]

    before = lru_order(stamps)
    assert buffers.steps_left() == (1 << 31) // 8192 - 1 - 123
    buffers.rebase()
    assert buffers.step == 0 and buffers.steps_left() == (1 << 31) // 8192 - 1
    assert lru_order(buffers.stamps) == before
    kept = buffers.stamps[buffers.stamps != INT32_MIN]
    assert int(kept.min()) >= -8 and int(kept.max()) < 0
    assert (buffers.stamps == INT32_MIN).sum() == 2


def test_block_segments_hand_case_and_plane_layout_equivalence():
    from adaptive_sparse.kv_pool import BlockSegments, PlanePoolLayout

    # Two segments, 100-byte pages in 256-byte chunks.
    seg = BlockSegments([(0, 100), (1000, 100)], page_bytes=100, num_blocks=8, allocation_bytes=1800,
                        chunk_bytes=256)
    assert seg.chunks([2]) == {0, 1, 4, 5}                      # bytes 200-299 and 1200-1299
    assert seg.sink_chunks() == {0, 3, 4}                        # block 0: bytes 0-99 and 1000-1099
    with pytest.raises(ValueError, match="Invalid KV block"):
        seg.chunks([8])
    with pytest.raises(ValueError, match="exceed"):
        BlockSegments([(0, 100), (1000, 100)], 100, 9, 1800, 256)
    # The block-gather geometry (36 layers x K/V planes of 20,000 blocks of 32 KiB) projects the
    # same chunks through either description.
    layout = PlanePoolLayout(layers=36, kv=2, rows=20000, row_bytes=32768)
    segments = BlockSegments([(layout.plane_offset(l, kv), 32768) for l in range(36) for kv in range(2)],
                             32768, 20000, layout.capacity_bytes, layout.chunk_bytes)
    for blocks in ([0], [1, 63, 64], [19999], list(range(100, 140))):
        assert segments.chunks(blocks) == layout.chunks_for_slots(blocks)


# ------------------------------------------------------------------ SGLang-convention swap-in (host checks)

def test_hisparse_swap_host_checks():
    import torch

    from adaptive_sparse.hisparse_swap import _row_layout, host_device_pointer, load_blocks_to_device_buffer_mha

    k = torch.zeros((10, 2, 8), dtype=torch.bfloat16)
    v = torch.zeros((10, 2, 8), dtype=torch.bfloat16)
    row_bytes, row_stride, _, rows = _row_layout(k, v, "cache")
    assert (row_bytes, row_stride, rows) == (32, 32, 10)
    with pytest.raises(ValueError, match="must share shape"):
        _row_layout(k, v[:, :1], "cache")
    with pytest.raises(ValueError, match="rows must be contiguous"):
        _row_layout(k.transpose(1, 2), v.transpose(1, 2), "cache")
    with pytest.raises(ValueError, match="pinned CPU memory"):
        host_device_pointer(k)                                     # pageable host memory
    small = torch.zeros((1, 1), dtype=torch.int32)
    with pytest.raises(ValueError, match="need GPU tensors"):     # no CPU fallback
        load_blocks_to_device_buffer_mha(small, small, small, small, k, v, k, v, small, small[0], small[0], small,
                                         32, 1, 1)


# ------------------------------------------------------------------ PlaneProjection


class _RecordingBacking:
    """Records the chunk ids a PlaneProjection sends to its backing."""

    def __init__(self, capacity_bytes, chunk_bytes, device):
        self.created = (capacity_bytes, chunk_bytes, device)
        self.calls = []
        self.backed_bytes = 0
        self.metrics = {"ensure_calls": 0}
        self.raw = None

    def ensure(self, ids):
        self.calls.append(("ensure", sorted(ids)))

    def precommit(self, ids):
        self.calls.append(("precommit", sorted(ids)))

    def reclaim(self, ids, *, synchronize):
        self.calls.append(("reclaim", sorted(ids), synchronize))


def test_plane_projection_commits_each_logical_chunk_in_every_plane():
    """elastic_kv/adapter.py:82-138: logical chunk c is chunk p * plane_chunks + c of plane p."""
    import torch

    from elastic_kv.adapter import PlaneProjection

    projection = PlaneProjection(20, 3, 8, 1, backing_factory=_RecordingBacking)
    backing = projection.backing
    assert (projection.plane_chunks, projection.plane_stride) == (3, 24)
    assert backing.created == (72, 8, 1)
    projection.ensure([0, 2])
    projection.ensure([2])                                   # held and ready: no call
    assert projection.precommit([2, 1]) == 1                 # only chunk 1 is new
    assert projection.precommit([1]) == 0
    assert projection.mapped_chunks == {0, 2} and projection.precommitted_chunks == {1}
    assert projection.metrics["precommitted_chunks"] == 1
    projection.ensure([1])                                   # waits for the precommitted chunk
    assert projection.mapped_chunks == {0, 1, 2} and projection.precommitted_chunks == set()
    projection.reclaim([2, 5], synchronize=False)
    assert projection.allocated_chunks == {0, 1}
    assert backing.calls == [("ensure", [0, 2, 3, 5, 6, 8]), ("precommit", [1, 4, 7]), ("ensure", [1, 4, 7]),
                             ("reclaim", [2, 5, 8], False)]
    backing.raw = torch.arange(72, dtype=torch.uint8)
    views = projection.views(torch.int16, (2, 5))
    assert [v.shape for v in views] == [(2, 5)] * 3
    assert [v.view(torch.uint8)[0, :2].tolist() for v in views] == [[0, 1], [24, 25], [48, 49]]


def test_hot_buffers_refuse_a_slot_base_on_the_sink():
    import torch

    from adaptive_sparse.swap_in import HotBuffers

    with pytest.raises(ValueError, match="slot_base must be >= 1"):
        HotBuffers(1, 2, 16, 4, "cpu", slot_base=torch.tensor([0, 4]))
    assert HotBuffers(1, 2, 16, 4, "cpu", slot_base=torch.tensor([1, 5])).slot_base.tolist() == [1, 5]
