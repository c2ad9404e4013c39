"""GPU tests of page migration: pack/unpack through pinned host, transactions.

The round trip is self-pinning: destination pages must hold exactly the
bytes the source pages held before demotion (the reference's bitwise
migration check, adaptive_sparse/logical_shadow.py:88-123, compares the same
way through int16 views). Packing is also checked against the oracle.
"""

import numpy as np
import pytest
import torch

from adaptive_sparse.kv_pool import BlockMajorLayout
from adaptive_sparse.migration import (
    MigrationCoordinator, MigrationRequest, abort_demote, abort_promote, commit_demote, commit_promote,
    prepare_demote, prepare_promote,
)
from adaptive_sparse.migration_engine import MigrationEngine, PagedKVPool

pytestmark = pytest.mark.gpu

# The migration block of the page-migration workload: 16 tokens x 8 heads x 128 bf16 per plane,
# 36 layers x K/V planes -> 2.25 MiB per block.
BLOCK = dict(layers=36, kv=2, row_bytes=16 * 8 * 128 * 2)


def fill(pool, pages, seed):
    gen = torch.Generator(device=pool.device).manual_seed(seed)
    for page in pages:
        pool.page_view(page).copy_(torch.randint(0, 256, (pool.layout.block_bytes,), dtype=torch.uint8,
                                                 device=pool.device, generator=gen))


@pytest.mark.parametrize("sub_batch", [5, 64])
def test_round_trip_is_byte_exact_and_pack_matches_oracle(gpu, coracle, sub_batch):
    layout = BlockMajorLayout(blocks=48, **BLOCK)
    pool = PagedKVPool(layout, device=0)
    try:
        rng = np.random.default_rng(sub_batch)
        live = sorted(rng.choice(np.arange(1, 48), size=24, replace=False).tolist())
        pool.allocate(live)
        fill(pool, live, 1)
        sources = rng.choice(live, size=13, replace=False).tolist()
        free = sorted(set(range(1, 48)) - set(live))
        targets = rng.choice(free, size=13, replace=False).tolist()
        before = {p: pool.page_view(p).clone() for p in sources}
        engine = MigrationEngine(pool, max_pages=16, sub_batch=sub_batch)
        pool.allocate(targets)
        host = engine.round_trip(sources, targets)
        engine.wait()
        for s, t in zip(sources, targets):
            assert torch.equal(pool.page_view(t), before[s]), (s, t)
        # the pinned host rows hold the demoted pages in order
        for i, s in enumerate(sources):
            assert torch.equal(engine.host[int(host.rows[i])], before[s].cpu())
        # pack == oracle gather of the same pool bytes (only mapped pages are copied to the host)
        raw = np.zeros(layout.capacity_bytes, dtype=np.uint8)
        for s in sources:
            raw[s * layout.block_bytes:(s + 1) * layout.block_bytes] = before[s].cpu().numpy()
        planes = pool.planes
        want = coracle.gather_kv(raw, planes.layer_stride, planes.kv_stride, planes.row_stride, planes.row_bytes,
                                 planes.rows, np.array(sources)[None, None, :].repeat(layout.layers, 0), layout.kv)
        packed = engine.out_staging[:13].view(13, layout.layers, layout.kv, layout.row_bytes).permute(1, 2, 0, 3)
        assert np.array_equal(packed.unsqueeze(0).cpu().numpy(), want)
        # demote side releases the sources; chunks only they used are unmapped
        backed = pool.backing.backed_bytes
        pool.release(sources)
        released = pool.trim()
        assert released > 0 and pool.backing.backed_bytes == backed - released
        for t in targets:
            assert torch.equal(pool.page_view(t), before[sources[targets.index(t)]])
    finally:
        pool.close()


def test_pack_and_unpack_take_a_device_tensor_of_pages(gpu):
    layout = BlockMajorLayout(blocks=16, **BLOCK)
    pool = PagedKVPool(layout, device=0)
    try:
        pages = [3, 7, 1, 12]
        pool.allocate(pages + [5, 9])
        fill(pool, pages, 2)
        engine = MigrationEngine(pool, max_pages=4)
        by_list, by_tensor = torch.zeros_like(engine.out_staging), torch.zeros_like(engine.out_staging)
        engine.pack(pages, by_list)
        engine.pack(torch.tensor(pages, device=pool.device), by_tensor)
        torch.cuda.synchronize()
        assert torch.equal(by_list, by_tensor)
        for i, page in enumerate(pages):
            assert torch.equal(by_list[i], pool.page_view(page))
        engine.unpack(torch.tensor([5, 9], device=pool.device), by_list, start=1)   # staging rows 1, 2: pages 7, 1
        engine.pack(torch.empty(0, dtype=torch.int64, device=pool.device), by_tensor)   # nothing to do
        torch.cuda.synchronize()
        assert torch.equal(pool.page_view(5), pool.page_view(7)) and torch.equal(pool.page_view(9), pool.page_view(1))
        assert torch.equal(by_list, by_tensor)
    finally:
        pool.close()


@pytest.mark.parametrize("sub_batch", [3, 64])
def test_trim_after_packed_event_overlaps_the_copies(gpu, sub_batch):
    # The sources are released and their chunks unmapped once the round trip's
    # pack has run (host waits on the `packed` event only), while the D2H,
    # H2D and unpacks queued behind them are still in flight; every target
    # page must still receive its source bytes.
    layout = BlockMajorLayout(blocks=64, **BLOCK)
    pool = PagedKVPool(layout, device=0)
    try:
        rng = np.random.default_rng(100 + sub_batch)
        live = sorted(rng.choice(np.arange(1, 64), size=30, replace=False).tolist())
        pool.allocate(live)
        fill(pool, live, 2)
        sources = rng.choice(live, size=20, replace=False).tolist()
        spare = next(p for p in live if p not in sources)      # released earlier, not fenced by the event
        free = sorted(set(range(1, 64)) - set(live))
        targets = rng.choice(free, size=20, replace=False).tolist()
        before = {p: pool.page_view(p).clone() for p in sources}
        torch.cuda.synchronize()
        engine = MigrationEngine(pool, max_pages=20, sub_batch=sub_batch)
        pool.allocate(targets)
        pool.release([spare])
        backed = pool.backing.backed_bytes
        host = engine.round_trip(sources, targets)
        assert host.packed is not None
        pool.release(sources)
        with pytest.raises(ValueError, match="released pages"):
            pool.trim(after=host.packed)
        idle = pool.pages.reclaimable_chunks()
        fenced = idle & set().union(*(pool.pages.chunks(p) for p in sources))
        released = pool.trim(after=host.packed, pages=sources)
        engine.wait()
        assert released == len(fenced) * layout.chunk_bytes > 0
        assert pool.backing.backed_bytes == backed - released
        # chunks the event does not fence (the spare's own) are left for a synchronized trim
        assert pool.pages.reclaimable_chunks() == idle - fenced
        assert pool.trim() == len(idle - fenced) * layout.chunk_bytes
        for s, t in zip(sources, targets):
            assert torch.equal(pool.page_view(t), before[s]), (s, t)
        for i, s in enumerate(sources):
            assert torch.equal(engine.host[int(host.rows[i])], before[s].cpu())
    finally:
        pool.close()


def test_transactions_demote_promote_cycle(gpu):
    layout = BlockMajorLayout(blocks=64, **BLOCK)
    pool = PagedKVPool(layout, device=0)
    try:
        engine = MigrationEngine(pool, max_pages=32, sub_batch=4)
        mapping = torch.zeros(100, dtype=torch.int64, device=gpu)
        pages = list(range(3, 3 + 20))
        pool.allocate(pages)
        fill(pool, pages, 7)
        logical = torch.arange(40, 60, device=gpu)
        mapping[logical] = torch.tensor(pages, device=gpu)
        original = {i: pool.page_view(p).clone() for i, p in enumerate(pages)}
        coordinator = MigrationCoordinator(pool, engine, mapping, keep_pages=6)
        request = MigrationRequest(row=2, logical=logical)
        published = []
        sync = torch.cuda.synchronize

        prepared = prepare_demote(coordinator, request, sync)
        assert len(prepared.retained_rows) == 6 and len(prepared.released_rows) == 14
        abort_demote(prepared)
        with pytest.raises(RuntimeError):
            abort_demote(prepared)
        assert engine.host_free.count == 32

        prepared = prepare_demote(coordinator, request, sync)
        backed = pool.backing.backed_bytes
        released = commit_demote(prepared, published.append, sync, trim_quiescent=pool.trim)
        assert published == [2] and prepared.status == "committed"
        assert (mapping[logical] == 0).all()
        assert released > 0 and pool.backing.backed_bytes == backed - released
        assert coordinator.hot[2] == tuple(pages[i] for i in prepared.retained_rows)
        with pytest.raises(RuntimeError):
            commit_demote(prepared, published.append, sync)

        promotion = prepare_promote(coordinator, request, sync)
        abort_promote(promotion)
        promotion = prepare_promote(coordinator, request, sync, destinations=list(range(40, 60)))
        grown = commit_promote(promotion, published.append, sync)
        assert published == [2, 2] and promotion.status == "committed"
        assert mapping[logical].tolist() == list(range(40, 60))
        assert grown >= 0 and 2 not in coordinator.host_backed and 2 not in coordinator.hot
        for i in range(20):
            assert torch.equal(pool.page_view(40 + i), original[i]), i
        assert engine.host_free.count == 32
        with pytest.raises(RuntimeError, match="missing committed host KV"):
            prepare_promote(coordinator, request, sync)
    finally:
        pool.close()


def test_back_to_back_demotes_and_promotes_without_host_syncs(gpu):
    # Consecutive calls reuse the device staging and released host rows; the
    # engine orders them with events, so no host synchronization is needed
    # between calls for every byte to land where it belongs.
    layout = BlockMajorLayout(blocks=40, **BLOCK)
    pool = PagedKVPool(layout, device=0)
    try:
        first, second = list(range(1, 9)), list(range(9, 17))
        pool.allocate(first + second)
        fill(pool, first + second, 3)
        before = {p: pool.page_view(p).clone() for p in first + second}
        engine = MigrationEngine(pool, max_pages=8, sub_batch=3)
        host_a = engine.demote(first)
        targets_a = list(range(17, 25))
        pool.allocate(targets_a)
        engine.promote(host_a, targets_a)
        engine.release_host(host_a)                  # its rows are reused by the next demote at once
        host_b = engine.demote(second)
        targets_b = list(range(25, 33))
        pool.allocate(targets_b)
        engine.promote(host_b, targets_b)
        engine.wait()
        for s, t in zip(first, targets_a):
            assert torch.equal(pool.page_view(t), before[s]), (s, t)
        for s, t in zip(second, targets_b):
            assert torch.equal(pool.page_view(t), before[s]), (s, t)
    finally:
        pool.close()


def test_full_tick_of_512_blocks_round_trips_byte_exact(gpu):
    # The page-migration workload at its own size: a 2048-block pool (4.5 GiB) with
    # 1024 live blocks; each of two ticks maps 512 fresh destination blocks, packs
    # 512 scattered sources into staging, copies them to pinned host and back,
    # unpacks them, and unmaps the chunks only the sources used once the packs have
    # run. Every destination must hold its source's bytes, every pinned host row its
    # source, and the pool must shrink by exactly the fenced chunks.
    blocks, live_count, move = 2048, 1024, 512
    layout = BlockMajorLayout(blocks=blocks, **BLOCK)
    pool = PagedKVPool(layout, device=0)
    try:
        rng = np.random.default_rng(512)
        live = sorted(rng.choice(np.arange(1, blocks), size=live_count, replace=False).tolist())
        pool.allocate(live)
        gen = torch.Generator(device=gpu).manual_seed(4)
        for page in live:
            pool.page_view(page).copy_(torch.randint(0, 256, (layout.block_bytes,), dtype=torch.uint8,
                                                     device=gpu, generator=gen))
        engine = MigrationEngine(pool, max_pages=move, sub_batch=64)
        for tick in range(2):
            sources = rng.choice(live, size=move, replace=False).tolist()
            free = sorted(set(range(1, blocks)) - set(live))
            targets = rng.choice(free, size=move, replace=False).tolist()
            snapshot = torch.empty((move, layout.block_bytes), dtype=torch.uint8, device=gpu)
            engine.pack(sources, snapshot)
            torch.cuda.synchronize()
            pool.allocate(targets)
            host = engine.round_trip(sources, targets)
            pool.release(sources)
            idle = pool.pages.reclaimable_chunks()
            fenced = idle & set().union(*(pool.pages.chunks(p) for p in sources))
            backed = pool.backing.backed_bytes
            released = pool.trim(after=host.packed, pages=sources)
            engine.wait()
            print(f"[migration] tick {tick}: {len(fenced)} chunks unmapped", flush=True)
            assert released == len(fenced) * layout.chunk_bytes > 0, tick
            assert pool.backing.backed_bytes == backed - released, tick
            for i, t in enumerate(targets):
                assert torch.equal(pool.page_view(t), snapshot[i]), (tick, i)
            rows = host.rows.tolist()
            for i in rng.choice(move, size=32, replace=False).tolist():   # pinned host rows, sampled
                assert torch.equal(engine.host[int(rows[i])], snapshot[i].cpu()), (tick, i)
            engine.release_host(host)
            live = sorted(set(live) - set(sources) | set(targets))
            del snapshot
    finally:
        torch.cuda.synchronize()
        pool.close()
