"""GPU tests of the HIP VMM backing and the gathers that read through it.

Mirror the reference's GPU tests: tests/test_backing.py:370-413 (map, hole,
reclaim, precommit, zero on commit, stable VA) and tests/test_graph_backing.py
(graph replay across reclaim and recommit at a stable VA), plus the gather
micro-benchmark's exact payload checks (scripts/bench_virtual_addressing.py:
43-88) run through a real VMM arena.
"""

import numpy as np
import pytest
import torch

from elastic_kv.backing import DEFAULT_CHUNK_BYTES, Backing
from experimental.resident_arena import VmmResidentArena
from experimental.sparse_read import gather_rows
from experimental.virtual_layout import VirtualKVLayout

pytestmark = pytest.mark.gpu


def test_spare_pool_recycles_reclaimed_chunks_zeroed(gpu):
    # With a spare pool, reclaimed chunks keep their physical memory and the next
    # ensure maps it at other addresses: the data written there before must not
    # show (every committed chunk is zero-filled), the accounting must follow,
    # and lowering the limit or closing must give the memory back.
    chunk = DEFAULT_CHUNK_BYTES
    backing = Backing(8 * chunk, chunk_bytes=chunk, device=0, spare_chunks=3)
    try:
        assert backing.ensure(range(6)) == 6
        raw = backing.raw
        for i in range(6):
            raw[i * chunk:(i + 1) * chunk].fill_(i + 1)
        assert backing.reclaim([2, 3, 4, 5]) == 4
        assert backing.spare_bytes == 3 * chunk and backing.backed_bytes == 2 * chunk
        assert backing.metrics["held_bytes"] == 5 * chunk and backing.metrics["spare_bytes"] == 3 * chunk
        assert backing.ensure([6, 7, 3]) == 3                     # all three from the pool
        assert backing.spare_bytes == 0 and backing.backed_bytes == 5 * chunk
        for i in (3, 6, 7):
            assert torch.count_nonzero(raw[i * chunk:(i + 1) * chunk]).item() == 0, i
        for i in (0, 1):
            assert raw[i * chunk:(i + 1) * chunk].eq(i + 1).all().item()
        raw[6 * chunk:7 * chunk].fill_(9)
        assert backing.reclaim([6, 7]) == 2 and backing.spare_bytes == 2 * chunk
        backing.set_spare_chunks(1)
        assert backing.spare_bytes == chunk
        assert backing.ensure([6]) == 1 and backing.spare_bytes == 0
        assert torch.count_nonzero(raw[6 * chunk:7 * chunk]).item() == 0
        backing.set_spare_chunks(0)
        assert backing.reclaim([6]) == 1 and backing.spare_bytes == 0
        with pytest.raises(ValueError, match="spare_chunks"):
            backing.set_spare_chunks(9)
        backing.set_spare_chunks(4)
        assert backing.reclaim([0, 1]) == 2 and backing.spare_bytes == 2 * chunk
        del raw
    finally:
        torch.cuda.synchronize()
        backing.close()


def test_release_and_recommit_one_hole(gpu):
    chunk = DEFAULT_CHUNK_BYTES
    backing = Backing(5 * chunk - 17, chunk_bytes=chunk, device=0)
    try:
        assert backing.ensure([0, 1, 2, 4]) == 4
        assert backing.reserved_bytes == 5 * chunk
        assert backing.backed_bytes == 4 * chunk
        raw = backing.raw
        base = raw.data_ptr()
        assert base == backing.base
        assert raw.numel() == 5 * chunk - 17
        assert base % chunk == 0, "reservation should be chunk aligned"
        views = {i: raw[i * chunk:(i + 1) * chunk] for i in (0, 1, 2, 4)}
        for i in (0, 1, 2, 4):
            assert torch.count_nonzero(views[i]).item() == 0, "new chunks are zero-filled"
        for i, value in ((0, 11), (1, 22), (2, 33), (4, 55)):
            views[i].fill_(value)
        assert backing.reclaim([1, 3, 1]) == 1
        assert backing.mapped_chunks == {0, 2, 4}
        assert backing.backed_bytes == 3 * chunk
        for i, value in ((0, 11), (2, 33), (4, 55)):
            assert views[i].eq(value).all().item()
        assert backing.precommit([1]) == 1
        assert backing.mapped_chunks == {0, 2, 4}
        assert backing.backed_bytes == 4 * chunk
        assert backing.ensure([1]) == 0
        assert backing.mapped_chunks == {0, 1, 2, 4}
        assert backing.raw.data_ptr() == base
        assert views[1].data_ptr() == base + chunk
        assert torch.count_nonzero(views[1]).item() == 0
        for i, value in ((0, 11), (2, 33), (4, 55)):
            assert views[i].data_ptr() == base + i * chunk
            assert views[i].eq(value).all().item()
        metrics = backing.metrics
        assert metrics["ensure_chunks"] == 4 and metrics["reclaim_chunks"] == 1
        assert metrics["precommit_chunks"] == 1
    finally:
        backing.close()


def test_admission_precommits_lookahead_chunks_of_a_real_backing(gpu):
    from elastic_kv.admission import PhysicalAdmission

    chunk = DEFAULT_CHUNK_BYTES
    slot_bytes = 512
    backing = Backing(8 * chunk, chunk_bytes=chunk, device=0)
    try:
        assert backing.ensure([0]) == 1
        ctrl = PhysicalAdmission([backing], slot_bytes, chunk, precommit_lookahead=2, precommit_limit=2,
                                 device=0)
        # The free device memory bounds nothing here: slots of chunks 0-2.
        per_chunk = chunk // slot_bytes
        assert ctrl.physical_available_tokens(3 * per_chunk - 1, [(1, 3 * per_chunk)]) == 3 * per_chunk - 1
        admitted = [(1, per_chunk + 5)]                    # ends inside chunk 1
        assert backing.ensure([0, 1]) == 1
        added = ctrl.precommit_after(admitted, backing.reserved_bytes // chunk,
                                     lambda c: c not in backing.mapped_chunks)
        assert added == [2]                                # chunk 1 is live; its successor is prewarmed
        assert ctrl.backed_chunks() == {0, 1, 2}
        assert backing.backed_bytes == 3 * chunk and backing.mapped_chunks == {0, 1}
        assert backing.ensure([2]) == 0                    # already mapped; the zero fill is fenced here
        ctrl.admitted([2])
        assert torch.count_nonzero(backing.raw[2 * chunk:3 * chunk]).item() == 0
        assert ctrl.counters["precommit_chunks"] == 1
    finally:
        backing.close()


def test_errors_are_reported_not_fatal(gpu):
    backing = Backing(2 * DEFAULT_CHUNK_BYTES, device=0)
    try:
        with pytest.raises(ValueError):
            backing.ensure([2])
        with pytest.raises(RuntimeError, match="sink"):
            backing.raw
        assert backing.ensure([0, 0, 1]) == 2
        assert backing.ensure([1]) == 0
        assert backing.reclaim([1]) == 1 and backing.reclaim([1]) == 0
    finally:
        backing.close()
    with pytest.raises(RuntimeError):
        Backing(DEFAULT_CHUNK_BYTES, chunk_bytes=DEFAULT_CHUNK_BYTES + 1, device=0)


def test_graph_replays_across_reclaim_and_recommit(gpu):
    chunk = 2 << 20
    backing = Backing(4 * chunk, chunk_bytes=chunk, device=0)
    try:
        assert backing.ensure([0, 1, 2]) == 3
        raw = backing.raw
        base = raw.data_ptr()
        raw[0] = 7
        raw[chunk] = 23
        raw[2 * chunk] = 41
        indices = torch.tensor([chunk, 2 * chunk, 0], device=gpu)
        graph = torch.cuda.CUDAGraph()
        torch.cuda.synchronize()
        with torch.cuda.graph(graph):
            result = torch.index_select(raw, 0, indices)

        def replay(offsets, expected):
            indices.copy_(torch.tensor(offsets, device=gpu))
            graph.replay()
            assert result.tolist() == expected
            assert backing.raw.data_ptr() == base

        replay([chunk, 2 * chunk, 0], [23, 41, 7])
        torch.cuda.synchronize()
        assert backing.reclaim([1], synchronize=False) == 1
        replay([2 * chunk, 0, 0], [41, 7, 7])
        assert backing.ensure([1]) == 1
        raw[chunk] = 97
        replay([chunk, 2 * chunk, 0], [97, 41, 7])
        del graph, result
    finally:
        torch.cuda.synchronize()
        backing.close()


def support_sets(length, selected, seed=137):
    import random

    rng = random.Random(seed)
    clustered = set()
    run = max(1, selected // 8)
    while len(clustered) < selected:
        begin = rng.randrange(length)
        for step in range(min(run, selected - len(clustered))):
            clustered.add((begin + step) % length)
    return {"contiguous": list(range(selected)), "uniform_random": rng.sample(range(length), selected),
            "synthetic_clustered": sorted(clustered)}


@pytest.mark.parametrize("width", [256, 3])
def test_gather_rows_through_vmm_arena(gpu, coracle, width):
    """scripts/bench_virtual_addressing.py:43-88 at reduced size, bit-exact."""
    batch, length, selected = 3, 4096 if width == 256 else 700, 512
    layout = VirtualKVLayout(batch, length, width)
    arena = VmmResidentArena(layout)
    try:
        for req in range(batch):
            arena.reserve(req, length)
            view = arena.row_view(req, length, torch.bfloat16)
            values = (torch.arange(length * width, device=gpu) + req * 17) % 97
            view.copy_(values.reshape(length, width))
        del view
        raw = arena.backing.raw.view(torch.bfloat16)
        request_ids = torch.arange(batch, device=gpu, dtype=torch.int64).flip(0)
        lengths = torch.full((batch,), length, device=gpu, dtype=torch.int64)
        count = batch * length
        table = torch.arange(count, 0, -1, device=gpu, dtype=torch.int64).reshape(batch, length)
        flat = torch.arange(count, device=gpu, dtype=torch.int64)
        addresses = (layout.chunk_bytes // layout.itemsize + (flat // length) * (layout.request_bytes // layout.itemsize)
                     + (flat % length) * width)
        offsets = torch.zeros(count + 1, device=gpu, dtype=torch.int64)
        offsets[table.flatten()] = addresses
        output = torch.empty((batch, selected, width), device=gpu, dtype=torch.bfloat16)
        raw_host = raw.view(torch.uint16).cpu().numpy()
        for name, support in support_sets(length, selected).items():
            positions = torch.tensor(support, device=gpu, dtype=torch.int64).expand(batch, -1).contiguous()
            columns = torch.arange(width, device=gpu)
            expected = ((positions.clamp_min(0)[..., None] * width + columns
                         + request_ids[:, None, None] * 17) % 97).to(torch.bfloat16)
            for indirect in (False, True):
                gather_rows(raw, positions, request_ids, lengths, table, offsets, output, layout,
                            indirect=indirect)
                assert torch.equal(output, expected), (name, indirect)
                for invalid in (-1, length):
                    bad = positions.clone()
                    bad[:, 0] = invalid
                    want = expected.clone()
                    want[:, 0] = 0
                    gather_rows(raw, bad, request_ids, lengths, table, offsets, output, layout,
                                indirect=indirect)
                    assert torch.equal(output, want), (name, invalid, indirect)
                oracle_out = coracle.gather_rows(raw_host, positions.cpu().numpy(), request_ids.cpu().numpy(),
                                                 lengths.cpu().numpy(), table.cpu().numpy(),
                                                 offsets.cpu().numpy(), width, layout.request_bytes // 2,
                                                 layout.chunk_bytes // 2, indirect)
                gather_rows(raw, positions, request_ids, lengths, table, offsets, output, layout,
                            indirect=indirect)
                assert np.array_equal(output.view(torch.uint16).cpu().numpy(), oracle_out)
        pointer, before = arena.backing.base, arena.backing.backed_bytes
        del raw, output, expected
        arena.resize_quiescent(0, 0)
        assert arena.backing.base == pointer
        assert before - arena.backing.backed_bytes == layout.request_bytes
    finally:
        arena.close()


def test_decode_step_graph_replays_across_remap(gpu):
    """Lookup + compaction + gather captured in one graph, replayed with new Top-K
    contents and across a reclaim/recommit of pool chunks (stable VA); every
    replay must equal an eager run of the same step."""
    from adaptive_sparse.kv_pool import PlanePoolLayout
    from adaptive_sparse.resident_lookup import build_residency_bits, resolve_resident
    from adaptive_sparse.sparse_read import gather_kv

    L, R, T, K, C = 3, 4, 2048, 64, 256
    layout = PlanePoolLayout(layers=L, kv=2, rows=1 + R * C, row_bytes=512)
    backing = Backing(layout.capacity_bytes, layout.chunk_bytes, device=0)
    try:
        backing.ensure(range(backing.chunk_count))
        raw = backing.raw
        gen = torch.Generator(device=gpu).manual_seed(5)
        raw.view(torch.bfloat16).normal_(generator=gen)
        planes = layout.kv_planes(backing.base, 0, owner=backing)
        table = torch.zeros((L, R, T), dtype=torch.int32, device=gpu)
        perm = torch.rand((L, R, C), generator=gen, device=gpu).argsort(-1).to(torch.int32)
        table[:, :, T - C:] = perm + (torch.arange(R, device=gpu, dtype=torch.int32) * C + 1).view(1, R, 1)
        bits = build_residency_bits(table)
        rows = torch.arange(R, device=gpu)
        lengths = torch.full((R,), T, dtype=torch.int32, device=gpu)
        topk = torch.zeros((L, R, K), dtype=torch.int32, device=gpu)
        slots = torch.zeros((L, R, K), dtype=torch.int32, device=gpu)
        misses = torch.zeros_like(slots)
        counts = torch.zeros((L, R), dtype=torch.int32, device=gpu)
        out = torch.zeros((R, L, 2, K, 256), dtype=torch.bfloat16, device=gpu)

        def step():
            resolve_resident(topk, table, None, rows, lengths, rows, slots, 1, misses=misses, miss_count=counts,
                             resident_bits=bits)
            gather_kv(planes, slots, out)

        def new_topk(seed):
            g = torch.Generator(device=gpu).manual_seed(seed)
            picks = torch.rand((L, R, T), generator=g, device=gpu).argsort(-1)[..., :K]
            topk.copy_(picks.to(torch.int32))

        new_topk(0)
        step()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        for seed in range(1, 6):
            new_topk(seed)
            step()                                   # eager reference of this step
            eager = (slots.clone(), misses.clone(), counts.clone(), out.clone())
            slots.zero_(), misses.zero_(), counts.zero_(), out.zero_()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(slots, eager[0]) and torch.equal(counts, eager[2]), seed
            assert torch.equal(out, eager[3]), seed
            for l in range(L):
                for r in range(R):
                    c = int(counts[l, r])
                    assert torch.equal(misses[l, r, :c], eager[1][l, r, :c])
            if seed == 3:
                # Unmap and recommit a pool chunk between replays (same VA, zero-filled), then
                # restore its bytes: the graph keeps working against the stable address.
                chunk = backing.chunk_count - 1
                saved = raw.narrow(0, chunk * layout.chunk_bytes, layout.chunk_bytes).clone()
                torch.cuda.synchronize()
                assert backing.reclaim([chunk], synchronize=False) == 1
                assert backing.ensure([chunk]) == 1
                restored = raw.narrow(0, chunk * layout.chunk_bytes, layout.chunk_bytes)
                assert torch.count_nonzero(restored).item() == 0
                restored.copy_(saved)
                assert backing.raw.data_ptr() == backing.base
        del graph
    finally:
        torch.cuda.synchronize()
        backing.close()
