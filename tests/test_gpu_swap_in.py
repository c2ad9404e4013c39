"""GPU parity of the LRU swap-in and the promote-from-host copy against the oracle.

Each step: HIP lookup (bitmap) -> HIP swap-in -> promote from pinned host
(move_kv) -> gather. After every step the whole LRU state (table, bitmap,
slot owners, stamps), the patched slots and the promotion lists must equal
the oracle's, and every gathered K/V row must equal the pinned-host row of
its token.
"""

import numpy as np
import pytest
import torch

from adaptive_sparse.host_arena import HostArena
from adaptive_sparse.kv_pool import KVPlanes
from adaptive_sparse.resident_lookup import resolve_resident
from adaptive_sparse.sparse_read import gather_kv
from adaptive_sparse.swap_in import HotBuffers, move_kv, swap_in
from oracle import oracle as ref

pytestmark = pytest.mark.gpu


def bits_match(got, want):
    """A bitmap padded to whole 16-byte pieces holds the oracle's ceil(T / 32) words, then zeros."""
    words = want.shape[-1]
    return (got.shape[-1] == -(-words // 4) * 4 and np.array_equal(got[..., :words], want)
            and not got[..., words:].any())


@pytest.mark.parametrize("capacity", [64, 50])
def test_lookup_swap_promote_gather_cycle(gpu, capacity):
    L, R, T, K, row_bytes = 2, 3, 300, 32, 64
    rng = np.random.default_rng(capacity)
    buffers = HotBuffers(L, R, T, capacity, gpu)
    # Start with the 40 most recent tokens resident in random slots.
    recent = torch.arange(T - 40, T).expand(L, R, 40)
    local = torch.stack([torch.stack([torch.tensor(rng.permutation(capacity)[:40]) for _ in range(R)])
                         for _ in range(L)])
    buffers.install(recent, local)
    host_table = torch.arange(R * T, dtype=torch.int32).reshape(R, T)
    plane = R * T * row_bytes
    arena = HostArena(L * 2 * plane)
    try:
        arena.host.copy_(torch.randint(0, 256, (L * 2 * plane,), dtype=torch.uint8))
        host_planes = KVPlanes(base=arena.device_ptr, device=0, layers=L, kv=2, layer_stride=2 * plane,
                               kv_stride=plane, row_stride=row_bytes, row_bytes=row_bytes, rows=R * T, owner=arena)
        pool_rows = 1 + R * capacity
        pool = torch.zeros(L * 2 * pool_rows * row_bytes, dtype=torch.uint8, device=gpu)
        pool_planes = KVPlanes(base=pool.data_ptr(), device=0, layers=L, kv=2, layer_stride=2 * pool_rows * row_bytes,
                               kv_stride=pool_rows * row_bytes, row_stride=row_bytes, row_bytes=row_bytes,
                               rows=pool_rows, owner=pool)
        # Prefill the resident rows from the host copy (as a promotion of the installed tokens).
        first_src = host_table.to(gpu)[torch.arange(R).view(1, R, 1), recent.to(gpu)].expand(L, R, 40).contiguous()
        first_dst = (local.to(gpu) + buffers.slot_base.view(1, R, 1)).to(torch.int32).contiguous()
        move_kv(host_planes, first_src.to(torch.int32), pool_planes, first_dst,
                torch.full((L, R), 40, dtype=torch.int32, device=gpu))
        host = arena.host.numpy().reshape(L, 2, R * T, row_bytes)
        rows = torch.arange(R, device=gpu)
        lengths = torch.full((R,), T, dtype=torch.int32, device=gpu)
        state = {"table": buffers.table.cpu().numpy(), "slot_token": buffers.slot_token.cpu().numpy(),
                 "stamps": buffers.stamps.cpu().numpy()}
        for step in range(6):
            near = [np.concatenate([rng.choice(np.arange(T - 50, T), 24, replace=False),
                                    rng.choice(np.arange(0, T - 50), 8, replace=False)])
                    for _ in range(L * R)]
            topk = np.stack([rng.permutation(x) for x in near]).reshape(L, R, K)
            topk_d = torch.tensor(topk, dtype=torch.int32, device=gpu)
            slots = torch.empty((L, R, K), dtype=torch.int32, device=gpu)
            misses = torch.full((L, R, K), -1, dtype=torch.int32, device=gpu)
            counts = torch.empty((L, R), dtype=torch.int32, device=gpu)
            resolve_resident(topk_d, buffers.table, None, rows, lengths, rows, slots, 1, misses=misses,
                             miss_count=counts, resident_bits=buffers.bits)
            want_slots, want_misses, want_counts = ref.resolve_resident(
                topk, state["table"], None, np.arange(R), np.full(R, T), np.arange(R), 1,
                np.zeros((L, R, K), np.int32), with_misses=True)
            assert np.array_equal(slots.cpu().numpy(), want_slots), step
            assert np.array_equal(counts.cpu().numpy(), want_counts), step
            miss_np = np.full((L, R, K), -1, np.int32)
            for (layer, r), lanes in want_misses.items():
                miss_np[layer, r, :len(lanes)] = lanes
            promote_src = torch.full((L, R, K), -9, dtype=torch.int32, device=gpu)
            promote_dst = torch.full((L, R, K), -9, dtype=torch.int32, device=gpu)
            swap_in(topk_d, 1, rows, rows, slots, misses, counts, buffers, host_table.to(gpu), promote_src,
                    promote_dst)
            state = ref.swap_in(step, 1, topk, np.arange(R), np.arange(R), want_slots, miss_np, want_counts,
                                state["table"], state["slot_token"], state["stamps"],
                                buffers.slot_base.cpu().numpy(), host_table.numpy())
            assert np.array_equal(slots.cpu().numpy(), state["slots"]), step
            assert np.array_equal(buffers.table.cpu().numpy(), state["table"]), step
            assert np.array_equal(buffers.slot_token.cpu().numpy(), state["slot_token"]), step
            assert np.array_equal(buffers.stamps.cpu().numpy(), state["stamps"]), step
            assert bits_match(buffers.bits.cpu().numpy(), ref.residency_bits(state["table"])), step
            got_src, got_dst = promote_src.cpu().numpy(), promote_dst.cpu().numpy()
            for layer in range(L):
                for r in range(R):
                    c = want_counts[layer, r]
                    assert np.array_equal(got_src[layer, r, :c], state["promote_src"][layer, r, :c])
                    assert np.array_equal(got_dst[layer, r, :c], state["promote_dst"][layer, r, :c])
            move_kv(host_planes, promote_src, pool_planes, promote_dst, counts)
            out = torch.empty((R, L, 2, K, row_bytes), dtype=torch.uint8, device=gpu)
            gather_kv(pool_planes, slots, out)
            got = out.cpu().numpy()
            for layer in range(L):
                for r in range(R):
                    host_rows = host_table.numpy()[r, topk[layer, r]]
                    for kv in range(2):
                        assert np.array_equal(got[r, layer, kv], host[layer, kv, host_rows]), (step, layer, r, kv)
    finally:
        torch.cuda.synchronize()
        arena.close()


def test_width_changes_between_calls_keep_the_lru_order(gpu):
    # Every call has its own row width (1 .. 16 lanes). The LRU state must equal
    # the oracle's after each call, and each (layer, request) stream's promotion
    # count must equal the reference's dict replay (lru_misses) over the same
    # selections: a narrower call never evicts a slot that one of its hits reads.
    L, R, T, C = 2, 3, 120, 16
    rng = np.random.default_rng(41)
    buffers = HotBuffers(L, R, T, C, gpu)
    host_table = torch.arange(R * T, dtype=torch.int32).reshape(R, T)
    rows = torch.arange(R, device=gpu)
    lengths = torch.full((R,), T, dtype=torch.int32, device=gpu)
    state = {"table": buffers.table.cpu().numpy(), "slot_token": buffers.slot_token.cpu().numpy(),
             "stamps": buffers.stamps.cpu().numpy()}
    streams = {(layer, r): [] for layer in range(L) for r in range(R)}
    promoted = {key: [] for key in streams}
    widths = [16, 2, 9, 1, 16, 5, 3, 12, 1, 7, 16, 4, 2, 10, 6, 1, 13, 8]
    for step, K in enumerate(widths):
        topk = np.stack([rng.choice(np.arange(T - 40, T), K, replace=False) for _ in range(L * R)]).reshape(L, R, K)
        topk_d = torch.tensor(topk, dtype=torch.int32, device=gpu)
        slots = torch.empty((L, R, K), dtype=torch.int32, device=gpu)
        misses = torch.full((L, R, K), -1, dtype=torch.int32, device=gpu)
        counts = torch.empty((L, R), dtype=torch.int32, device=gpu)
        resolve_resident(topk_d, buffers.table, None, rows, lengths, rows, slots, 1, misses=misses,
                         miss_count=counts, resident_bits=buffers.bits)
        want_slots, want_misses, want_counts = ref.resolve_resident(
            topk, state["table"], None, np.arange(R), np.full(R, T), np.arange(R), 1,
            np.zeros((L, R, K), np.int32), with_misses=True)
        miss_np = np.full((L, R, K), -1, np.int32)
        for (layer, r), lanes in want_misses.items():
            miss_np[layer, r, :len(lanes)] = lanes
        src = torch.full((L, R, K), -9, dtype=torch.int32, device=gpu)
        dst = torch.full((L, R, K), -9, dtype=torch.int32, device=gpu)
        swap_in(topk_d, 1, rows, rows, slots, misses, counts, buffers, host_table.to(gpu), src, dst, check=True)
        state = ref.swap_in(step, 1, topk, np.arange(R), np.arange(R), want_slots, miss_np, want_counts,
                            state["table"], state["slot_token"], state["stamps"], buffers.slot_base.cpu().numpy(),
                            host_table.numpy())
        got_slots = slots.cpu().numpy()
        assert np.array_equal(got_slots, state["slots"]), (step, K)
        assert np.array_equal(buffers.table.cpu().numpy(), state["table"]), (step, K)
        assert np.array_equal(buffers.slot_token.cpu().numpy(), state["slot_token"]), (step, K)
        assert np.array_equal(buffers.stamps.cpu().numpy(), state["stamps"]), (step, K)
        for (layer, r), stream in streams.items():
            stream.append(topk[layer, r].tolist())
            promoted[(layer, r)].append(int(want_counts[layer, r]))
            # every lane reads its own token's slot after the call
            held = buffers.slot_token.cpu().numpy()[layer, r]
            local = got_slots[layer, r] - int(buffers.slot_base[r])
            assert held[local].tolist() == topk[layer, r].tolist(), (step, layer, r)
    for key, stream in streams.items():
        assert promoted[key] == ref.lru_misses(stream, C), key


def test_miss_entries_without_a_lane_record_empty_promotions(gpu):
    # A miss list the lookup did not write (lane -1, lane past the row) must not
    # leave stale promotion records behind for the move that follows.
    L, R, T, C, K = 1, 1, 64, 8, 4
    buffers = HotBuffers(L, R, T, C, gpu)
    topk = torch.tensor([[[5, 6, 7, 9]]], dtype=torch.int32, device=gpu)
    rows = torch.arange(R, device=gpu)
    slots = torch.zeros((L, R, K), dtype=torch.int32, device=gpu)
    misses = torch.tensor([[[0, -1, 99, 2]]], dtype=torch.int32, device=gpu)
    counts = torch.tensor([[4]], dtype=torch.int32, device=gpu)
    host_table = torch.arange(R * T, dtype=torch.int32, device=gpu).reshape(R, T)
    promote_src = torch.full((L, R, K), 77, dtype=torch.int32, device=gpu)
    promote_dst = torch.full((L, R, K), 77, dtype=torch.int32, device=gpu)
    swap_in(topk, 1, rows, rows, slots, misses, counts, buffers, host_table, promote_src, promote_dst)
    src, dst = promote_src.cpu().tolist()[0][0], promote_dst.cpu().tolist()[0][0]
    assert src[1] == dst[1] == -1 and src[2] == dst[2] == -1
    assert src[0] == 5 and src[3] == 7                      # lanes 0 and 2 select tokens 5 and 7
    assert dst[0] > 0 and dst[3] > 0 and dst[0] != dst[3]
    assert slots.cpu().tolist()[0][0][0] == dst[0] and slots.cpu().tolist()[0][0][2] == dst[3]
    table = buffers.table.cpu()[0, 0]
    assert table[5] == dst[0] and table[7] == dst[3] and int((table != 0).sum()) == 2


@pytest.mark.parametrize("counted", [False, True])
def test_an_empty_batch_leaves_the_hot_buffers_alone(gpu, counted):
    # topk [L, 0, K]: the selection's entries name batch rows that do not exist, so nothing is resident, evicted
    # or promoted; the call is still one step.
    L, R, T, C, K = 2, 3, 64, 8, 4
    buffers = HotBuffers(L, R, T, C, gpu, step_counter=counted)
    tokens = torch.arange(C, device=gpu).view(1, 1, C).expand(L, R, C)
    buffers.install(tokens, torch.arange(C, device=gpu).flip(0).view(1, 1, C).expand(L, R, C))
    before = [t.clone() for t in (buffers.table, buffers.bits, buffers.slot_token, buffers.stamps)]
    empty = torch.zeros((L, 0, K), dtype=torch.int32, device=gpu)
    selected = torch.tensor([0, 1], device=gpu)
    host_table = torch.arange(R * T, dtype=torch.int32, device=gpu).reshape(R, T)
    swap_in(empty, 1, torch.zeros(0, dtype=torch.int64, device=gpu), selected, empty.clone(), empty.clone(),
            torch.zeros((L, 0), dtype=torch.int32, device=gpu), buffers, host_table, empty.clone(), empty.clone(),
            check=True)
    torch.cuda.synchronize()
    for got, want in zip((buffers.table, buffers.bits, buffers.slot_token, buffers.stamps), before):
        assert torch.equal(got, want)
    assert buffers.step == 1
    if counted:
        assert int(buffers.step_counter.item()) == 1


def test_a_table_without_positions_is_refused(gpu):
    # With no token positions no miss can be inserted, and the promotions' host rows are read at position 0:
    # refused before anything is queued.
    L, R, C, K = 1, 2, 8, 4
    buffers = HotBuffers(L, R, 0, C, gpu)
    topk = torch.zeros((L, R, K), dtype=torch.int32, device=gpu)
    rows = torch.arange(R, device=gpu)
    lists = [torch.full((L, R, K), -7, dtype=torch.int32, device=gpu) for _ in range(4)]
    counts = torch.full((L, R), K, dtype=torch.int32, device=gpu)
    with pytest.raises(RuntimeError, match="no positions"):
        swap_in(topk, 1, rows, rows, lists[0], lists[1], counts, buffers,
                torch.zeros((R, 0), dtype=torch.int32, device=gpu), lists[2], lists[3])
    torch.cuda.synchronize()
    assert all(bool((t == -7).all()) for t in lists)


@pytest.mark.parametrize("bs", [2, 3])
def test_paged_blocks_lookup_and_swap_in_match_oracle(gpu, bs):
    # Top-K over blocks of bs tokens, -1 padding and rows shorter than the
    # table: lookup and swap-in state after every step equal the oracle's.
    L, R, T, C, K = 2, 3, 240, 32, 8   # C >= W = 16 or 24; evictions start within the 5 steps
    W = K * bs
    rng = np.random.default_rng(40 + bs)
    buffers = HotBuffers(L, R, T, C, gpu)
    host_table = torch.arange(R * T, dtype=torch.int32).reshape(R, T)
    lengths = np.array([T, T - 5, T - 17])
    rows = torch.arange(R, device=gpu)
    state = {"table": buffers.table.cpu().numpy(), "slot_token": buffers.slot_token.cpu().numpy(),
             "stamps": buffers.stamps.cpu().numpy()}
    blocks_total = T // bs
    for step in range(5):
        topk = np.empty((L, R, K), np.int64)
        for layer in range(L):
            for r in range(R):
                recent = rng.choice(np.arange(blocks_total - 12, blocks_total), 6, replace=False)
                old = rng.choice(np.arange(0, blocks_total - 12), K - 6, replace=False)
                picks = rng.permutation(np.concatenate([recent, old]))
                picks[rng.random(K) < 0.15] = -1
                topk[layer, r] = picks
        topk_d = torch.tensor(topk, dtype=torch.int32, device=gpu)
        slots = torch.empty((L, R, W), dtype=torch.int32, device=gpu)
        misses = torch.full((L, R, W), -1, dtype=torch.int32, device=gpu)
        counts = torch.empty((L, R), dtype=torch.int32, device=gpu)
        resolve_resident(topk_d, buffers.table, None, rows, torch.tensor(lengths, dtype=torch.int32, device=gpu),
                         rows, slots, bs, misses=misses, miss_count=counts, resident_bits=buffers.bits)
        want_slots, want_misses, want_counts = ref.resolve_resident(
            topk, state["table"], None, np.arange(R), lengths, np.arange(R), bs,
            np.zeros((L, R, W), np.int32), with_misses=True)
        assert np.array_equal(slots.cpu().numpy(), want_slots), step
        assert np.array_equal(counts.cpu().numpy(), want_counts), step
        miss_np = np.full((L, R, W), -1, np.int32)
        for (layer, r), lanes in want_misses.items():
            miss_np[layer, r, :len(lanes)] = lanes
        assert np.array_equal(misses.cpu().numpy(), miss_np), step
        promote_src = torch.full((L, R, W), -9, dtype=torch.int32, device=gpu)
        promote_dst = torch.full((L, R, W), -9, dtype=torch.int32, device=gpu)
        swap_in(topk_d, bs, rows, rows, slots, misses, counts, buffers, host_table.to(gpu), promote_src,
                promote_dst)
        state = ref.swap_in(step, bs, topk, np.arange(R), np.arange(R), want_slots, miss_np, want_counts,
                            state["table"], state["slot_token"], state["stamps"], buffers.slot_base.cpu().numpy(),
                            host_table.numpy())
        assert np.array_equal(slots.cpu().numpy(), state["slots"]), step
        assert np.array_equal(buffers.table.cpu().numpy(), state["table"]), step
        assert np.array_equal(buffers.slot_token.cpu().numpy(), state["slot_token"]), step
        assert np.array_equal(buffers.stamps.cpu().numpy(), state["stamps"]), step
        assert bits_match(buffers.bits.cpu().numpy(), ref.residency_bits(state["table"])), step
        got_src, got_dst = promote_src.cpu().numpy(), promote_dst.cpu().numpy()
        for layer in range(L):
            for r in range(R):
                c = want_counts[layer, r]
                assert np.array_equal(got_src[layer, r, :c], state["promote_src"][layer, r, :c])
                assert np.array_equal(got_dst[layer, r, :c], state["promote_dst"][layer, r, :c])


def test_rebase_mid_stream_changes_no_decision(gpu):
    # Two hot-buffer sets see the same Top-K stream; one is rebased after step 2
    # (as swap_in does before its stamps would overflow). Every later table,
    # slot and promotion must be the same.
    L, R, T, C, K = 2, 2, 400, 24, 16
    rng = np.random.default_rng(77)
    plain, rebased = HotBuffers(L, R, T, C, gpu), HotBuffers(L, R, T, C, gpu)
    rows = torch.arange(R, device=gpu)
    lengths = torch.full((R,), T, dtype=torch.int32, device=gpu)
    host_table = torch.arange(R * T, dtype=torch.int32, device=gpu).reshape(R, T)
    for step in range(6):
        topk = torch.tensor(np.stack([rng.permutation(np.concatenate([
            rng.choice(np.arange(T - 40, T), 12, replace=False), rng.choice(np.arange(0, T - 40), 4, replace=False)]))
            for _ in range(L * R)]).reshape(L, R, K), dtype=torch.int32, device=gpu)
        results = []
        for buffers in (plain, rebased):
            if buffers is rebased and step == 3:
                buffers.rebase()
            slots = torch.empty((L, R, K), dtype=torch.int32, device=gpu)
            misses = torch.full((L, R, K), -1, dtype=torch.int32, device=gpu)
            counts = torch.empty((L, R), dtype=torch.int32, device=gpu)
            resolve_resident(topk, buffers.table, None, rows, lengths, rows, slots, 1, misses=misses,
                             miss_count=counts, resident_bits=buffers.bits)
            src = torch.full((L, R, K), -9, dtype=torch.int32, device=gpu)
            dst = torch.full((L, R, K), -9, dtype=torch.int32, device=gpu)
            swap_in(topk, 1, rows, rows, slots, misses, counts, buffers, host_table, src, dst)
            results.append((slots.cpu(), counts.cpu(), src.cpu(), dst.cpu(), buffers.table.cpu(),
                            buffers.slot_token.cpu()))
        for a, b in zip(*results):
            assert torch.equal(a, b), step
    assert rebased.step == 3 and plain.step == 6


def global_table(buffers):
    """The token -> global slot table of a HotBuffers, whichever form it keeps."""
    table = buffers.table.cpu().numpy().astype(np.int64)
    if buffers.table.dtype == torch.int16:
        base = buffers.slot_base.cpu().numpy().reshape(1, -1, 1)
        table = np.where(table > 0, base + table - 1, 0)
    return table


@pytest.mark.parametrize("table_dtype", [torch.int32, torch.int16])
def test_whole_decode_step_replays_from_one_graph(gpu, table_dtype):
    # Lookup -> swap-in (device step counter) -> promote from pinned host -> gather,
    # captured once and replayed for five steps with new Top-K contents. After every
    # replay the LRU state equals the oracle's at that step and every gathered row is
    # its token's host row. Replays 3 and 4 carry a padded batch row (length 0, as a
    # graph captured for a larger batch runs): it must yield -1 slots, no misses, no
    # promotions and zero rows, and leave its hot buffer untouched.
    L, R, T, K, row_bytes, capacity = 2, 3, 300, 32, 64, 64
    rng = np.random.default_rng(21)
    buffers = HotBuffers(L, R, T, capacity, gpu, step_counter=True, table_dtype=table_dtype)
    local = buffers.slot_base if table_dtype == torch.int16 else None
    host_table = torch.arange(R * T, dtype=torch.int32).reshape(R, T)
    host_table_d = host_table.to(gpu)
    plane = R * T * row_bytes
    arena = HostArena(L * 2 * plane)
    try:
        arena.host.copy_(torch.randint(0, 256, (L * 2 * plane,), dtype=torch.uint8))
        host_planes = KVPlanes(base=arena.device_ptr, device=0, layers=L, kv=2, layer_stride=2 * plane,
                               kv_stride=plane, row_stride=row_bytes, row_bytes=row_bytes, rows=R * T, owner=arena)
        pool_rows = 1 + R * capacity
        pool = torch.zeros(L * 2 * pool_rows * row_bytes, dtype=torch.uint8, device=gpu)
        pool_planes = KVPlanes(base=pool.data_ptr(), device=0, layers=L, kv=2, layer_stride=2 * pool_rows * row_bytes,
                               kv_stride=pool_rows * row_bytes, row_stride=row_bytes, row_bytes=row_bytes,
                               rows=pool_rows, owner=pool)
        host = arena.host.numpy().reshape(L, 2, R * T, row_bytes)
        rows = torch.arange(R, device=gpu)
        lengths = torch.full((R,), T, dtype=torch.int32, device=gpu)
        topk_d = torch.zeros((L, R, K), dtype=torch.int32, device=gpu)
        slots = torch.empty((L, R, K), dtype=torch.int32, device=gpu)
        misses = torch.full((L, R, K), -1, dtype=torch.int32, device=gpu)
        counts = torch.empty((L, R), dtype=torch.int32, device=gpu)
        promote_src = torch.full((L, R, K), -9, dtype=torch.int32, device=gpu)
        promote_dst = torch.full((L, R, K), -9, dtype=torch.int32, device=gpu)
        out = torch.empty((R, L, 2, K, row_bytes), dtype=torch.uint8, device=gpu)

        def decode_step():
            resolve_resident(topk_d, buffers.table, None, rows, lengths, rows, slots, 1, misses=misses,
                             miss_count=counts, resident_bits=buffers.bits, slot_base=local)
            swap_in(topk_d, 1, rows, rows, slots, misses, counts, buffers, host_table_d, promote_src, promote_dst)
            move_kv(host_planes, promote_src, pool_planes, promote_dst, counts)
            gather_kv(pool_planes, slots, out)

        state = {"table": global_table(buffers), "slot_token": buffers.slot_token.cpu().numpy(),
                 "stamps": buffers.stamps.cpu().numpy()}
        graph = None
        for step in range(6):
            near = [np.concatenate([rng.choice(np.arange(T - 50, T), 24, replace=False),
                                    rng.choice(np.arange(0, T - 50), 8, replace=False)]) for _ in range(L * R)]
            topk = np.stack([rng.permutation(x) for x in near]).reshape(L, R, K)
            topk_d.copy_(torch.tensor(topk, dtype=torch.int32))
            step_lengths = np.full(R, T)
            if step in (3, 4):
                step_lengths[1] = 0                  # a padded row
            lengths.copy_(torch.tensor(step_lengths, dtype=torch.int32))
            if step == 0:
                decode_step()                        # eager step 0, also loads every kernel
                torch.cuda.synchronize()
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph):
                    decode_step()                    # recorded, not run
            else:
                graph.replay()
            torch.cuda.synchronize()
            assert int(buffers.step_counter.item()) == step + 1
            want_slots, want_misses, want_counts = ref.resolve_resident(
                topk, state["table"], None, np.arange(R), step_lengths, np.arange(R), 1,
                np.zeros((L, R, K), np.int32), with_misses=True)
            miss_np = np.full((L, R, K), -1, np.int32)
            for (layer, r), lanes in want_misses.items():
                miss_np[layer, r, :len(lanes)] = lanes
            state = ref.swap_in(step, 1, topk, np.arange(R), np.arange(R), want_slots, miss_np, want_counts,
                                state["table"], state["slot_token"], state["stamps"],
                                buffers.slot_base.cpu().numpy(), host_table.numpy())
            assert np.array_equal(slots.cpu().numpy(), state["slots"]), step
            assert np.array_equal(global_table(buffers), state["table"]), step
            assert np.array_equal(buffers.stamps.cpu().numpy(), state["stamps"]), step
            got = out.cpu().numpy()
            for layer in range(L):
                for r in range(R):
                    if step_lengths[r] == 0:
                        assert (slots[layer, r] == -1).all() and int(counts[layer, r]) == 0, step
                        assert not got[r, layer].any(), step
                        continue
                    host_rows = host_table.numpy()[r, topk[layer, r]]
                    for kv in range(2):
                        assert np.array_equal(got[r, layer, kv], host[layer, kv, host_rows]), (step, layer, r, kv)
        del graph
    finally:
        torch.cuda.synchronize()
        arena.close()


def test_local_slot_tables_follow_the_global_slot_stream(gpu):
    # Two hot-buffer sets, one with int32 global-slot tables and one with int16
    # local-slot tables, see the same Top-K stream over rows long enough for the
    # lookup's window staging. Every slot, miss list, promotion and LRU state must
    # be the same, and the int16 table must be the local form of the int32 one.
    L, R, T, C, K = 2, 3, 5000, 600, 512
    rng = np.random.default_rng(88)
    base = torch.tensor([1, 700, 1500], dtype=torch.int64, device=gpu)
    wide = HotBuffers(L, R, T, C, gpu, slot_base=base)
    narrow = HotBuffers(L, R, T, C, gpu, slot_base=base, table_dtype=torch.int16)
    recent = torch.arange(T - 300, T).expand(L, R, 300)
    local = torch.stack([torch.stack([torch.tensor(rng.permutation(C)[:300]) for _ in range(R)]) for _ in range(L)])
    for buffers in (wide, narrow):
        buffers.install(recent, local)
    rows = torch.arange(R, device=gpu)
    lengths = torch.tensor([T, T - 7, T - 130], dtype=torch.int32, device=gpu)
    host_table = torch.arange(R * T, dtype=torch.int32, device=gpu).reshape(R, T)
    for step in range(5):
        topk = torch.tensor(np.stack([rng.permutation(np.concatenate([
            rng.choice(np.arange(T - 1500, T - 130), 400, replace=False),
            rng.choice(np.arange(0, T - 1500), 112, replace=False)])) for _ in range(L * R)]).reshape(L, R, K),
            dtype=torch.int32, device=gpu)
        results = []
        for buffers in (wide, narrow):
            slots = torch.empty((L, R, K), dtype=torch.int32, device=gpu)
            misses = torch.full((L, R, K), -1, dtype=torch.int32, device=gpu)
            counts = torch.empty((L, R), dtype=torch.int32, device=gpu)
            resolve_resident(topk, buffers.table, None, rows, lengths, rows, slots, 1, misses=misses,
                             miss_count=counts, resident_bits=buffers.bits,
                             slot_base=buffers.slot_base if buffers.table.dtype == torch.int16 else None)
            looked_up = slots.clone()
            src = torch.full((L, R, K), -9, dtype=torch.int32, device=gpu)
            dst = torch.full((L, R, K), -9, dtype=torch.int32, device=gpu)
            swap_in(topk, 1, rows, rows, slots, misses, counts, buffers, host_table, src, dst)
            results.append((looked_up.cpu(), counts.cpu(), misses.cpu(), slots.cpu(), src.cpu(), dst.cpu(),
                            buffers.slot_token.cpu(), buffers.stamps.cpu(), buffers.bits.cpu()))
        for a, b in zip(*results):
            assert torch.equal(a, b), step
        table32, table16 = wide.table.cpu().long(), narrow.table.cpu().long()
        local_form = torch.where(table32 > 0, table32 - base.cpu().view(1, R, 1) + 1, torch.zeros_like(table32))
        assert torch.equal(table16, local_form), step
        assert int(results[0][1].sum()) > 0 and int((results[0][0] > 0).sum()) > 0   # hits and misses both occur
