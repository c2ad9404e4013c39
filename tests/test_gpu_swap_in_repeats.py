"""GPU swap-in with repeated tokens, shared requests and stamp overflow, against the oracle.

A Top-K block listed twice expands to repeated tokens. The swap-in treats a
repeat as one access by its first lane (the reference's batch-token LRU
replay applied to the selection with later repeats dropped): one victim per
distinct missed token, shared by every lane of it, and one promotion. Rows
that would race (two selected rows naming one request) or whose stamps would
overflow are refused and reported through the status word.
"""

import numpy as np
import pytest
import torch

from adaptive_sparse.resident_lookup import resolve_resident
from adaptive_sparse.swap_in import STEP_STAMPS, SWAP_SHARED_REQUEST, SWAP_STAMP_OVERFLOW, HotBuffers, swap_in
from oracle import oracle as ref

pytestmark = pytest.mark.gpu


def _global(buffers):
    table = buffers.table.cpu().numpy().astype(np.int64)
    if buffers.table.dtype == torch.int16:
        base = buffers.slot_base.cpu().numpy().reshape(1, -1, 1)
        table = np.where(table > 0, base + table - 1, 0)
    return table


def _step(gpu, buffers, topk, bs, lengths, state, step, host_table, rows=None, selected=None):
    """One lookup + swap-in on the GPU and in the oracle; asserts equal state, returns the oracle's."""
    L, B, K = topk.shape
    W = K * bs
    rows = np.arange(B) if rows is None else rows
    selected = np.arange(B) if selected is None else selected
    rows_d, sel_d = torch.tensor(rows, device=gpu), torch.tensor(selected, device=gpu)
    topk_d = torch.tensor(topk, dtype=torch.int32, device=gpu)
    slots = torch.zeros((L, B, W), dtype=torch.int32, device=gpu)
    misses = torch.full((L, B, W), -1, dtype=torch.int32, device=gpu)
    counts = torch.zeros((L, B), dtype=torch.int32, device=gpu)
    local = buffers.slot_base if buffers.table.dtype == torch.int16 else None
    resolve_resident(topk_d, buffers.table, None, rows_d, torch.tensor(lengths, dtype=torch.int32, device=gpu),
                     sel_d, slots, bs, misses=misses, miss_count=counts, resident_bits=buffers.bits,
                     bits_shift=buffers.bits_shift, slot_base=local)
    want_slots, want_misses, want_counts = ref.resolve_resident(
        topk, state["table"], None, rows, lengths, selected, bs, np.zeros((L, B, W), np.int32), with_misses=True)
    assert np.array_equal(slots.cpu().numpy(), want_slots), step
    assert np.array_equal(counts.cpu().numpy(), want_counts), step
    miss_np = np.full((L, B, W), -1, np.int32)
    for (layer, r), lanes in want_misses.items():
        miss_np[layer, r, :len(lanes)] = lanes
    src = torch.full((L, B, W), -9, dtype=torch.int32, device=gpu)
    dst = torch.full((L, B, W), -9, dtype=torch.int32, device=gpu)
    swap_in(topk_d, bs, rows_d, sel_d, slots, misses, counts, buffers, host_table.to(gpu), src, dst)
    torch.cuda.synchronize()
    new = ref.swap_in(step, bs, topk, rows, selected, want_slots, miss_np, want_counts, state["table"],
                      state["slot_token"], state["stamps"], buffers.slot_base.cpu().numpy(), host_table.numpy())
    assert int(buffers.status.item()) == new["status"], step
    buffers.status.zero_()
    assert np.array_equal(slots.cpu().numpy(), new["slots"]), step
    assert np.array_equal(_global(buffers), new["table"]), step
    assert np.array_equal(buffers.slot_token.cpu().numpy(), new["slot_token"]), step
    assert np.array_equal(buffers.stamps.cpu().numpy(), new["stamps"]), step
    got_src, got_dst = src.cpu().numpy(), dst.cpu().numpy()
    for layer in range(L):
        for b in range(B):
            c = want_counts[layer, b]
            assert np.array_equal(got_src[layer, b, :c], new["promote_src"][layer, b, :c]), (step, layer, b)
            assert np.array_equal(got_dst[layer, b, :c], new["promote_dst"][layer, b, :c]), (step, layer, b)
    if buffers.bits is not None and buffers.bits_shift == 0:
        exact = ref.residency_bits(new["table"])
        assert np.array_equal(buffers.bits.cpu().numpy()[..., :exact.shape[-1]], exact), step
    return new


@pytest.mark.parametrize("table_dtype", [torch.int32, torch.int16])
def test_access_trace_kat_repeated_block_through_lookup_and_swap_in(gpu, table_dtype):
    """tests/test_hisparse_access_trace.py:170-199: blocks [1, -1, 3, 1, 4], bs 2, seq_len 7, prestate
    [2, 1, -1, 6] in the first four slots; token 3 misses at lanes 1 and 7 and takes one slot. The kernel
    needs a hot buffer of at least K * bs = 10 slots (the KAT's capacity 4 only decides its short path,
    which seq_len 7 does not take); the empty slot 2 is still the first victim."""
    buffers = HotBuffers(1, 1, 10, 10, gpu, table_dtype=table_dtype)
    buffers.install(torch.tensor([[[1, 2, 6]]]), torch.tensor([[[1, 0, 3]]]))   # prestate order: 1, 2, 6
    host_table = torch.arange(10, dtype=torch.int32).reshape(1, 10) + 100
    state = {"table": _global(buffers), "slot_token": buffers.slot_token.cpu().numpy(),
             "stamps": buffers.stamps.cpu().numpy()}
    assert state["slot_token"][0, 0, :4].tolist() == [2, 1, -1, 6]
    new = _step(gpu, buffers, np.array([[[1, -1, 3, 1, 4]]]), 2, np.array([7]), state, 0, host_table)
    assert new["promote_src"][0, 0, :2].tolist() == [103, -1]
    assert new["slots"][0, 0, 1] == new["slots"][0, 0, 7] == int(buffers.slot_base[0]) + 2
    assert buffers.slot_token.cpu()[0, 0, :4].tolist() == [2, 1, 3, 6]


@pytest.mark.parametrize("bs", [1, 2])
@pytest.mark.parametrize("table_dtype", [torch.int32, torch.int16])
def test_random_streams_with_repeated_blocks(gpu, bs, table_dtype):
    L, R, T, C, K = 2, 4, 400, 48, 16
    rng = np.random.default_rng(100 + bs)
    buffers = HotBuffers(L, R, T, C, gpu, table_dtype=table_dtype)
    host_table = torch.arange(R * T, dtype=torch.int32).reshape(R, T)
    state = {"table": _global(buffers), "slot_token": buffers.slot_token.cpu().numpy(),
             "stamps": buffers.stamps.cpu().numpy()}
    lengths = np.array([T, T - 3, T - 11, T])
    blocks_total = T // bs
    repeats = 0
    for step in range(8):
        topk = rng.integers(blocks_total - 30, blocks_total, (L, R, K))
        topk[..., :4] = rng.integers(0, blocks_total, (L, R, 4))
        dup = rng.random((L, R, K)) < 0.25                      # ~a quarter of the ids repeat an earlier one
        src = rng.integers(0, K, (L, R, K))
        topk = np.where(dup, np.take_along_axis(topk, src, -1), topk)
        topk[rng.random((L, R, K)) < 0.05] = -1
        repeats += sum(len(set(x[x >= 0].tolist())) < int((x >= 0).sum()) for x in topk.reshape(-1, K))
        state = _step(gpu, buffers, topk, bs, lengths, state, step, host_table)
    assert repeats > 0


def test_shared_request_rows_are_refused_and_reported(gpu):
    L, R, T, C, K = 2, 3, 64, 16, 4
    buffers = HotBuffers(L, R, T, C, gpu)
    host_table = torch.arange(R * T, dtype=torch.int32).reshape(R, T)
    state = {"table": _global(buffers), "slot_token": buffers.slot_token.cpu().numpy(),
             "stamps": buffers.stamps.cpu().numpy()}
    topk = np.array([[[1, 2, 3, 4], [5, 6, 7, 8], [9, 10, 11, 12], [13, 14, 15, 16]]] * L)
    # batch rows 0 and 3 both name request 2
    new = _step(gpu, buffers, topk, 1, np.full(4, T), state, 0, host_table, rows=np.array([2, 0, 1, 2]))
    assert new["status"] == SWAP_SHARED_REQUEST
    assert not _global(buffers)[:, 2].any()
    swap_in_rows = torch.tensor([2, 0, 1, 2], device=gpu)
    slots = torch.zeros((L, 4, K), dtype=torch.int32, device=gpu)
    counts = torch.zeros((L, 4), dtype=torch.int32, device=gpu)
    with pytest.raises(RuntimeError, match="same request"):
        swap_in(torch.tensor(topk, dtype=torch.int32, device=gpu), 1, swap_in_rows, torch.arange(4, device=gpu),
                slots, torch.zeros_like(slots), counts, buffers, host_table.to(gpu), torch.zeros_like(slots),
                torch.zeros_like(slots), check=True)


def test_counted_step_past_the_stamp_range_is_reported(gpu):
    # The device step counter is set past the int32 stamp range from the host: the
    # swap-in must change nothing, record empty promotions and report the overflow.
    L, R, T, C, K = 1, 2, 64, 8, 4
    buffers = HotBuffers(L, R, T, C, gpu, step_counter=True)
    buffers.step_counter.fill_((1 << 31) // STEP_STAMPS - 1)     # the first step whose stamps leave int32
    topk = torch.tensor([[[1, 2, 3, 4], [5, 6, 7, 8]]], dtype=torch.int32, device=gpu)
    rows = torch.arange(R, device=gpu)
    slots = torch.zeros((L, R, K), dtype=torch.int32, device=gpu)
    misses = torch.arange(K, dtype=torch.int32, device=gpu).expand(L, R, K).contiguous()
    counts = torch.full((L, R), K, dtype=torch.int32, device=gpu)
    src = torch.full((L, R, K), 7, dtype=torch.int32, device=gpu)
    dst = torch.full((L, R, K), 7, dtype=torch.int32, device=gpu)
    host_table = torch.arange(R * T, dtype=torch.int32, device=gpu).reshape(R, T)
    swap_in(topk, 1, rows, rows, slots, misses, counts, buffers, host_table, src, dst)
    torch.cuda.synchronize()
    assert int(buffers.status.item()) == SWAP_STAMP_OVERFLOW
    assert (src == -1).all() and (dst == -1).all() and (slots == 0).all()
    assert not buffers.table.any() and (buffers.slot_token == -1).all()
    with pytest.raises(RuntimeError, match="overflow"):
        buffers.check_status()
    assert int(buffers.status.item()) == 0


@pytest.mark.parametrize("seed", range(24))
def test_swap_in_random_configurations(gpu, seed):
    """Seeded shapes, block sizes, table forms, summaries, lengths and selections, 2-5 steps each.

    Every step runs lookup + swap-in on the GPU and in the oracle and compares
    slots, miss counts, the token table, slot tokens, stamps, promotion lists
    and (per-position summary) the residency bits.
    """
    rng = np.random.default_rng(7000 + seed)
    L, R = int(rng.integers(1, 4)), int(rng.integers(1, 6))
    B = int(rng.integers(1, R + 1))
    bs = int(rng.choice([1, 1, 2, 4, 16]))
    K = int(rng.integers(1, 9))
    W = K * bs
    T = int(rng.integers(max(W, 8), 700))
    C = int(rng.integers(W, W + 64))
    table_dtype = torch.int16 if rng.random() < 0.5 else torch.int32
    with_bits = rng.random() < 0.8
    shift = int(rng.choice([0, 0, 3, 6])) if with_bits else 0
    buffers = HotBuffers(L, R, T, C, gpu, table_dtype=table_dtype, with_bits=with_bits, bits_shift=shift)
    host_table = torch.tensor(rng.permutation(R * T), dtype=torch.int32).reshape(R, T)
    state = {"table": _global(buffers), "slot_token": buffers.slot_token.cpu().numpy(),
             "stamps": buffers.stamps.cpu().numpy()}
    rows = rng.permutation(R)[:B]                       # distinct requests: no row is refused
    lengths = np.where(rng.random(B) < 0.2, rng.integers(1, T + 1, B), rng.integers(T // 2 + 1, T + 1, B))
    blocks_total = -(-T // bs)
    row_blocks = -(-lengths // bs)                      # blocks holding a valid position, per batch row
    span = np.minimum(row_blocks, 2 * K)
    promoted = 0
    for step in range(int(rng.integers(2, 6))):
        selected = np.sort(rng.permutation(B)[:int(rng.integers(1, B + 1))])
        # a recent-heavy share: the last 2K blocks of each row's own context
        topk = row_blocks[None, :, None] - 1 - (rng.random((L, B, K)) * span[None, :, None]).astype(np.int64)
        old = rng.random((L, B, K)) < 0.3
        topk = np.where(old, rng.integers(0, blocks_total + 3, (L, B, K)), topk)  # some past the length
        dup = rng.random((L, B, K)) < 0.15
        topk = np.where(dup, np.take_along_axis(topk, rng.integers(0, K, (L, B, K)), -1), topk)
        topk[rng.random((L, B, K)) < 0.1] = -1
        if step == 0:   # every row selected with one valid pick: the first step has misses to promote
            selected = np.arange(B)
            topk[:, :, 0] = row_blocks[None, :] - 1
        state = _step(gpu, buffers, topk, bs, lengths, state, step, host_table, rows=rows, selected=selected)
        promoted += int((state["promote_dst"] >= 0).sum())
    assert promoted > 0


@pytest.mark.parametrize("capacity", [2500, 4096, 5000, 8192])
def test_large_hot_buffers_evict_in_lru_order(gpu, capacity):
    """Hot buffers of more than 2048 slots (their 4096 or 8192 sort keys are sorted in registers): nearly full
    buffers, so every step's misses evict least-recently-used entries; 3 steps against the oracle."""
    rng = np.random.default_rng(capacity)
    L, R, K, bs = 2, 2, 64, 4                                    # 256 lanes per row
    T = capacity + 3000
    table_dtype = torch.int16 if capacity % 2 else torch.int32
    buffers = HotBuffers(L, R, T, capacity, gpu, table_dtype=table_dtype)
    filled = capacity - 5                                        # five empty slots, taken first
    tokens = np.stack([[rng.choice(T, filled, replace=False) for _ in range(R)] for _ in range(L)])
    local = np.stack([[rng.permutation(capacity)[:filled] for _ in range(R)] for _ in range(L)])
    buffers.install(torch.tensor(tokens), torch.tensor(local))
    host_table = torch.tensor(rng.permutation(R * T), dtype=torch.int32).reshape(R, T)
    state = {"table": _global(buffers), "slot_token": buffers.slot_token.cpu().numpy(),
             "stamps": buffers.stamps.cpu().numpy()}
    evicted = 0
    for step in range(3):
        topk = rng.integers(0, T // bs, (L, R, K))
        before = state["slot_token"].copy()
        state = _step(gpu, buffers, topk, bs, np.full(R, T), state, step, host_table)
        evicted += int(((before >= 0) & (state["slot_token"] != before)).sum())
    assert evicted > 0


@pytest.mark.parametrize("capacity", [4096, 8192])
@pytest.mark.parametrize("K,bs", [(2049, 1), (1000, 3), (1024, 4)])
def test_rows_wider_than_2048_lanes_evict_in_lru_order(gpu, capacity, K, bs):
    """Rows of 2049 to 4096 lanes (their lane state is held 16 lanes per thread) over hot buffers of 4096 and
    8192 slots, nearly full, with repeated blocks: 3 steps against the oracle."""
    rng = np.random.default_rng(K * 7 + capacity)
    L, R = 1, 2
    W = K * bs
    T = capacity + 2 * W
    buffers = HotBuffers(L, R, T, capacity, gpu, table_dtype=torch.int16 if bs == 3 else torch.int32)
    filled = capacity - 3
    tokens = np.stack([[rng.choice(T, filled, replace=False) for _ in range(R)] for _ in range(L)])
    local = np.stack([[rng.permutation(capacity)[:filled] for _ in range(R)] for _ in range(L)])
    buffers.install(torch.tensor(tokens), torch.tensor(local))
    host_table = torch.tensor(rng.permutation(R * T), dtype=torch.int32).reshape(R, T)
    state = {"table": _global(buffers), "slot_token": buffers.slot_token.cpu().numpy(),
             "stamps": buffers.stamps.cpu().numpy()}
    evicted = 0
    for step in range(3):
        topk = rng.integers(0, T // bs, (L, R, K))
        topk[..., 1::97] = topk[..., 0:1]                        # repeated blocks
        topk[..., 5::211] = -1
        before = state["slot_token"].copy()
        state = _step(gpu, buffers, topk, bs, np.array([T, T - 5]), state, step, host_table)
        evicted += int(((before >= 0) & (state["slot_token"] != before)).sum())
    assert evicted > 0
