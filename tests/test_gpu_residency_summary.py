"""GPU parity of the coarse residency summary (one bit per group of 2**shift positions).

The summary builder must equal the oracle's, and every lookup kernel that
reads a summary (the prefetching int16 kernel, the contiguous-pieces kernel,
the strided int16 and int32 kernels) must give the oracle's plain lookup -
slots, miss lists and counts - for exact summaries and for supersets of
them (stale group bits). The swap-in keeps a coarse summary exact through
its group counts; without them it leaves a superset behind.
"""

import numpy as np
import pytest
import torch

from adaptive_sparse.resident_lookup import build_residency_bits, resolve_resident, summary_words
from adaptive_sparse.swap_in import HotBuffers, swap_in
from oracle import oracle as ref

pytestmark = pytest.mark.gpu


def test_summary_words_cover_whole_pieces():
    assert summary_words(65536, 0) == 2048 and summary_words(65536, 6) == 32
    assert summary_words(70, 0) == 4 and summary_words(70, 6) == 4 and summary_words(1, 20) == 4


@pytest.mark.parametrize("dtype", [torch.int16, torch.int32, torch.int64])
@pytest.mark.parametrize("shift", [0, 1, 5, 6, 7, 10])
def test_summary_builder_matches_oracle(gpu, dtype, shift):
    rng = np.random.default_rng(shift * 7 + dtype.itemsize)
    for L, R, T in ((1, 3, 70), (2, 5, 4099), (3, 2, 65536)):
        table = rng.integers(1, 100, (L, R, T)) * (rng.random((L, R, T)) < 0.003)
        table[0, 0, T - 1] = 5                                   # the last position of a ragged group
        got = build_residency_bits(torch.tensor(table, dtype=dtype, device=gpu), shift=shift).cpu().numpy()
        want = ref.residency_bits(table, shift)
        words = want.shape[-1]
        assert got.shape[-1] == summary_words(T, shift)
        assert np.array_equal(got[..., :words], want), (L, R, T)
        assert not got[..., words:].any()
    # a strided [R, T] view
    table = rng.integers(0, 3, (4, 300))
    view = torch.tensor(table, dtype=dtype, device=gpu).t().contiguous().t()
    assert np.array_equal(build_residency_bits(view, shift=shift).cpu().numpy()[:, :ref.residency_bits(table, shift)
                                                                                    .shape[-1]],
                          ref.residency_bits(table, shift))


def _decode_case(rng, L, R, T, K, C, recent):
    """Top-K (most from the last `recent` positions) and an int16 local-slot table of the C newest tokens."""
    topk = np.empty((L, R, K), np.int64)
    for i in range(L * R):
        near = rng.choice(np.arange(T - recent, T), (K * 4) // 5, replace=False)
        far = rng.choice(np.arange(0, T - recent), K - len(near), replace=False)
        topk.flat[i * K:(i + 1) * K] = rng.permutation(np.concatenate([near, far]))
    topk[rng.random(topk.shape) < 0.02] = -1
    local = np.zeros((L, R, T), np.int64)
    for layer in range(L):
        for r in range(R):
            local[layer, r, T - C:] = rng.permutation(C) + 1
            stray = rng.choice(T - C, 5, replace=False)                 # a few old resident tokens
            local[layer, r, stray] = rng.choice(np.arange(1, C + 1), 5, replace=False)
    return topk, local


def _superset(bits, rng, density=0.3):
    extra = (rng.random(bits.shape) < density) * rng.integers(0, 1 << 31, bits.shape)
    return bits | torch.tensor(extra, dtype=torch.int32, device=bits.device)


@pytest.mark.parametrize("shift", [3, 6])
@pytest.mark.parametrize("shape", ["pipe", "runs", "strided"])
def test_lookup_with_summary_matches_oracle(gpu, shift, shape):
    rng = np.random.default_rng({"pipe": 1, "runs": 2, "strided": 3}[shape] * 10 + shift)
    L, R, T, C = 3, 6, 9000, 1500
    K = {"pipe": 1024, "runs": 2560, "strided": 1024}[shape]
    topk, local = _decode_case(rng, L, R, T, K, C, 3000)
    base = np.arange(R) * C + 1
    lengths = np.full(R, T)
    lengths[1] = T - 40                                                # a short row
    table16 = torch.tensor(local, dtype=torch.int16, device=gpu)
    global_table = np.where(local > 0, base.reshape(1, R, 1) + local - 1, 0)
    want, want_misses, want_counts = ref.resolve_resident(topk, global_table, None, np.arange(R), lengths,
                                                          np.arange(R), 1, np.full((L, R, K), -7, np.int32),
                                                          with_misses=True)
    topk_d = torch.tensor(topk, dtype=torch.int32, device=gpu)
    if shape == "strided":
        # a Top-K view shifted by one element is not 16-byte aligned: the strided kernel runs
        wide = torch.zeros((L, R, K + 1), dtype=torch.int32, device=gpu)
        wide[..., 1:] = topk_d
        topk_d = wide[..., 1:]
    exact = build_residency_bits(table16, shift=shift)
    rows = torch.arange(R, device=gpu)
    for bits in (exact, _superset(exact, rng)):
        for table, slot_base in ((table16, torch.tensor(base, device=gpu)),
                                 (torch.tensor(global_table, dtype=torch.int32, device=gpu), None)):
            slots = torch.full((L, R, K), -7, dtype=torch.int32, device=gpu)
            misses = torch.full((L, R, K), -3, dtype=torch.int32, device=gpu)
            counts = torch.empty((L, R), dtype=torch.int32, device=gpu)
            resolve_resident(topk_d, table, None, rows, torch.tensor(lengths, device=gpu), rows, slots, 1,
                             misses=misses, miss_count=counts, resident_bits=bits, bits_shift=shift,
                             slot_base=slot_base)
            assert np.array_equal(slots.cpu().numpy(), want)
            assert np.array_equal(counts.cpu().numpy(), want_counts)
            got = misses.cpu().numpy()
            for (layer, r), lanes in want_misses.items():
                assert np.array_equal(got[layer, r, :len(lanes)], lanes)


def test_summary_rejects_a_short_row_and_bad_shift(gpu):
    table = torch.zeros((2, 4096), dtype=torch.int16, device=gpu)
    topk = torch.zeros((1, 2, 8), dtype=torch.int32, device=gpu)
    out = torch.empty((1, 2, 8), dtype=torch.int32, device=gpu)
    rows = torch.arange(2, device=gpu)
    lengths = torch.full((2,), 4096, device=gpu)
    base = torch.tensor([1, 9], device=gpu)
    with pytest.raises(RuntimeError, match="words per row"):
        resolve_resident(topk, table, None, rows, lengths, rows, out, 1, slot_base=base,
                         resident_bits=torch.zeros((2, 1), dtype=torch.int32, device=gpu), bits_shift=6)
    with pytest.raises(RuntimeError, match="bits_shift"):
        resolve_resident(topk, table, None, rows, lengths, rows, out, 1, slot_base=base,
                         resident_bits=torch.zeros((2, 4), dtype=torch.int32, device=gpu), bits_shift=21)


def _stream_step(rng, buffers, L, R, T, K, recent):
    """One lookup + swap-in step of a locality stream; returns the oracle's lookup of the table before it."""
    topk = np.stack([rng.permutation(np.concatenate([
        rng.choice(np.arange(T - recent, T), K - K // 4, replace=False),
        rng.choice(np.arange(0, T - recent), K // 4, replace=False)])) for _ in range(L * R)]).reshape(L, R, K)
    topk_d = torch.tensor(topk, dtype=torch.int32, device=buffers.device)
    table_before = _global(buffers)
    rows = torch.arange(R, device=buffers.device)
    lengths = torch.full((R,), T, dtype=torch.int32, device=buffers.device)
    slots = torch.empty((L, R, K), dtype=torch.int32, device=buffers.device)
    misses = torch.full((L, R, K), -1, dtype=torch.int32, device=buffers.device)
    counts = torch.empty((L, R), dtype=torch.int32, device=buffers.device)
    resolve_resident(topk_d, buffers.table, None, rows, lengths, rows, slots, 1, misses=misses,
                     miss_count=counts, resident_bits=buffers.bits, bits_shift=buffers.bits_shift,
                     slot_base=buffers.slot_base if buffers.table.dtype == torch.int16 else None)
    want, _, want_counts = ref.resolve_resident(topk, table_before, None, np.arange(R), np.full(R, T), np.arange(R),
                                                1, np.zeros((L, R, K), np.int32), with_misses=True)
    got_slots, got_counts = slots.cpu().numpy(), counts.cpu().numpy()
    host_table = torch.arange(R * T, dtype=torch.int32, device=buffers.device).reshape(R, T)
    src = torch.full((L, R, K), -9, dtype=torch.int32, device=buffers.device)
    dst = torch.full((L, R, K), -9, dtype=torch.int32, device=buffers.device)
    swap_in(topk_d, 1, rows, rows, slots, misses, counts, buffers, host_table, src, dst, check=True)
    return np.array_equal(got_slots, want) and np.array_equal(got_counts, want_counts)


def _group_counts(table, shift):
    """Resident positions per group of 2**shift positions (the last group ragged)."""
    T = table.shape[-1]
    groups = -(-T // (1 << shift))
    padded = np.zeros((*table.shape[:-1], groups << shift), bool)
    padded[..., :T] = table != 0
    return padded.reshape(*table.shape[:-1], groups, 1 << shift).sum(-1)


@pytest.mark.parametrize("table_dtype,shift", [(torch.int16, 6), (torch.int32, 6), (torch.int16, 3)])
def test_swap_in_keeps_the_coarse_summary_exact(gpu, table_dtype, shift):
    # A stream through lookup + swap-in with a coarse summary: after every step
    # the summary the swap-in maintains equals a fresh build_residency_bits of
    # the table (and the oracle's), its group counts equal the table's, and the
    # lookup through it equals the oracle's plain lookup. Old groups fill and
    # empty as uniform picks come and go, so bits are cleared as well as set.
    L, R, T, C, K = 2, 3, 3001, 256, 128
    rng = np.random.default_rng(5 + shift)
    buffers = HotBuffers(L, R, T, C, gpu, table_dtype=table_dtype, bits_shift=shift)
    ever = np.zeros(ref.residency_bits(_global(buffers), shift).shape, np.uint32)
    for step in range(12):
        assert _stream_step(rng, buffers, L, R, T, K, 400), step
        table = _global(buffers)
        exact = ref.residency_bits(table, shift)
        words = exact.shape[-1]
        kept = buffers.bits.cpu().numpy()
        assert np.array_equal(kept[..., :words], exact), step
        assert not kept[..., words:].any()
        assert torch.equal(buffers.bits, build_residency_bits(buffers.table, shift=shift)), step
        assert np.array_equal(buffers.resident_counts.cpu().numpy(), _group_counts(table, shift)), step
        ever |= exact.view(np.uint32)
    assert (ever != exact.view(np.uint32)).any()       # groups emptied: bits were cleared, not only set


def test_swap_in_without_group_counts_keeps_a_superset(gpu):
    # The ABI's count-less form: a coarse summary only gains bits (a superset
    # that lookups still read correctly); refresh_bits() makes it exact again.
    L, R, T, C, K = 2, 3, 3000, 256, 128
    rng = np.random.default_rng(5)
    buffers = HotBuffers(L, R, T, C, gpu, table_dtype=torch.int16, bits_shift=6)
    buffers.resident_counts = None
    for step in range(8):
        assert _stream_step(rng, buffers, L, R, T, K, 400), step
        exact = ref.residency_bits(_global(buffers), 6).view(np.uint32)
        kept = buffers.bits.cpu().numpy()[..., :exact.shape[-1]].view(np.uint32)
        assert np.array_equal(kept & exact, exact), step
    assert (kept != exact).any()                       # evictions left stale bits
    buffers.refresh_bits()
    exact = ref.residency_bits(_global(buffers), 6)
    assert np.array_equal(buffers.bits.cpu().numpy()[..., :exact.shape[-1]], exact)


def _global(buffers):
    table = buffers.table.cpu().numpy().astype(np.int64)
    if buffers.table.dtype == torch.int16:
        base = buffers.slot_base.cpu().numpy().reshape(1, -1, 1)
        table = np.where(table > 0, base + table - 1, 0)
    return table
