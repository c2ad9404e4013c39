"""GPU tests of the logical shadow (bitwise oracle contract) and its row-compare kernel.

LogicalShadow.check runs the tensor mask arithmetic and the HIP row comparison
(ekv_compare_kv). Its counts, cleaned blocks and physical slots must equal the
oracle's lane-by-lane restatement (oracle.shadow_check) on random inputs.
check_complete must pass over a faithful migration, and must name exactly the
corrupted token when one byte of a migrated row is changed.
"""

import json

import numpy as np
import pytest
import torch

from adaptive_sparse.kv_pool import KVPlanes
from adaptive_sparse.logical_shadow import COUNT_KEYS, LogicalShadow, compare_rows
from oracle import oracle as ref

pytestmark = pytest.mark.gpu


def test_compare_rows_flags_equal_different_and_out_of_range(gpu):
    rows = torch.randint(0, 256, (2, 10, 48), dtype=torch.uint8, device=gpu)   # [kv, slot, bytes]
    other = rows.clone()
    other[1, 4, 47] ^= 1                                                        # V row 4 differs in its last byte
    make = lambda t: KVPlanes(base=t.data_ptr(), device=0, layers=1, kv=2, layer_stride=0,  # noqa: E731
                              kv_stride=t.stride(0), row_stride=t.stride(1), row_bytes=48, rows=10, owner=t)
    a_rows = torch.tensor([[[0, 4, 9, -1, 10, 3]]], dtype=torch.int32, device=gpu)
    b_rows = torch.tensor([[[0, 4, 9, 2, 1, 3]]], dtype=torch.int64, device=gpu)
    equal = compare_rows(make(rows), a_rows, make(other), b_rows)
    assert equal.cpu().tolist() == [[[1, 0, 1, -1, -1, 1]]]


@pytest.mark.parametrize("seed", range(4))
def test_check_matches_the_oracle_lane_by_lane(gpu, seed):
    rng = np.random.default_rng(seed)
    B, K, bs, T, capacity, N, page = 5, 6, 4, 200, 600, 700, 4
    heads, dim = 2, 16
    W = K * bs
    lengths = rng.integers(-2, T + 10, size=B)
    rows = rng.permutation(B)
    table = rng.integers(-2, capacity + 5, size=(B, T))
    blocks = rng.integers(-1, (T + 10) // bs + 3, size=(1, B, K))
    blocks[rng.random(blocks.shape) < 0.2] = -1
    blocks[:, :, 0] = rng.integers(0, 3, size=B)            # most rows start with a valid block
    physical = rng.integers(-3, N + 3, size=(1, B, W))
    live = rng.random(N // page + 1) < 0.8
    shadow = LogicalShadow(capacity, gpu)
    written = np.zeros(capacity, dtype=bool)
    shadow_k = np.zeros((capacity, heads * dim * 2), np.uint8)
    shadow_v = np.zeros_like(shadow_k)
    locations = np.flatnonzero(rng.random(capacity) < 0.8)
    key = torch.randn((len(locations), heads, dim), dtype=torch.bfloat16, device=gpu)
    value = torch.randn((len(locations), heads, dim), dtype=torch.bfloat16, device=gpu)
    shadow.write(3, torch.tensor(locations, device=gpu), key, value)
    written[locations] = True
    shadow_k[locations] = key.view(len(locations), -1).view(torch.uint8).cpu().numpy()
    shadow_v[locations] = value.view(len(locations), -1).view(torch.uint8).cpu().numpy()
    # Pool rows: random, then 70 % of lanes' physical rows made equal to their logical shadow rows.
    k_cache = torch.randn((N, heads, dim), dtype=torch.bfloat16, device=gpu)
    v_cache = torch.randn((N, heads, dim), dtype=torch.bfloat16, device=gpu)
    pool_k = k_cache.view(N, -1).view(torch.uint8).cpu().numpy()
    pool_v = v_cache.view(N, -1).view(torch.uint8).cpu().numpy()
    for b in range(B):
        for o in range(W):
            p = int(physical[0, b, o])
            logical = int(table[rows[b], min(max(0, int(blocks[0, b, o // bs]) * bs + o % bs), T - 1)])
            if 0 <= p < N and 0 <= logical < capacity and rng.random() < 0.7:
                pool_k[p], pool_v[p] = shadow_k[logical], shadow_v[logical]
    k_cache.view(N, -1).view(torch.uint8).copy_(torch.from_numpy(pool_k))
    v_cache.view(N, -1).view(torch.uint8).copy_(torch.from_numpy(pool_v))

    t = lambda a: torch.tensor(a, device=gpu)  # noqa: E731
    clean, out = shadow.check(3, k_cache, v_cache, t(table), t(lengths), t(rows), bs, t(blocks), t(physical),
                              t(live), page)
    want_counts, want_clean, want_out = ref.shadow_check(blocks, table, lengths, rows, bs, physical, live, page,
                                                         capacity, written, pool_k, pool_v, shadow_k, shadow_v)
    assert tuple(shadow.counts.tolist()) == want_counts
    assert np.array_equal(clean.cpu().numpy(), want_clean)
    assert np.array_equal(out.cpu().numpy(), want_out)
    assert want_counts[0] > 0 and want_counts[4] > 0      # the case checks tokens and finds mismatches


def test_check_complete_after_a_migration_and_a_planted_corruption(gpu, tmp_path):
    layers, capacity, N, heads, dim = 2, 64, 80, 2, 16
    row_bytes = heads * dim * 2
    shadow = LogicalShadow(capacity, gpu)
    logical = torch.arange(1, 41, device=gpu)
    physical = torch.randperm(N - 1, device=gpu)[:40] + 1
    pool = torch.zeros((layers, 2, N, row_bytes), dtype=torch.uint8, device=gpu)
    for layer in range(layers):
        key = torch.randn((40, heads, dim), dtype=torch.bfloat16, device=gpu)
        value = torch.randn((40, heads, dim), dtype=torch.bfloat16, device=gpu)
        shadow.write(layer, logical, key, value)
        pool[layer, 0, physical] = key.view(40, -1).view(torch.uint8)      # the migration's result
        pool[layer, 1, physical] = value.view(40, -1).view(torch.uint8)
    planes = KVPlanes(base=pool.data_ptr(), device=0, layers=layers, kv=2, layer_stride=pool.stride(0),
                      kv_stride=pool.stride(1), row_stride=pool.stride(2), row_bytes=row_bytes, rows=N, owner=pool)
    report = shadow.check_complete(planes, logical, physical, "promote")
    assert report == {"migration_checked_tokens": 80, "migration_checked_bytes": 80 * 2 * row_bytes,
                      "migration_invalid_tokens": 0, "migration_mismatched_tokens": 0}
    pool[1, 1, physical[17], 5] ^= 0x80
    with pytest.raises(RuntimeError, match="'migration_mismatched_tokens': 1"):
        shadow.check_complete(planes, logical, physical, "promote")
    pool[1, 1, physical[17], 5] ^= 0x80
    shadow.check_complete(planes, logical, physical, "promote")
    shadow.publish(tmp_path, 0)
    stats = json.loads((tmp_path / "shadow-tp-0.json").read_text())
    assert stats["migration_checked_tokens"] == 240 and stats["migration_mismatched_tokens"] == 1
    assert all(stats[key] == 0 for key in COUNT_KEYS)


def test_decode_check_through_a_vmm_backed_pool(gpu):
    # One layer of a VMM pool: the rows a lookup resolves are the shadow's rows, then one is corrupted.
    from elastic_kv.backing import Backing

    capacity, heads, dim, bs = 1024, 2, 128, 1
    chunk = 2 << 20
    row_bytes = heads * dim * 2
    backing = Backing(2 * chunk, chunk_bytes=chunk, device=0)
    raw = k_cache = v_cache = None
    try:
        backing.ensure([0, 1])
        raw = backing.raw
        slots_per_plane = chunk // row_bytes
        k_cache = raw.narrow(0, 0, chunk).view(torch.bfloat16).view(slots_per_plane, heads, dim)
        v_cache = raw.narrow(0, chunk, chunk).view(torch.bfloat16).view(slots_per_plane, heads, dim)
        shadow = LogicalShadow(capacity, gpu)
        locations = torch.arange(1, 301, device=gpu)
        key = torch.randn((300, heads, dim), dtype=torch.bfloat16, device=gpu)
        value = torch.randn((300, heads, dim), dtype=torch.bfloat16, device=gpu)
        shadow.write(0, locations, key, value)
        physical_of = torch.randperm(slots_per_plane - 1, device=gpu)[:300] + 1
        k_cache[physical_of] = key
        v_cache[physical_of] = value
        table = torch.arange(300, device=gpu).view(1, 300) + 1                  # position p -> logical p + 1
        blocks = torch.randperm(300, device=gpu)[:64].view(1, 1, 64)
        physical = physical_of[blocks[0] + 0].view(1, 1, 64)                     # logical p + 1 lives at physical_of[p]
        lengths = torch.tensor([300], device=gpu)
        rows = torch.tensor([0], device=gpu)
        _, out = shadow.check(0, k_cache, v_cache, table, lengths, rows, bs, blocks, physical, None, 1)
        assert torch.equal(out, physical.to(torch.int32))
        assert shadow.stats()["checked_tokens"] == 64 and shadow.stats()["mismatched_tokens"] == 0
        v_cache[physical[0, 0, 7], 1, 3] += 1.0
        shadow.check(0, k_cache, v_cache, table, lengths, rows, bs, blocks, physical, None, 1)
        assert shadow.stats()["checked_tokens"] == 128 and shadow.stats()["mismatched_tokens"] == 1
        torch.cuda.synchronize()
    finally:
        del k_cache, v_cache, raw
        backing.close()
