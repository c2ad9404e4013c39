"""Full-size GPU checks of the decode read and the block gather.

At full size the oracle would take minutes, so these tests check properties
that do not depend on size instead:
- the HiSparse decode read (128 requests x 65,536 tokens x 60 layers,
  Top-K 2048, hot capacity 4096) is built so that its results have closed
  forms. Each (layer, request) selects 1638 distinct tokens from the last
  4096 positions, all resident, and 410 distinct tokens from the rest, none
  resident. So every row has exactly 410 misses, and those misses are exactly
  the lanes that selected an old token;
- every gathered K/V plane must equal torch.index_select of the pool plane
  at the resolved slots, with zero rows for misses. index_select is the
  textbook gather.
- the block gather (64 requests x 256 blocks of 16 tokens, 36 layers, a
  20,000-block pool) is checked plane by plane the same way.
The pools are VMM Backings of 2 MiB chunks, as in the benchmarks.
"""

import numpy as np
import pytest
import torch

from adaptive_sparse.kv_pool import PlanePoolLayout
from adaptive_sparse.resident_lookup import build_residency_bits, resolve_resident
from adaptive_sparse.sparse_read import gather_kv
from elastic_kv.backing import Backing

pytestmark = pytest.mark.gpu


def committed_pool(layout, device, seed):
    backing = Backing(layout.capacity_bytes, layout.chunk_bytes, device=device.index or 0)
    backing.ensure(range(backing.chunk_count))
    raw = backing.raw
    gen = torch.Generator(device=device).manual_seed(seed)
    for plane in range(layout.planes):
        raw.narrow(0, plane * layout.plane_stride, layout.plane_bytes).view(torch.bfloat16).normal_(generator=gen)
    return backing, raw


def plane_rows(raw, layout, layer, kv):
    return raw.narrow(0, layout.plane_offset(layer, kv), layout.plane_bytes).view(layout.rows, layout.row_bytes)


def test_decode_read_at_full_size(gpu):
    L, R, T, K, C, W = 60, 128, 65536, 2048, 4096, 4096
    recent_count, old_count = 1638, 410
    row_bytes = 512
    gen = torch.Generator(device=gpu).manual_seed(31)
    recent = torch.rand((L, R, W), generator=gen, device=gpu).argsort(-1)[..., :recent_count] + (T - W)
    old = torch.rand((L, R, T - W), generator=gen, device=gpu).topk(old_count, dim=-1).indices
    topk = torch.cat([recent, old], dim=-1)
    del recent, old
    topk = torch.gather(topk, -1, torch.rand((L, R, K), generator=gen, device=gpu).argsort(-1))
    topk = topk.to(torch.int32).contiguous()
    table = torch.zeros((L, R, T), dtype=torch.int32, device=gpu)
    base = (torch.arange(R, device=gpu, dtype=torch.int32) * C + 1).view(1, R, 1)
    table[:, :, T - C:] = torch.rand((L, R, C), generator=gen, device=gpu).argsort(-1).to(torch.int32) + base
    bits = build_residency_bits(table)
    rows = torch.arange(R, device=gpu)
    lengths = torch.full((R,), T, dtype=torch.int32, device=gpu)
    slots = torch.full((L, R, K), -7, dtype=torch.int32, device=gpu)
    misses = torch.full((L, R, K), -5, dtype=torch.int32, device=gpu)
    counts = torch.full((L, R), -5, dtype=torch.int32, device=gpu)
    resolve_resident(topk, table, None, rows, lengths, rows, slots, 1, misses=misses, miss_count=counts,
                     resident_bits=bits)
    torch.cuda.synchronize()
    print(f"[full-size decode] lookup done, counts {int(counts.min())}..{int(counts.max())}", flush=True)

    # Lookup: closed forms.
    assert bool((counts == old_count).all())
    is_old = topk < T - C
    lanes = torch.arange(K, device=gpu, dtype=torch.int32).expand(L, R, K)
    want_misses = torch.sort(torch.where(is_old, lanes, K), dim=-1).values[..., :old_count]
    assert torch.equal(misses[..., :old_count], want_misses)
    assert bool((misses[..., old_count:] == -5).all())
    assert bool((slots[is_old] == 0).all())
    assert torch.equal(torch.where(is_old, 0, torch.gather(table, -1, topk.long())), slots)
    del is_old, lanes, want_misses, table, bits

    # Gather: every plane against index_select, misses as zero rows.
    layout = PlanePoolLayout(layers=L, kv=2, rows=1 + R * C, row_bytes=row_bytes)
    backing, raw = committed_pool(layout, gpu, 32)
    try:
        out = torch.empty((R, L, 2, K, row_bytes), dtype=torch.uint8, device=gpu)
        gather_kv(layout.kv_planes(backing.base, 0, owner=backing), slots, out)
        torch.cuda.synchronize()
        print("[full-size decode] gather done", flush=True)
        for layer in range(L):
            hit = (slots[layer] > 0).unsqueeze(-1)
            for kv in range(2):
                want = plane_rows(raw, layout, layer, kv).index_select(0, slots[layer].reshape(-1).long())
                want = torch.where(hit, want.view(R, K, row_bytes), 0)
                assert torch.equal(out[:, layer, kv], want), (layer, kv)
        del out
    finally:
        torch.cuda.synchronize()
        del raw
        backing.close()


def test_block_gather_at_full_size(gpu):
    R, NB, L, POOL = 64, 256, 36, 20000
    row_bytes = 16 * 8 * 128 * 2
    tables = np.random.default_rng(2024).permutation(POOL)[: R * NB].reshape(R, NB)
    layout = PlanePoolLayout(layers=L, kv=2, rows=POOL, row_bytes=row_bytes)
    backing, raw = committed_pool(layout, gpu, 7)
    try:
        tables_d = torch.tensor(tables, dtype=torch.int32, device=gpu)
        out = torch.empty((R, L, 2, NB, row_bytes), dtype=torch.uint8, device=gpu)
        gather_kv(layout.kv_planes(backing.base, 0, owner=backing), tables_d.unsqueeze(0).expand(L, R, NB), out,
                  zero_below=0)
        torch.cuda.synchronize()
        print("[full-size block gather] gather done", flush=True)
        index = tables_d.reshape(-1).long()
        for layer in range(L):
            for kv in range(2):
                want = plane_rows(raw, layout, layer, kv).index_select(0, index).view(R, NB, row_bytes)
                assert torch.equal(out[:, layer, kv], want), (layer, kv)
        del out
    finally:
        torch.cuda.synchronize()
        del raw
        backing.close()
