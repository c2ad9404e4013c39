"""Full-size GPU checks of the decode read and the block gather.

At full size the oracle would take minutes, so these tests check properties
that do not depend on size instead:
- the HiSparse decode read (128 requests x 65,536 tokens x 60 layers,
  Top-K 2048, hot capacity 2048, 4096 or 8192 holding the most recent
  tokens) is built so that its results have closed forms. Each (layer,
  request) selects 1638 distinct tokens from the last 4096 positions and 410
  distinct tokens from the rest; a lane misses exactly when its token lies
  below T - C (at C = 4096: exactly the 410 old picks of every row), its miss
  list is those lanes in order, and a hit's slot is its table entry. Every
  table form is checked: int32 global slots and int16 local slots behind the
  per-position bitmap, and the decode default, int16 behind the line summary;
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


@pytest.mark.parametrize("capacity", [2048, 4096, 8192])
def test_decode_read_at_full_size(gpu, capacity):
    """Closed forms of the decode read at every hot capacity, through each table form.

    The hot set is the C most recent tokens, so a lane misses exactly when it
    picked a token below T - C: at C = 4096 that is the 410 old picks of every
    row, at C = 2048 also the recent picks in [T - 4096, T - 2048), at
    C = 8192 only the old picks below T - 8192.
    """
    L, R, T, K, C, W = 60, 128, 65536, 2048, capacity, 4096
    recent_count, old_count = 1638, 410
    row_bytes = 512
    gen = torch.Generator(device=gpu).manual_seed(31 + capacity)
    recent = torch.rand((L, R, W), generator=gen, device=gpu).argsort(-1)[..., :recent_count] + (T - W)
    old = torch.rand((L, R, T - W), generator=gen, device=gpu).topk(old_count, dim=-1).indices
    topk = torch.cat([recent, old], dim=-1)
    del recent, old
    topk = torch.gather(topk, -1, torch.rand((L, R, K), generator=gen, device=gpu).argsort(-1))
    topk = topk.to(torch.int32).contiguous()
    table = torch.zeros((L, R, T), dtype=torch.int32, device=gpu)
    base = torch.arange(R, device=gpu, dtype=torch.int64) * C + 1
    table[:, :, T - C:] = (torch.rand((L, R, C), generator=gen, device=gpu).argsort(-1)
                           + base.view(1, R, 1)).to(torch.int32)
    table16 = torch.where(table > 0, table - base.view(1, R, 1) + 1, 0).to(torch.int16)
    rows = torch.arange(R, device=gpu)
    lengths = torch.full((R,), T, dtype=torch.int32, device=gpu)
    is_old = topk < T - C
    miss_count = is_old.sum(-1).to(torch.int32)
    lanes = torch.arange(K, device=gpu, dtype=torch.int32).expand(L, R, K)
    want_misses = torch.sort(torch.where(is_old, lanes, K), dim=-1).values
    want_slots = torch.where(is_old, 0, torch.gather(table, -1, topk.long()))
    forms = {"int32 table + position bitmap": dict(table=table, resident_bits=build_residency_bits(table)),
             "int16 table + position bitmap": dict(table=table16, resident_bits=build_residency_bits(table16),
                                                   slot_base=base),
             "int16 table + line summary (decode default)": dict(table=table16, slot_base=base, bits_shift=6,
                                                                 resident_bits=build_residency_bits(table16, shift=6))}
    slots = None
    for name, form in forms.items():
        slots = torch.full((L, R, K), -7, dtype=torch.int32, device=gpu)
        misses = torch.full((L, R, K), -5, dtype=torch.int32, device=gpu)
        counts = torch.full((L, R), -5, dtype=torch.int32, device=gpu)
        resolve_resident(topk, form.pop("table"), None, rows, lengths, rows, slots, 1, misses=misses,
                         miss_count=counts, **form)
        torch.cuda.synchronize()
        print(f"[full-size decode C={C}] {name}: counts {int(counts.min())}..{int(counts.max())}", flush=True)
        assert torch.equal(counts, miss_count), name
        filled = lanes < counts.unsqueeze(-1)
        assert torch.equal(torch.where(filled, misses, K), want_misses), name
        assert bool((misses[~filled] == -5).all()), name
        assert torch.equal(slots, want_slots), name
    if C == 4096:
        assert bool((miss_count == old_count).all())
    hit_rate = float((want_slots > 0).float().mean())
    print(f"[full-size decode C={C}] hit rate {hit_rate:.4f}", flush=True)
    del is_old, lanes, want_misses, table, table16, forms, want_slots

    # Gather: every plane against index_select, misses as zero rows.
    layout = PlanePoolLayout(layers=L, kv=2, rows=1 + R * C, row_bytes=row_bytes)
    backing, raw = committed_pool(layout, gpu, 32)
    try:
        out = torch.empty((R, L, 2, K, row_bytes), dtype=torch.uint8, device=gpu)
        gather_kv(layout.kv_planes(backing.base, 0, owner=backing), slots, out)
        torch.cuda.synchronize()
        print(f"[full-size decode C={C}] gather done", flush=True)
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
