"""GPU parity of whole configurations against the oracle.

- Config 1, the reference's CPU-runnable case, at full size: 8 requests x
  8192-token context, the two-level lookup req_to_token -> mapping
  (adaptive_sparse/resident_lookup.py:6-40), Top-K 2048 shared by 28 layers
  of 8 KV heads, and the gather of their 2 KiB K and V rows from a VMM pool
  (experimental/sparse_read.py:11-30 in multi-plane form). Slots, miss lists
  and every gathered byte equal the C oracle's.
- Config 5, the composite elastic decode step, at a reduced size (8 requests
  x 4 layers, contexts uniform in [4096, 32768], Top-K 2048 with the decode
  locality mix, hot capacity 4096): every step remaps 5 % of the pool's
  chunks (their hot slots are invalidated, the chunks unmapped and committed
  again, zero-filled), then lookup, LRU swap-in, promote from pinned host and
  gather. The lookup, the LRU state and the promotions equal the oracle's
  (adaptive_sparse/request_residency.py:805-832 with the batch-token LRU of
  benchmarks/hisparse_locality_replay.py:90-99), and every gathered row equals
  its token's host row.
- Config 5 at full size (128 requests x 60 layers), two steps, each with
  its 5 % chunk remap: every gathered K/V row equals its token's host row,
  the hot-buffer state stays a bijection between tokens and slots, every
  selected lane is resident in the slot it read, and the residency summary
  kept by the swap-ins equals a fresh build, per position and per 64
  positions with its group counts (size-independent checks; the oracle
  itself runs at the reduced size above).
- The prefetching lookup with more items than 16 per resident workgroup, the
  launch shape where the host raises the grid above the resident count.
"""

import numpy as np
import pytest
import torch

from adaptive_sparse.host_arena import HostArena
from adaptive_sparse.kv_pool import KVPlanes, PlanePoolLayout
from adaptive_sparse.resident_lookup import build_residency_bits, resolve_resident
from adaptive_sparse.sparse_read import gather_kv
from adaptive_sparse.swap_in import INT32_MIN, HotBuffers, move_kv, residency_counts, swap_in
from elastic_kv.backing import Backing
from oracle import oracle as ref

pytestmark = pytest.mark.gpu


def _filled_pool(layout, device, seed):
    backing = Backing(layout.capacity_bytes, layout.chunk_bytes, device=device.index or 0)
    backing.ensure(range(backing.chunk_count))
    raw = backing.raw
    gen = torch.Generator(device=device).manual_seed(seed)
    for plane in range(layout.planes):
        raw.narrow(0, plane * layout.plane_stride, layout.plane_bytes).view(torch.bfloat16).normal_(generator=gen)
    return backing, raw


def test_config1_full_size_matches_the_oracle(gpu, coracle):
    R, T, L, K, C = 8, 8192, 28, 2048, 4096
    row_bytes = 8 * 128 * 2
    rng = np.random.default_rng(2024)
    table = np.arange(R * T, dtype=np.int64).reshape(R, T) + 1          # req_to_token: logical ids
    mapping = np.zeros(R * T + 1, dtype=np.int64)                        # logical id -> hot slot (0 = miss)
    for r in range(R):
        resident = rng.choice(T, C, replace=False)
        mapping[r * T + resident + 1] = r * C + rng.permutation(C) + 1
    topk = np.stack([rng.choice(T, K, replace=False) for _ in range(R)])[None].astype(np.int32)
    layout = PlanePoolLayout(layers=L, kv=2, rows=1 + R * C, row_bytes=row_bytes)
    backing, raw = _filled_pool(layout, gpu, 7)
    try:
        planes = layout.kv_planes(backing.base, 0, owner=backing)
        rows = torch.arange(R, device=gpu)
        lengths = torch.full((R,), T, dtype=torch.int32, device=gpu)
        slots = torch.full((1, R, K), -7, dtype=torch.int32, device=gpu)
        misses = torch.full((1, R, K), -5, dtype=torch.int32, device=gpu)
        counts = torch.empty((1, R), dtype=torch.int32, device=gpu)
        resolve_resident(torch.tensor(topk, device=gpu), torch.tensor(table, device=gpu),
                         torch.tensor(mapping, device=gpu), rows, lengths, rows, slots, 1, misses=misses,
                         miss_count=counts)
        output = torch.empty((R, L, 2, K, row_bytes), dtype=torch.uint8, device=gpu)
        gather_kv(planes, slots.expand(L, R, K), output)
        torch.cuda.synchronize()
        print("[config 1] lookup + gather done", flush=True)
        idx, full = np.arange(R), np.full(R, T)
        want_slots, want_misses, want_counts = coracle.resolve_resident(
            topk, table, mapping, idx, full, idx, 1, np.full((1, R, K), -7, np.int32), with_misses=True)
        assert np.array_equal(slots.cpu().numpy(), want_slots)
        assert np.array_equal(counts.cpu().numpy(), want_counts)
        got_misses = misses.cpu().numpy()
        for r in range(R):
            c = int(want_counts[0, r])
            assert np.array_equal(got_misses[0, r, :c], want_misses[0, r, :c]), r
            assert (got_misses[0, r, c:] == -5).all(), r
        hit_rate = float((want_slots > 0).mean())
        assert 0.45 < hit_rate < 0.55
        pool = raw.cpu().numpy()
        want_rows = coracle.gather_kv(pool, planes.layer_stride, planes.kv_stride, row_bytes, row_bytes,
                                      layout.rows, want_slots[0], 2, shared_layers=L)
        assert np.array_equal(output.cpu().numpy().reshape(want_rows.shape), want_rows)
    finally:
        torch.cuda.synchronize()
        del raw
        backing.close()


def _composite_topk(rng, L, R, K, lengths, window=4096):
    """Per (layer, request): K distinct tokens, 80 % from the last `window` of its context, the rest older."""
    topk = np.empty((L, R, K), np.int64)
    for layer in range(L):
        for r in range(R):
            n = int(lengths[r])
            older = max(0, n - window)
            far = min(older, K - (K * 4) // 5)
            near = rng.choice(np.arange(older, n), K - far, replace=False)
            old = rng.choice(older, far, replace=False) if far else np.empty(0, np.int64)
            topk[layer, r] = rng.permutation(np.concatenate([near, old]))
    return topk


def test_config5_composite_steps_match_the_oracle(gpu):
    L, R, K, C, HOST_ROWS, row_bytes = 4, 8, 2048, 4096, 65536, 512
    rng = np.random.default_rng(55)
    lengths = rng.integers(4096, 32769, R)
    T = int(lengths.max())
    layout = PlanePoolLayout(layers=L, kv=2, rows=1 + R * C, row_bytes=row_bytes)
    backing = Backing(layout.capacity_bytes, layout.chunk_bytes, device=0)
    arena = None
    try:
        backing.ensure(range(backing.chunk_count))
        planes = layout.kv_planes(backing.base, 0, owner=backing)
        host_plane = HOST_ROWS * row_bytes
        arena = HostArena(2 * L * host_plane)
        arena.host.copy_(torch.randint(0, 256, (2 * L * host_plane,), dtype=torch.uint8))
        host = arena.host.numpy().reshape(L, 2, HOST_ROWS, row_bytes)
        host_planes = KVPlanes(base=arena.device_ptr, device=0, layers=L, kv=2, layer_stride=2 * host_plane,
                               kv_stride=host_plane, row_stride=row_bytes, row_bytes=row_bytes, rows=HOST_ROWS,
                               owner=arena)
        host_table = ((np.arange(R)[:, None] * T + np.arange(T)[None, :]) % HOST_ROWS).astype(np.int32)
        host_table_d = torch.tensor(host_table, device=gpu)
        # The C most recent tokens of every request are resident, in a seeded permutation of its slots.
        buffers = HotBuffers(L, R, T, C, gpu, table_dtype=torch.int16, bits_shift=6)
        recent = torch.tensor(lengths, device=gpu).view(1, R, 1) - C + torch.arange(C, device=gpu).view(1, 1, C)
        local = torch.tensor(np.stack([[rng.permutation(C) for _ in range(R)] for _ in range(L)]), device=gpu)
        buffers.install(recent.expand(L, R, C), local)
        src = torch.tensor(host_table, device=gpu)[torch.arange(R, device=gpu).view(1, R, 1), recent.expand(L, R, C)]
        move_kv(host_planes, src.to(torch.int32).contiguous(), planes,
                (local + buffers.slot_base.view(1, R, 1)).to(torch.int32).contiguous(),
                torch.full((L, R), C, dtype=torch.int32, device=gpu))
        base = buffers.slot_base.cpu().numpy()

        def global_table():
            t = buffers.table.cpu().numpy().astype(np.int64)
            return np.where(t > 0, base.reshape(1, R, 1) + t - 1, 0)

        state = {"table": global_table(), "slot_token": buffers.slot_token.cpu().numpy(),
                 "stamps": buffers.stamps.cpu().numpy()}
        rows = torch.arange(R, device=gpu)
        lengths_d = torch.tensor(lengths, dtype=torch.int32, device=gpu)
        chunk_rows = layout.chunk_bytes // row_bytes
        remap_count = max(1, round(0.05 * backing.chunk_count))
        for step in range(3):
            # Remap 5 % of the chunks (never the sink): their hot slots become empty, on the GPU
            # state and on the oracle's, then the chunks are unmapped and committed again.
            chosen = rng.choice(np.arange(1, backing.chunk_count), size=remap_count, replace=False)
            slot_token, stamps, table = state["slot_token"], state["stamps"], state["table"]
            for chunk in chosen.tolist():
                plane, within = divmod(chunk, layout.plane_chunks)
                layer = plane // 2
                for slot in range(within * chunk_rows, (within + 1) * chunk_rows):
                    if not 1 <= slot < layout.rows:
                        continue
                    r, loc = divmod(slot - 1, C)
                    token = slot_token[layer, r, loc]
                    if token >= 0:
                        table[layer, r, token] = 0
                    slot_token[layer, r, loc] = -1
                    stamps[layer, r, loc] = INT32_MIN
            local_table = np.where(table > 0, table - base.reshape(1, R, 1) + 1, 0)
            buffers.table.copy_(torch.tensor(local_table, dtype=torch.int16))
            buffers.slot_token.copy_(torch.tensor(slot_token))
            buffers.stamps.copy_(torch.tensor(stamps))
            buffers.refresh_bits()
            backing.reclaim(chosen.tolist())
            backing.ensure(chosen.tolist())
            # lookup -> swap-in -> promote -> gather
            topk = _composite_topk(rng, L, R, K, lengths)
            topk_d = torch.tensor(topk, dtype=torch.int32, device=gpu)
            slots = torch.empty((L, R, K), dtype=torch.int32, device=gpu)
            misses = torch.full((L, R, K), -1, dtype=torch.int32, device=gpu)
            counts = torch.empty((L, R), dtype=torch.int32, device=gpu)
            promote_src = torch.full((L, R, K), -9, dtype=torch.int32, device=gpu)
            promote_dst = torch.full((L, R, K), -9, dtype=torch.int32, device=gpu)
            output = torch.empty((R, L, 2, K, row_bytes), dtype=torch.uint8, device=gpu)
            resolve_resident(topk_d, buffers.table, None, rows, lengths_d, rows, slots, 1, misses=misses,
                             miss_count=counts, resident_bits=buffers.bits, bits_shift=buffers.bits_shift,
                             slot_base=buffers.slot_base)
            looked_up = slots.cpu().numpy()
            swap_in(topk_d, 1, rows, rows, slots, misses, counts, buffers, host_table_d, promote_src, promote_dst,
                    check=True)
            move_kv(host_planes, promote_src, planes, promote_dst, counts)
            gather_kv(planes, slots, output)
            torch.cuda.synchronize()
            print(f"[config 5] step {step}: {int(counts.sum())} misses", flush=True)
            want_slots, want_misses, want_counts = ref.resolve_resident(
                topk, state["table"], None, np.arange(R), lengths, np.arange(R), 1, np.zeros((L, R, K), np.int32),
                with_misses=True)
            assert np.array_equal(looked_up, want_slots), step
            assert np.array_equal(counts.cpu().numpy(), want_counts), step
            miss_np = np.full((L, R, K), -1, np.int32)
            for (layer, r), lanes in want_misses.items():
                miss_np[layer, r, :len(lanes)] = lanes
            state = ref.swap_in(step, 1, topk, np.arange(R), np.arange(R), want_slots, miss_np, want_counts,
                                state["table"], state["slot_token"], state["stamps"], base, host_table)
            assert np.array_equal(slots.cpu().numpy(), state["slots"]), step
            assert np.array_equal(global_table(), state["table"]), step
            assert np.array_equal(buffers.slot_token.cpu().numpy(), state["slot_token"]), step
            assert np.array_equal(buffers.stamps.cpu().numpy(), state["stamps"]), step
            got_src, got_dst = promote_src.cpu().numpy(), promote_dst.cpu().numpy()
            for layer in range(L):
                for r in range(R):
                    c = int(want_counts[layer, r])
                    assert np.array_equal(got_src[layer, r, :c], state["promote_src"][layer, r, :c])
                    assert np.array_equal(got_dst[layer, r, :c], state["promote_dst"][layer, r, :c])
            got = output.cpu().numpy()
            for layer in range(L):
                for r in range(R):
                    host_rows = host_table[r, topk[layer, r]]
                    for kv in range(2):
                        assert np.array_equal(got[r, layer, kv], host[layer, kv, host_rows]), (step, layer, r, kv)
    finally:
        torch.cuda.synchronize()
        backing.close()
        if arena is not None:
            arena.close()


def _composite_topk_gpu(gen, L, R, K, lengths, window=4096):
    """Per (layer, request) on the device: K distinct tokens, 80 % from the last `window`, the rest uniform older."""
    device = lengths.device
    T = int(lengths.max())
    far_want = K - (K * 4) // 5
    older = (lengths - window).clamp_min(0)
    far = torch.minimum(older, torch.full_like(older, far_want))
    near_count = K - far
    near = torch.rand((L, R, window), generator=gen, device=device).argsort(-1)[..., :K] + older.view(1, R, 1)
    keys = torch.rand((L, R, T), generator=gen, device=device)
    keys.masked_fill_(torch.arange(T, device=device).view(1, 1, T) >= older.view(1, R, 1), 2.0)
    old = keys.topk(far_want, dim=-1, largest=False).indices
    del keys
    lane = torch.arange(K, device=device).view(1, 1, K)
    pick = torch.where(lane < near_count.view(1, R, 1), near,
                       torch.gather(old, -1, (lane - near_count.view(1, R, 1)).clamp(0, far_want - 1)))
    order = torch.rand((L, R, K), generator=gen, device=device).argsort(-1)
    return torch.gather(pick, -1, order).to(torch.int32).contiguous()


@pytest.mark.parametrize("shift", [0, 6])
def test_config5_full_size_steps_keep_rows_and_lru_invariants(gpu, shift):
    # shift 0: the per-position summary that the composite workload of bench.py runs; shift 6: the line summary
    # with the group counts that the swap-in keeps.
    L, R, K, C, HOST_ROWS, row_bytes = 60, 128, 2048, 4096, 65536, 512
    gen = torch.Generator(device=gpu).manual_seed(505)
    rng = np.random.default_rng(505)
    lengths = torch.randint(4096, 32769, (R,), generator=gen, device=gpu)
    T = int(lengths.max())
    layout = PlanePoolLayout(layers=L, kv=2, rows=1 + R * C, row_bytes=row_bytes)
    backing = Backing(layout.capacity_bytes, layout.chunk_bytes, device=0)
    arena = None
    try:
        backing.ensure(range(backing.chunk_count))
        planes = layout.kv_planes(backing.base, 0, owner=backing)
        host_plane = HOST_ROWS * row_bytes
        arena = HostArena(2 * L * host_plane)
        host_gpu = torch.randint(0, 256, (L, 2, HOST_ROWS, row_bytes), dtype=torch.uint8, device=gpu,
                                 generator=gen)
        arena.host.copy_(host_gpu.view(-1).cpu())
        host_planes = KVPlanes(base=arena.device_ptr, device=0, layers=L, kv=2, layer_stride=2 * host_plane,
                               kv_stride=host_plane, row_stride=row_bytes, row_bytes=row_bytes, rows=HOST_ROWS,
                               owner=arena)
        host_table = ((torch.arange(R, device=gpu).view(R, 1) * T + torch.arange(T, device=gpu).view(1, T))
                      % HOST_ROWS).to(torch.int32)
        buffers = HotBuffers(L, R, T, C, gpu, table_dtype=torch.int16, bits_shift=shift)
        recent = (lengths.view(1, R, 1) - C + torch.arange(C, device=gpu).view(1, 1, C)).expand(L, R, C)
        local = torch.rand((L, R, C), generator=gen, device=gpu).argsort(-1)
        buffers.install(recent, local)
        rows = torch.arange(R, device=gpu)
        move_kv(host_planes, host_table[rows.view(1, R, 1), recent].contiguous(), planes,
                (local + buffers.slot_base.view(1, R, 1)).to(torch.int32).contiguous(),
                torch.full((L, R), C, dtype=torch.int32, device=gpu))
        lengths32 = lengths.to(torch.int32)
        slots = torch.empty((L, R, K), dtype=torch.int32, device=gpu)
        misses = torch.empty_like(slots)
        counts = torch.empty((L, R), dtype=torch.int32, device=gpu)
        src, dst = torch.empty_like(slots), torch.empty_like(slots)
        output = torch.empty((R, L, 2, K, row_bytes), dtype=torch.uint8, device=gpu)
        chunk_rows = layout.chunk_bytes // row_bytes
        remap_count = round(0.05 * backing.chunk_count)
        torch.cuda.synchronize()
        print(f"[config 5 full, shift {shift}] ready: {backing.chunk_count} chunks, remap {remap_count} per step",
              flush=True)
        for step in range(2):
            # remap: empty the chosen chunks' hot slots, unmap them and commit them again (zero-filled)
            chosen = rng.choice(np.arange(1, backing.chunk_count), size=remap_count, replace=False)
            ids = torch.tensor(chosen, device=gpu)
            plane, within = ids // layout.plane_chunks, ids % layout.plane_chunks
            slot = within.view(-1, 1) * chunk_rows + torch.arange(chunk_rows, device=gpu).view(1, -1)
            layer = (plane // 2).view(-1, 1).expand_as(slot)
            keep = (slot >= 1) & (slot < layout.rows)
            slot, layer = slot[keep], layer[keep]
            req, loc = (slot - 1) // C, (slot - 1) % C
            token = buffers.slot_token[layer, req, loc].long()
            held = token >= 0
            buffers.table[layer[held], req[held], token[held]] = 0
            buffers.slot_token[layer, req, loc] = -1
            buffers.stamps[layer, req, loc] = INT32_MIN
            buffers.refresh_bits()
            backing.reclaim(chosen.tolist())
            backing.ensure(chosen.tolist())
            topk = _composite_topk_gpu(gen, L, R, K, lengths)
            resolve_resident(topk, buffers.table, None, rows, lengths32, rows, slots, 1, misses=misses,
                             miss_count=counts, resident_bits=buffers.bits, bits_shift=buffers.bits_shift,
                             slot_base=buffers.slot_base)
            swap_in(topk, 1, rows, rows, slots, misses, counts, buffers, host_table, src, dst, check=True)
            move_kv(host_planes, src, planes, dst, counts)
            gather_kv(planes, slots, output)
            torch.cuda.synchronize()
            print(f"[config 5 full, shift {shift}] step {step}: {int(counts.sum())} of {L * R * K} lanes promoted",
                  flush=True)
            # every gathered row is its token's host row
            for layer_index in range(L):
                host_rows = torch.gather(host_table, 1, topk[layer_index].long()).long()          # [R, K]
                for kv in range(2):
                    want = host_gpu[layer_index, kv][host_rows]                                    # [R, K, row]
                    assert torch.equal(output[:, layer_index, kv], want), (step, layer_index, kv)
            # every selected lane is resident in the slot it read
            local_slot = slots.long() - buffers.slot_base.view(1, R, 1)
            assert bool(((local_slot >= 0) & (local_slot < C)).all()), step
            assert torch.equal(torch.gather(buffers.slot_token, 2, local_slot).long(), topk.long()), step
            # the token <-> slot state is a bijection, and the summary (and its group counts) are exact
            slot_token = buffers.slot_token.long()
            held = slot_token >= 0
            entry = torch.gather(buffers.table.long(), 2, slot_token.clamp_min(0))              # [L, R, C]
            assert torch.equal(entry[held], (torch.arange(C, device=gpu).expand(L, R, C) + 1)[held]), step
            assert int((buffers.table != 0).sum()) == int(held.sum()), step
            assert torch.equal(buffers.bits, build_residency_bits(buffers.table, shift=shift)), step
            if shift:
                assert torch.equal(buffers.resident_counts, residency_counts(buffers.table, shift)), step
    finally:
        torch.cuda.synchronize()
        backing.close()
        if arena is not None:
            arena.close()


def test_prefetching_lookup_with_a_raised_grid(gpu):
    # 40 layers x 1000 rows = 40,000 items: more than 16 per resident workgroup
    # (2048 on MI355X), so the host raises the grid; K = 8 lanes per row.
    L, B, R, T, K, C = 40, 1000, 50, 512, 8, 64
    rng = np.random.default_rng(8)
    local = np.zeros((L, R, T), np.int64)
    for layer in range(L):
        for r in range(R):
            held = rng.choice(T, C, replace=False)
            local[layer, r, held] = rng.permutation(C) + 1
    base = np.arange(R) * C + 1
    rows = rng.integers(0, R, B)
    lengths = rng.integers(0, T + 1, B)
    topk = rng.integers(-1, T, (L, B, K))
    selected = rng.permutation(B)[: B - 7]
    global_table = np.where(local > 0, base.reshape(1, R, 1) + local - 1, 0)
    want, want_misses, want_counts = ref.resolve_resident(topk, global_table, None, rows, lengths, selected, 1,
                                                          np.full((L, B, K), -3, np.int32), with_misses=True)
    table16 = torch.tensor(local, dtype=torch.int16, device=gpu)
    for shift in (0, 6):
        slots = torch.full((L, B, K), -3, dtype=torch.int32, device=gpu)
        misses = torch.full((L, B, K), -2, dtype=torch.int32, device=gpu)
        counts = torch.full((L, B), -2, dtype=torch.int32, device=gpu)
        resolve_resident(torch.tensor(topk, dtype=torch.int32, device=gpu), table16, None,
                         torch.tensor(rows, device=gpu), torch.tensor(lengths, device=gpu),
                         torch.tensor(selected, device=gpu), slots, 1, misses=misses, miss_count=counts,
                         resident_bits=build_residency_bits(table16, shift=shift), bits_shift=shift,
                         slot_base=torch.tensor(base, device=gpu))
        assert np.array_equal(slots.cpu().numpy(), want), shift
        got_counts, got_misses = counts.cpu().numpy(), misses.cpu().numpy()
        for layer in range(L):
            for b in selected:
                c = int(want_counts[layer, b])
                assert got_counts[layer, b] == c
                assert np.array_equal(got_misses[layer, b, :c], want_misses[(layer, int(b))])
        unselected = np.setdiff1d(np.arange(B), selected)
        assert (got_counts[:, unselected] == -2).all()
