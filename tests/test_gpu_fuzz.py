"""Seeded random configurations of the HIP kernels against the oracle (bit-exact).

Each case draws its shapes, dtypes, strides (views of larger buffers), block
size, table form (single or two level, with or without a layer dimension,
with or without the residency bitmap), lengths, selections, row sizes and
vector widths, plane strides and zero_below from a seed, including request
rows outside the table and selection entries outside the batch. The cases are small
(the oracle runs in milliseconds) and together cover the kernels' branches:
the recent-window staging, the bitmap staged in LDS or read per lane, the
int16 local-slot tables, the dense and strided addressing, every vector width of the copy engine, and
large rows cut into segments.
"""

import numpy as np
import pytest
import torch

from adaptive_sparse.kv_pool import KVPlanes
from adaptive_sparse.resident_lookup import build_residency_bits, resolve_resident
from adaptive_sparse.sparse_read import gather_kv, scatter_kv
from adaptive_sparse.swap_in import move_kv
from oracle import oracle as ref

pytestmark = pytest.mark.gpu


def bits_match(got, want):
    """A bitmap padded to whole 16-byte pieces holds the oracle's ceil(T / 32) words, then zeros."""
    words = want.shape[-1]
    return (got.shape[-1] == -(-words // 4) * 4 and np.array_equal(got[..., :words], want)
            and not got[..., words:].any())

INDEX_DTYPES = (torch.int32, torch.int64)


def on_gpu(array, dtype, device, strided):
    """`array` on the device, optionally as a view with stride 2 along the last dimension."""
    source = torch.tensor(array, dtype=dtype)
    if not strided:
        return source.to(device)
    spread = torch.zeros((*source.shape, 2), dtype=dtype)
    spread[..., 0] = source
    return spread.to(device)[..., 0]


@pytest.mark.parametrize("seed", range(100))
def test_lookup_random_configurations(gpu, coracle, seed):
    rng = np.random.default_rng(7000 + seed)
    layers = int(rng.integers(1, 4))
    batch = int(rng.integers(1, 9))
    bs = int(rng.choice([1, 1, 1, 2, 3, 8, 16]))
    k = int(rng.integers(1, 2600 // bs + 2))
    rrows = int(rng.integers(1, 10))
    cols = int(rng.integers(1, 7000))
    layered = bool(rng.random() < 0.5)
    mapped = bool(rng.random() < 0.35)
    use_bits = (not mapped) and bool(rng.random() < 0.6)
    local = (not mapped) and bool(rng.random() < 0.3)     # int16 table of local slots + per-request bases
    compact = bool(rng.random() < 0.8)
    strided = {name: bool(rng.random() < 0.25) for name in ("topk", "table", "output")}
    topk_dtype, table_dtype, map_dtype = (INDEX_DTYPES[int(rng.integers(2))] for _ in range(3))

    lengths = rng.integers(-2, cols + 5, size=batch)
    rows = rng.integers(0, rrows, size=batch)
    stray = rng.random(batch) < 0.1          # request rows outside the table resolve to -1
    rows[stray] = rng.choice([-1, rrows, rrows + 7], size=int(stray.sum()))
    width = k * bs
    topk = rng.integers(-1, cols // bs + 2, size=(layers, batch, k))
    for r in range(batch):  # a recent-heavy share, as decode Top-K sets are
        hi = max(1, min(int(lengths[r]), cols) // bs)
        near = rng.random((layers, k)) < 0.6
        topk[:, r][near] = rng.integers(max(0, hi - 1200 // bs), hi + 1, size=(layers, k))[near]
    shape = (layers, rrows, cols) if layered else (rrows, cols)
    n = 5000
    mapping = None
    if mapped:
        table = rng.integers(-2, n + 2, size=shape)
        mapping = rng.integers(1, 1 << 20, size=n)
        mapping[rng.random(n) < 0.3] = 0
    else:
        table = rng.integers(1, 1 << 20, size=shape)
        table[rng.random(shape) < 0.4] = 0
    slot_base = None
    if local:
        local_table = rng.integers(1, 1 << 15, size=shape)
        local_table[rng.random(shape) < 0.4] = 0
        local_table[rng.random(shape) < 0.02] = -int(rng.integers(1, 1 << 15))   # negative: not resident
        slot_base = rng.integers(1, 1 << 20, size=rrows)
        req_axis = 1 if layered else 0
        bases = np.expand_dims(slot_base, tuple(a for a in range(len(shape)) if a != req_axis))
        table = np.where(local_table > 0, bases + local_table - 1, 0)          # the oracle's global form
    selected = rng.permutation(batch)[: int(rng.integers(1, batch + 1))]
    if rng.random() < 0.2:                   # selection entries outside the batch are skipped
        selected = np.concatenate([selected, [-1, batch]])
    initial = np.full((layers, batch, width), -77, np.int32)
    want, want_misses, want_counts = coracle.resolve_resident(topk, table, mapping, rows, lengths, selected, bs,
                                                              initial, with_misses=True)

    table_d = on_gpu(local_table if local else table, torch.int16 if local else table_dtype, gpu, strided["table"])
    bits = build_residency_bits(table_d) if use_bits else None
    output = on_gpu(initial, torch.int32, gpu, strided["output"])
    misses = torch.full((layers, batch, width), -5, dtype=torch.int32, device=gpu) if compact else None
    counts = torch.full((layers, batch), -5, dtype=torch.int32, device=gpu) if compact else None
    resolve_resident(on_gpu(topk, topk_dtype, gpu, strided["topk"]), table_d,
                     None if mapping is None else torch.tensor(mapping, dtype=map_dtype, device=gpu),
                     torch.tensor(rows, device=gpu), torch.tensor(lengths, dtype=torch.int32, device=gpu),
                     torch.tensor(selected, device=gpu), output, bs, misses=misses, miss_count=counts,
                     resident_bits=bits,
                     slot_base=None if slot_base is None else torch.tensor(slot_base, device=gpu))
    assert np.array_equal(output.cpu().numpy(), want), (seed, layers, batch, bs, k, cols, layered, mapped, use_bits,
                                                        local)
    if compact:
        got_counts, got_misses = counts.cpu().numpy(), misses.cpu().numpy()
        for layer in range(layers):
            for row in range(batch):
                if row in selected:
                    c = want_counts[layer, row]
                    assert got_counts[layer, row] == c
                    assert np.array_equal(got_misses[layer, row, :c], want_misses[layer, row, :c])
                else:
                    assert got_counts[layer, row] == -5


@pytest.mark.parametrize("seed", range(40))
def test_local_slot_runs_random_configurations(gpu, coracle, seed):
    # The decode default: int32 Top-K, int16 local-slot table with slot bases,
    # residency bitmap, block size 1, K a multiple of 8 and 16-byte aligned
    # rows, which the contiguous 8-lane-run kernel serves. Widths past one
    # 2048-lane chunk, bitmaps too wide to stage (T > 131072), stray rows and
    # partial selections; a Top-K view shifted by one element must give the
    # same answer through the strided kernel.
    rng = np.random.default_rng(9100 + seed)
    layers = int(rng.integers(1, 4))
    batch = int(rng.integers(1, 9))
    k = 8 * int(rng.integers(1, 700 if seed % 2 == 0 else 257))    # odd seeds: one 2048-lane chunk
    rrows = int(rng.integers(1, 10))
    cols = int(rng.integers(1, 7000)) if seed % 8 else int(rng.integers(131_073, 140_000))
    if seed % 4 == 1:
        cols = 8 * ((cols + 7) // 8)        # 16-byte aligned table rows
    layered = bool(rng.random() < 0.7)
    compact = bool(rng.random() < 0.85)
    lengths = rng.integers(-2, cols + 5, size=batch)
    rows = rng.integers(0, rrows, size=batch)
    stray = rng.random(batch) < 0.1
    rows[stray] = rng.choice([-1, rrows, rrows + 7], size=int(stray.sum()))
    topk = rng.integers(-1, cols + 2, size=(layers, batch, k))
    for r in range(batch):
        hi = max(1, min(int(lengths[r]), cols))
        near = rng.random((layers, k)) < 0.7
        topk[:, r][near] = rng.integers(max(0, hi - 4096), hi + 1, size=(layers, k))[near]
    shape = (layers, rrows, cols) if layered else (rrows, cols)
    local_table = rng.integers(1, 1 << 15, size=shape)
    local_table[rng.random(shape) < 0.5] = 0
    local_table[rng.random(shape) < 0.02] = -int(rng.integers(1, 1 << 15))
    slot_base = rng.integers(1, 1 << 20, size=rrows)
    req_axis = 1 if layered else 0
    bases = np.expand_dims(slot_base, tuple(a for a in range(len(shape)) if a != req_axis))
    table = np.where(local_table > 0, bases + local_table - 1, 0)
    selected = rng.permutation(batch)[: int(rng.integers(1, batch + 1))]
    if rng.random() < 0.2:
        selected = np.concatenate([selected, [-1, batch]])
    initial = np.full((layers, batch, k), -77, np.int32)
    want, want_misses, want_counts = coracle.resolve_resident(topk, table, None, rows, lengths, selected, 1,
                                                              initial, with_misses=True)
    table_d = torch.tensor(local_table, dtype=torch.int16, device=gpu)
    bits = build_residency_bits(table_d)
    base_d = torch.tensor(slot_base, device=gpu)
    topk_aligned = torch.tensor(topk, dtype=torch.int32, device=gpu)
    topk_shifted = torch.zeros(topk.size + 1, dtype=torch.int32, device=gpu)[1:].view(topk.shape)
    topk_shifted.copy_(topk_aligned)
    assert topk_aligned.data_ptr() % 16 == 0 and topk_shifted.data_ptr() % 16 == 4
    for topk_d in (topk_aligned, topk_shifted):
        output = torch.tensor(initial, device=gpu)
        misses = torch.full((layers, batch, k), -5, dtype=torch.int32, device=gpu) if compact else None
        counts = torch.full((layers, batch), -5, dtype=torch.int32, device=gpu) if compact else None
        resolve_resident(topk_d, table_d, None, torch.tensor(rows, device=gpu),
                         torch.tensor(lengths, dtype=torch.int32, device=gpu), torch.tensor(selected, device=gpu),
                         output, 1, misses=misses, miss_count=counts, resident_bits=bits, slot_base=base_d)
        case = (seed, layers, batch, k, cols, layered, topk_d.data_ptr() % 16)
        assert np.array_equal(output.cpu().numpy(), want), case
        if compact:
            got_counts, got_misses = counts.cpu().numpy(), misses.cpu().numpy()
            for layer in range(layers):
                for row in range(batch):
                    if row in selected:
                        c = want_counts[layer, row]
                        assert got_counts[layer, row] == c, case
                        assert np.array_equal(got_misses[layer, row, :c], want_misses[layer, row, :c]), case
                    else:
                        assert got_counts[layer, row] == -5, case


@pytest.mark.parametrize("seed", range(6))
def test_local_slot_prefetch_many_items_per_workgroup(gpu, coracle, seed):
    # Rows of one 2048-lane chunk over bitmap rows of whole 16-byte pieces take
    # the prefetching kernel (int16 local-slot and int32 global-slot tables),
    # whose persistent grid gives each workgroup
    # several (row, layer) items once there are more items than resident
    # workgroups (about 2048 on MI355X): here 3,000-8,000 items, with stray
    # request rows, stray selections, short lengths and negative entries.
    rng = np.random.default_rng(9400 + seed)
    layers = int(rng.integers(20, 41))
    batch = int(rng.integers(150, 201))
    k = 8 * int(rng.integers(1, 257))
    rrows = int(rng.integers(batch // 2, batch + 1))
    cols = int(rng.integers(1, 8193)) if seed % 2 else 128 * int(rng.integers(1, 65))   # odd seeds: any T
    layered = seed != 5
    compact = seed != 4
    lengths = rng.integers(-2, cols + 5, size=batch)
    rows = rng.integers(0, rrows, size=batch)
    stray = rng.random(batch) < 0.05
    rows[stray] = rng.choice([-1, rrows, rrows + 7], size=int(stray.sum()))
    topk = rng.integers(-1, cols + 2, size=(layers, batch, k))
    shape = (layers, rrows, cols) if layered else (rrows, cols)
    local_table = rng.integers(1, 1 << 15, size=shape)
    local_table[rng.random(shape) < 0.5] = 0
    local_table[rng.random(shape) < 0.02] = -int(rng.integers(1, 1 << 15))
    slot_base = rng.integers(-(1 << 20), 1 << 31, size=rrows)
    req_axis = 1 if layered else 0
    bases = np.expand_dims(slot_base, tuple(a for a in range(len(shape)) if a != req_axis))
    # Bases up to 2^31: the oracle's int32 cast of base + local - 1 must equal the kernel's 32-bit sum.
    table = np.where(local_table > 0, bases + local_table - 1, 0)
    selected = rng.permutation(batch)[: int(rng.integers(batch - 10, batch + 1))]
    if seed % 2:
        selected = np.concatenate([selected, [-1, batch]])
    initial = np.full((layers, batch, k), -77, np.int32)
    want, want_misses, want_counts = coracle.resolve_resident(topk, table, None, rows, lengths, selected, 1,
                                                              initial, with_misses=True)
    table_d = torch.tensor(local_table, dtype=torch.int16, device=gpu)
    bits = build_residency_bits(table_d)
    assert bits.stride(-2) % 4 == 0 and bits.data_ptr() % 16 == 0
    output = torch.tensor(initial, device=gpu)
    misses = torch.full((layers, batch, k), -5, dtype=torch.int32, device=gpu) if compact else None
    counts = torch.full((layers, batch), -5, dtype=torch.int32, device=gpu) if compact else None
    resolve_resident(torch.tensor(topk, dtype=torch.int32, device=gpu), table_d, None, torch.tensor(rows, device=gpu),
                     torch.tensor(lengths, dtype=torch.int32, device=gpu), torch.tensor(selected, device=gpu),
                     output, 1, misses=misses, miss_count=counts, resident_bits=bits,
                     slot_base=torch.tensor(slot_base, device=gpu))
    chosen = np.zeros(batch, bool)
    chosen[selected[(selected >= 0) & (selected < batch)]] = True
    lanes = np.arange(k)
    valid = lanes[None, None, :] < want_counts[:, :, None]

    def check(output, misses, counts, case):
        assert np.array_equal(output.cpu().numpy(), want), case
        if compact:
            got_counts, got_misses = counts.cpu().numpy(), misses.cpu().numpy()
            assert np.array_equal(got_counts[:, chosen], want_counts[:, chosen]), case
            assert (got_counts[:, ~chosen] == -5).all(), case
            assert np.array_equal(np.where(valid, got_misses, 0)[:, chosen],
                                  np.where(valid, want_misses, 0)[:, chosen]), case

    check(output, misses, counts, (seed, layers, batch, k, cols, layered, "int16"))
    # The same residency as an int32 table of global slots (the int32 cast of
    # base + local - 1, which is what the oracle compares against).
    wrapped = (table + (1 << 31)) % (1 << 32) - (1 << 31)
    table32 = torch.tensor(wrapped, dtype=torch.int32, device=gpu)
    output = torch.tensor(initial, device=gpu)
    misses = torch.full((layers, batch, k), -5, dtype=torch.int32, device=gpu) if compact else None
    counts = torch.full((layers, batch), -5, dtype=torch.int32, device=gpu) if compact else None
    resolve_resident(torch.tensor(topk, dtype=torch.int32, device=gpu), table32, None, torch.tensor(rows, device=gpu),
                     torch.tensor(lengths, dtype=torch.int32, device=gpu), torch.tensor(selected, device=gpu),
                     output, 1, misses=misses, miss_count=counts, resident_bits=build_residency_bits(table32))
    check(output, misses, counts, (seed, layers, batch, k, cols, layered, "int32"))


@pytest.mark.parametrize("seed", range(40))
def test_summary_lookup_random_configurations(gpu, coracle, seed):
    # Single-level lookups behind residency summaries of random coarseness
    # (shift 0-9): summaries of at most 64 words per row take the one-wave-per-
    # item kernel (its rows are walked in passes of 512 lanes, here 1-10 of
    # them, the last one partial), wider ones the prefetching or strided
    # kernels. int16 local-slot and int32 global-slot tables; exact summaries
    # and supersets with stray bits past the length and past the table; stray
    # rows and selections, lengths past the table, negative entries.
    rng = np.random.default_rng(9700 + seed)
    layers = int(rng.integers(1, 5))
    batch = int(rng.integers(1, 13))
    k = 8 * int(rng.integers(1, 600))
    rrows = int(rng.integers(1, 10))
    cols = int(rng.integers(1, 140_000)) if seed % 3 else int(rng.integers(1, 3000))
    shift = int(rng.integers(0, 10))
    layered = bool(rng.random() < 0.7)
    compact = bool(rng.random() < 0.85)
    local = seed % 2 == 0
    lengths = rng.integers(-2, cols + 5, size=batch)
    rows = rng.integers(0, rrows, size=batch)
    stray = rng.random(batch) < 0.1
    rows[stray] = rng.choice([-1, rrows, rrows + 7], size=int(stray.sum()))
    topk = rng.integers(-1, cols + 2, size=(layers, batch, k))
    for r in range(batch):
        hi = max(1, min(int(lengths[r]), cols))
        near = rng.random((layers, k)) < 0.7
        topk[:, r][near] = rng.integers(max(0, hi - 4096), hi + 1, size=(layers, k))[near]
    shape = (layers, rrows, cols) if layered else (rrows, cols)
    local_table = rng.integers(1, 1 << 15, size=shape)
    local_table[rng.random(shape) < 0.9] = 0
    local_table[rng.random(shape) < 0.01] = -int(rng.integers(1, 1 << 15))
    slot_base = rng.integers(1, 1 << 20, size=rrows)
    req_axis = 1 if layered else 0
    bases = np.expand_dims(slot_base, tuple(a for a in range(len(shape)) if a != req_axis))
    table = np.where(local_table > 0, bases + local_table - 1, 0)
    selected = rng.permutation(batch)[: int(rng.integers(1, batch + 1))]
    if rng.random() < 0.2:
        selected = np.concatenate([selected, [-1, batch]])
    initial = np.full((layers, batch, k), -77, np.int32)
    want, want_misses, want_counts = coracle.resolve_resident(topk, table, None, rows, lengths, selected, 1,
                                                              initial, with_misses=True)
    if local:
        table_d, base_d = torch.tensor(local_table, dtype=torch.int16, device=gpu), torch.tensor(slot_base, device=gpu)
    else:
        table_d, base_d = torch.tensor(table, dtype=torch.int32, device=gpu), None
    bits = build_residency_bits(table_d, shift=shift)
    if seed % 4 >= 2:
        extra = (rng.random(bits.shape) < 0.3) * rng.integers(0, 1 << 31, bits.shape)
        bits |= torch.tensor(extra, dtype=torch.int32, device=gpu)
    output = torch.tensor(initial, device=gpu)
    misses = torch.full((layers, batch, k), -5, dtype=torch.int32, device=gpu) if compact else None
    counts = torch.full((layers, batch), -5, dtype=torch.int32, device=gpu) if compact else None
    resolve_resident(torch.tensor(topk, dtype=torch.int32, device=gpu), table_d, None, torch.tensor(rows, device=gpu),
                     torch.tensor(lengths, dtype=torch.int32, device=gpu), torch.tensor(selected, device=gpu),
                     output, 1, misses=misses, miss_count=counts, resident_bits=bits, bits_shift=shift,
                     slot_base=base_d)
    case = (seed, layers, batch, k, cols, shift, layered, local)
    assert np.array_equal(output.cpu().numpy(), want), case
    if compact:
        got_counts, got_misses = counts.cpu().numpy(), misses.cpu().numpy()
        for layer in range(layers):
            for row in range(batch):
                if row in selected:
                    c = want_counts[layer, row]
                    assert got_counts[layer, row] == c, case
                    assert np.array_equal(got_misses[layer, row, :c], want_misses[layer, row, :c]), case
                else:
                    assert got_counts[layer, row] == -5, case


def random_planes(rng, gpu, layers, kv, rows, row_bytes):
    row_stride = row_bytes + int(rng.choice([0, 0, 2, 8, 16, 48]))
    plane = rows * row_stride + int(rng.choice([0, 16, 64, 100]))
    layer_gap = int(rng.choice([0, 32, 4096]))
    total = layers * (kv * plane + layer_gap) + 64
    offset = int(rng.choice([0, 0, 2, 4, 8, 16]))                 # base alignment below 16 bytes
    host = rng.integers(0, 256, total + offset, dtype=np.uint8)
    device = torch.tensor(host, device=gpu)
    planes = KVPlanes(base=device.data_ptr() + offset, device=gpu.index or 0, layers=layers, kv=kv,
                      layer_stride=kv * plane + layer_gap, kv_stride=plane, row_stride=row_stride,
                      row_bytes=row_bytes, rows=rows, owner=device)
    return device, host[offset:], planes


ROW_BYTES = (2, 6, 8, 24, 64, 128, 512, 1000, 2048, 4096, 40960)


@pytest.mark.parametrize("seed", range(60))
def test_gather_and_scatter_random_configurations(gpu, coracle, seed):
    rng = np.random.default_rng(8000 + seed)
    layers, kv = int(rng.integers(1, 4)), int(rng.choice([1, 2]))
    row_bytes = int(rng.choice(ROW_BYTES))
    rows = int(rng.integers(1, 200 if row_bytes < 4096 else 12))
    batch = int(rng.integers(1, 5))
    k = int(rng.integers(1, 300 if row_bytes < 4096 else 6))
    zero_below = int(rng.choice([0, 1, 3]))
    device, host, planes = random_planes(rng, gpu, layers, kv, rows, row_bytes)
    slots = rng.integers(-2, rows + 3, size=(layers, batch, k))
    slot_dtype = INDEX_DTYPES[int(rng.integers(2))]
    spare = int(rng.choice([0, 0, 3]))
    big = torch.full((batch, layers, kv, k + spare, row_bytes), 0xAB, dtype=torch.uint8, device=gpu)
    out = big[:, :, :, spare:]
    gather_kv(planes, torch.tensor(slots, dtype=slot_dtype, device=gpu), out, zero_below=zero_below)
    want = coracle.gather_kv(host, planes.layer_stride, planes.kv_stride, planes.row_stride, row_bytes, rows,
                             slots, kv, zero_below=zero_below)
    assert np.array_equal(out.cpu().numpy(), want), (seed, layers, kv, rows, row_bytes, batch, k, zero_below)

    # Scatter distinct in-range slots back from new rows; every other byte stays.
    valid = np.arange(zero_below, rows)
    if valid.size:
        count = min(valid.size, batch * k)
        distinct = rng.permutation(valid)[:count]
        targets = np.full(batch * k, -1, dtype=np.int64)
        targets[rng.permutation(batch * k)[:count]] = distinct
        targets = np.broadcast_to(targets.reshape(1, batch, k), (layers, batch, k)).copy()
        source = rng.integers(0, 256, size=(batch, layers, kv, k, row_bytes), dtype=np.uint8)
        scatter_kv(planes, torch.tensor(targets, device=gpu), torch.tensor(source, device=gpu),
                   zero_below=zero_below)
        want_pool = coracle.scatter_kv(host, planes.layer_stride, planes.kv_stride, planes.row_stride, row_bytes,
                                       rows, targets, kv, source, zero_below=zero_below)
        offset = planes.base - device.data_ptr()
        assert np.array_equal(device.cpu().numpy()[offset:], want_pool), seed


@pytest.mark.parametrize("seed", range(30))
def test_move_random_configurations(gpu, seed):
    rng = np.random.default_rng(9000 + seed)
    layers, kv = int(rng.integers(1, 4)), int(rng.choice([1, 2]))
    row_bytes = int(rng.choice(ROW_BYTES[:9]))
    src_rows_n, dst_rows_n = int(rng.integers(1, 150)), int(rng.integers(1, 150))
    batch, k = int(rng.integers(1, 5)), int(rng.integers(1, 40))
    zero_below = int(rng.choice([0, 1]))
    src_dev, src_host, src_planes = random_planes(rng, gpu, layers, kv, src_rows_n, row_bytes)
    dst_dev, dst_host, dst_planes = random_planes(rng, gpu, layers, kv, dst_rows_n, row_bytes)
    src_rows = rng.integers(-2, src_rows_n + 2, size=(layers, batch, k))
    # Destinations are distinct within a layer (two moves into one row would race).
    dst_rows = np.full((layers, batch, k), -1, dtype=np.int64)
    for layer in range(layers):
        picks = rng.permutation(np.arange(-1, dst_rows_n + 2))[: batch * k]
        dst_rows[layer].flat[: picks.size] = picks
    counts = rng.integers(-1, k + 2, size=(layers, batch))
    dst_before = dst_dev.cpu().numpy().copy()
    t = lambda a: torch.tensor(a, dtype=torch.int32, device=gpu)  # noqa: E731
    move_kv(src_planes, t(src_rows), dst_planes, t(dst_rows), t(counts), zero_below=zero_below)
    offset = dst_planes.base - dst_dev.data_ptr()
    layout = lambda p, n: (p.layer_stride, p.kv_stride, p.row_stride, row_bytes, n)  # noqa: E731
    want = ref.move_kv(src_host, layout(src_planes, src_rows_n), dst_before[offset:], layout(dst_planes, dst_rows_n),
                       src_rows, dst_rows, counts, kv, zero_below=zero_below)
    assert np.array_equal(dst_dev.cpu().numpy()[offset:], want), seed
    assert np.array_equal(dst_dev.cpu().numpy()[:offset], dst_before[:offset])


@pytest.mark.parametrize("seed", range(20))
def test_swap_in_random_configurations(gpu, seed):
    from adaptive_sparse.swap_in import HotBuffers, swap_in

    rng = np.random.default_rng(9500 + seed)
    L, R = int(rng.integers(1, 3)), int(rng.integers(1, 5))
    bs = int(rng.choice([1, 1, 2, 3]))
    K = int(rng.integers(2, 24))
    W = K * bs
    T = int(rng.integers(max(W, 2 * K) * 2, 600))
    C = int(rng.integers(W, W + 40))
    lengths = np.maximum(rng.integers(T // 2, T + 3, size=R), 1)
    buffers = HotBuffers(L, R, T, C, gpu)
    host_table = rng.permutation(R * T).astype(np.int32).reshape(R, T)
    state = {"table": buffers.table.cpu().numpy(), "slot_token": buffers.slot_token.cpu().numpy(),
             "stamps": buffers.stamps.cpu().numpy()}
    rows = torch.arange(R, device=gpu)
    selected = rng.permutation(R)[: int(rng.integers(1, R + 1))]
    blocks_total = T // bs
    for step in range(4):
        topk = np.stack([rng.permutation(blocks_total)[:K] for _ in range(L * R)]).reshape(L, R, K)
        topk[rng.random(topk.shape) < 0.1] = -1
        topk_d = torch.tensor(topk, dtype=torch.int32, device=gpu)
        slots = torch.full((L, R, W), -3, dtype=torch.int32, device=gpu)
        misses = torch.full((L, R, W), -1, dtype=torch.int32, device=gpu)
        counts = torch.zeros((L, R), dtype=torch.int32, device=gpu)
        resolve_resident(topk_d, buffers.table, None, rows, torch.tensor(lengths, dtype=torch.int32, device=gpu),
                         torch.tensor(selected, device=gpu), slots, bs, misses=misses, miss_count=counts,
                         resident_bits=buffers.bits)
        want_slots, want_misses, want_counts = ref.resolve_resident(
            topk, state["table"], None, np.arange(R), lengths, selected, bs, np.full((L, R, W), -3, np.int32),
            with_misses=True)
        want_counts_full = np.zeros((L, R), np.int32)
        miss_np = np.full((L, R, W), -1, np.int32)
        for (layer, r), lanes in want_misses.items():
            miss_np[layer, r, :len(lanes)] = lanes
            want_counts_full[layer, r] = len(lanes)
        assert np.array_equal(slots.cpu().numpy(), want_slots), (seed, step)
        promote_src = torch.full((L, R, W), -9, dtype=torch.int32, device=gpu)
        promote_dst = torch.full((L, R, W), -9, dtype=torch.int32, device=gpu)
        swap_in(topk_d, bs, rows, torch.tensor(selected, device=gpu), slots, misses, counts, buffers,
                torch.tensor(host_table, device=gpu), promote_src, promote_dst)
        state = ref.swap_in(step, bs, topk, np.arange(R), selected, want_slots, miss_np, want_counts_full,
                            state["table"], state["slot_token"], state["stamps"], buffers.slot_base.cpu().numpy(),
                            host_table)
        assert np.array_equal(slots.cpu().numpy(), state["slots"]), (seed, step)
        assert np.array_equal(buffers.table.cpu().numpy(), state["table"]), (seed, step)
        assert np.array_equal(buffers.slot_token.cpu().numpy(), state["slot_token"]), (seed, step)
        assert np.array_equal(buffers.stamps.cpu().numpy(), state["stamps"]), (seed, step)
        assert bits_match(buffers.bits.cpu().numpy(), ref.residency_bits(state["table"])), (seed, step)
        got_src, got_dst = promote_src.cpu().numpy(), promote_dst.cpu().numpy()
        for layer in range(L):
            for r in selected:
                c = want_counts_full[layer, r]
                assert np.array_equal(got_src[layer, r, :c], state["promote_src"][layer, r, :c]), (seed, step)
                assert np.array_equal(got_dst[layer, r, :c], state["promote_dst"][layer, r, :c]), (seed, step)


@pytest.mark.parametrize("seed", range(30))
def test_gather_rows_random_configurations(gpu, coracle, seed):
    """experimental/sparse_read.py's gather_rows on seeded layouts: row widths of 1-300 bf16 elements, direct and
    indirect addressing, positions, requests, table entries and element offsets in and out of range (odd offsets
    take the unaligned path), against the C oracle bit for bit."""
    from types import SimpleNamespace

    from experimental.sparse_read import gather_rows

    rng = np.random.default_rng(9000 + seed)
    width = int(rng.choice([1, 2, 3, 8, 64, 128, 256, 300]))
    batch, selected, requests = int(rng.integers(1, 5)), int(rng.integers(1, 200)), int(rng.integers(1, 5))
    length = int(rng.integers(1, 300))
    request_stride = length * width + int(rng.integers(0, 3))       # elements per request region
    sink = int(rng.integers(0, 64))
    raw_elems = max(1, sink + requests * request_stride + int(rng.integers(-width, 50)))
    raw = rng.integers(0, 1 << 16, raw_elems, dtype=np.uint16)
    positions = rng.integers(-3, length + 3, (batch, selected))
    request_ids = rng.integers(-1, requests + 1, batch)
    lengths = rng.integers(0, length + 1, batch)
    table = rng.integers(-2, requests * length + 3, (requests, length))
    offsets = rng.integers(-5, raw_elems + 5, requests * length + 1)
    indirect = bool(rng.random() < 0.5)
    layout = SimpleNamespace(row_elements=width, request_bytes=2 * request_stride, chunk_bytes=2 * sink, itemsize=2)
    raw_d = torch.tensor(raw.view(np.int16)).view(torch.bfloat16).to(gpu)
    output = torch.full((batch, selected, width), 7.0, dtype=torch.bfloat16, device=gpu)
    gather_rows(raw_d, torch.tensor(positions, device=gpu), torch.tensor(request_ids, device=gpu),
                torch.tensor(lengths, device=gpu), torch.tensor(table, device=gpu), torch.tensor(offsets, device=gpu),
                output, layout, indirect=indirect)
    want = coracle.gather_rows(raw, positions, request_ids, lengths, table, offsets, width, request_stride, sink,
                               indirect)
    assert np.array_equal(output.view(torch.int16).cpu().numpy().view(np.uint16), want)
