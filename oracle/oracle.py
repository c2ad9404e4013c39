"""CPU oracle of the sparse-KV residency hot path.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
CPU-baseline leg of bench.py, to verify the HIP kernels' results. Product code
never imports it.

Two independent restatements of the reference semantics live here:
  * numpy functions (vectorized, following the torch indexing sequence of
    adaptive_sparse/request_residency.py:819-825 and the Triton gather of
    experimental/sparse_read.py:11-30), and
  * COracle, a ctypes binding of ekv_oracle.c (scalar C, following the
    Triton lookup adaptive_sparse/resident_lookup.py:14-26 lane by lane),
plus restatements of the reference's hit semantics
(adaptive_sparse/hisparse_access_trace.py:59-71), its batch-token LRU replay
(benchmarks/hisparse_locality_replay.py:90-99), and the swap-in in SGLang's
calling convention that its decode path and swap smoke test use
(tests/smoke_minimax_swap.py:18-67). tests/test_oracle.py pins all of them
against the reference's known-answer vectors, closed forms, its smoke
scenarios and brute-force loops.

Parity unpinned: which free hot slot hisparse_swap gives a particular miss.
The reference's swap smoke test accepts any free slot and the engine kernel
that chooses it is not part of the reference; hisparse_swap takes batch-token
LRU order, empty slots first, and its hits, miss counts, LRU order and bytes
are pinned as above.
"""

import ctypes as ct
import subprocess
from collections import OrderedDict
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
LIBRARY = ORACLE_DIR / "libekv_oracle.so"


def build(force=True):
    """Compile ekv_oracle.c into libekv_oracle.so with the oracle Makefile."""
    command = ["make", "-s", "-C", str(ORACLE_DIR)] + (["-B"] if force else [])
    subprocess.run(command, check=True)
    return LIBRARY


# ---------------------------------------------------------------- lookup (numpy)

def resolve_resident(topk, table, mapping, rows, lengths, selected, block_size, output,
                     with_misses=False):
    """Return (output, misses, counts) after the lookup; inputs are not modified.

    topk [L, B, K]; table [R, T] or [L, R, T]; mapping None, [N] or [L, N];
    output [L, B, K * bs] int32 initial contents (unselected rows survive).
    misses is a list over (l, row) of int32 lane arrays (None if not asked).
    """
    topk = np.asarray(topk, dtype=np.int64)
    table = np.asarray(table, dtype=np.int64)
    rows = np.asarray(rows, dtype=np.int64)
    lengths = np.asarray(lengths, dtype=np.int64)
    selected = np.asarray(selected, dtype=np.int64)
    out = np.array(output, dtype=np.int32, copy=True)
    L, B, K = topk.shape
    width = K * block_size
    misses = {} if with_misses else None
    counts = np.zeros((L, B), dtype=np.int32) if with_misses else None
    sel = selected[(selected >= 0) & (selected < B)]
    for layer in range(L):
        layer_table = table[layer] if table.ndim == 3 else table
        R, T = layer_table.shape
        blocks = topk[layer, sel]                                            # [S, K]
        positions = (blocks[:, :, None] * block_size + np.arange(block_size)).reshape(len(sel), width)
        valid = (positions >= 0) & (positions < lengths[sel, None])
        req = rows[sel]
        req_ok = (req >= 0) & (req < R)
        in_bounds = valid & req_ok[:, None] & (positions < T)
        logical = layer_table[np.where(req_ok, req, 0)[:, None], np.where(in_bounds, positions, 0)]
        if mapping is None:
            physical = logical
        else:
            layer_map = np.asarray(mapping, dtype=np.int64)
            layer_map = layer_map[layer] if layer_map.ndim == 2 else layer_map
            in_bounds &= (logical >= 0) & (logical < layer_map.shape[0])
            physical = layer_map[np.where(in_bounds, logical, 0)]
        result = np.where(in_bounds, physical, -1).astype(np.int32)
        out[layer, sel] = result
        if with_misses:
            for i, row in enumerate(sel):
                lanes = np.nonzero(in_bounds[i] & (result[i] == 0))[0].astype(np.int32)
                misses[(layer, int(row))] = lanes
                counts[layer, row] = lanes.size
    return out, misses, counts


def residency_bits(table, shift=0):
    """int32 words of a residency summary: bit j of word w of a row = any(table[.., ((32w + j) << shift) + i] != 0
    for i < 2**shift); shift 0 is the per-position bitmap (bit p = table[.., p] != 0)."""
    table = np.asarray(table)
    resident = table != 0
    group = 1 << shift
    groups = -(-table.shape[-1] // group)
    pad = groups * group - table.shape[-1]
    resident = np.concatenate([resident, np.zeros((*table.shape[:-1], pad), bool)], axis=-1)
    resident = resident.reshape(*table.shape[:-1], groups, group).any(-1)
    words = -(-groups // 32)
    resident = np.concatenate([resident, np.zeros((*table.shape[:-1], words * 32 - groups), bool)], axis=-1)
    weights = (np.uint64(1) << np.arange(32, dtype=np.uint64))
    packed = (resident.reshape(*table.shape[:-1], words, 32).astype(np.uint64) * weights).sum(-1)
    return packed.astype(np.uint32).view(np.int32)


def access_tokens(blocks, block_size, seq_len, hot_capacity, prestate):
    """Selected tokens and sorted hit tokens of one HiSparse swap-in.

    Restates adaptive_sparse/hisparse_access_trace.py:59-71: every token of a
    non-negative block below seq_len is selected; when seq_len fits the hot
    capacity everything hits, otherwise hits are selected tokens that were
    resident before the swap or are the newest token seq_len - 1.
    """
    selected = []
    for block in blocks:
        if block < 0:
            continue
        stop = min((block + 1) * block_size, seq_len)
        selected.extend(range(block * block_size, stop))
    if seq_len <= hot_capacity:
        return selected, sorted(set(selected))
    resident = set(prestate) | {seq_len - 1}
    return selected, sorted(resident & set(selected))


def lru_misses(steps, capacity):
    """Misses per step of the batch-token LRU of one (request, layer) stream.

    Restates benchmarks/hisparse_locality_replay.py:90-99: misses are counted
    on entry, hits are touched (moved to most recent) before eviction, least
    recent entries are evicted until the misses fit, then misses are inserted
    in selection order.
    """
    cache = OrderedDict()
    result = []
    for selected in steps:
        missing = [token for token in selected if token not in cache]
        for token in selected:
            if token in cache:
                cache.move_to_end(token)
        while len(cache) + len(missing) > capacity:
            cache.popitem(last=False)
        for token in missing:
            cache[token] = None
        result.append(len(missing))
    return result


SWAP_STEP_STAMPS = 8192   # recency stamps per LRU step: 2 x the 4096 lanes a row may have


def swap_in(step, block_size, topk, rows, selected, slots, misses, counts, table, slot_token, stamps, slot_base,
            host_table):
    """Batch-token LRU swap-in after a lookup, on numpy arrays (copies are returned).

    Per selected row b (request r = rows[b]) of every layer: hits touch their
    slot (stamp = step*8192 + the lowest lane that hit it); with u distinct
    missed tokens, the victims are the slots of the u smallest (stamp, slot)
    keys - empty slots (-2^31) first - and the first miss entry of the i-th
    distinct token (in miss-list order) takes the i-th victim in slot order;
    a victim's old token leaves the table, the new token enters it, its stamp
    becomes step*8192 + 4096 + lane, and promotion i records
    (host_table[r, token], global slot). A later miss entry of the same token
    gets that slot and an empty promotion (-1, -1), as does an entry naming
    no valid lane. This is benchmarks/hisparse_locality_replay.py:90-99
    applied to the selection with repeated tokens reduced to their first
    lane. A step spans 8192 stamps whatever the row width W (at most 4096),
    so the stamps of a call with a smaller W than the call before still
    rank above the earlier ones. Selected rows that share a request with
    another selected row, and every row when (step + 1) * 8192 reaches 2^31,
    change nothing and record
    empty promotions; "status" returns the error bits (1 = stamp overflow,
    2 = shared request). Returns a dict of the new arrays.
    """
    topk = np.asarray(topk, dtype=np.int64)
    L, B, K = topk.shape
    W = K * block_size
    slots = np.array(slots, dtype=np.int32, copy=True)
    table = np.array(table, dtype=np.int32, copy=True)
    slot_token = np.array(slot_token, dtype=np.int32, copy=True)
    stamps = np.array(stamps, dtype=np.int64, copy=True)
    R, T = table.shape[1], table.shape[2]
    C = slot_token.shape[2]
    src = np.full((L, B, W), -1, dtype=np.int32)
    dst = np.full((L, B, W), -1, dtype=np.int32)
    live = [int(b) for b in selected if 0 <= int(b) < B and 0 <= int(rows[int(b)]) < R]
    named = [int(rows[b]) for b in live]
    status = 0
    overflow = step < 0 or (step + 1) * SWAP_STEP_STAMPS >= 1 << 31
    for layer in range(L):
        for b in live:
            r = int(rows[b])
            if named.count(r) > 1 or overflow:
                status |= 2 if named.count(r) > 1 else 1
                continue
            base = int(slot_base[r])
            stamp = stamps[layer, r]
            first_hit = {}
            for lane in range(W):
                slot = int(slots[layer, b, lane])
                if slot > 0 and 0 <= slot - base < C:
                    first_hit.setdefault(slot - base, lane)
            for local, lane in first_hit.items():
                stamp[local] = step * SWAP_STEP_STAMPS + lane
            order = sorted(range(C), key=lambda v: (stamp[v], v))
            m = max(0, min(int(counts[layer, b]), W))
            # The victims are the slots of the u smallest keys (u = distinct valid missed tokens), handed
            # out in slot order.
            distinct = set()
            for i in range(m):
                lane = int(misses[layer, b, i])
                if 0 <= lane < W:
                    token = int(topk[layer, b, lane // block_size]) * block_size + lane % block_size
                    if 0 <= token < T:
                        distinct.add(token)
            victims = sorted(order[:len(distinct)])
            taken = {}
            for i in range(m):
                lane = int(misses[layer, b, i])
                if not 0 <= lane < W:
                    continue
                token = int(topk[layer, b, lane // block_size]) * block_size + lane % block_size
                if not 0 <= token < T:
                    continue
                if token in taken:
                    slots[layer, b, lane] = base + taken[token]
                    continue
                victim = victims[len(taken)]
                taken[token] = victim
                old = int(slot_token[layer, r, victim])
                if old >= 0:
                    table[layer, r, old] = 0
                table[layer, r, token] = base + victim
                slot_token[layer, r, victim] = token
                stamp[victim] = step * SWAP_STEP_STAMPS + SWAP_STEP_STAMPS // 2 + lane
                src[layer, b, i] = host_table[r, token]
                dst[layer, b, i] = base + victim
                slots[layer, b, lane] = base + victim
    return {"slots": slots, "table": table, "slot_token": slot_token, "stamps": stamps.astype(np.int32),
            "promote_src": src, "promote_dst": dst, "status": status}


def hisparse_swap(top_k_blocks, tokens, host_locs, dev_locs, host_k, host_v, dev_k, dev_v, req, seq, lru, hot,
                  block_size, num_real=None):
    """HiSparse swap-in with SGLang's calling convention, token by token (copies are returned).

    The swap the reference's decode path makes through
    load_blocks_to_device_buffer_mha (adaptive_sparse/request_residency.py
    :805-809; checked in tests/smoke_minimax_swap.py:18-67). Per real batch
    row b with request r and length s > 0:
    - selected tokens: every non-negative Top-K block expanded, tokens below
      s and below T = host_locs width, in Top-K order
      (adaptive_sparse/hisparse_access_trace.py:59-64);
    - the newest token s - 1 takes the reserved slot `hot`;
    - another token is a hit when a hot slot holds it (the lowest such slot);
    - the other tokens are misses, taken once each in order of first
      appearance; those whose host row lies outside host_k are dropped;
    - batch-token LRU (benchmarks/hisparse_locality_replay.py:90-99): the
      misses take the empty slots, then the untouched occupied slots, in
      lru order; the new order is the unused empty slots, the untouched
      survivors, the hit slots in order of first hit, the misses' slots;
    - each miss's K and V rows are copied from its host row to its slot's
      device row; device rows outside dev_k are reported as -1, never written.
    Returns (out [B, K*bs] int32, tokens, lru, dev_k, dev_v).
    """
    top_k_blocks = np.asarray(top_k_blocks, dtype=np.int64)
    tokens = np.array(tokens, dtype=np.int64, copy=True)
    lru = np.array(lru, dtype=np.int64, copy=True)
    dev_k = np.array(dev_k, copy=True)
    dev_v = np.array(dev_v, copy=True)
    host_locs = np.asarray(host_locs, dtype=np.int64)
    dev_locs = np.asarray(dev_locs, dtype=np.int64)
    B, K = top_k_blocks.shape
    W = K * block_size
    R, T = host_locs.shape
    out = np.full((B, W), -1, dtype=np.int32)
    real = B if num_real is None else int(num_real)
    for b in range(B):
        r, s = int(req[b]), int(seq[b])
        if b >= real or not 0 <= r < R or s <= 0:
            continue

        def location(slot):
            row = int(dev_locs[r, slot])
            return row if 0 <= row < dev_k.shape[0] else -1

        selected = [int(block) * block_size + j for block in top_k_blocks[b] if block >= 0
                    for j in range(block_size) if int(block) * block_size + j < min(s, T)]
        resident = {}
        for slot in range(hot):
            if tokens[r, slot] >= 0:
                resident.setdefault(int(tokens[r, slot]), slot)
        hit_slots, missed, dropped, seen = [], [], set(), set()
        for token in selected:
            if token == s - 1 or token in seen:
                continue
            seen.add(token)
            if token in resident:
                hit_slots.append(resident[token])
            elif 0 <= host_locs[r, token] < host_k.shape[0]:
                missed.append(token)
            else:
                dropped.add(token)
        slot_of = {}
        if hit_slots or missed:
            touched = set(hit_slots)
            listed = [int(x) for x in lru[r] if 0 <= x < hot]
            empty = [x for x in listed if x not in touched and tokens[r, x] < 0]
            untouched = [x for x in listed if x not in touched and tokens[r, x] >= 0]
            taken_empty = min(len(missed), len(empty))
            taken_untouched = min(len(missed) - taken_empty, len(untouched))
            victims = empty[:taken_empty] + untouched[:taken_untouched]
            order = empty[taken_empty:] + untouched[taken_untouched:] + hit_slots + victims
            for position, slot in enumerate(order[:hot]):
                lru[r, position] = slot
            for token, slot in zip(missed, victims):
                tokens[r, slot] = token
                slot_of[token] = slot
                row = location(slot)
                if row >= 0:
                    dev_k[row] = host_k[host_locs[r, token]]
                    dev_v[row] = host_v[host_locs[r, token]]
        position = 0
        for token in selected:
            if token in dropped:
                continue
            if token == s - 1:
                out[b, position] = location(hot)
            elif token in resident:
                out[b, position] = location(resident[token])
            else:
                out[b, position] = location(slot_of[token]) if token in slot_of else -1
            position += 1
    return out, tokens.astype(np.int32), lru, dev_k, dev_v


# ---------------------------------------------------------------- gathers (numpy)

def gather_rows(raw, positions, request_ids, lengths, request_table, slot_offsets, width,
                request_stride, sink, indirect):
    """Restates experimental/sparse_read.py:18-30 on a 1-D numpy payload."""
    raw = np.asarray(raw)
    positions = np.asarray(positions, dtype=np.int64)
    B, S = positions.shape
    out = np.zeros((B, S, width), dtype=raw.dtype)
    for b in range(B):
        req = int(request_ids[b])
        for s in range(S):
            pos = int(positions[b, s])
            if not 0 <= pos < int(lengths[b]):
                continue
            if indirect:
                table = np.asarray(request_table)
                if not (0 <= req < table.shape[0] and pos < table.shape[1]):
                    continue
                logical = int(table[req, pos])
                if not 0 <= logical < len(slot_offsets):
                    continue
                element = int(slot_offsets[logical])
            else:
                element = sink + req * request_stride + pos * width
            if 0 <= element and element + width <= raw.shape[0]:
                out[b, s] = raw[element:element + width]
    return out


def gather_kv(pool, layer_stride, kv_stride, row_stride, row_bytes, rows, slots, kv, zero_below=1):
    """Dense [B, L, KV, K, row_bytes] uint8 gather from a byte pool.

    pool is a 1-D uint8 array; slots [L, B, K]. Rows with a slot outside
    [zero_below, rows) are zero.
    """
    pool = np.asarray(pool, dtype=np.uint8)
    slots = np.asarray(slots, dtype=np.int64)
    L, B, K = slots.shape
    out = np.zeros((B, L, kv, K, row_bytes), dtype=np.uint8)
    cols = np.arange(row_bytes)
    for layer in range(L):
        for plane in range(kv):
            valid = (slots[layer] >= zero_below) & (slots[layer] < rows)            # [B, K]
            starts = layer * layer_stride + plane * kv_stride + np.where(valid, slots[layer], 0) * row_stride
            values = pool[starts[..., None] + cols]                                  # [B, K, row_bytes]
            out[:, layer, plane] = np.where(valid[..., None], values, 0)
    return out


def shadow_check(blocks, table, lengths, rows, block_size, physical, live_pages, page_size, capacity, written,
                 pool_k, pool_v, shadow_k, shadow_v):
    """One LogicalShadow.check, lane by lane (adaptive_sparse/logical_shadow.py:46-86).

    Arrays are numpy: blocks [1, B, K]; table [R, T]; lengths, rows [B];
    physical [1, B, K * block_size] or None; live_pages [P] bool or None;
    written [capacity] bool; pool_k/pool_v [N, row] and shadow_k/shadow_v
    [capacity, row] uint8 rows. Returns (counts, clean_blocks, physical_out)
    with counts = (checked tokens, checked bytes, uninitialized logical,
    invalid physical, mismatched, calls = 1, malformed blocks).
    """
    blocks = np.asarray(blocks)
    _, B, K = blocks.shape
    W = K * block_size
    N = pool_k.shape[0]
    T = table.shape[1]
    row_bytes = pool_k.shape[1] + pool_v.shape[1]
    clean = np.full_like(blocks, -1)
    out = np.zeros((1, B, W), dtype=np.int64)
    tokens = uninitialized = invalid = mismatched = malformed = 0
    for b in range(B):
        length = int(lengths[b])
        limit = (length + block_size - 1) // block_size
        leading = True
        for k in range(K):
            block = int(blocks[0, b, k])
            valid_block = 0 <= block < limit
            leading = leading and valid_block
            if (block != -1 and not valid_block) or (valid_block and not leading):
                malformed += 1
            clean[0, b, k] = block if leading else -1
            for j in range(block_size):
                o = k * block_size + j
                position = int(clean[0, b, k]) * block_size + j
                selected = 0 <= position < length
                bounded = selected and position < T
                logical = int(table[int(rows[b]), position if bounded else 0])
                logical_ok = bounded and page_size <= logical < capacity
                logical = logical if logical_ok else 0
                source_ok = logical_ok and bool(written[logical])
                phys = logical if physical is None else int(physical[0, b, o])
                in_range = page_size <= phys < N
                safe = phys if in_range else 0
                backed = in_range if live_pages is None else in_range and bool(live_pages[safe // page_size])
                safe = safe if backed else 0
                same = (np.array_equal(pool_k[safe], shadow_k[logical])
                        and np.array_equal(pool_v[safe], shadow_v[logical]))
                checked = selected and source_ok and backed
                tokens += checked
                uninitialized += selected and not source_ok
                invalid += selected and not backed
                mismatched += checked and not same
                out[0, b, o] = 0 if (selected and not backed) else phys
    counts = (tokens, tokens * row_bytes, uninitialized, invalid, mismatched, 1, malformed)
    return counts, clean, out


def move_kv(src, src_layout, dst, dst_layout, src_rows, dst_rows, counts, kv, zero_below=0):
    """Row moves between two byte pools (the promote of a swap-in), returning a new dst.

    layouts are (layer_stride, kv_stride, row_stride, row_bytes, rows). For
    every layer l, row b, i < min(counts[l, b], K) and plane kv: row dst_rows[l, b, i]
    of dst takes row src_rows[l, b, i] of src, when 0 <= src row < rows and
    zero_below <= dst row < rows; other entries move nothing.
    """
    src = np.asarray(src, dtype=np.uint8)
    out = np.array(dst, dtype=np.uint8, copy=True)
    s_ls, s_kvs, s_rs, row_bytes, s_rows = src_layout
    d_ls, d_kvs, d_rs, _, d_rows = dst_layout
    L, B, K = np.shape(src_rows)
    for layer in range(L):
        for b in range(B):
            for i in range(min(K, max(0, int(counts[layer][b])))):
                frm, to = int(src_rows[layer][b][i]), int(dst_rows[layer][b][i])
                if not (0 <= frm < s_rows and zero_below <= to < d_rows):
                    continue
                for plane in range(kv):
                    a = layer * s_ls + plane * s_kvs + frm * s_rs
                    z = layer * d_ls + plane * d_kvs + to * d_rs
                    out[z:z + row_bytes] = src[a:a + row_bytes]
    return out


# ---------------------------------------------------------------- C oracle

_I64P = ct.POINTER(ct.c_int64)
_I32P = ct.POINTER(ct.c_int32)
_U8P = ct.POINTER(ct.c_uint8)


def _i64(array):
    return np.ascontiguousarray(array, dtype=np.int64)


def _ptr(array, kind):
    return array.ctypes.data_as(kind) if array is not None else None


class COracle:
    """ctypes binding of ekv_oracle.c (built by build())."""

    def __init__(self, path=LIBRARY):
        if not Path(path).exists():
            build()
        self.lib = ct.CDLL(str(path))
        self.lib.oracle_resolve_resident.restype = None
        self.lib.oracle_gather_rows.restype = None
        self.lib.oracle_gather_kv.restype = None
        self.lib.oracle_scatter_kv.restype = None

    def resolve_resident(self, topk, table, mapping, rows, lengths, selected, block_size, output,
                         with_misses=False):
        topk, table, rows, lengths, selected = map(_i64, (topk, table, rows, lengths, selected))
        L, B, K = topk.shape
        width = K * block_size
        out = np.array(output, dtype=np.int32, copy=True, order="C")
        misses = np.full((L, B, width), -1, dtype=np.int32) if with_misses else None
        counts = np.zeros((L, B), dtype=np.int32) if with_misses else None
        layered = table.ndim == 3
        R, T = table.shape[-2:]
        map_arr = _i64(mapping) if mapping is not None else None
        N = map_arr.shape[-1] if map_arr is not None else 0
        self.lib.oracle_resolve_resident(
            ct.c_int64(L), ct.c_int64(B), ct.c_int64(K), ct.c_int64(block_size), _ptr(topk, _I64P),
            _ptr(table, _I64P), ct.c_int(int(layered)), ct.c_int64(R), ct.c_int64(T),
            _ptr(map_arr, _I64P), ct.c_int(int(map_arr is not None and map_arr.ndim == 2)), ct.c_int64(N),
            _ptr(rows, _I64P), _ptr(lengths, _I64P), _ptr(selected, _I64P), ct.c_int64(selected.shape[0]),
            _ptr(out, _I32P), _ptr(misses, _I32P), _ptr(counts, _I32P))
        return out, misses, counts

    def gather_rows(self, raw, positions, request_ids, lengths, request_table, slot_offsets, width,
                    request_stride, sink, indirect):
        raw = np.ascontiguousarray(raw)
        positions, request_ids, lengths = map(_i64, (positions, request_ids, lengths))
        B, S = positions.shape
        table = _i64(request_table) if indirect else np.zeros((0, 0), np.int64)
        offsets = _i64(slot_offsets) if indirect else np.zeros(0, np.int64)
        out = np.empty((B, S, width), dtype=raw.dtype)
        self.lib.oracle_gather_rows(
            raw.ctypes.data_as(_U8P), ct.c_int64(raw.shape[0]), ct.c_int64(raw.itemsize),
            _ptr(positions, _I64P), ct.c_int64(B), ct.c_int64(S), _ptr(request_ids, _I64P),
            _ptr(lengths, _I64P), _ptr(table, _I64P), ct.c_int64(table.shape[0]),
            ct.c_int64(table.shape[1]), _ptr(offsets, _I64P), ct.c_int64(offsets.shape[0]),
            ct.c_int(int(bool(indirect))), ct.c_int64(width), ct.c_int64(request_stride), ct.c_int64(sink),
            out.ctypes.data_as(_U8P))
        return out

    def gather_kv(self, pool, layer_stride, kv_stride, row_stride, row_bytes, rows, slots, kv,
                  zero_below=1, shared_layers=None):
        """Dense [B, L, KV, K, row_bytes] gather. shared_layers=L uses one [B, K] slot list."""
        pool = np.ascontiguousarray(pool, dtype=np.uint8)
        slots = _i64(slots)
        if shared_layers is not None:
            B, K = slots.shape
            L, layer_step = shared_layers, 0
        else:
            L, B, K = slots.shape
            layer_step = B * K
        out = np.empty((B, L, kv, K, row_bytes), dtype=np.uint8)
        self.lib.oracle_gather_kv(
            pool.ctypes.data_as(_U8P), ct.c_int64(layer_stride), ct.c_int64(kv_stride), ct.c_int64(row_stride),
            ct.c_int64(row_bytes), ct.c_int64(rows), ct.c_int64(L), ct.c_int64(B), ct.c_int64(kv), ct.c_int64(K),
            _ptr(slots, _I64P), ct.c_int64(layer_step), ct.c_int64(zero_below), out.ctypes.data_as(_U8P))
        return out

    def scatter_kv(self, pool, layer_stride, kv_stride, row_stride, row_bytes, rows, slots, kv, source,
                   zero_below=1):
        """Return a copy of the byte pool after scattering dense [B, L, KV, K, row_bytes] rows."""
        pool = np.array(pool, dtype=np.uint8, copy=True)
        slots = _i64(slots)
        L, B, K = slots.shape
        source = np.ascontiguousarray(source, dtype=np.uint8)
        self.lib.oracle_scatter_kv(
            pool.ctypes.data_as(_U8P), ct.c_int64(layer_stride), ct.c_int64(kv_stride), ct.c_int64(row_stride),
            ct.c_int64(row_bytes), ct.c_int64(rows), ct.c_int64(L), ct.c_int64(B), ct.c_int64(kv), ct.c_int64(K),
            _ptr(slots, _I64P), ct.c_int64(B * K), ct.c_int64(zero_below), source.ctypes.data_as(_U8P))
        return pool
