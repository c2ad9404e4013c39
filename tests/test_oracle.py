"""Pin the CPU oracle before trusting it (CPU only).

Each oracle function is checked against at least one of: a known-answer
vector from the reference's tests, a closed form the reference states, a
brute-force loop written directly from the reference's per-lane definition,
and the other (independent) restatement.
"""

import random

import numpy as np
import pytest

from oracle import oracle as ref

# ------------------------------------------------------------------ helpers


def brute_force_lookup(topk, table, mapping, rows, lengths, selected, block_size, initial):
    """Per-lane loop of adaptive_sparse/resident_lookup.py:14-26 on Python lists."""
    out = [[list(row) for row in layer] for layer in initial]
    for layer in range(len(topk)):
        for row in selected:
            for lane in range(len(topk[layer][row]) * block_size):
                block = topk[layer][row][lane // block_size]
                position = block * block_size + lane % block_size
                if block >= 0 and position < lengths[row]:
                    logical = table[rows[row]][position]
                    out[layer][row][lane] = logical if mapping is None else mapping[logical]
                else:
                    out[layer][row][lane] = -1
    return out


def smoke_inputs():
    """Inputs of the reference's tests/smoke_resident_lookup.py:8-13."""
    topk = [[[1, -1, 2] + [-1] * 13, [0] * 16, [0, 2, -1] + [-1] * 13]]
    rows = [3, 0, 1]
    lengths = [130, 0, 0]
    table = [[i * 300 + j for j in range(300)] for i in range(4)]
    mapping = [i * 3 + 5 for i in range(1200)]
    selected = [2, 0]
    initial = np.full((1, 3, 2048), -77, dtype=np.int32)
    return topk, table, mapping, rows, lengths, selected, initial


def random_lookup_case(rng, layers, batch, k, block_size, table_rows, table_cols, layered, with_map):
    topk = rng.integers(-1, table_cols // block_size + 2, size=(layers, batch, k))
    rows = rng.integers(0, table_rows, size=batch)
    lengths = rng.integers(0, table_cols + 3, size=batch)
    shape = (layers, table_rows, table_cols) if layered else (table_rows, table_cols)
    n = 97
    table = rng.integers(0, n, size=shape)
    mapping = None
    if with_map:
        mapping = rng.integers(-3, 40, size=(n,))
        mapping[rng.random(n) < 0.4] = 0  # not resident
    selected = rng.permutation(batch)[: max(1, batch - 1)]
    initial = np.full((layers, batch, k * block_size), -77, dtype=np.int32)
    return topk, table, mapping, rows, lengths, selected, initial


# ------------------------------------------------------------------ lookup


@pytest.mark.parametrize("which", ["numpy", "c"])
def test_lookup_reference_smoke_vectors(which, coracle):
    topk, table, mapping, rows, lengths, selected, initial = smoke_inputs()
    run = ref.resolve_resident if which == "numpy" else coracle.resolve_resident
    out, _, _ = run(topk, table, mapping, rows, lengths, selected, 128, initial)
    expected = out[0].tolist()
    # Known answers from tests/smoke_resident_lookup.py:21-23.
    assert expected[0][:3] == [3089, 3092, -1]
    assert expected[0][-1] == -1 and expected[2] == [-1] * 2048
    assert expected[1] == [-77] * 2048
    brute = brute_force_lookup(topk, table, mapping, rows, lengths, selected, 128, initial.tolist())
    assert expected == brute[0]


@pytest.mark.parametrize("batch", [1, 2, 4])
@pytest.mark.parametrize("which", ["numpy", "c"])
def test_lookup_reference_closed_form(batch, which, coracle):
    """tests/bench_resident_lookup.py:24-42 inputs against its closed form."""
    selected = np.arange(batch)
    rows = selected[::-1].copy()
    lengths = np.full(batch, 8192)
    table = np.arange(batch * 8192).reshape(batch, 8192) + 1
    mapping = np.arange(batch * 8192 + 1) * 3 + 5
    topk = np.broadcast_to(np.arange(16) * 4, (1, batch, 16))
    run = ref.resolve_resident if which == "numpy" else coracle.resolve_resident
    out, _, _ = run(topk, table, mapping, rows, lengths, selected, 128,
                    np.zeros((1, batch, 2048), np.int32))
    closed = [[((batch - 1 - row) * 8192 + block * 512 + offset + 1) * 3 + 5
               for block in range(16) for offset in range(128)] for row in range(batch)]
    assert out[0].tolist() == closed


@pytest.mark.parametrize("seed", range(6))
def test_lookup_numpy_c_and_brute_force_agree(seed, coracle):
    rng = np.random.default_rng(seed)
    block_size = [1, 2, 3, 4, 8, 1][seed]
    layered = seed % 2 == 0
    with_map = seed % 3 != 2
    case = random_lookup_case(rng, layers=2, batch=5, k=7, block_size=block_size, table_rows=6,
                              table_cols=23, layered=layered, with_map=with_map)
    topk, table, mapping, rows, lengths, selected, initial = case
    a, am, ac = ref.resolve_resident(*case[:6], block_size, initial, with_misses=True)
    b, bm, bc = coracle.resolve_resident(*case[:6], block_size, initial, with_misses=True)
    assert np.array_equal(a, b)
    assert np.array_equal(ac, bc)
    for (layer, row), lanes in am.items():
        assert bm[layer, row, : bc[layer, row]].tolist() == lanes.tolist()
    # brute force needs in-range indices: restrict to rows whose lanes are all in bounds
    safe = [row for row in selected
            if all(0 <= p < table.shape[-1] for p in range(lengths[row]))]
    tables = [table[layer] if layered else table for layer in range(2)]
    for layer in range(2):
        brute = brute_force_lookup([topk[layer]], tables[layer],
                                   None if mapping is None else mapping, rows, lengths, safe,
                                   block_size, [initial[layer]])
        for row in safe:
            assert a[layer, row].tolist() == brute[0][row]


def test_miss_list_is_ordered_nonzero_of_resident_zero():
    """Miss compaction == torch.nonzero(valid & out == 0), row-major, built by hand."""
    topk = [[[0, 1, -1, 2]]]
    table = [[5, 6, 7, 8, 9, 10, 11, 12]]
    mapping = [0] * 5 + [3, 0, 4, 0, 0, 9, 0, 0]
    out, misses, counts = ref.resolve_resident(topk, table, mapping, [0], [5], [0], 2,
                                               np.zeros((1, 1, 8), np.int32), with_misses=True)
    # lanes: blk0 -> pos 0,1 -> logical 5,6 -> 3,0 ; blk1 -> pos 2,3 -> 4,0 ;
    # blk -1 -> -1,-1 ; blk2 -> pos 4 -> logical 9 -> 0, pos 5 >= length -> -1
    assert out[0, 0].tolist() == [3, 0, 4, 0, -1, -1, 0, -1]
    assert misses[(0, 0)].tolist() == [1, 3, 6]
    assert counts[0, 0] == 3


def test_miss_semantics_match_reference_access_trace_kat():
    """tests/test_hisparse_access_trace.py:170-199 through the lookup."""
    # Long path: hot capacity 4, prestate [2, 1, -1, 6], seq_len 7, blocks [1, -1, 3, 1, 4], bs 2.
    selected, hits = ref.access_tokens([1, -1, 3, 1, 4], 2, 7, 4, [2, 1, -1, 6])
    assert selected == [2, 3, 6, 2, 3] and hits == [2, 6]
    resident = {2, 1, 6} | {7 - 1}
    table = [[slot + 1 if pos in resident else 0 for slot, pos in enumerate(range(10))]]
    out, misses, _ = ref.resolve_resident([[[1, -1, 3, 1, 4]]], table, None, [0], [7], [0], 2,
                                          np.zeros((1, 1, 10), np.int32), with_misses=True)
    lanes = out[0, 0]
    positions = [b * 2 + j for b in [1, -1, 3, 1, 4] for j in range(2)]
    valid = [i for i, p in enumerate(positions) if [1, -1, 3, 1, 4][i // 2] >= 0 and p < 7]
    assert [positions[i] for i in valid] == selected
    miss_lanes = set(misses[(0, 0)].tolist())
    assert sorted({positions[i] for i in valid if i not in miss_lanes}) == hits
    assert all(lanes[i] > 0 for i in valid if i not in miss_lanes)
    # Short path: seq_len 4 <= capacity 4, everything resident.
    selected, hits = ref.access_tokens([1, 0, 2], 2, 4, 4, [3, 4, 5, 0])
    assert selected == [2, 3, 0, 1] and hits == [0, 1, 2, 3]
    out, misses, _ = ref.resolve_resident([[[1, 0, 2]]], [[1, 2, 3, 4, 5, 6]], None, [0], [4], [0], 2,
                                          np.zeros((1, 1, 6), np.int32), with_misses=True)
    assert misses[(0, 0)].tolist() == []
    assert out[0, 0].tolist() == [3, 4, 1, 2, -1, -1]


def test_access_tokens_agree_with_lookup_on_random_hot_sets():
    rng = random.Random(11)
    for _ in range(200):
        seq_len = rng.randint(1, 40)
        capacity = rng.randint(1, 12)
        bs = rng.randint(1, 4)
        blocks = [rng.randint(-1, seq_len // bs + 1) for _ in range(rng.randint(1, 6))]
        prestate = rng.sample(range(seq_len), min(capacity, seq_len))
        selected, hits = ref.access_tokens(blocks, bs, seq_len, capacity, prestate)
        if seq_len <= capacity:
            resident = set(range(seq_len))
        else:
            resident = set(prestate) | {seq_len - 1}
        width = 48
        table = [[(p + 1) if p in resident else 0 for p in range(width)]]
        out, misses, _ = ref.resolve_resident([[blocks]], table, None, [0], [seq_len], [0], bs,
                                              np.zeros((1, 1, len(blocks) * bs), np.int32),
                                              with_misses=True)
        lane_pos = [b * bs + j for b in blocks for j in range(bs)]
        valid = [i for i in range(len(lane_pos)) if blocks[i // bs] >= 0 and lane_pos[i] < seq_len]
        assert [lane_pos[i] for i in valid] == selected
        miss = set(misses[(0, 0)].tolist())
        assert sorted({lane_pos[i] for i in valid if i not in miss}) == hits


def test_lru_replay_reference_kat():
    """tests/test_hisparse_locality_replay.py:15-24 (windows of 2 steps)."""
    steps = [[0, 1], [2, 0], [1, 0]]
    cap2 = ref.lru_misses(steps, 2)
    cap3 = ref.lru_misses(steps, 3)
    assert sum(cap2[:2]) == 3 and cap2[2] == 1
    assert cap3[2] == 0


# ------------------------------------------------------------------ gathers


def bf16_bits(values):
    """uint16 bit patterns of small integers as bfloat16 (exact)."""
    return (np.asarray(values, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)


def support_sets(length, selected, seed=137):
    """Support sets of scripts/analyze_virtual_layout.py:11-27 (stdlib random)."""
    rng = random.Random(seed)
    clustered = set()
    run = max(1, selected // 8)
    while len(clustered) < selected:
        begin = rng.randrange(length)
        for step in range(min(run, selected - len(clustered))):
            clustered.add((begin + step) % length)
    return {
        "contiguous": list(range(selected)),
        "uniform_random": rng.sample(range(length), selected),
        "synthetic_clustered": sorted(clustered),
    }


def virtual_addressing_case(batch=3, length=64, width=8, chunk_bytes=256):
    """Payload and tables of scripts/bench_virtual_addressing.py:43-63 in numpy."""
    row_bytes = width * 2
    request_bytes = -(-length * row_bytes // chunk_bytes) * chunk_bytes
    capacity = chunk_bytes + batch * request_bytes
    raw = np.zeros(capacity // 2, dtype=np.uint16)
    for req in range(batch):
        start = (chunk_bytes + req * request_bytes) // 2
        raw[start:start + length * width] = bf16_bits((np.arange(length * width) + req * 17) % 97)
    request_ids = np.arange(batch)[::-1].copy()
    lengths = np.full(batch, length)
    count = batch * length
    table = np.arange(count, 0, -1).reshape(batch, length)
    flat = np.arange(count)
    addresses = chunk_bytes // 2 + (flat // length) * (request_bytes // 2) + (flat % length) * width
    offsets = np.zeros(count + 1, dtype=np.int64)
    offsets[table.flatten()] = addresses
    return raw, request_ids, lengths, table, offsets, request_bytes // 2, chunk_bytes // 2


@pytest.mark.parametrize("indirect", [False, True])
@pytest.mark.parametrize("which", ["numpy", "c"])
def test_gather_rows_reference_closed_form(indirect, which, coracle):
    batch, length, width, selected = 3, 64, 8, 16
    raw, request_ids, lengths, table, offsets, request_stride, sink = virtual_addressing_case(
        batch, length, width)
    run = ref.gather_rows if which == "numpy" else coracle.gather_rows
    for name, support in support_sets(length, selected).items():
        positions = np.broadcast_to(np.array(support), (batch, selected)).copy()
        expected = bf16_bits((np.clip(positions, 0, None)[..., None] * width + np.arange(width)
                              + request_ids[:, None, None] * 17) % 97)
        out = run(raw, positions, request_ids, lengths, table, offsets, width, request_stride, sink, indirect)
        assert np.array_equal(out, expected), name
        for invalid in (-1, length):
            bad = positions.copy()
            bad[:, 0] = invalid
            want = expected.copy()
            want[:, 0] = 0
            out = run(raw, bad, request_ids, lengths, table, offsets, width, request_stride, sink, indirect)
            assert np.array_equal(out, want), (name, invalid)


def test_support_sets_reproduce_reference_geometry():
    """results/virtual-addressing-cpu/geometry.json chunk counts (1 / 16 / 8)."""
    import json

    from conftest import GOLDEN
    from experimental.virtual_layout import VirtualKVLayout

    geometry = json.loads((GOLDEN / "virtual_addressing_geometry.json").read_text())
    layout = VirtualKVLayout(1, geometry["length"], geometry["row_elements"],
                             chunk_bytes=geometry["chunk_bytes"])
    sets = support_sets(geometry["length"], geometry["selected"])
    for case in geometry["cases"]:
        positions = sets[case["pattern"]]
        assert len(set(positions)) == case["unique_tokens"]
        assert len(layout.selected_chunks(0, positions)) == case["fixed_position_chunks"]
    assert len(layout.prefix_chunks(0, geometry["length"])) * geometry["chunk_bytes"] == \
        geometry["full_request_backing_bytes"]


@pytest.mark.parametrize("seed", range(4))
def test_gather_kv_numpy_c_and_closed_form_agree(seed, coracle):
    rng = np.random.default_rng(100 + seed)
    layers, kv, rows, row_bytes = 3, 2, 11, 24
    plane = rows * row_bytes + 8
    pool_bytes = layers * kv * plane
    # Closed-form payload: byte j of row (l, v, s) is (31*l + 7*v + 3*s + j) % 251.
    pool = np.zeros(pool_bytes, dtype=np.uint8)
    for l in range(layers):
        for v in range(kv):
            for s in range(rows):
                start = (l * kv + v) * plane + s * row_bytes
                pool[start:start + row_bytes] = (31 * l + 7 * v + 3 * s + np.arange(row_bytes)) % 251
    slots = rng.integers(-1, rows + 2, size=(layers, 4, 5))
    a = ref.gather_kv(pool, kv * plane, plane, row_bytes, row_bytes, rows, slots, kv)
    b = coracle.gather_kv(pool, kv * plane, plane, row_bytes, row_bytes, rows, slots, kv)
    assert np.array_equal(a, b)
    for bi in range(4):
        for l in range(layers):
            for v in range(kv):
                for k in range(5):
                    s = slots[l, bi, k]
                    want = ((31 * l + 7 * v + 3 * s + np.arange(row_bytes)) % 251 if 1 <= s < rows
                            else np.zeros(row_bytes))
                    assert np.array_equal(a[bi, l, v, k], want)


def test_scatter_inverts_gather(coracle):
    rng = np.random.default_rng(7)
    layers, kv, rows, row_bytes = 2, 2, 40, 16
    plane = rows * row_bytes
    pool = rng.integers(0, 256, size=layers * kv * plane, dtype=np.uint8)
    slots = np.stack([rng.permutation(np.arange(1, rows))[:12].reshape(3, 4) for _ in range(layers)])
    dense = coracle.gather_kv(pool, kv * plane, plane, row_bytes, row_bytes, rows, slots, kv)
    cleared = pool.copy()
    for l in range(layers):
        for v in range(kv):
            for s in slots[l].ravel():
                start = l * kv * plane + v * plane + s * row_bytes
                cleared[start:start + row_bytes] = 0
    restored = coracle.scatter_kv(cleared, kv * plane, plane, row_bytes, row_bytes, rows, slots, kv, dense)
    assert np.array_equal(restored, pool)


def test_residency_bits_little_endian_words():
    table = np.zeros((2, 70), np.int64)
    table[0, [0, 31, 32, 69]] = [5, 6, 7, 8]
    table[1, 33] = -1
    words = ref.residency_bits(table).view(np.uint32)
    assert words.shape == (2, 3)
    assert words[0].tolist() == [1 | (1 << 31), 1, 1 << 5]
    assert words[1].tolist() == [0, 1 << 1, 0]


def test_residency_summary_groups_the_bitmap():
    """A summary at shift s is the OR of each group of 2**s bitmap bits (brute force from the definition)."""
    table = np.zeros((2, 200), np.int64)
    table[0, [0, 63, 64, 199]] = [5, 6, 7, 8]
    table[1, 130] = -1
    words = ref.residency_bits(table, shift=6).view(np.uint32)
    assert words.shape == (2, 1)
    assert words[0].tolist() == [0b1011] and words[1].tolist() == [0b100]
    rng = np.random.default_rng(3)
    for shift in (0, 1, 3, 5, 6, 7):
        t = rng.integers(0, 2, (3, 4, 1000)) * rng.integers(1, 9, (3, 4, 1000))
        got = ref.residency_bits(t, shift).view(np.uint32)
        for layer in range(3):
            for row in range(4):
                for group in range(-(-1000 // (1 << shift))):
                    want = bool(t[layer, row, group << shift:(group + 1) << shift].any())
                    assert bool((got[layer, row, group // 32] >> (group % 32)) & 1) == want


def _lookup_swap_steps(step_tokens, capacity, context, block_size=1, fixed_width=True):
    """Drive lookup + swap-in for one (layer, request) stream; returns per-step promotion counts.

    Checks after every step that the hot buffer holds exactly the tokens of
    an OrderedDict run of the reference policy (hisparse_locality_replay.py
    :90-99) over the selections with repeated tokens reduced to their first
    occurrence, in the same recency order. With fixed_width=False every step
    is a call whose row width is that step's selection size.
    """
    from collections import OrderedDict

    table = np.zeros((1, 1, context), np.int32)
    slot_token = np.full((1, 1, capacity), -1, np.int32)
    stamps = np.full((1, 1, capacity), -(1 << 31), np.int32)
    host_table = np.arange(context)[None] + 1000
    model = OrderedDict()
    promoted_per_step = []
    widest = max(len(t) for t in step_tokens)
    for step, tokens in enumerate(step_tokens):
        K = widest if fixed_width else len(tokens)
        topk = np.full((1, 1, K), -1, np.int64)
        topk[0, 0, :len(tokens)] = tokens
        out, miss_lists, counts = ref.resolve_resident(topk, table[0], None, [0], [context], [0], block_size,
                                                       np.zeros((1, 1, K), np.int32), with_misses=True)
        miss = np.zeros((1, 1, K), np.int32)
        lanes = miss_lists[(0, 0)]
        miss[0, 0, :len(lanes)] = lanes
        state = ref.swap_in(step, block_size, topk, [0], [0], out, miss, counts, table, slot_token, stamps,
                            [1], host_table)
        table, slot_token, stamps = state["table"], state["slot_token"], state["stamps"]
        assert state["status"] == 0
        # every selected token is now resident, in the slot the patched output names
        assert all(state["slots"][0, 0, i] == table[0, 0, t] > 0 for i, t in enumerate(tokens))
        # one promotion per distinct missed token, at its first miss entry
        first_entry = {}
        for i, lane in enumerate(lanes.tolist()):
            first_entry.setdefault(tokens[lane], i)
        want_src = [1000 + tokens[lane] if first_entry[tokens[lane]] == i else -1 for i, lane in enumerate(lanes)]
        assert state["promote_src"][0, 0, :counts[0, 0]].tolist() == want_src
        promoted_per_step.append(len(first_entry))
        # the cache contents and order equal an OrderedDict run of the reference policy
        unique = list(dict.fromkeys(tokens))
        missing = [t for t in unique if t not in model]
        for t in unique:
            if t in model:
                model.move_to_end(t)
        while len(model) + len(missing) > capacity:
            model.popitem(last=False)
        model.update((t, None) for t in missing)
        held = slot_token[0, 0]
        by_recency = sorted((int(stamps[0, 0, v]), int(held[v])) for v in range(capacity) if held[v] >= 0)
        assert [t for _, t in by_recency] == list(model)
        assert set(np.nonzero(table[0, 0])[0].tolist()) == set(model)
    return promoted_per_step


def test_swap_in_reproduces_reference_lru_kat():
    """tests/test_hisparse_locality_replay.py:15-24 through lookup + swap-in."""
    steps = [[0, 1], [2, 0], [1, 0]]
    assert _lookup_swap_steps(steps, capacity=2, context=4) == ref.lru_misses(steps, 2) == [2, 1, 1]
    assert _lookup_swap_steps(steps, capacity=3, context=4) == ref.lru_misses(steps, 3) == [2, 1, 0]


def test_swap_in_matches_lru_replay_on_random_streams():
    rng = random.Random(29)
    for capacity, context, k in ((8, 40, 6), (16, 100, 16), (5, 12, 5)):
        steps = [rng.sample(range(context), rng.randint(1, k)) for _ in range(40)]
        assert _lookup_swap_steps(steps, capacity, context) == ref.lru_misses(steps, capacity)


def test_swap_in_order_survives_a_narrower_call():
    """Step 0 fills 8 slots with 8 lanes; step 1 has 2 lanes: token 10 hits, token 40 misses.

    The miss must evict the least recent token of step 0 (token 0), never the
    slot of the hit it sits beside, whatever the two calls' widths."""
    context, capacity = 64, 8
    table = np.zeros((1, 1, context), np.int32)
    slot_token = np.full((1, 1, capacity), -1, np.int32)
    stamps = np.full((1, 1, capacity), -(1 << 31), np.int32)
    host = np.arange(context)[None] + 1000
    for step, tokens in enumerate(([0, 10, 20, 30, 1, 2, 3, 4], [10, 40])):
        topk = np.array([[tokens]], np.int64)
        out, miss_lists, counts = ref.resolve_resident(topk, table[0], None, [0], [context], [0], 1,
                                                       np.zeros((1, 1, len(tokens)), np.int32), with_misses=True)
        miss = np.zeros((1, 1, len(tokens)), np.int32)
        miss[0, 0, :len(miss_lists[(0, 0)])] = miss_lists[(0, 0)]
        state = ref.swap_in(step, 1, topk, [0], [0], out, miss, counts, table, slot_token, stamps, [1], host)
        table, slot_token, stamps = state["table"], state["slot_token"], state["stamps"]
    assert state["slots"][0, 0].tolist() == [2, 1]          # token 10 keeps slot 2, token 40 takes token 0's slot 1
    assert table[0, 0, 10] == 2 and table[0, 0, 40] == 1 and table[0, 0, 0] == 0
    assert sorted(slot_token[0, 0].tolist()) == sorted([40, 10, 20, 30, 1, 2, 3, 4])


def test_swap_in_matches_lru_replay_when_the_width_changes_every_call():
    rng = random.Random(37)
    for capacity, context, k in ((8, 40, 8), (16, 100, 16), (6, 20, 6)):
        steps = [rng.sample(range(context), rng.randint(1, k)) for _ in range(60)]
        assert len({len(s) for s in steps}) > 2
        assert _lookup_swap_steps(steps, capacity, context, fixed_width=False) == ref.lru_misses(steps, capacity)


def test_swap_in_repeated_tokens_follow_the_deduplicated_replay():
    """Repeats (a Top-K block listed twice) are one access of the first lane."""
    rng = random.Random(31)
    for capacity, context, k in ((8, 30, 8), (12, 50, 12), (4, 9, 4)):
        steps = [rng.choices(range(context), k=rng.randint(1, k)) for _ in range(40)]
        assert any(len(set(s)) < len(s) for s in steps)
        unique = [list(dict.fromkeys(s)) for s in steps]
        assert _lookup_swap_steps(steps, capacity, context) == ref.lru_misses(unique, capacity)


def test_swap_in_access_trace_kat_with_a_repeated_block():
    """tests/test_hisparse_access_trace.py:170-199: blocks [1, -1, 3, 1, 4], bs 2, seq_len 7, hot capacity 4,
    prestate [2, 1, -1, 6] selects [2, 3, 6, 2, 3] and hits [2, 6]; token 3 misses twice and takes one slot."""
    prestate = [2, 1, -1, 6]
    context, bs = 10, 2
    slot_token = np.array([[prestate]], np.int32)
    table = np.zeros((1, 1, context), np.int32)
    stamps = np.full((1, 1, 4), -(1 << 31), np.int32)
    for slot, token in enumerate(prestate):
        if token >= 0:
            table[0, 0, token] = 1 + slot
            stamps[0, 0, slot] = slot - 8
    blocks = np.array([[[1, -1, 3, 1, 4]]])
    out, miss_lists, counts = ref.resolve_resident(blocks, table[0], None, [0], [7], [0], bs,
                                                   np.zeros((1, 1, 10), np.int32), with_misses=True)
    lanes = miss_lists[(0, 0)].tolist()
    assert lanes == [1, 7]              # token 3 at lanes 1 and 7 (block 1 twice)
    miss = np.zeros((1, 1, 10), np.int32)
    miss[0, 0, :2] = lanes
    state = ref.swap_in(0, bs, blocks, [0], [0], out, miss, counts, table, slot_token, stamps, [1],
                        np.arange(context)[None] + 100)
    # the one promotion fills the empty slot 2 (global slot 3) for both lanes
    assert state["promote_src"][0, 0, :2].tolist() == [103, -1]
    assert state["promote_dst"][0, 0, :2].tolist() == [3, -1]
    assert state["slots"][0, 0, 1] == state["slots"][0, 0, 7] == 3
    assert state["slot_token"][0, 0].tolist() == [2, 1, 3, 6]
    hits = sorted({2 * b + j for b in [1, 3] for j in range(bs) if 2 * b + j < 7} - {3})
    assert hits == [2, 6]               # the KAT's prestate hits
    # touch order: token 2 (lane 0) then 6 (lane 4), then the inserted 3; token 1 stays least recent
    order = [int(state["slot_token"][0, 0, v]) for v in np.argsort(state["stamps"][0, 0], kind="stable")]
    assert order == [1, 2, 6, 3]


def test_swap_in_refuses_shared_requests_and_overflowing_steps():
    table = np.zeros((1, 2, 8), np.int32)
    slot_token = np.full((1, 2, 4), -1, np.int32)
    stamps = np.full((1, 2, 4), -(1 << 31), np.int32)
    topk = np.array([[[1, 2], [3, 4], [5, 6]]])
    out = np.zeros((1, 3, 2), np.int32)
    miss = np.array([[[0, 1], [0, 1], [0, 1]]], np.int32)
    counts = np.full((1, 3), 2, np.int32)
    host = np.arange(16).reshape(2, 8)
    # rows 0 and 2 name request 1: both refused; row 1 (request 0) proceeds
    state = ref.swap_in(0, 1, topk, [1, 0, 1], [0, 1, 2], out, miss, counts, table, slot_token, stamps, [1, 5],
                        host)
    assert state["status"] == 2
    assert state["promote_src"][0, 0].tolist() == [-1, -1] and state["promote_src"][0, 2].tolist() == [-1, -1]
    assert state["promote_src"][0, 1].tolist() == [3, 4]
    assert state["table"][0, 1].tolist() == [0] * 8
    state = ref.swap_in((1 << 30) // 2, 1, topk, [1, 0, 1], [1], out, miss, counts, table, slot_token, stamps,
                        [1, 5], host)
    assert state["status"] == 1 and state["promote_src"][0, 1].tolist() == [-1, -1]


def _shadow_case():
    """Two rows over a capacity-8 shadow: row 0 reads logical 2, 3 (written) and 4 (never
    written); row 1 has a leading block, then an out-of-range block (malformed) and a
    valid block after the break (malformed); its table maps to logical 0 and 9, both invalid."""
    rowb = 4
    table = np.array([[0, 1, 2, 3, 4, 5, 6, 7], [0, 9, 7, 7, 1, 0, 3, 3]])
    written = np.array([0, 1, 1, 1, 0, 1, 1, 1], dtype=bool)
    rng = np.random.default_rng(5)
    shadow_k = rng.integers(0, 256, (8, rowb), dtype=np.uint8)
    shadow_v = rng.integers(0, 256, (8, rowb), dtype=np.uint8)
    pool_k, pool_v = shadow_k.copy(), shadow_v.copy()
    return table, written, shadow_k, shadow_v, pool_k, pool_v, rowb


def test_shadow_check_hand_counted_case():
    table, written, shadow_k, shadow_v, pool_k, pool_v, rowb = _shadow_case()
    pool_v[3, 1] ^= 0x40                       # logical 3 differs in its V row
    blocks = np.array([[[1, 2, -1], [0, 5, 1]]])
    counts, clean, out = ref.shadow_check(blocks, table, np.array([5, 6]), np.array([0, 1]), 2, None, None, 1, 8,
                                          written, pool_k, pool_v, shadow_k, shadow_v)
    # checked: logical 2 and 3; uninitialized: logical 4 and row 1's two lanes;
    # invalid physical: row 1's two lanes (physical = logical 0); mismatched: logical 3.
    assert counts == (2, 2 * 2 * rowb, 3, 2, 1, 1, 2)
    assert clean.tolist() == [[[1, 2, -1], [0, -1, -1]]]
    assert out.tolist() == [[[2, 3, 4, 0, 0, 0], [0, 0, 0, 0, 0, 0]]]


def test_shadow_check_with_physical_slots_and_live_pages():
    table, written, shadow_k, shadow_v, pool_k, pool_v, rowb = _shadow_case()
    pool_k[6], pool_v[6] = shadow_k[3], shadow_v[3]   # physical 6 holds logical 3
    physical = np.array([[[5, 6, 7, 8, 2, 3]]])
    live = np.array([1, 1, 1, 1, 1, 0, 1, 1], dtype=bool)
    counts, _, out = ref.shadow_check(np.array([[[1, 2, -1]]]), table[:1], np.array([5]), np.array([0]), 2,
                                      physical, live, 1, 8, written, pool_k, pool_v, shadow_k, shadow_v)
    # lane 0: page 5 not live (invalid, zeroed); lane 1: checked, equal; lane 2: logical 4 never
    # written; lanes 3-5 are not selected and keep their physical slots.
    assert counts == (1, 2 * rowb, 1, 1, 0, 1, 0)
    assert out.tolist() == [[[0, 6, 7, 8, 2, 3]]]


def test_move_kv_hand_case_and_gather_identity():
    rng = np.random.default_rng(9)
    kv, row = 2, 4
    src = rng.integers(1, 256, 2 * kv * 5 * row, dtype=np.uint8)          # 2 layers x 2 planes x 5 rows
    dst = np.zeros(2 * kv * 6 * row, dtype=np.uint8)                      # 2 layers x 2 planes x 6 rows
    src_layout = (kv * 5 * row, 5 * row, row, row, 5)
    dst_layout = (kv * 6 * row, 6 * row, row, row, 6)
    src_rows = [[[1, 4, 7]], [[0, 2, 3]]]
    dst_rows = [[[2, 0, 3]], [[5, 1, 4]]]
    counts = [[3], [2]]                                                   # layer 1 moves only its first two
    out = ref.move_kv(src, src_layout, dst, dst_layout, src_rows, dst_rows, counts, kv, zero_below=1)
    planes = out.reshape(2, kv, 6, row)
    source = src.reshape(2, kv, 5, row)
    # layer 0: 1 -> 2 moves; 4 -> 0 is below zero_below; 7 is past the source rows.
    assert np.array_equal(planes[0, :, 2], source[0, :, 1])
    assert not planes[0, :, [0, 1, 3, 4, 5]].any()
    # layer 1: 0 -> 5 and 2 -> 1 move; the third entry is past the count.
    assert np.array_equal(planes[1, :, 5], source[1, :, 0]) and np.array_equal(planes[1, :, 1], source[1, :, 2])
    assert not planes[1, :, [0, 2, 3, 4]].any()
    # Reading the moved rows back at their destinations gives the source rows.
    moved_src = np.array([[[1]], [[0]]]); moved_dst = np.array([[[2]], [[5]]])
    assert np.array_equal(ref.gather_kv(out, *dst_layout[:4], 6, moved_dst, kv),
                          ref.gather_kv(src, *src_layout[:4], 5, moved_src, kv, zero_below=0))


# ------------------------------------------------------------------ HiSparse swap (SGLang convention)

def bf16_rows(values):
    """bfloat16 bytes of float32 values that bfloat16 holds exactly."""
    bits = np.asarray(values, dtype=np.float32).view(np.uint32) >> 16
    return bits.astype(np.uint16).view(np.uint8).reshape(*np.shape(values)[:-1], -1)


def smoke_swap_scenario(swap, layer):
    """tests/smoke_minimax_swap.py:18-62 for one layer; `swap` runs one call.

    Returns (selected device rows per newest token, host K/V rows, device
    K/V rows after the last call) and asserts the reference's checks.
    """
    block, hot, width = 128, 256, 128
    t = np.arange(3 * block)[:, None] % 43
    d = np.arange(width)[None, :] % 13
    host = [bf16_rows(t + d + layer * 64 + plane * 128) for plane in range(2)]     # [384, 256 B]
    device = [np.zeros((hot + 2, width * 2), np.uint8) for _ in range(2)]
    locs = np.arange(1, hot + 2).reshape(1, -1)
    tokens = np.full((1, hot + 1), -1)
    tokens[0, :block] = np.arange(block, 2 * block)
    for dst, src in zip(device, host):
        dst[1:block + 1] = src[block:2 * block]
    lru = np.arange(hot).reshape(1, -1)
    results = []
    for newest in range(2 * block, 2 * block + 3):
        for dst, src in zip(device, host):
            if newest > 2 * block:
                src[newest - 1] = dst[hot + 1]          # back up the previous newest token
            dst[hot + 1] = src[newest]
        out, tokens, lru, device[0], device[1] = swap(
            np.array([[0, 2]]), tokens, np.arange(3 * block).reshape(1, -1), locs, host[0], host[1],
            device[0], device[1], [0], [newest + 1], lru, hot, block, 1)
        valid = block + newest - 2 * block + 1
        selected = out[0, :valid]
        assert (selected > 0).all()
        assert selected[-1] == hot + 1
        assert (out[0, valid:] == -1).all()
        for dst, src in zip(device, host):
            expected = np.concatenate((src[:block], src[2 * block:newest + 1]))
            assert np.array_equal(dst[selected], expected), (layer, newest)
        results.append(selected.tolist())
    return results


def test_hisparse_swap_reproduces_reference_smoke_scenario():
    """The reference's swap smoke test (valid locations > 0, newest token in the reserved slot,
    -1 tail, every selected device row equal to its host row) holds for the oracle."""
    first = smoke_swap_scenario(ref.hisparse_swap, 0)
    second = smoke_swap_scenario(ref.hisparse_swap, 1)
    assert first == second                               # locations do not depend on the payload
    assert first[0][:3] == [129, 130, 131]               # block 0 fills the empty slots 128.. in order


def _swap_state(rng, hot, context, resident_count):
    tokens = np.full((1, hot + 1), -1)
    resident = rng.choice(context, size=resident_count, replace=False)
    slots = rng.choice(hot, size=resident_count, replace=False)
    tokens[0, slots] = resident
    lru = rng.permutation(hot).reshape(1, -1)
    return tokens, lru


def test_hisparse_swap_hits_follow_reference_access_model():
    """Hits are selected ∩ (prestate ∪ {newest}) (adaptive_sparse/hisparse_access_trace.py:59-71),
    and a short request whose tokens are all resident hits everywhere."""
    rng = np.random.default_rng(41)
    row_bytes = 8
    for case in range(60):
        hot, bs, k = int(rng.integers(4, 40)), int(rng.choice([1, 2, 4])), int(rng.integers(1, 6))
        k = min(k, hot // bs)
        short = case % 4 == 0
        context = int(rng.integers(2, hot + 1)) if short else int(rng.integers(hot + 1, 4 * hot))
        seq = context
        if short:
            tokens = np.full((1, hot + 1), -1)
            tokens[0, :seq - 1] = np.arange(seq - 1)       # every token before the newest is resident
            lru = rng.permutation(hot).reshape(1, -1)
        else:
            tokens, lru = _swap_state(rng, hot, seq, int(rng.integers(0, hot + 1)))
        k = min(k, -(-seq // bs) + 1)
        blocks = rng.choice(-(-seq // bs) + 1, size=k, replace=False) - 1      # distinct, -1 = padding
        locs = rng.permutation(hot + 1).reshape(1, -1) + 3
        host = rng.integers(0, 256, (seq, row_bytes), dtype=np.uint8)
        device = np.zeros((hot + 4, row_bytes), np.uint8)
        out, *_ = ref.hisparse_swap(blocks[None], tokens, np.arange(seq)[None], locs, host, host, device,
                                    device, [0], [seq], lru, hot, bs)
        selected, hits = ref.access_tokens(blocks.tolist(), bs, seq, hot, tokens[0, :hot][tokens[0, :hot] >= 0])
        slot_of = {int(tok): slot for slot, tok in enumerate(tokens[0, :hot]) if tok >= 0}
        got = {tok for tok, loc in zip(selected, out[0])
               if (tok == seq - 1 and loc == locs[0, hot]) or (tok in slot_of and loc == locs[0, slot_of[tok]])}
        assert sorted(got) == hits, case
        assert (out[0, :len(selected)] >= 3).all() and (out[0, len(selected):] == -1).all()


def test_hisparse_swap_lru_matches_reference_replay():
    """Resident tokens in LRU order and miss counts follow benchmarks/hisparse_locality_replay.py:90-99
    step by step (distinct selections, newest token never selected)."""
    rng = np.random.default_rng(43)
    for hot, context, k in ((8, 60, 6), (16, 200, 16), (5, 30, 5), (32, 500, 20)):
        tokens = np.full((1, hot + 1), -1)
        lru = rng.permutation(hot).reshape(1, -1)
        locs = np.arange(hot + 1).reshape(1, -1)
        host = np.zeros((context + 1, 4), np.uint8)
        device = np.zeros((hot + 1, 4), np.uint8)
        cache = ref.OrderedDict()
        for _ in range(30):
            chosen = rng.choice(context, size=int(rng.integers(1, k + 1)), replace=False)
            out, tokens, lru, *_ = ref.hisparse_swap(chosen[None], tokens, np.arange(context + 1)[None], locs,
                                                     host, host, device, device, [0], [context + 1], lru, hot, 1)
            missing = [t for t in chosen.tolist() if t not in cache]
            for t in chosen.tolist():
                if t in cache:
                    cache.move_to_end(t)
            while len(cache) + len(missing) > hot:
                cache.popitem(last=False)
            cache.update((t, None) for t in missing)
            resident = [int(tokens[0, slot]) for slot in lru[0] if tokens[0, slot] >= 0]
            assert resident == list(cache)
            assert sorted(lru[0].tolist()) == list(range(hot))


def test_hisparse_swap_repeated_blocks_padding_and_bounds():
    hot, bs, row = 6, 2, 4
    host = np.arange(20 * row, dtype=np.uint8).reshape(20, row)
    device = np.zeros((8, row), np.uint8)
    tokens = np.full((3, hot + 1), -1)
    tokens[0, 2] = 5                                       # request 0 holds token 5 in slot 2
    lru = np.tile(np.arange(hot), (3, 1))
    locs = np.tile(np.array([1, 2, 3, 4, 5, 6, 7]), (3, 1))
    locs[0, 1] = 99                                        # slot 1's device row lies outside the buffer
    host_locs = np.tile(np.arange(20), (3, 1))
    host_locs[0, 8] = 50                                   # token 8 has no host row
    blocks = np.array([[2, 0, 2, 4], [1, -1, -1, -1], [0, 1, -1, -1]])
    out, tokens2, lru2, dk, _ = ref.hisparse_swap(blocks, tokens, host_locs, locs, host, host, device, device,
                                                  [0, 1, 2], [10, 0, 4], lru, hot, bs, num_real=2)
    # row 0: tokens 4 5 | 0 1 | 4 5 | 8 9; 9 is the newest (reserved row 7); 5 hits slot 2 (row 3);
    # 4, 0, 1 miss into empty slots 0, 1, 3 (rows 1, 99 -> -1, 4); the repeated block reuses them;
    # token 8 is dropped (no host row).
    assert out[0].tolist() == [1, 3, -1, 4, 1, 3, 7, -1]
    assert tokens2[0, :hot].tolist() == [4, 0, 5, 1, -1, -1]
    assert lru2[0].tolist() == [4, 5, 2, 0, 1, 3]
    assert np.array_equal(dk[1], host[4]) and np.array_equal(dk[4], host[1]) and not dk[[2, 3, 5, 6, 7]].any()
    # row 1 has length 0 and row 2 is past num_real: -1 only, state unchanged.
    assert (out[1:] == -1).all()
    assert np.array_equal(tokens2[1:], tokens[1:]) and np.array_equal(lru2[1:], lru[1:])


def test_torch_cpu_path_reproduces_reference_smoke_vectors():
    """tests/smoke_resident_lookup.py:8-23 through the torch restatement of request_residency.py:819-825."""
    import torch

    from oracle import torch_path

    topk = torch.tensor([[1, -1, 2] + [-1] * 13, [0] * 16, [0, 2, -1] + [-1] * 13])
    rows, lengths = torch.tensor([3, 0, 1]), torch.tensor([130, 0, 0])
    table = torch.tensor([[(i * 300 + j) for j in range(300)] for i in range(4)])
    mapping = torch.tensor([i * 3 + 5 for i in range(1200)])
    slots, misses = torch_path.lookup(topk, table, mapping, rows, lengths, torch.tensor([2, 0]), 128)
    assert slots[1, :3].tolist() == [3089, 3092, -1] and slots[1, -1] == -1
    assert slots[0].tolist() == [-1] * 2048
    assert misses.numel() == 0


def test_torch_cpu_path_matches_the_numpy_oracle():
    import torch

    from oracle import torch_path

    rng = np.random.default_rng(17)
    for block_size in (1, 2, 4):
        B, R, T, K, N = 6, 5, 300, 24, 900
        topk = rng.integers(-1, T // block_size + 3, (1, B, K))
        req_to_token = rng.integers(0, N, (R, T))
        mapping = rng.integers(0, 40, N) * (rng.random(N) < 0.6)
        rows, lengths = rng.integers(0, R, B), rng.integers(0, T + 1, B)
        selected = np.array([4, 0, 2])
        want, want_misses, _ = ref.resolve_resident(topk, req_to_token, mapping, rows, lengths, selected,
                                                    block_size, np.zeros((1, B, K * block_size), np.int32),
                                                    with_misses=True)
        got, misses = torch_path.lookup(*(torch.tensor(a) for a in (topk[0], req_to_token, mapping, rows, lengths,
                                                                     selected)), block_size)
        assert np.array_equal(got.numpy(), want[0, selected])
        for i, row in enumerate(selected):
            lanes = misses[misses[:, 0] == i, 1].numpy()
            assert np.array_equal(lanes, want_misses[(0, int(row))])
        planes = torch.tensor(rng.integers(0, 256, (2, 41, 8), dtype=np.uint8))
        flat = got.flatten()
        rows_out = torch_path.gather(planes, flat)
        pool = planes.numpy().reshape(-1)
        expect = ref.gather_kv(pool, 2 * 41 * 8, 41 * 8, 8, 8, 41, flat.numpy().reshape(1, 1, -1), 2)
        assert np.array_equal(rows_out.numpy().reshape(-1), expect.reshape(-1))
