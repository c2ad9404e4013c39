"""GPU parity of the HIP resident lookup + miss compaction against the oracle.

Bar: bit-exact output, miss list and miss counts. Inputs are seeded and
identical for both sides; the oracle runs on the same host arrays.
"""

import numpy as np
import pytest
import torch

from adaptive_sparse.resident_lookup import resolve_resident

pytestmark = pytest.mark.gpu


def bits_match(got, want):
    """A bitmap padded to whole 16-byte pieces holds the oracle's ceil(T / 32) words, then zeros."""
    words = want.shape[-1]
    return (got.shape[-1] == -(-words // 4) * 4 and np.array_equal(got[..., :words], want)
            and not got[..., words:].any())


def strided(values, dtype, device):
    """A non-contiguous view holding `values` (tests/smoke_resident_lookup.py:28-33)."""
    source = torch.tensor(values, dtype=dtype, device=device)
    backing = torch.empty((*source.shape, 2), dtype=dtype, device=device)
    view = backing[..., 1]
    view.copy_(source)
    return view


def test_reference_smoke_on_strided_inputs(gpu, coracle):
    topk = [[[1, -1, 2] + [-1] * 13, [0] * 16, [0, 2, -1] + [-1] * 13]]
    rows, lengths, selected = [3, 0, 1], [130, 0, 0], [2, 0]
    table = [[i * 300 + j for j in range(300)] for i in range(4)]
    mapping = [i * 3 + 5 for i in range(1200)]
    output = torch.full((1, 3, 4096), -77, device=gpu, dtype=torch.int32)[..., ::2]
    resolve_resident(strided(topk, torch.int32, gpu), strided(table, torch.long, gpu),
                     strided(mapping, torch.long, gpu), strided(rows, torch.long, gpu),
                     strided(lengths, torch.int32, gpu), strided(selected, torch.long, gpu),
                     output, 128)
    got = output.cpu().numpy()
    assert got[0, 0, :3].tolist() == [3089, 3092, -1]
    assert (got[0, 2] == -1).all() and (got[0, 1] == -77).all()
    want, _, _ = coracle.resolve_resident(topk, table, mapping, rows, lengths, selected, 128,
                                          np.full((1, 3, 2048), -77, np.int32))
    assert np.array_equal(got, want)


@pytest.mark.parametrize("batch", [1, 2, 4])
def test_reference_closed_form(gpu, batch):
    device = gpu
    selected = torch.arange(batch, device=device)
    rows = selected.flip(0)
    lengths = torch.full((batch,), 8192, dtype=torch.int32, device=device)
    table = torch.arange(batch * 8192, device=device).reshape(batch, 8192) + 1
    mapping = torch.arange(batch * 8192 + 1, device=device) * 3 + 5
    topk = (torch.arange(16, device=device) * 4).int().expand(1, batch, 16).contiguous()
    result = torch.empty((1, batch, 2048), device=device, dtype=torch.int32)
    resolve_resident(topk, table, mapping, rows, lengths, selected, result, 128)
    closed = torch.tensor([[((batch - 1 - row) * 8192 + block * 512 + offset + 1) * 3 + 5
                            for block in range(16) for offset in range(128)] for row in range(batch)],
                          dtype=torch.int32).unsqueeze(0)
    assert torch.equal(result.cpu(), closed)


CASES = [
    # layers, batch, k, block_size, table_rows, table_cols, layered, map dtype, topk/table dtypes
    (1, 3, 16, 128, 4, 2100, False, torch.int64, torch.int32, torch.int64),
    (2, 5, 37, 3, 6, 130, True, torch.int32, torch.int64, torch.int32),
    (3, 4, 2053, 1, 4, 4100, True, None, torch.int32, torch.int32),
    (1, 7, 64, 1, 9, 70, False, None, torch.int64, torch.int64),
    (2, 2, 5, 7, 3, 40, False, torch.int64, torch.int32, torch.int32),
    (1, 1, 4096, 2, 2, 9000, False, torch.int32, torch.int32, torch.int64),
]


@pytest.mark.parametrize("case", range(len(CASES)))
@pytest.mark.parametrize("compact", [True, False])
def test_random_parity_with_oracle(gpu, coracle, case, compact):
    layers, batch, k, bs, rrows, cols, layered, map_dtype, topk_dtype, table_dtype = CASES[case]
    rng = np.random.default_rng(1000 + case)
    topk = rng.integers(-1, cols // bs + 2, size=(layers, batch, k))
    rows = rng.integers(0, rrows, size=batch)
    lengths = rng.integers(0, cols + 3, size=batch)
    n = 5000
    table = rng.integers(0, n, size=(layers, rrows, cols) if layered else (rrows, cols))
    mapping = None
    if map_dtype is not None:
        mapping = rng.integers(1, 1 << 20, size=n)
        mapping[rng.random(n) < 0.3] = 0
    else:
        table[rng.random(table.shape) < 0.3] = 0
    selected = rng.permutation(batch)[: max(1, batch - 1)]
    width = k * bs
    initial = np.full((layers, batch, width), -77, np.int32)
    want, want_misses, want_counts = coracle.resolve_resident(topk, table, mapping, rows, lengths, selected,
                                                              bs, initial, with_misses=True)
    t = lambda a, dt: torch.tensor(a, dtype=dt, device=gpu)  # noqa: E731
    output = t(initial, torch.int32)
    misses = torch.full((layers, batch, width), -5, dtype=torch.int32, device=gpu) if compact else None
    counts = torch.full((layers, batch), -5, dtype=torch.int32, device=gpu) if compact else None
    resolve_resident(t(topk, topk_dtype), t(table, table_dtype),
                     None if mapping is None else t(mapping, map_dtype), t(rows, torch.int64),
                     t(lengths, torch.int32), t(selected, torch.int64), output, bs,
                     misses=misses, miss_count=counts)
    assert np.array_equal(output.cpu().numpy(), want)
    if compact:
        got_counts = counts.cpu().numpy()
        got_misses = misses.cpu().numpy()
        for layer in range(layers):
            for row in range(batch):
                if row in selected:
                    c = want_counts[layer, row]
                    assert got_counts[layer, row] == c
                    assert np.array_equal(got_misses[layer, row, :c], want_misses[layer, row, :c])
                    assert (got_misses[layer, row, c:] == -5).all()
                else:
                    assert got_counts[layer, row] == -5


def test_empty_selection_and_zero_width_do_nothing(gpu):
    output = torch.full((1, 2, 8), 9, dtype=torch.int32, device=gpu)
    topk = torch.zeros((1, 2, 4), dtype=torch.int32, device=gpu)
    table = torch.ones((2, 8), dtype=torch.int64, device=gpu)
    rows = torch.arange(2, device=gpu)
    lengths = torch.full((2,), 8, dtype=torch.int32, device=gpu)
    resolve_resident(topk, table, None, rows, lengths, torch.empty(0, dtype=torch.long, device=gpu), output, 2)
    resolve_resident(topk[:, :, :0], table, None, rows, lengths, rows, output[:, :, :0], 2)
    torch.cuda.synchronize()
    assert (output == 9).all()


def test_shape_errors_raise(gpu):
    topk = torch.zeros((1, 2, 4), dtype=torch.int32, device=gpu)
    table = torch.ones((2, 8), dtype=torch.int64, device=gpu)
    rows = torch.arange(2, device=gpu)
    lengths = torch.full((2,), 8, dtype=torch.int32, device=gpu)
    with pytest.raises(RuntimeError, match="output"):
        resolve_resident(topk, table, None, rows, lengths, rows,
                         torch.zeros((1, 2, 7), dtype=torch.int32, device=gpu), 2)
    with pytest.raises(RuntimeError, match="int32"):
        resolve_resident(topk, table, None, rows, lengths, rows,
                         torch.zeros((1, 2, 8), dtype=torch.int64, device=gpu), 2)


@pytest.mark.parametrize("dtype", [torch.int16, torch.int32, torch.int64])
def test_residency_summary_matches_oracle_on_every_layout(gpu, dtype):
    # Rows in whole 16-byte pieces take the vectorized kernel; ragged, strided
    # and misaligned tables the general one. Both must write the oracle's
    # words over whatever the output held and leave the padding words past
    # them as they were.
    from adaptive_sparse.resident_lookup import build_residency_bits, summary_words
    from oracle import oracle as ref

    rng = np.random.default_rng(300 + dtype.itemsize)
    per_piece = 16 // dtype.itemsize
    for case in range(48):
        shift = int(rng.choice([0, 1, 2, 3, 4, 5, 6, 7, 9, 12, 20]))
        layered = bool(rng.random() < 0.5)
        layers, rows = int(rng.integers(1, 4)), int(rng.integers(1, 5))
        cols = per_piece * int(rng.integers(1, 900)) if rng.random() < 0.7 else int(rng.integers(1, 5000))
        shape = (layers, rows, cols) if layered else (rows, cols)
        table = rng.integers(-5, 100, size=shape)
        table[rng.random(shape) < rng.random()] = 0
        form = int(rng.integers(0, 4))   # 0, 1: contiguous; 2: strided entries; 3: one entry off the alignment
        if form == 2:
            view = strided(table, dtype, gpu)
        elif form == 3:
            backing = torch.zeros((*shape[:-1], cols + 1), dtype=dtype, device=gpu)
            view = backing[..., 1:]
            view.copy_(torch.tensor(table, dtype=dtype, device=gpu))
        else:
            view = torch.tensor(table, dtype=dtype, device=gpu)
        before = rng.integers(-(1 << 31), 1 << 31, size=(*shape[:-1], summary_words(cols, shift))).astype(np.int32)
        out = torch.tensor(before, device=gpu)
        build_residency_bits(view, out=out, shift=shift)
        want = ref.residency_bits(table, shift)
        got = out.cpu().numpy()
        words = want.shape[-1]
        assert np.array_equal(got[..., :words], want), (case, shape, shift, form)
        assert np.array_equal(got[..., words:], before[..., words:]), (case, shape, shift, form)


@pytest.mark.parametrize("layered", [False, True])
@pytest.mark.parametrize("bs", [1, 3])
def test_bitmap_lookup_equals_plain_lookup_and_oracle(gpu, coracle, layered, bs):
    from adaptive_sparse.resident_lookup import build_residency_bits
    from oracle import oracle as ref

    rng = np.random.default_rng(77 + bs + 10 * layered)
    layers, batch, k, rrows, cols = 2, 5, 300, 6, 1000
    topk = rng.integers(-1, cols // bs + 2, size=(layers, batch, k))
    rows = rng.integers(0, rrows, size=batch)
    lengths = rng.integers(0, cols + 3, size=batch)
    table = rng.integers(1, 1 << 20, size=(layers, rrows, cols) if layered else (rrows, cols))
    table[rng.random(table.shape) < 0.6] = 0
    selected = np.arange(batch)
    t = lambda a, dt: torch.tensor(a, dtype=dt, device=gpu)  # noqa: E731
    table_d = t(table, torch.int32)
    bits = build_residency_bits(table_d)
    assert bits_match(bits.cpu().numpy(), ref.residency_bits(table))
    width = k * bs
    outs = []
    for use_bits in (False, True):
        out = torch.full((layers, batch, width), -7, dtype=torch.int32, device=gpu)
        misses = torch.full_like(out, -5)
        counts = torch.zeros((layers, batch), dtype=torch.int32, device=gpu)
        resolve_resident(t(topk, torch.int32), table_d, None, t(rows, torch.int64), t(lengths, torch.int32),
                         t(selected, torch.int64), out, bs, misses=misses, miss_count=counts,
                         resident_bits=bits if use_bits else None)
        outs.append((out.cpu().numpy(), misses.cpu().numpy(), counts.cpu().numpy()))
    assert np.array_equal(outs[0][0], outs[1][0])
    assert np.array_equal(outs[0][2], outs[1][2])
    want, want_misses, want_counts = coracle.resolve_resident(topk, table, None, rows, lengths, selected, bs,
                                                              np.full((layers, batch, width), -7, np.int32),
                                                              with_misses=True)
    assert np.array_equal(outs[1][0], want)
    assert np.array_equal(outs[1][2], want_counts)
    for layer in range(layers):
        for row in range(batch):
            c = want_counts[layer, row]
            assert np.array_equal(outs[1][1][layer, row, :c], want_misses[layer, row, :c])


# Rows wide enough (>= 1024 lanes) that the kernels stage the table entries of
# the recent window (the last 4096 positions before the row's length) in LDS.
WINDOW_CASES = [
    # layers, batch, k, block_size, table_rows, table_cols, layered, two-level, table dtype, table layout, bitmap
    (2, 4, 1536, 1, 5, 10000, True, False, torch.int32, "dense", True),
    (1, 3, 512, 4, 4, 9001, False, False, torch.int32, "offset", True),
    (2, 3, 1200, 1, 3, 6000, False, False, torch.int64, "dense", False),
    (1, 4, 1024, 1, 4, 7000, True, False, torch.int32, "strided", True),
    (1, 2, 2048, 1, 2, 140000, False, False, torch.int32, "dense", True),
    (2, 3, 1500, 1, 4, 5000, False, True, torch.int32, "dense", False),
    (1, 3, 2048, 1, 3, 3000, False, False, torch.int32, "offset", False),
]


def laid_out(values, dtype, layout, device):
    """`values` as a dense tensor, a view whose rows start 4 bytes off 16-byte
    alignment, or a view with element stride 2 along the last dimension."""
    source = torch.tensor(values, dtype=dtype, device=device)
    if layout == "dense":
        return source
    if layout == "offset":
        backing = torch.zeros((*source.shape[:-1], source.shape[-1] + 1), dtype=dtype, device=device)
        view = backing[..., 1:]
    else:
        backing = torch.zeros((*source.shape, 2), dtype=dtype, device=device)
        view = backing[..., 0]
    view.copy_(source)
    return view


@pytest.mark.parametrize("case", range(len(WINDOW_CASES)))
def test_recent_window_parity_with_oracle(gpu, coracle, case):
    from adaptive_sparse.resident_lookup import build_residency_bits

    layers, batch, k, bs, rrows, cols, layered, mapped, table_dtype, layout, use_bits = WINDOW_CASES[case]
    rng = np.random.default_rng(500 + case)
    choices = [cols, cols + 5, cols - 77, 4000, 0, 130, -3, cols - 4096 - 1]
    lengths = np.array([choices[rng.integers(len(choices))] for _ in range(batch)])
    lengths[0] = cols - 1
    rows = rng.integers(0, rrows, size=batch)
    topk = rng.integers(-1, cols // bs + 2, size=(layers, batch, k))
    for r in range(batch):
        hi = max(1, min(lengths[r], cols) // bs)
        recent = rng.integers(max(0, hi - 4300 // bs), hi + 1, size=(layers, k))
        near = rng.random((layers, k)) < 0.8
        topk[:, r][near] = recent[near]
    shape = (layers, rrows, cols) if layered else (rrows, cols)
    n = 6000
    mapping = None
    if mapped:
        table = rng.integers(-2, n + 2, size=shape)
        mapping = rng.integers(1, 1 << 20, size=n)
        mapping[rng.random(n) < 0.3] = 0
    else:
        table = rng.integers(1, 1 << 20, size=shape)
        table[rng.random(shape) < 0.4] = 0
    selected = rng.permutation(batch)
    width = k * bs
    initial = np.full((layers, batch, width), -77, np.int32)
    want, want_misses, want_counts = coracle.resolve_resident(topk, table, mapping, rows, lengths, selected,
                                                              bs, initial, with_misses=True)
    t = lambda a, dt: torch.tensor(a, dtype=dt, device=gpu)  # noqa: E731
    table_d = laid_out(table, table_dtype, layout, gpu)
    bits = None
    if use_bits:
        bits = build_residency_bits(table_d.to(torch.int32).contiguous())
        if layout == "strided":
            spread = torch.zeros((*bits.shape, 2), dtype=torch.int32, device=gpu)
            spread[..., 1].copy_(bits)
            bits = spread[..., 1]
    output = t(initial, torch.int32)
    misses = torch.full((layers, batch, width), -5, dtype=torch.int32, device=gpu)
    counts = torch.full((layers, batch), -5, dtype=torch.int32, device=gpu)
    resolve_resident(t(topk, torch.int32), table_d, None if mapping is None else t(mapping, torch.int32),
                     t(rows, torch.int64), t(lengths, torch.int32), t(selected, torch.int64), output, bs,
                     misses=misses, miss_count=counts, resident_bits=bits)
    assert np.array_equal(output.cpu().numpy(), want)
    assert np.array_equal(counts.cpu().numpy(), want_counts)
    got_misses = misses.cpu().numpy()
    for layer in range(layers):
        for row in range(batch):
            c = want_counts[layer, row]
            assert np.array_equal(got_misses[layer, row, :c], want_misses[layer, row, :c])
            assert (got_misses[layer, row, c:] == -5).all()


def test_launch_goes_to_the_current_stream(gpu):
    """The lookup is issued on torch's current stream: a side stream's work is ordered before the host reads it."""
    from elastic_kv import _native

    batch, context = 4, 8192
    selected = torch.arange(batch, device=gpu)
    rows = selected.flip(0)
    lengths = torch.full((batch,), context, dtype=torch.int32, device=gpu)
    table = torch.arange(batch * context, device=gpu).reshape(batch, context) + 1
    mapping = torch.arange(batch * context + 1, device=gpu) * 3 + 5
    topk = (torch.arange(16, device=gpu) * 4).int().expand(1, batch, 16).contiguous()
    want = ((rows.view(batch, 1, 1) * context + topk[0].long().view(batch, 16, 1) * 128
             + torch.arange(128, device=gpu) + 1) * 3 + 5).view(1, batch, 2048).int()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        assert _native.stream_handle(gpu).value == side.cuda_stream
        out = torch.full((1, batch, 2048), -7, dtype=torch.int32, device=gpu)
        for _ in range(20):
            resolve_resident(topk, table, mapping, rows, lengths, selected, out, 128)
        side.synchronize()
    # torch's default stream is the null stream: handle 0, which ctypes reads back as None.
    assert (_native.stream_handle(gpu).value or 0) == torch.cuda.current_stream(gpu).cuda_stream
    assert torch.equal(out, want)
