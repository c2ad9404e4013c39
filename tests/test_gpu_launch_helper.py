"""The compiled launch helper describes tensors exactly as the ctypes path does.

resolve_resident and gather_rows call their entry points through the launch
helper (csrc/py_launch.cpp). Here the same inputs also go through the ctypes
descriptors (elastic_kv._native.packed / describe) straight to the entry
point: every output must be identical, on torch's current stream, and the
argument errors must name the argument as the ctypes path does.
"""

import ctypes as ct
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from adaptive_sparse.resident_lookup import build_residency_bits, resolve_resident
from elastic_kv import _native
from experimental.sparse_read import gather_rows
from oracle import oracle as ref

pytestmark = pytest.mark.gpu


def _ctypes_resolve(form, topk, table, mapping, slot_base, bits, shift, rows, lengths, selected, out, misses,
                    counts, block_size):
    lib = _native.kernel_library()
    pack = lambda t, name: _native.packed(t, name) if t is not None else None  # noqa: E731
    stream = _native.stream_handle(topk.device)
    head = [pack(topk, "topk"), pack(table, "table")]
    tail = [pack(rows, "rows"), pack(lengths, "lengths"), pack(selected, "selected"), pack(out, "output"),
            pack(misses, "misses"), pack(counts, "miss_count"), block_size, stream]
    if form == 2:
        status = lib.ekv_resolve_resident_local(*head, pack(slot_base, "slot_base"), pack(bits, "bits"), shift,
                                                *tail)
    elif form == 1:
        status = lib.ekv_resolve_resident_bits(*head, pack(bits, "bits"), shift, *tail)
    else:
        status = lib.ekv_resolve_resident(*head, pack(mapping, "mapping"), *tail)
    _native.check(lib, status, "resolve_resident (ctypes)")


@pytest.mark.parametrize("form", [0, 1, 2])
def test_lookup_through_the_helper_equals_the_ctypes_descriptors(gpu, form):
    rng = np.random.default_rng(70 + form)
    L, B, R, T, K, C = 3, 5, 6, 700, 40, 64
    topk = torch.tensor(rng.integers(-2, T, (L, B, K)), dtype=torch.int32, device=gpu)
    rows = torch.tensor(rng.permutation(R)[:B], device=gpu)
    lengths = torch.tensor(rng.integers(0, T + 50, B), dtype=torch.int32, device=gpu)
    selected = torch.tensor([4, 0, 2, 7, 1], device=gpu)            # 7 is a stray entry
    slot_base = torch.arange(R, device=gpu) * C + 1
    local = np.zeros((L, R, T), np.int16)
    for l in range(L):
        for r in range(R):
            picked = rng.choice(T, C // 2, replace=False)
            local[l, r, picked] = rng.choice(C, C // 2, replace=False) + 1
    mapping = None
    if form == 2:
        table = torch.tensor(local, device=gpu)
    else:
        table = torch.tensor(np.where(local > 0, slot_base.cpu().numpy()[None, :, None] + local - 1, 0),
                             dtype=torch.int32, device=gpu)
    if form == 0:
        mapping = torch.tensor(rng.integers(0, 1 << 20, 1 + R * C), dtype=torch.int64, device=gpu)
        table = (table % (1 + R * C)).to(torch.int64)
    bits = build_residency_bits(table, shift=0) if form else None
    outs = []
    for route in ("helper", "ctypes"):
        out = torch.full((L, B, K), -9, dtype=torch.int32, device=gpu)
        misses = torch.full((L, B, K), -9, dtype=torch.int32, device=gpu)
        counts = torch.full((L, B), -9, dtype=torch.int32, device=gpu)
        if route == "helper":
            resolve_resident(topk, table, mapping, rows, lengths, selected, out, 1, misses=misses, miss_count=counts,
                             resident_bits=bits, bits_shift=0, slot_base=slot_base if form == 2 else None)
        else:
            _ctypes_resolve(form, topk, table, mapping, slot_base if form == 2 else None, bits, 0, rows, lengths,
                            selected, out, misses, counts, 1)
        torch.cuda.synchronize()
        outs.append((out.cpu(), misses.cpu(), counts.cpu()))
    for got, want in zip(*outs):
        assert torch.equal(got, want)
    if form == 0:   # and both equal the oracle's two-level lookup
        want, _, _ = ref.resolve_resident(topk.cpu().numpy(), table.cpu().numpy(), mapping.cpu().numpy(),
                                          rows.cpu().numpy(), lengths.cpu().numpy(), selected.cpu().numpy(), 1,
                                          np.full((L, B, K), -9, np.int32), with_misses=True)
        assert np.array_equal(outs[0][0].numpy(), want)


@pytest.mark.parametrize("indirect", [False, True])
def test_row_gather_through_the_helper_equals_the_ctypes_descriptors(gpu, indirect):
    rng = np.random.default_rng(81)
    width, batch, selected, requests, length, sink = 64, 3, 50, 4, 256, 32
    stride = length * width
    layout = SimpleNamespace(row_elements=width, request_bytes=2 * stride, chunk_bytes=2 * sink, itemsize=2)
    raw = torch.empty(sink + requests * stride, dtype=torch.bfloat16, device=gpu).normal_()
    positions = torch.tensor(rng.integers(-3, length + 3, (batch, selected)), dtype=torch.int32, device=gpu)
    request_ids = torch.tensor([2, 0, 3], device=gpu)
    lengths = torch.tensor([256, 100, 7], dtype=torch.int32, device=gpu)
    table = torch.tensor(rng.integers(-1, requests * length, (requests, length)), device=gpu)
    offsets = torch.tensor(rng.integers(0, raw.numel() - width, requests * length), device=gpu)
    outs = []
    for route in ("helper", "ctypes"):
        out = torch.full((batch, selected, width), 7.0, dtype=torch.bfloat16, device=gpu)
        if route == "helper":
            gather_rows(raw, positions, request_ids, lengths, table, offsets, out, layout, indirect=indirect)
        else:
            lib = _native.kernel_library()
            views = [_native.describe(t) for t in (raw, positions, request_ids, lengths, table, offsets, out)]
            refs = [ct.byref(v) for v in views]
            status = lib.ekv_gather_rows(refs[0], refs[1], refs[2], refs[3], refs[4] if indirect else None,
                                         refs[5] if indirect else None, refs[6], stride, sink, int(indirect),
                                         _native.stream_handle(raw.device))
            _native.check(lib, status, "gather_rows (ctypes)")
        torch.cuda.synchronize()
        outs.append(out.view(torch.int16).cpu())
    assert torch.equal(outs[0], outs[1])
    assert not torch.equal(outs[0], torch.full_like(outs[0], 7.0, dtype=torch.bfloat16).view(torch.int16))


def test_the_helper_launches_on_torchs_current_stream(gpu):
    # On a side stream, a long fill runs before the table is written and the lookup reads it. A lookup
    # launched on any other stream would run ahead of the fill and read the zeroed table (slot -1 or 0).
    L, B, T, K = 1, 2, 64, 8
    side = torch.cuda.Stream(gpu)
    topk = torch.arange(K, dtype=torch.int32, device=gpu).repeat(L, B, 1).contiguous()
    rows = torch.arange(B, device=gpu)
    lengths = torch.full((B,), T, dtype=torch.int32, device=gpu)
    mapping = torch.arange(1000, dtype=torch.int64, device=gpu) * 3
    table = torch.zeros((B, T), dtype=torch.int64, device=gpu)
    out = torch.full((L, B, K), -9, dtype=torch.int32, device=gpu)
    filler = torch.empty(1 << 28, dtype=torch.int32, device=gpu)
    torch.cuda.synchronize()
    with torch.cuda.stream(side):
        for _ in range(4):
            filler.fill_(1)
        table.copy_(torch.arange(B * T, device=gpu).view(B, T) + 1)
        resolve_resident(topk, table, mapping, rows, lengths, rows, out, 1)
    side.synchronize()
    want = (torch.arange(B, device=gpu).view(B, 1) * T + torch.arange(K, device=gpu).view(1, K) + 1) * 3
    assert torch.equal(out[0].long(), want)


def test_argument_errors_name_the_argument(gpu):
    i32 = lambda *shape: torch.zeros(shape, dtype=torch.int32, device=gpu)  # noqa: E731
    rows = torch.arange(2, device=gpu)
    with pytest.raises(TypeError, match="rows has unsupported dtype"):
        resolve_resident(i32(1, 2, 4), i32(2, 8), None, rows.double(), i32(2), rows, i32(1, 2, 4), 1)
    with pytest.raises(ValueError, match="topk has more than 4 dimensions"):
        resolve_resident(i32(1, 1, 1, 2, 4), i32(2, 8), None, rows, i32(2), rows, i32(1, 2, 4), 1)
    with pytest.raises(ValueError, match="share one device"):
        resolve_resident(i32(1, 2, 4), i32(2, 8), None, rows.cpu(), i32(2), rows, i32(1, 2, 4), 1)
    with pytest.raises(RuntimeError, match="resolve_resident"):   # the entry point's own shape check
        resolve_resident(i32(1, 2, 4), i32(2, 8), None, rows, i32(2), rows, i32(1, 2, 5), 1)


def test_hisparse_argument_errors_match_the_python_checks(gpu):
    from adaptive_sparse.hisparse_swap import load_blocks_to_device_buffer_mha

    H, W, ROWS, WIDTH = 8, 4, 16, 64
    dev_k = torch.zeros((ROWS, WIDTH), dtype=torch.bfloat16, device=gpu)
    host_k = torch.zeros((ROWS, WIDTH), dtype=torch.bfloat16).pin_memory()
    args = dict(top_k_blocks=torch.zeros((1, W), dtype=torch.int32, device=gpu),
                device_buffer_tokens=torch.full((1, H + 1), -1, dtype=torch.int32, device=gpu),
                host_cache_locs=torch.zeros((1, ROWS), dtype=torch.int64, device=gpu),
                device_buffer_locs=torch.arange(1, H + 2, device=gpu).view(1, -1),
                host_cache_k=host_k, host_cache_v=torch.zeros_like(host_k).pin_memory(),
                device_buffer_k=dev_k, device_buffer_v=torch.zeros_like(dev_k),
                top_k_device_locs=torch.full((1, W), -7, dtype=torch.int32, device=gpu),
                req_pool_indices=torch.zeros(1, dtype=torch.int64, device=gpu),
                seq_lens=torch.ones(1, dtype=torch.int32, device=gpu),
                lru_slots=torch.arange(H, dtype=torch.int16, device=gpu).view(1, -1),
                item_size_bytes=WIDTH * 2, hot_buffer_size=H, sparse_block_size=1)
    cases = [
        (dict(host_cache_k=torch.zeros((ROWS, WIDTH), dtype=torch.bfloat16),
              host_cache_v=torch.zeros((ROWS, WIDTH), dtype=torch.bfloat16)), ValueError, "pinned CPU memory"),
        (dict(host_cache_v=torch.zeros((ROWS, WIDTH // 2), dtype=torch.bfloat16).pin_memory()), ValueError,
         "host cache K and V must share shape"),
        (dict(device_buffer_k=dev_k[:, ::2], device_buffer_v=torch.zeros_like(dev_k)[:, ::2]), ValueError,
         "device buffer rows must be contiguous"),
        (dict(item_size_bytes=WIDTH * 4), ValueError, "item_size_bytes is 256"),
        (dict(seq_lens=torch.ones(1, dtype=torch.int32)), ValueError, "share one device"),
        (dict(top_k_blocks=torch.zeros((1, W), dtype=torch.float64, device=gpu)), TypeError,
         "top_k_blocks has unsupported dtype"),
    ]
    for change, error, message in cases:
        with pytest.raises(error, match=message):
            load_blocks_to_device_buffer_mha(**{**args, **change})
    torch.cuda.synchronize()
    assert bool((args["top_k_device_locs"] == -7).all())   # nothing ran
    load_blocks_to_device_buffer_mha(**args)                 # and the unchanged arguments are accepted
    torch.cuda.synchronize()
    assert args["top_k_device_locs"][0, 0].item() == args["device_buffer_locs"][0, H].item()   # the newest token
