"""GPU tests of the HiSparse swap-in with SGLang's calling convention (ekv_hisparse_swap_in).

- The reference's swap smoke test (tests/smoke_minimax_swap.py:18-79) on
  stock device tensors and on VMM-backed planes: valid locations > 0, the
  newest token in the reserved slot, -1 tail, every selected device row
  equal to its host row, and the same locations for both layouts.
- Seeded random multi-step streams against the oracle, bit-exact in the
  output locations, the hot tokens, the LRU lists and every device row:
  hot sizes 1..4096, block sizes 1..128, index dtypes, strided views, row
  sizes for every copy width, padding rows, repeated blocks, lengths past
  the host table, host rows and device rows out of range.
- One decode-sized call: 128 requests, 4096 hot slots, 16 blocks of 128
  tokens, 512-byte K and V rows.
"""

import numpy as np
import pytest
import torch

from adaptive_sparse.hisparse_swap import load_blocks_to_device_buffer_mha
from oracle import oracle as ref

pytestmark = pytest.mark.gpu

BLOCK, HOT, WIDTH = 128, 256, 128


def smoke_check(planes, gpu):
    """tests/smoke_minimax_swap.py:18-67 through this library's swap-in; returns the locations."""
    results = []
    for layer in range(2):
        device_k, device_v = planes[layer], planes[layer + 2]
        host = [(torch.arange(3 * BLOCK)[:, None, None] % 43 + torch.arange(WIDTH)[None, None, :] % 13
                 + layer * 64 + plane * 128).to(torch.bfloat16).pin_memory() for plane in range(2)]
        locs = torch.arange(1, HOT + 2, dtype=torch.int32, device=gpu).view(1, -1)
        tokens = torch.full((1, HOT + 1), -1, dtype=torch.int32, device=gpu)
        tokens[0, :BLOCK] = torch.arange(BLOCK, 2 * BLOCK, device=gpu)        # the hot buffer holds block 1
        for dst, src in zip((device_k, device_v), host):
            dst[1:BLOCK + 1].copy_(src[BLOCK:2 * BLOCK], non_blocking=True)
        lru = torch.arange(HOT, dtype=torch.int16, device=gpu).view(1, -1)
        out = torch.empty((1, 2 * BLOCK), dtype=torch.int32, device=gpu)
        for newest in range(2 * BLOCK, 2 * BLOCK + 3):
            for dst, src in zip((device_k, device_v), host):
                if newest > 2 * BLOCK:
                    src[newest - 1].copy_(dst[HOT + 1], non_blocking=True)   # back up the previous newest
                dst[HOT + 1].copy_(src[newest], non_blocking=True)
            torch.cuda.synchronize()
            load_blocks_to_device_buffer_mha(
                top_k_blocks=torch.tensor([[0, 2]], dtype=torch.int32, device=gpu),
                device_buffer_tokens=tokens,
                host_cache_locs=torch.arange(3 * BLOCK, dtype=torch.int64, device=gpu).view(1, -1),
                device_buffer_locs=locs, host_cache_k=host[0], host_cache_v=host[1],
                device_buffer_k=device_k, device_buffer_v=device_v, top_k_device_locs=out,
                req_pool_indices=torch.tensor([0], dtype=torch.int64, device=gpu),
                seq_lens=torch.tensor([newest + 1], dtype=torch.int32, device=gpu),
                lru_slots=lru, item_size_bytes=WIDTH * 2, hot_buffer_size=HOT, sparse_block_size=BLOCK,
                num_real_reqs=torch.tensor([1], dtype=torch.int32, device=gpu))
            torch.cuda.synchronize()
            valid = BLOCK + newest - 2 * BLOCK + 1
            selected = out[0, :valid].long()
            assert (selected > 0).all().item()
            assert selected[-1].item() == HOT + 1
            assert (out[0, valid:] == -1).all().item()
            for dst, src in zip((device_k, device_v), host):
                expected = torch.cat((src[:BLOCK], src[2 * BLOCK:newest + 1]))
                assert torch.equal(dst[selected].cpu(), expected), (layer, newest)
            results.append(selected.tolist())
    return results


def test_reference_smoke_on_stock_and_vmm_planes(gpu):
    from elastic_kv.backing import Backing

    chunk = 2 << 20
    shape = (HOT + 2, 1, WIDTH)
    stock = [torch.zeros(shape, dtype=torch.bfloat16, device=gpu) for _ in range(4)]
    backing = Backing(4 * chunk, chunk, device=0)
    raw = vmm = None
    try:
        backing.ensure(range(4))
        raw = backing.raw
        length = (HOT + 2) * WIDTH * 2
        vmm = [raw.narrow(0, plane * chunk, length).view(torch.bfloat16).view(shape) for plane in range(4)]
        first = smoke_check(stock, gpu)
        assert first == smoke_check(vmm, gpu)
        assert first[0][:3] == [129, 130, 131]        # block 0 fills the empty slots 128.. in order
        torch.cuda.synchronize()
    finally:
        del vmm, raw
        backing.close()


def index(array, dtype, device, strided=False):
    source = torch.tensor(np.asarray(array), dtype=dtype)
    if not strided:
        return source.to(device)
    spread = torch.zeros((*source.shape, 2), dtype=dtype)
    spread[..., 0] = source
    return spread.to(device)[..., 0]


def random_stream(seed):
    rng = np.random.default_rng(9100 + seed)
    hot = int(rng.choice([1, 3, 7, 64, 256, 1000, 4096]))
    bs = int(rng.choice([1, 1, 2, 16, 128]))
    bs = min(bs, hot)
    k = int(rng.integers(1, max(1, min(hot, 2048) // bs) + 1))
    batch = int(rng.integers(1, 7))
    requests = batch + int(rng.integers(0, 3))
    context = int(rng.integers(max(2, k * bs // 2), 3 * hot + 2 * k * bs + 8))
    row_bytes = int(rng.choice([16, 256, 512, 36, 7, 2]))
    host_rows = requests * context + 5
    dev_rows = requests * (hot + 1) + 3
    host_locs = rng.permutation(host_rows)[:requests * context].reshape(requests, context)
    host_locs[rng.random(host_locs.shape) < 0.03] = host_rows + 7                       # no host row
    dev_locs = rng.permutation(dev_rows)[:requests * (hot + 1)].reshape(requests, hot + 1)
    dev_locs[rng.random(dev_locs.shape) < 0.03] = -2                                      # outside the buffer
    tokens = np.full((requests, hot + 1), -1)
    lru = np.zeros((requests, hot), dtype=np.int64)
    for r in range(requests):
        n = int(rng.integers(0, min(hot, context) + 1))
        tokens[r, rng.choice(hot, size=n, replace=False)] = rng.choice(context, size=n, replace=False)
        lru[r] = rng.permutation(hot)
    return rng, hot, bs, k, batch, requests, context, row_bytes, host_rows, dev_rows, host_locs, dev_locs, tokens, lru


@pytest.mark.parametrize("seed", range(24))
def test_random_streams_match_the_oracle(gpu, seed):
    (rng, hot, bs, k, batch, requests, context, row_bytes, host_rows, dev_rows, host_locs, dev_locs, tokens,
     lru) = random_stream(seed)
    dtypes = [torch.int32 if rng.random() < 0.5 else torch.int64 for _ in range(5)]
    lru_dtype = torch.int16 if rng.random() < 0.7 else torch.int32
    strided = bool(rng.random() < 0.3)
    host = torch.randint(0, 256, (2, host_rows, row_bytes), dtype=torch.uint8).pin_memory()
    device_k = torch.randint(0, 256, (dev_rows, row_bytes), dtype=torch.uint8, device=gpu)
    device_v = torch.randint(0, 256, (dev_rows, row_bytes), dtype=torch.uint8, device=gpu)
    tokens_d = index(tokens, torch.int32, gpu, strided)
    lru_d = index(lru, lru_dtype, gpu, strided)
    host_locs_d = index(host_locs, dtypes[0], gpu, strided)
    dev_locs_d = index(dev_locs, dtypes[1], gpu)
    want_tokens, want_lru = tokens, lru
    want_k, want_v = device_k.cpu().numpy(), device_v.cpu().numpy()
    seq = rng.integers(1, context + 3, size=batch)
    for step in range(3):
        req = rng.permutation(requests)[:batch]
        seq = seq + 1
        seq[rng.random(batch) < 0.15] = 0                                  # padding rows of length 0
        blocks = np.stack([rng.permutation(max(k, -(-context // bs) + 2))[:k] - 1 for _ in range(batch)])
        for b in range(batch):
            if rng.random() < 0.2 and k > 1:
                blocks[b, -1] = blocks[b, 0]                               # a repeated Top-K block
            recent = (int(seq[b]) - 1) // bs
            if rng.random() < 0.7 and recent >= 0:
                blocks[b, int(rng.integers(k))] = recent                   # select the newest token's block
        num_real = int(rng.integers(0, batch + 1)) if rng.random() < 0.3 else None
        out = torch.full((batch, k * bs), -9, dtype=torch.int32, device=gpu)
        load_blocks_to_device_buffer_mha(
            top_k_blocks=index(blocks, dtypes[2], gpu, strided), device_buffer_tokens=tokens_d,
            host_cache_locs=host_locs_d, device_buffer_locs=dev_locs_d, host_cache_k=host[0], host_cache_v=host[1],
            device_buffer_k=device_k, device_buffer_v=device_v, top_k_device_locs=out,
            req_pool_indices=index(req, dtypes[3], gpu), seq_lens=index(seq, dtypes[4], gpu), lru_slots=lru_d,
            item_size_bytes=row_bytes, hot_buffer_size=hot, sparse_block_size=bs,
            num_real_reqs=None if num_real is None else torch.tensor([num_real], dtype=torch.int32, device=gpu))
        want_out, want_tokens, want_lru, want_k, want_v = ref.hisparse_swap(
            blocks, want_tokens, host_locs, dev_locs, host[0].numpy(), host[1].numpy(), want_k, want_v, req, seq,
            want_lru, hot, bs, num_real)
        case = (seed, step, hot, bs, k, batch, row_bytes)
        assert np.array_equal(out.cpu().numpy(), want_out), case
        assert np.array_equal(tokens_d.cpu().numpy(), want_tokens), case
        assert np.array_equal(lru_d.cpu().numpy().astype(np.int64), want_lru), case
        assert np.array_equal(device_k.cpu().numpy(), want_k), case
        assert np.array_equal(device_v.cpu().numpy(), want_v), case


def test_decode_sized_call_matches_the_oracle(gpu):
    # 128 requests, hot buffers of 4096 slots, 16 blocks x 128 tokens, 2 KV heads x 128 bf16 per row.
    rng = np.random.default_rng(77)
    batch, hot, bs, k, context, row_bytes = 128, 4096, 128, 16, 32768, 512
    host_rows = 1 << 16
    host_locs = (np.arange(context)[None, :] * 7 + np.arange(batch)[:, None] * 131) % host_rows
    dev_locs = np.arange(batch * (hot + 1)).reshape(batch, hot + 1) + 1
    tokens = np.full((batch, hot + 1), -1)
    lru = np.zeros((batch, hot), dtype=np.int64)
    for r in range(batch):
        tokens[r, :hot - 512] = rng.choice(context - 1, size=hot - 512, replace=False)
        lru[r] = rng.permutation(hot)
    host = torch.randint(0, 256, (2, host_rows, row_bytes), dtype=torch.uint8).pin_memory()
    device_k = torch.zeros((batch * (hot + 1) + 1, row_bytes), dtype=torch.uint8, device=gpu)
    device_v = torch.zeros_like(device_k)
    tokens_d = torch.tensor(tokens, dtype=torch.int32, device=gpu)
    lru_d = torch.tensor(lru, dtype=torch.int16, device=gpu)
    host_locs_d = torch.tensor(host_locs, device=gpu)
    dev_locs_d = torch.tensor(dev_locs, dtype=torch.int32, device=gpu)
    seq = np.full(batch, context)
    blocks = np.stack([rng.choice(context // bs, size=k, replace=False) for _ in range(batch)])
    blocks[:, 0] = context // bs - 1                                       # the newest block
    out = torch.empty((batch, k * bs), dtype=torch.int32, device=gpu)
    load_blocks_to_device_buffer_mha(
        top_k_blocks=torch.tensor(blocks, dtype=torch.int32, device=gpu), device_buffer_tokens=tokens_d,
        host_cache_locs=host_locs_d, device_buffer_locs=dev_locs_d, host_cache_k=host[0], host_cache_v=host[1],
        device_buffer_k=device_k, device_buffer_v=device_v, top_k_device_locs=out,
        req_pool_indices=torch.arange(batch, device=gpu), seq_lens=torch.tensor(seq, device=gpu),
        lru_slots=lru_d, item_size_bytes=row_bytes, hot_buffer_size=hot, sparse_block_size=bs)
    want_out, want_tokens, want_lru, want_k, want_v = ref.hisparse_swap(
        blocks, tokens, host_locs, dev_locs, host[0].numpy(), host[1].numpy(), device_k.cpu().numpy(),
        device_v.cpu().numpy(), np.arange(batch), seq, lru, hot, bs)
    assert np.array_equal(out.cpu().numpy(), want_out)
    assert np.array_equal(tokens_d.cpu().numpy(), want_tokens)
    assert np.array_equal(lru_d.cpu().numpy().astype(np.int64), want_lru)
    assert np.array_equal(device_k.cpu().numpy(), want_k) and np.array_equal(device_v.cpu().numpy(), want_v)
    assert (out >= 0).all().item()                                          # every lane selected a valid token


def test_graph_replays_with_padding_rows_match_the_oracle(gpu):
    # SGLang replays decode from captured graphs; rows at or past num_real_reqs are padding.
    rng = np.random.default_rng(505)
    batch, hot, bs, k, context, row_bytes = 4, 64, 4, 6, 400, 64
    host_rows = batch * context
    host_locs = rng.permutation(host_rows).reshape(batch, context)
    dev_locs = rng.permutation(batch * (hot + 1)).reshape(batch, hot + 1) + 1
    host = torch.randint(0, 256, (2, host_rows, row_bytes), dtype=torch.uint8).pin_memory()
    device_k = torch.zeros((batch * (hot + 1) + 1, row_bytes), dtype=torch.uint8, device=gpu)
    device_v = torch.zeros_like(device_k)
    tokens = torch.full((batch, hot + 1), -1, dtype=torch.int32, device=gpu)
    lru = torch.arange(hot, dtype=torch.int16, device=gpu).repeat(batch, 1)
    blocks_d = torch.zeros((batch, k), dtype=torch.int32, device=gpu)
    seq_d = torch.zeros(batch, dtype=torch.int32, device=gpu)
    real_d = torch.zeros(1, dtype=torch.int32, device=gpu)
    req = torch.arange(batch, device=gpu)
    out = torch.empty((batch, k * bs), dtype=torch.int32, device=gpu)
    host_locs_d, dev_locs_d = torch.tensor(host_locs, device=gpu), torch.tensor(dev_locs, device=gpu)

    def call():
        load_blocks_to_device_buffer_mha(
            top_k_blocks=blocks_d, device_buffer_tokens=tokens, host_cache_locs=host_locs_d,
            device_buffer_locs=dev_locs_d, host_cache_k=host[0], host_cache_v=host[1], device_buffer_k=device_k,
            device_buffer_v=device_v, top_k_device_locs=out, req_pool_indices=req, seq_lens=seq_d, lru_slots=lru,
            item_size_bytes=row_bytes, hot_buffer_size=hot, sparse_block_size=bs, num_real_reqs=real_d)

    want = (tokens.cpu().numpy(), lru.cpu().numpy().astype(np.int64), device_k.cpu().numpy(),
            device_v.cpu().numpy())
    seq = np.full(batch, 150)
    graph = torch.cuda.CUDAGraph()
    for step in range(6):
        seq = seq + 1
        blocks = np.stack([rng.choice(-(-int(s) // bs), size=k, replace=False) for s in seq])
        real = int(rng.integers(1, batch + 1))
        blocks_d.copy_(torch.tensor(blocks, dtype=torch.int32))
        seq_d.copy_(torch.tensor(seq, dtype=torch.int32))
        real_d.fill_(real)
        if step == 0:
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                call()                                     # eager first call
            torch.cuda.current_stream().wait_stream(side)
            torch.cuda.synchronize()
            with torch.cuda.graph(graph):
                call()                                     # recorded, not run
        else:
            graph.replay()
        torch.cuda.synchronize()
        want_out, *rest = ref.hisparse_swap(blocks, *want[:1], host_locs, dev_locs, host[0].numpy(),
                                            host[1].numpy(), want[2], want[3], np.arange(batch), seq, want[1], hot,
                                            bs, real)
        want = (rest[0], rest[1], rest[2], rest[3])
        assert np.array_equal(out.cpu().numpy()[:real], want_out[:real]), step
        assert (out.cpu().numpy()[real:] == -1).all(), step
        assert np.array_equal(tokens.cpu().numpy(), want[0]), step
        assert np.array_equal(lru.cpu().numpy().astype(np.int64), want[1]), step
        assert np.array_equal(device_k.cpu().numpy(), want[2]) and np.array_equal(device_v.cpu().numpy(), want[3])
        torch.randn(1000, device=gpu).sum().item()        # eager work between replays
