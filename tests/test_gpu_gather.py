"""GPU parity of the HIP gather family against the oracle (bit-exact bytes)."""

import numpy as np
import pytest
import torch

from adaptive_sparse.kv_pool import KVPlanes
from adaptive_sparse.sparse_read import gather_kv, scatter_kv

pytestmark = pytest.mark.gpu


def make_pool(gpu, seed, layers, kv, rows, row_bytes, row_stride=None, pad=0):
    row_stride = row_stride or row_bytes
    plane = rows * row_stride + pad
    gen = torch.Generator(device="cpu").manual_seed(seed)
    host = torch.randint(0, 256, (layers * kv * plane,), dtype=torch.uint8, generator=gen)
    pool = host.to(gpu)
    planes = KVPlanes(base=pool.data_ptr(), device=gpu.index or 0, layers=layers, kv=kv,
                      layer_stride=kv * plane, kv_stride=plane, row_stride=row_stride,
                      row_bytes=row_bytes, rows=rows, owner=pool)
    return pool, host.numpy(), planes


GATHER_CASES = [
    # layers, kv, rows, row_bytes, batch, k, zero_below, row_stride
    (2, 2, 300, 512, 3, 70, 1, None),       # config-3 rows (2 heads x 128 bf16)
    (3, 2, 90, 2048, 2, 33, 1, None),       # config-1 rows (8 heads x 128 bf16)
    (2, 1, 50, 6, 4, 300, 1, None),         # 2-byte lanes
    (1, 2, 40, 24, 3, 17, 0, 40),           # 8-byte lanes, padded rows, block mode (0 valid)
    (1, 2, 12, 32768, 2, 5, 0, None),       # one 32 KiB row per tile (config-2 blocks)
    (1, 1, 6, 40960, 1, 4, 1, None),        # large rows split into 2 segments
]


@pytest.mark.parametrize("case", range(len(GATHER_CASES)))
def test_gather_kv_matches_oracle(gpu, coracle, case):
    layers, kv, rows, row_bytes, batch, k, zero_below, row_stride = GATHER_CASES[case]
    pool, host, planes = make_pool(gpu, 10 + case, layers, kv, rows, row_bytes, row_stride, pad=64)
    rng = np.random.default_rng(case)
    slots = rng.integers(-1, rows + 2, size=(layers, batch, k))
    out = torch.full((batch, layers, kv, k, row_bytes), 0xAB, dtype=torch.uint8, device=gpu)
    gather_kv(planes, torch.tensor(slots, dtype=torch.int32, device=gpu), out, zero_below=zero_below)
    want = coracle.gather_kv(host, planes.layer_stride, planes.kv_stride, planes.row_stride, row_bytes, rows,
                             slots, kv, zero_below=zero_below)
    assert np.array_equal(out.cpu().numpy(), want)


def test_gather_kv_shared_layer_slots_and_strided_output(gpu, coracle):
    layers, kv, rows, row_bytes, batch, k = 4, 2, 128, 256, 3, 50
    pool, host, planes = make_pool(gpu, 3, layers, kv, rows, row_bytes)
    rng = np.random.default_rng(5)
    slots = rng.integers(0, rows, size=(batch, k))
    shared = torch.tensor(slots, dtype=torch.int64, device=gpu).unsqueeze(0).expand(layers, batch, k)
    big = torch.zeros((batch, layers, kv, k + 3, row_bytes // 2), dtype=torch.bfloat16, device=gpu)
    out = big[:, :, :, 2:k + 2]
    gather_kv(planes, shared, out)
    want = coracle.gather_kv(host, planes.layer_stride, planes.kv_stride, planes.row_stride, row_bytes, rows,
                             slots, kv, shared_layers=layers)
    got = out.contiguous().view(torch.uint8).reshape(batch, layers, kv, k, row_bytes).cpu().numpy()
    assert np.array_equal(got, want)
    assert (big[:, :, :, :2] == 0).all() and (big[:, :, :, k + 2:] == 0).all()


@pytest.mark.parametrize("row_bytes", [512, 24, 40960])
def test_scatter_kv_matches_oracle_and_inverts_gather(gpu, coracle, row_bytes):
    layers, kv, rows, batch, k = 2, 2, 64, 2, 9
    pool, host, planes = make_pool(gpu, 21, layers, kv, rows, row_bytes)
    rng = np.random.default_rng(row_bytes)
    slots = np.stack([rng.permutation(np.arange(1, rows))[: batch * k].reshape(batch, k) for _ in range(layers)])
    slots[0, 0, 0] = -1  # padding lane writes nothing
    src = torch.randint(0, 256, (batch, layers, kv, k, row_bytes), dtype=torch.uint8, device=gpu)
    scatter_kv(planes, torch.tensor(slots, dtype=torch.int32, device=gpu), src)
    want = coracle.scatter_kv(host, planes.layer_stride, planes.kv_stride, planes.row_stride, row_bytes, rows,
                              slots, kv, src.cpu().numpy())
    assert np.array_equal(pool.cpu().numpy(), want)
    back = torch.zeros_like(src)
    gather_kv(planes, torch.tensor(slots, dtype=torch.int32, device=gpu), back)
    expect = src.clone()
    expect[0, 0, :, 0] = 0  # the padding lane gathers zeros
    assert torch.equal(back, expect)


def test_gather_kv_rejects_bad_shapes(gpu):
    pool, _, planes = make_pool(gpu, 1, 1, 2, 8, 16)
    slots = torch.zeros((1, 2, 3), dtype=torch.int32, device=gpu)
    with pytest.raises(ValueError):
        gather_kv(planes, slots, torch.zeros((2, 1, 2, 4, 16), dtype=torch.uint8, device=gpu))
    with pytest.raises(ValueError):
        gather_kv(planes, slots, torch.zeros((2, 1, 2, 3, 15), dtype=torch.uint8, device=gpu))
    with pytest.raises(ValueError):
        gather_kv(planes, torch.zeros((2, 2, 3), dtype=torch.int32, device=gpu),
                  torch.zeros((2, 2, 2, 3, 16), dtype=torch.uint8, device=gpu))
