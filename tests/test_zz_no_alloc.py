"""ekv_decode_step_static (no workspace, no allocation) against ekv_decode_step, through the C ABI.

Two copies of the same hot buffers, pool and pinned host copy: one runs the
workspace entry point, the other the static one, on two calls in a row - the
second over fewer layers and rows, so the static array holds the first
call's contents when the second starts. Slots, gathered rows, pool bytes and
LRU state must be identical after each call; a step larger than the static
array is refused with a message.
"""

import ctypes as ct
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from adaptive_sparse.decode_step import decode_step_workspace, step_args
from adaptive_sparse.host_arena import HostArena
from adaptive_sparse.kv_pool import KVPlanes
from adaptive_sparse.swap_in import HotBuffers, move_kv
from elastic_kv import _native

pytestmark = pytest.mark.gpu

L, R, T, C, ROW = 4, 6, 4000, 1024, 64


def _side(gpu, host_planes, host_table, seed):
    rng = np.random.default_rng(seed)
    buffers = HotBuffers(L, R, T, C, gpu, table_dtype=torch.int16, bits_shift=6)
    recent = torch.arange(T - 500, T, device=gpu).expand(L, R, 500)
    local = torch.tensor(np.stack([[rng.permutation(C)[:500] for _ in range(R)] for _ in range(L)]), device=gpu)
    buffers.install(recent, local)
    rows = 1 + R * C
    pool = torch.zeros(L * 2 * rows * ROW, dtype=torch.uint8, device=gpu)
    planes = KVPlanes(base=pool.data_ptr(), device=0, layers=L, kv=2, layer_stride=2 * rows * ROW,
                      kv_stride=rows * ROW, row_stride=ROW, row_bytes=ROW, rows=rows, owner=pool)
    src = host_table[torch.arange(R, device=gpu).view(1, R, 1), recent].contiguous()
    dst = (local + buffers.slot_base.view(1, R, 1)).to(torch.int32).contiguous()
    move_kv(host_planes, src, planes, dst, torch.full((L, R), 500, dtype=torch.int32, device=gpu))
    return buffers, pool, planes


def _first_layers(buffers, n):
    """The hot-buffer state of the first n layers (views), as step_args reads it."""
    return SimpleNamespace(table=buffers.table[:n], bits=buffers.bits[:n], bits_shift=buffers.bits_shift,
                           resident_counts=buffers.resident_counts[:n],
                           slot_base=buffers.slot_base, slot_token=buffers.slot_token[:n],
                           stamps=buffers.stamps[:n], step_counter=None, status=buffers.status)


def test_static_step_equals_the_workspace_step_on_two_calls(gpu):
    plane = R * T * ROW
    arena = HostArena(L * 2 * plane)
    try:
        arena.host.copy_(torch.randint(0, 256, (L * 2 * plane,), dtype=torch.uint8))
        host_planes = KVPlanes(base=arena.device_ptr, device=0, layers=L, kv=2, layer_stride=2 * plane,
                               kv_stride=plane, row_stride=ROW, row_bytes=ROW, rows=R * T, owner=arena)
        host_table = torch.arange(R * T, dtype=torch.int32, device=gpu).reshape(R, T)
        sides = [_side(gpu, host_planes, host_table, 4) for _ in range(2)]
        lib = _native.kernel_library()
        stream = _native.stream_handle(gpu)
        rng = np.random.default_rng(12)
        # call 1: every layer and row, 512 lanes, LRU step 0; call 2: 2 layers x 4 rows,
        # 128 lanes, step 1 (a step spans 8192 stamps whatever its width, so the
        # narrower call's stamps are still the newest)
        for call, (layers, batch, K, step) in enumerate(((L, R, 512, 0), (2, 4, 128, 1))):
            topk = torch.tensor(np.stack([rng.permutation(np.concatenate([
                rng.choice(np.arange(T - 900, T), K - K // 8, replace=False),
                rng.choice(np.arange(0, T - 900), K // 8, replace=False)])) for _ in range(layers * batch)])
                .reshape(layers, batch, K), dtype=torch.int32, device=gpu)
            rows = torch.arange(batch, device=gpu) + (R - batch)         # the last `batch` requests
            selected = torch.arange(batch, device=gpu)                   # batch rows, all served
            lengths = torch.full((batch,), T, dtype=torch.int32, device=gpu)
            results = []
            for index, (buffers, pool, planes) in enumerate(sides):
                slots = torch.full((layers, batch, K), -9, dtype=torch.int32, device=gpu)
                out = torch.empty((batch, layers, 2, K, ROW), dtype=torch.uint8, device=gpu)
                args, keep = step_args(topk, rows, lengths, selected, _first_layers(buffers, layers), host_table,
                                       host_planes, planes, slots, out, 1, step)
                if index == 0:
                    workspace = torch.empty(decode_step_workspace(layers, batch, K), dtype=torch.uint8, device=gpu)
                    status = lib.ekv_decode_step(ct.addressof(args), ct.c_void_p(workspace.data_ptr()),
                                                 workspace.numel(), stream)
                else:
                    status = lib.ekv_decode_step_static(ct.addressof(args), stream)
                _native.check(lib, status, "decode step")
                torch.cuda.synchronize()
                del keep
                results.append([slots.cpu(), out.cpu(), pool.cpu(), buffers.table.cpu(), buffers.bits.cpu(),
                                buffers.resident_counts.cpu(), buffers.slot_token.cpu(), buffers.stamps.cpu(),
                                buffers.status.cpu()])
            print(f"[no-alloc] call {call}: {layers} layers x {batch} rows x {K} lanes", flush=True)
            for a, b in zip(*results):
                assert torch.equal(a, b), call
            assert int(results[1][-1]) == 0
            assert int((results[0][0] > 0).sum()) == layers * batch * K          # every lane resident after
        # a step whose intermediates exceed the static array is refused
        big = torch.zeros((16, 128, 4096), dtype=torch.int32, device=gpu)
        buffers, _, planes = sides[1]
        row = torch.empty(ROW, dtype=torch.uint8, device=gpu)
        out = row.as_strided((128, 16, 2, 4096, ROW), (0, 0, 0, 0, 1))     # never written: refused first
        args, keep = step_args(big, torch.arange(128, device=gpu), torch.zeros(128, dtype=torch.int32, device=gpu),
                               torch.arange(128, device=gpu), buffers, host_table, host_planes, planes, big, out, 1, 5)
        assert lib.ekv_decode_step_static(ct.addressof(args), stream) == -1
        assert b"static workspace" in lib.ev_error()
    finally:
        torch.cuda.synchronize()
        arena.close()
