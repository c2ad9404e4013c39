"""The one-call decode step (ekv_decode_step) against its four stages called one by one.

Two copies of the same hot buffers, pool and pinned host copy see the same
Top-K stream. One copy runs resolve_resident -> swap_in -> move_kv ->
gather_kv (each parity-checked against the oracle elsewhere), the other runs
decode_step; after every step the slots, gathered rows, pool bytes and LRU
state must be identical. The step also replays from a captured HIP graph
(device step counter, caller workspace) with new Top-K contents.
"""

import numpy as np
import pytest
import torch

from adaptive_sparse.decode_step import decode_step, decode_step_workspace
from adaptive_sparse.host_arena import HostArena
from adaptive_sparse.kv_pool import KVPlanes
from adaptive_sparse.resident_lookup import resolve_resident
from adaptive_sparse.sparse_read import gather_kv
from adaptive_sparse.swap_in import HotBuffers, move_kv, swap_in

pytestmark = pytest.mark.gpu

L, R, T, C, K, ROW = 3, 5, 3000, 512, 256, 64


class Side:
    """Hot buffers + pool of one copy."""

    def __init__(self, gpu, host, table_dtype, shift, counter, seed):
        host_planes, host_table, _ = host
        rng = np.random.default_rng(seed)
        self.buffers = HotBuffers(L, R, T, C, gpu, table_dtype=table_dtype, bits_shift=shift, step_counter=counter)
        recent = torch.arange(T - 300, T, device=gpu).expand(L, R, 300)
        local = torch.tensor(np.stack([[rng.permutation(C)[:300] for _ in range(R)] for _ in range(L)]), device=gpu)
        self.buffers.install(recent, local)
        rows = 1 + R * C
        self.pool = torch.zeros(L * 2 * rows * ROW, dtype=torch.uint8, device=gpu)
        self.planes = KVPlanes(base=self.pool.data_ptr(), device=0, layers=L, kv=2, layer_stride=2 * rows * ROW,
                               kv_stride=rows * ROW, row_stride=ROW, row_bytes=ROW, rows=rows, owner=self.pool)
        # The installed tokens' rows come from the host copy.
        src = host_table[torch.arange(R, device=gpu).view(1, R, 1), recent].contiguous()
        dst = (local + self.buffers.slot_base.view(1, R, 1)).to(torch.int32).contiguous()
        move_kv(host_planes, src, self.planes, dst, torch.full((L, R), 300, dtype=torch.int32, device=gpu))

    def state(self):
        b = self.buffers
        counts = [b.resident_counts.cpu()] if b.resident_counts is not None else []
        return [b.table.cpu(), b.bits.cpu(), b.slot_token.cpu(), b.stamps.cpu(), self.pool.cpu()] + counts


def _topk(rng):
    return torch.tensor(np.stack([rng.permutation(np.concatenate([
        rng.choice(np.arange(T - 600, T), K - 40, replace=False), rng.choice(np.arange(0, T - 600), 40, replace=False)]))
        for _ in range(L * R)]).reshape(L, R, K), dtype=torch.int32)


@pytest.fixture(scope="module")
def host(gpu):
    plane = R * T * ROW
    arena = HostArena(L * 2 * plane)
    arena.host.copy_(torch.randint(0, 256, (L * 2 * plane,), dtype=torch.uint8))
    planes = KVPlanes(base=arena.device_ptr, device=0, layers=L, kv=2, layer_stride=2 * plane, kv_stride=plane,
                      row_stride=ROW, row_bytes=ROW, rows=R * T, owner=arena)
    table = torch.arange(R * T, dtype=torch.int32, device=gpu).reshape(R, T)
    yield planes, table, arena.host.numpy().reshape(L, 2, R * T, ROW)
    torch.cuda.synchronize()
    arena.close()


@pytest.mark.parametrize("table_dtype,shift", [(torch.int16, 6), (torch.int32, 0)])
def test_decode_step_equals_its_stages(gpu, host, table_dtype, shift):
    host_planes, host_table, host_rows = host
    staged, fused = Side(gpu, host, table_dtype, shift, False, 1), Side(gpu, host, table_dtype, shift, False, 1)
    rows = torch.arange(R, device=gpu)
    lengths = torch.tensor([T, T - 3, T - 50, T, T - 7], dtype=torch.int32, device=gpu)
    rng = np.random.default_rng(3)
    workspace = torch.empty(decode_step_workspace(L, R, K), dtype=torch.uint8, device=gpu)
    for step in range(4):
        topk = _topk(rng).to(gpu)
        # steps 1 and 3 serve a subset of the rows: the others must promote nothing
        selected = torch.tensor([0, 2, 4] if step % 2 else list(range(R)), device=gpu)
        outputs = []
        for side in (staged, fused):
            slots = torch.full((L, R, K), -9, dtype=torch.int32, device=gpu)
            out = torch.empty((R, L, 2, K, ROW), dtype=torch.uint8, device=gpu)
            b = side.buffers
            if side is staged:
                misses = torch.empty((L, R, K), dtype=torch.int32, device=gpu)
                counts = torch.zeros((L, R), dtype=torch.int32, device=gpu)
                resolve_resident(topk, b.table, None, rows, lengths, selected, slots, 1, misses=misses,
                                 miss_count=counts, resident_bits=b.bits, bits_shift=b.bits_shift,
                                 slot_base=b.slot_base if table_dtype == torch.int16 else None)
                src, dst = torch.empty_like(slots), torch.empty_like(slots)
                swap_in(topk, 1, rows, selected, slots, misses, counts, b, host_table, src, dst)
                move_kv(host_planes, src, side.planes, dst, counts)
                gather_kv(side.planes, slots, out)
            else:
                if step % 2:
                    workspace.fill_(0x7f)          # stale contents from "an earlier call" must not matter
                decode_step(topk, rows, lengths, b, host_table, host_planes, side.planes, slots, out,
                            selected=selected, workspace=workspace if step % 2 else None)
            outputs.append([slots.cpu(), out.cpu()] + side.state())
        torch.cuda.synchronize()
        for a, b in zip(*outputs):
            assert torch.equal(a, b), step
        got = outputs[1][1].numpy()
        tokens = topk.cpu().numpy()
        for layer in range(L):
            for r in selected.tolist():
                valid = tokens[layer, r] < int(lengths[r])
                want = host_rows[layer, :, host_table[r].cpu().numpy()[tokens[layer, r]]]     # [K, 2, ROW]
                assert np.array_equal(got[r, layer][:, valid], np.swapaxes(want, 0, 1)[:, valid]), (step, layer, r)
                assert not got[r, layer][:, ~valid].any()
    assert fused.buffers.step == staged.buffers.step == 4
    with pytest.raises(RuntimeError, match="workspace bytes"):
        decode_step(topk, rows, lengths, fused.buffers, host_table, host_planes, fused.planes,
                    torch.empty((L, R, K), dtype=torch.int32, device=gpu),
                    torch.empty((R, L, 2, K, ROW), dtype=torch.uint8, device=gpu), workspace=workspace[:-256])


def test_decode_step_without_selected_serves_every_batch_row(gpu, host):
    # A batch of 3 rows naming requests 4, 2 and 3 (ids outside 0 .. B - 1 and
    # permuted) with no `selected`: every batch row must be looked up, swapped
    # in and gathered, as the staged path does with selected = 0 .. B - 1.
    host_planes, host_table, host_rows = host
    staged, fused = Side(gpu, host, torch.int16, 6, False, 7), Side(gpu, host, torch.int16, 6, False, 7)
    rows = torch.tensor([4, 2, 3], device=gpu)
    B = rows.numel()
    lengths = torch.full((B,), T, dtype=torch.int32, device=gpu)
    rng = np.random.default_rng(13)
    for step in range(2):
        topk = _topk(rng)[:, :B].contiguous().to(gpu)
        outputs = []
        for side in (staged, fused):
            slots = torch.full((L, B, K), -9, dtype=torch.int32, device=gpu)
            out = torch.empty((B, L, 2, K, ROW), dtype=torch.uint8, device=gpu)
            b = side.buffers
            if side is staged:
                every = torch.arange(B, device=gpu)
                misses = torch.empty((L, B, K), dtype=torch.int32, device=gpu)
                counts = torch.zeros((L, B), dtype=torch.int32, device=gpu)
                resolve_resident(topk, b.table, None, rows, lengths, every, slots, 1, misses=misses,
                                 miss_count=counts, resident_bits=b.bits, bits_shift=b.bits_shift,
                                 slot_base=b.slot_base)
                src, dst = torch.empty_like(slots), torch.empty_like(slots)
                swap_in(topk, 1, rows, every, slots, misses, counts, b, host_table, src, dst)
                move_kv(host_planes, src, side.planes, dst, counts)
                gather_kv(side.planes, slots, out)
            else:
                decode_step(topk, rows, lengths, b, host_table, host_planes, side.planes, slots, out)
            outputs.append([slots.cpu(), out.cpu()] + side.state())
        torch.cuda.synchronize()
        for a, b in zip(*outputs):
            assert torch.equal(a, b), step
        assert int((outputs[1][0] > 0).sum()) == L * B * K          # no batch row left unserved
        got, tokens = outputs[1][1].numpy(), topk.cpu().numpy()
        for layer in range(L):
            for i, r in enumerate(rows.tolist()):
                want = host_rows[layer, :, host_table[r].cpu().numpy()[tokens[layer, i]]]
                assert np.array_equal(got[i, layer], np.swapaxes(want, 0, 1)), (step, layer, i)


def test_decode_step_replays_from_a_graph(gpu, host):
    host_planes, host_table, _ = host
    eager, graphed = Side(gpu, host, torch.int16, 6, True, 5), Side(gpu, host, torch.int16, 6, True, 5)
    rows = torch.arange(R, device=gpu)
    lengths = torch.full((R,), T, dtype=torch.int32, device=gpu)
    rng = np.random.default_rng(9)
    topk = torch.zeros((L, R, K), dtype=torch.int32, device=gpu)
    slots = [torch.empty((L, R, K), dtype=torch.int32, device=gpu) for _ in range(2)]
    out = [torch.empty((R, L, 2, K, ROW), dtype=torch.uint8, device=gpu) for _ in range(2)]
    workspace = torch.empty(decode_step_workspace(L, R, K), dtype=torch.uint8, device=gpu)

    def step_of(side, i):
        decode_step(topk, rows, lengths, side.buffers, host_table, host_planes, side.planes, slots[i], out[i],
                    workspace=workspace)

    graph = None
    for step in range(4):
        topk.copy_(_topk(rng))
        step_of(eager, 0)
        if graph is None:
            step_of(graphed, 1)                   # eager first step, also loads every kernel
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                step_of(graphed, 1)               # recorded, not run
        else:
            graph.replay()
        torch.cuda.synchronize()
        assert int(graphed.buffers.step_counter.item()) == step + 1
        assert torch.equal(slots[0], slots[1]) and torch.equal(out[0], out[1]), step
        for a, b in zip(eager.state(), graphed.state()):
            assert torch.equal(a, b), step
    del graph


def test_a_stage_that_refuses_its_arguments_leaves_nothing_queued(gpu, host):
    """The step checks all four stages before it launches any: a refusal by the swap-in or the
    promote leaves the slots, the hot buffers, the pool and the output as they were."""
    host_planes, host_table, _ = host
    side = Side(gpu, host, torch.int16, 6, False, 5)
    rows = torch.arange(R, device=gpu)
    lengths = torch.full((R,), T, dtype=torch.int32, device=gpu)
    rng = np.random.default_rng(11)
    narrow_host = KVPlanes(base=host_planes.base, device=0, layers=L, kv=2, layer_stride=host_planes.layer_stride,
                           kv_stride=host_planes.kv_stride, row_stride=ROW, row_bytes=ROW // 2, rows=host_planes.rows,
                           owner=host_planes.owner)
    wide = C + 8                                    # more lanes per row than a hot buffer holds
    cases = [
        (torch.tensor(rng.integers(0, T, (L, R, wide)), dtype=torch.int32, device=gpu), host_planes, "swap-in"),
        (_topk(rng).to(gpu), narrow_host, "promote"),
    ]
    for topk, planes, stage in cases:
        width = topk.shape[2]
        before = side.state()
        slots = torch.full((L, R, width), -9, dtype=torch.int32, device=gpu)
        out = torch.full((R, L, 2, width, ROW), 0x5a, dtype=torch.uint8, device=gpu)
        with pytest.raises(RuntimeError, match=stage):
            decode_step(topk, rows, lengths, side.buffers, host_table, planes, side.planes, slots, out)
        torch.cuda.synchronize()
        assert bool((slots == -9).all()), stage
        assert bool((out == 0x5a).all()), stage
        for a, b in zip(before, side.state()):
            assert torch.equal(a, b), stage
        assert side.buffers.step == 0


def test_argument_errors_name_the_argument(gpu, host):
    """The launch helper's own checks of the step's planes and output rows (before the entry point's)."""
    host_planes, host_table, _ = host
    side = Side(gpu, host, torch.int16, 6, False, 6)
    rows = torch.arange(R, device=gpu)
    lengths = torch.full((R,), T, dtype=torch.int32, device=gpu)
    topk = _topk(np.random.default_rng(12)).to(gpu)
    slots = torch.full((L, R, K), -9, dtype=torch.int32, device=gpu)
    out = torch.full((R, L, 2, K, ROW), 0x5a, dtype=torch.uint8, device=gpu)
    cases = [
        (dict(out=out[:, :, :1]), ValueError, r"output leading shape \(5, 3, 1, 256\) != \(5, 3, 2, 256\)"),
        (dict(out=out[..., :ROW // 2]), ValueError, "output rows hold 32 bytes, pool rows 64"),
        (dict(out=out[..., ::2]), ValueError, "output rows hold 32 bytes"),
        (dict(out=torch.zeros((R, L, 2, K, 2 * ROW), dtype=torch.uint8, device=gpu)[..., ::2]), ValueError,
         "output rows must be contiguous"),
        (dict(host_planes=(host_planes,)), TypeError, "must be KVPlanes"),
        (dict(lengths=lengths.cpu()), ValueError, "share one device"),
    ]
    for change, error, message in cases:
        arguments = dict(topk=topk, rows=rows, lengths=lengths, buffers=side.buffers, host_table=host_table,
                         host_planes=host_planes, pool_planes=side.planes, slots=slots, output=out)
        arguments.update({("output" if k == "out" else k): v for k, v in change.items()})
        with pytest.raises(error, match=message):
            decode_step(**arguments)
    torch.cuda.synchronize()
    assert bool((slots == -9).all()) and bool((out == 0x5a).all())
    assert side.buffers.step == 0
