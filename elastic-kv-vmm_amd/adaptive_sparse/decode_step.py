"""One decode step in one native call: lookup, LRU swap-in, promote from host, gather.

The sequence of the reference's decode path per layer
(adaptive_sparse/request_residency.py:805-832: resolve the Top-K blocks,
swap the missing ones in from the host copy, then read the selected rows),
as the single entry point ekv_decode_step of csrc/decode_step.hip. Its
intermediates (the miss list and counts, the promotion lists) live in a
device workspace: pass one (decode_step_workspace gives its size) to keep a
serving loop or a captured graph free of allocations, or let the call take
one from torch's caching allocator.
"""

import ctypes as ct

import torch

from elastic_kv import _native

from .kv_pool import KVPlanes
from .profile_ranges import profile_range
from .sparse_read import _dense_struct, _planes_struct
from .swap_in import STEP_STAMPS

_P_TENSOR = ct.POINTER(_native.EkvTensor)


class StepArgs(ct.Structure):
    """ekv_step_args of include/ekv_kernels.h."""

    _fields_ = [
        ("topk", _P_TENSOR), ("block_size", ct.c_int64), ("rows", _P_TENSOR), ("lengths", _P_TENSOR),
        ("selected", _P_TENSOR), ("table", _P_TENSOR), ("resident_bits", _P_TENSOR), ("bits_shift", ct.c_int64),
        ("resident_counts", _P_TENSOR), ("slot_base", _P_TENSOR), ("slot_token", _P_TENSOR), ("stamps", _P_TENSOR),
        ("step", ct.c_int64),
        ("step_counter", _P_TENSOR), ("status", _P_TENSOR), ("host_table", _P_TENSOR),
        ("host", ct.POINTER(_native.EkvPlanes)), ("pool", ct.POINTER(_native.EkvPlanes)), ("slots", _P_TENSOR),
        ("out", ct.POINTER(_native.EkvKvRows)),
    ]


def decode_step_workspace(layers, batch, width):
    """Bytes of workspace a step over layers x batch rows x width lanes needs."""
    lib = _native.kernel_library()
    size = lib.ekv_decode_step_workspace_bytes(int(layers), int(batch), int(width))
    if size == (1 << 64) - 1:
        raise ValueError(lib.ev_error().decode())
    return size


def step_args(topk, rows, lengths, selected, buffers, host_table, host_planes, pool_planes, slots, output,
              block_size, step):
    """StepArgs over the given tensors, plus the descriptors it points to (keep them alive with it)."""
    for planes in (host_planes, pool_planes):
        if not isinstance(planes, KVPlanes):
            raise TypeError("host_planes and pool_planes must be KVPlanes")
    keep = []

    def ref(obj):
        keep.append(obj)
        return ct.pointer(obj)

    def tensor(t, name):
        return ref(_native.describe(t, name)) if t is not None else None

    args = StepArgs(
        topk=tensor(topk, "topk"), block_size=int(block_size), rows=tensor(rows, "rows"),
        lengths=tensor(lengths, "lengths"), selected=tensor(selected, "selected"),
        table=tensor(buffers.table, "table"), resident_bits=tensor(buffers.bits, "resident_bits"),
        bits_shift=int(buffers.bits_shift),
        resident_counts=tensor(getattr(buffers, "resident_counts", None), "resident_counts"),
        slot_base=tensor(buffers.slot_base, "slot_base"),
        slot_token=tensor(buffers.slot_token, "slot_token"), stamps=tensor(buffers.stamps, "stamps"),
        step=int(step), step_counter=tensor(buffers.step_counter if step < 0 else None, "step_counter"),
        status=tensor(buffers.status, "status"), host_table=tensor(host_table, "host_table"),
        host=ref(_planes_struct(host_planes)), pool=ref(_planes_struct(pool_planes)), slots=tensor(slots, "slots"),
        out=ref(_dense_struct(output, pool_planes, slots, "output")))
    return args, keep


@profile_range("native/decode_step")
def decode_step(topk, rows, lengths, buffers, host_table, host_planes, pool_planes, slots, output, *,
                block_size=1, selected=None, step=None, workspace=None):
    """Lookup -> swap-in -> promote -> gather for the selected rows of every layer of `topk`.

    topk [L, B, K]; rows, lengths [B]; selected [S]: batch rows in [0, B)
    (default: every batch row, 0 .. B - 1, built on each call: a serving
    loop passes one it keeps);
    buffers: the HotBuffers of the pool; host_table [R, T] and host_planes:
    the pinned host copy (device-mapped); pool_planes: the hot pool; slots
    [L, B, K * block_size] int32 and output [B, L, KV, K * block_size, row]:
    the results (every selected lane's slot after the swap-in, and its row).
    The LRU step follows swap_in's rules (the device counter when buffers
    has one and no step is given). Refused rows show in buffers.status.
    """
    L, B = topk.shape[0], topk.shape[1]
    width = topk.shape[2] * block_size
    if selected is None:
        selected = torch.arange(B, device=topk.device)
    counted = buffers.step_counter is not None and step is None
    if step is None and not counted:
        if (buffers.step + 1) * STEP_STAMPS >= (1 << 31):
            buffers.rebase()
        step = buffers.step
    for planes in (host_planes, pool_planes):
        if not isinstance(planes, KVPlanes):
            raise TypeError("host_planes and pool_planes must be KVPlanes")
    if workspace is None:
        workspace = torch.empty(decode_step_workspace(L, B, width), dtype=torch.uint8, device=topk.device)
    # The launch helper checks the devices, builds the step's descriptors (those of step_args) in C++ and
    # calls ekv_decode_step: at small shapes the step's GPU work is shorter than building them in Python.
    helper, entries = _native.launch_helper()
    status = helper.decode_step(
        entries["ekv_decode_step"], topk, rows, lengths, selected, buffers.table, buffers.bits,
        int(buffers.bits_shift), getattr(buffers, "resident_counts", None), buffers.slot_base, buffers.slot_token,
        buffers.stamps, -1 if counted else int(step), buffers.step_counter if counted else None, buffers.status,
        host_table, host_planes, pool_planes, slots, output, int(block_size), workspace)
    _native.launch_check(status, "decode_step")
    if not counted:
        buffers.step = step + 1
