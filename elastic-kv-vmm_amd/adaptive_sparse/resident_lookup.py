"""Resolve Top-K selected blocks of resident decode rows to device slots (HIP).

Drop-in for the reference's adaptive_sparse/resident_lookup.py:29-40
(resolve_resident, a Triton kernel). Same arguments, same in-place contract:
only the `selected` rows of `output` are written, any strides are accepted,
and an empty selection or zero width launches nothing. The work runs in the
HIP kernel of csrc/lookup.hip; there is no Python or torch fallback.

Extensions (all optional, none changes the reference behaviour):
  * misses / miss_count: per row, the lanes whose slot is 0 (valid but not
    resident) in ascending lane order, and their number;
  * mapping=None: single-level lookup, the table value is the slot itself;
  * a leading layer dimension L on topk / output (table and mapping may then
    carry it too), so all layers of a decode step resolve in one launch.
"""

import ctypes as ct

import torch

from elastic_kv import _native


def resolve_resident(topk, table, mapping, rows, lengths, selected, output, block_size, *,
                     misses=None, miss_count=None):
    """Write only selected rows into an existing [L, B, K * block_size] tensor.

    For selected row r, layer l and lane o: block = topk[l, r, o // bs],
    pos = block * bs + o % bs; the lane is valid when block >= 0 and
    pos < lengths[r]; output[l, r, o] = int32(mapping[table[rows[r], pos]])
    for valid lanes and -1 otherwise. With misses/miss_count given,
    misses[l, r, :miss_count[l, r]] lists the valid lanes whose slot is 0.
    """
    width = topk.shape[2] * block_size
    if not selected.numel() or not width:
        return
    if (misses is None) != (miss_count is None):
        raise ValueError("misses and miss_count must be given together")
    tensors = [topk, table, rows, lengths, selected, output]
    if mapping is not None:
        tensors.append(mapping)
    if misses is not None:
        tensors += [misses, miss_count]
    device = _native.device_of(*tensors)
    lib = _native.kernel_library()
    views = [_native.describe(t, name) for t, name in (
        (topk, "topk"), (table, "table"), (rows, "rows"), (lengths, "lengths"),
        (selected, "selected"), (output, "output"))]
    mapping_view = ct.byref(_native.describe(mapping, "mapping")) if mapping is not None else None
    miss_view = ct.byref(_native.describe(misses, "misses")) if misses is not None else None
    count_view = ct.byref(_native.describe(miss_count, "miss_count")) if miss_count is not None else None
    with torch.cuda.device(device):
        status = lib.ekv_resolve_resident(
            ct.byref(views[0]), ct.byref(views[1]), mapping_view, ct.byref(views[2]),
            ct.byref(views[3]), ct.byref(views[4]), ct.byref(views[5]), miss_view, count_view,
            int(block_size), _native.stream_handle(device))
    _native.check(lib, status, "resolve_resident")
