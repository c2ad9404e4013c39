"""Gather selected rows of a fixed-position virtual layout (HIP).

Drop-in for the reference's experimental/sparse_read.py:33-51 (gather_rows, a
Triton kernel): same arguments and checks; the rows are copied by the HIP
row-copy engine of csrc/gather.hip.
"""

import ctypes as ct

from elastic_kv import _native


def gather_rows(raw, positions, request_ids, lengths, request_table, slot_offsets,
                output, layout, *, indirect):
    """Copy row `positions[b, s]` of request `request_ids[b]` into output[b, s].

    Rows with pos < 0 or pos >= lengths[b] are zero. Direct mode addresses
    raw by the layout (sink chunk + request region + pos * row_elements);
    indirect mode reads the ELEMENT offset slot_offsets[request_table[req,
    pos]]. All tensors are GPU tensors on one device; output is contiguous in
    its last dimension and has raw's dtype.
    """
    batch, selected = positions.shape
    if output.shape != (batch, selected, layout.row_elements):
        raise ValueError("output shape does not match positions and row width")
    if not batch or not selected:
        return
    tensors = [raw, positions, request_ids, lengths, output]
    if indirect:
        tensors += [request_table, slot_offsets]
    device = _native.device_of(*tensors)
    lib = _native.kernel_library()
    views = [_native.describe(t, n) for t, n in (
        (raw, "raw"), (positions, "positions"), (request_ids, "request_ids"),
        (lengths, "lengths"))]
    table_view = ct.byref(_native.describe(request_table, "request_table")) if indirect else None
    offsets_view = ct.byref(_native.describe(slot_offsets, "slot_offsets")) if indirect else None
    out_view = _native.describe(output, "output")
    with _native.on_device(device):
        status = lib.ekv_gather_rows(
            ct.byref(views[0]), ct.byref(views[1]), ct.byref(views[2]), ct.byref(views[3]),
            table_view, offsets_view, ct.byref(out_view),
            layout.request_bytes // layout.itemsize, layout.chunk_bytes // layout.itemsize,
            1 if indirect else 0, _native.stream_handle(device))
    _native.check(lib, status, "gather_rows")
