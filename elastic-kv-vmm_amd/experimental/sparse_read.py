"""Gather selected rows of a fixed-position virtual layout (HIP).

Drop-in for the reference's experimental/sparse_read.py:33-51 (gather_rows, a
Triton kernel): same arguments and checks; the rows are copied by the HIP
row-copy engine of csrc/gather.hip.
"""

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
    # Launch-bound (a few microseconds of GPU work): the launch helper describes
    # the tensors in C++ and calls ekv_gather_rows by address.
    helper, entries = _native.launch_helper()
    status = helper.gather_rows(entries["ekv_gather_rows"], raw, positions, request_ids, lengths,
                                request_table if indirect else None, slot_offsets if indirect else None, output,
                                layout.request_bytes // layout.itemsize, layout.chunk_bytes // layout.itemsize,
                                1 if indirect else 0)
    _native.launch_check(status, "gather_rows")
