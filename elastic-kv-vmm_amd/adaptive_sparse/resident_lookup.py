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
    carry it too), so all layers of a decode step resolve in one launch;
  * resident_bits / bits_shift (single level only): a residency summary
    built by build_residency_bits, one bit per group of 2**bits_shift
    positions (0: per position; 6: per 128-byte line of an int16 table);
    lanes whose group bit is clear skip their table read. A summary may be a
    superset of the table's residency (a set bit over unresident positions
    only costs their table reads), never a subset;
  * slot_base (single level only): the table is int16 and holds local slots
    (0 = not resident, v >= 1 = local slot v - 1 of the request); the slot
    written is slot_base[rows[r]] + v - 1. Half the bytes of an int32 table
    of global slots, with the same output.
"""

import ctypes as ct

import torch

from elastic_kv import _native

from .profile_ranges import profile_range


@profile_range("native/lookup")
def resolve_resident(topk, table, mapping, rows, lengths, selected, output, block_size, *,
                     misses=None, miss_count=None, resident_bits=None, bits_shift=0, slot_base=None):
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
    if resident_bits is not None and mapping is not None:
        raise ValueError("resident_bits needs the single-level form (mapping=None)")
    if (slot_base is not None) != (table.dtype == torch.int16):
        raise ValueError("an int16 table holds local slots and needs slot_base (and only it)")
    if slot_base is not None and mapping is not None:
        raise ValueError("slot_base needs the single-level form (mapping=None)")
    # The call is bound by its host launch cost: the launch helper describes the
    # tensors in C++ (device checks, descriptors, torch's current stream) and
    # calls the entry point by address.
    helper, entries = _native.launch_helper()
    if slot_base is not None:
        form, entry = 2, entries["ekv_resolve_resident_local"]
    elif resident_bits is not None:
        form, entry = 1, entries["ekv_resolve_resident_bits"]
    else:
        form, entry = 0, entries["ekv_resolve_resident"]
    status = helper.resolve(form, entry, topk, table, mapping, slot_base, resident_bits, int(bits_shift), rows,
                            lengths, selected, output, misses, miss_count, int(block_size))
    _native.launch_check(status, "resolve_resident")


def summary_words(context, shift=0):
    """int32 words per row of a residency summary over `context` positions, in whole 16-byte pieces."""
    groups = -(-context // (1 << shift))
    return -(-(-(-groups // 32)) // 4) * 4


def build_residency_bits(table, out=None, shift=0):
    """Exact residency summary of a single-level table.

    Bit q of row r is set when any position in [q << shift, (q + 1) << shift)
    of table[.., r, :] is non-zero (shift 0: bit p = table[.., r, p] != 0).
    Returns an int32 tensor [.., R, W] (or fills `out`, which needs at least
    ceil(ceil(T / 2**shift) / 32) words per row). W = summary_words(T, shift):
    ceil(ceil(T / 2**shift) / 32) rounded up to a multiple of 4, so every row
    is whole 16-byte pieces, and the words past the summary are zero, so the
    lookup can stage a row with 16-byte loads for any T.
    """
    if table.dim() not in (2, 3):
        raise ValueError("table must be [R, T] or [L, R, T]")
    if out is None:
        out = torch.zeros((*table.shape[:-1], summary_words(table.shape[-1], shift)), dtype=torch.int32,
                          device=table.device)
    device = _native.device_of(table, out)
    lib = _native.kernel_library()
    table_view, out_view = _native.describe(table, "table"), _native.describe(out, "resident_bits")
    with _native.on_device(device):
        status = lib.ekv_residency_bits(ct.byref(table_view), ct.byref(out_view), int(shift),
                                        _native.stream_handle(device))
    _native.check(lib, status, "build_residency_bits")
    return out
