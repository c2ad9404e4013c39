"""Top-K sparse KV reads from a chunked pool (HIP).

gather_rows is the reference's experimental/sparse_read.py:33-51 API (also
importable from experimental.sparse_read). gather_kv is its multi-plane form
for decode: the slot lists of every (layer, request) - as written by
resolve_resident - are read from the K and V planes of every layer in one
launch. scatter_kv is the inverse, used to unpack migrated rows.
"""

from math import prod

from elastic_kv import _native
from experimental.sparse_read import gather_rows  # noqa: F401  (re-export)

from .kv_pool import KVPlanes
from .profile_ranges import profile_range


def _planes_struct(planes):
    if not isinstance(planes, KVPlanes):
        raise TypeError("planes must be a KVPlanes")
    return _native.EkvPlanes(planes.base, planes.layers, planes.kv, planes.layer_stride,
                             planes.kv_stride, planes.row_stride, planes.row_bytes, planes.rows)


def _dense_struct(tensor, planes, slots, name):
    """EkvKvRows for a (B, L, KV, K, *row) tensor of planes.row_bytes rows."""
    if tensor.dim() < 4:
        raise ValueError(f"{name} must be shaped (B, L, KV, K, ...)")
    layers, batch, lanes = slots.shape
    expected = (batch, layers, planes.kv, lanes)
    if tuple(tensor.shape[:4]) != expected:
        raise ValueError(f"{name} leading shape {tuple(tensor.shape[:4])} != {expected}")
    item = tensor.element_size()
    tail = tensor.shape[4:]
    if prod(tail) * item != planes.row_bytes:
        raise ValueError(f"{name} rows hold {prod(tail) * item} bytes, pool rows {planes.row_bytes}")
    expect = 1
    for extent, stride in zip(reversed(tail), reversed(tensor.stride()[4:])):
        if extent > 1 and stride != expect:
            raise ValueError(f"{name} rows must be contiguous")
        expect *= extent
    s = tensor.stride()
    return _native.EkvKvRows(tensor.data_ptr(), s[1] * item, s[0] * item, s[2] * item, s[3] * item)


def _kv_call(entry, planes, slots, dense, zero_below, name):
    if not isinstance(planes, KVPlanes):
        raise TypeError("planes must be a KVPlanes")
    if slots.dim() != 3:
        raise ValueError("slots must be shaped [L, B, K]")
    if slots.shape[0] > planes.layers:
        raise ValueError("slots name more layers than the pool holds")
    if not slots.numel():
        if _native.device_of(slots, dense).index != planes.device:
            raise ValueError("slots and pool live on different devices")
        return
    # The launch helper checks the devices and the dense rows (those of _dense_struct) and builds the
    # descriptors in C++.
    helper, entries = _native.launch_helper()
    status = helper.kv(entries[entry], planes, slots, dense, int(zero_below), name)
    _native.launch_check(status, entry)


@profile_range("native/gather")
def gather_kv(planes, slots, output, *, zero_below=1):
    """output[b, l, kv, k] = plane(l, kv)[slots[l, b, k]] for valid slots.

    A slot is valid when zero_below <= slot < planes.rows; other lanes get
    zero rows (slot 0 is the sink / not resident, -1 is padding). slots may
    have stride 0 over layers to share one list across layers.
    """
    _kv_call("ekv_gather_kv", planes, slots, output, zero_below, "output")


@profile_range("native/scatter")
def scatter_kv(planes, slots, source, *, zero_below=1):
    """plane(l, kv)[slots[l, b, k]] = source[b, l, kv, k] for valid slots."""
    _kv_call("ekv_scatter_kv", planes, slots, source, zero_below, "source")
