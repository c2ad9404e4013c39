"""HiSparse hot-buffer swap-in with SGLang's calling convention, on the HIP kernel.

The reference's decode path hands host-backed rows to SGLang's
load_blocks_to_device_buffer_mha (through its HiSparse coordinator,
adaptive_sparse/request_residency.py:805-809,829-832; called directly in
tests/smoke_minimax_swap.py:38-67). This function takes the same keyword
arguments and runs ekv_hisparse_swap_in:
- the selected tokens of each row are its Top-K blocks expanded to tokens
  below seq_len, in Top-K order;
- the newest token (seq_len - 1) maps to the reserved slot
  device_buffer_locs[r, hot_buffer_size];
- a token held by a hot slot hits;
- misses take slots in batch-token LRU order (empty slots first), are copied
  from the pinned host cache and enter the hot state;
- top_k_device_locs receives the device locations in selection order,
  followed by -1.

The host cache must be pinned host memory (torch's pin_memory), which the
kernel reads through its device mapping. There is no CPU fallback.
"""

import ctypes as ct
from math import prod

from elastic_kv import _native

from .profile_ranges import profile_range

MAX_HOT = 4096
MAX_LANES = 2048


def _row_layout(first, second, name):
    """(row_bytes, row_stride_bytes, kv_stride_bytes, rows) of a K/V tensor pair."""
    if first.shape != second.shape or first.dtype != second.dtype or first.stride() != second.stride():
        raise ValueError(f"{name} K and V must share shape, dtype and strides")
    if first.dim() < 1 or first.shape[0] == 0:
        raise ValueError(f"{name} needs at least one row")
    item = first.element_size()
    expect = 1
    for extent, stride in zip(reversed(first.shape[1:]), reversed(first.stride()[1:])):
        if extent > 1 and stride != expect:
            raise ValueError(f"{name} rows must be contiguous")
        expect *= extent
    row_bytes = prod(first.shape[1:]) * item
    return row_bytes, first.stride(0) * item, second.data_ptr() - first.data_ptr(), first.shape[0]


def host_device_pointer(tensor):
    """Device address of a pinned host tensor's first byte."""
    if tensor.device.type != "cpu" or not tensor.is_pinned():
        raise ValueError("the host cache must be pinned CPU memory (pin_memory)")
    lib = _native.kernel_library()
    device = ct.c_void_p()
    _native.check(lib, lib.ekv_host_device_pointer(ct.c_void_p(tensor.data_ptr()), ct.byref(device)),
                  "host_device_pointer")
    return device.value


@profile_range("native/hisparse_swap")
def load_blocks_to_device_buffer_mha(top_k_blocks, device_buffer_tokens, host_cache_locs, device_buffer_locs,
                                     host_cache_k, host_cache_v, device_buffer_k, device_buffer_v,
                                     top_k_device_locs, req_pool_indices, seq_lens, lru_slots, item_size_bytes,
                                     hot_buffer_size, sparse_block_size, num_real_reqs=None):
    """Swap the selected blocks of every row into its hot buffer; see the module docstring.

    top_k_blocks [B, K]; device_buffer_tokens [R, >= H+1] int32;
    host_cache_locs [R, T]; device_buffer_locs [R, >= H+1]; lru_slots [R, H]
    int16/int32; top_k_device_locs [B, K * sparse_block_size] int32;
    req_pool_indices, seq_lens [B]; num_real_reqs [1] on the device (rows at
    or past it are padding) or None. host_cache_k/v: pinned CPU tensors
    [host rows, ...]; device_buffer_k/v: GPU tensors [device rows, ...]; both
    with rows of item_size_bytes. Updates the hot state in place; returns None.
    """
    # Called once per layer and step: the launch helper runs these checks (those of _row_layout and
    # host_device_pointer, in this order) and builds the descriptors in C++.
    helper, entries = _native.launch_helper()
    status = helper.hisparse(entries["ekv_hisparse_swap_in"], entries["ekv_host_device_pointer"], top_k_blocks,
                             device_buffer_tokens, host_cache_locs, device_buffer_locs, host_cache_k, host_cache_v,
                             device_buffer_k, device_buffer_v, top_k_device_locs, req_pool_indices, seq_lens,
                             lru_slots, int(item_size_bytes), int(hot_buffer_size), int(sparse_block_size),
                             num_real_reqs)
    _native.launch_check(status, "load_blocks_to_device_buffer_mha")
