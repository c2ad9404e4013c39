"""Pinned host memory that HIP kernels read and write directly.

The host KV copy of demoted / host-backed tokens lives here. Kernels reach it
through the mapped device pointer (ekv_host_alloc: hipHostMalloc +
hipHostGetDevicePointer), so a promote is one gather kernel over PCIe instead
of a host-side pack followed by a copy.
"""

import ctypes as ct
import weakref

import torch

from elastic_kv import _dlpack, _native


def _release(lib, host_ptr):
    # Kernels may still read or write the memory: let the device drain first.
    if torch.cuda.is_initialized():
        torch.cuda.synchronize()
    lib.ekv_host_free(ct.c_void_p(host_ptr))


class HostArena:
    """`nbytes` of pinned, device-mapped host memory.

    `host` is a CPU uint8 tensor over the memory (keeps the arena alive);
    `device_ptr` is the address kernels use. Closing (or collecting) the
    arena synchronizes the device before freeing the memory; views of `host`
    taken by the caller must be dropped first.
    """

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        if self.nbytes <= 0:
            raise ValueError("arena size must be positive")
        self._lib = _native.kernel_library()
        host, device = ct.c_void_p(), ct.c_void_p()
        _native.check(self._lib, self._lib.ekv_host_alloc(self.nbytes, ct.byref(host), ct.byref(device)),
                      "ekv_host_alloc")
        self.host_ptr = host.value
        self.device_ptr = device.value
        self._finalizer = weakref.finalize(self, _release, self._lib, self.host_ptr)
        self.host = _dlpack.borrow_bytes(self.host_ptr, self.nbytes, _dlpack.KDL_CPU, 0, self)

    def close(self):
        self.host = None
        self._finalizer()


class HostKVCache:
    """Pinned host K/V token rows, plane-major: the host image of host-backed requests.

    `view` [layers, kv, rows, row_bytes] uint8 is the host tensor (torch's
    pinned memory, so SGLang-convention callers can pass per-layer slices as
    host_cache_k / host_cache_v); `planes` addresses the same rows through
    their device mapping for the kernels. Rows are handed out one per token
    (`alloc` / `free`), the role of SGLang's paged host token slots.
    """

    def __init__(self, layers, kv, rows, row_bytes):
        from elastic_kv.slots import FreeSlots

        from .hisparse_swap import host_device_pointer
        from .kv_pool import KVPlanes

        self.layers, self.kv, self.rows, self.row_bytes = layers, kv, rows, row_bytes
        self.view = torch.empty((layers, kv, rows, row_bytes), dtype=torch.uint8, pin_memory=True)
        plane = rows * row_bytes
        self.planes = KVPlanes(base=host_device_pointer(self.view), device=0, layers=layers, kv=kv,
                               layer_stride=kv * plane, kv_stride=plane, row_stride=row_bytes,
                               row_bytes=row_bytes, rows=rows, owner=self.view)
        self._free = FreeSlots(rows)

    def alloc(self, count):
        """int64 CPU tensor of `count` free rows (lowest first), or None when too few are free."""
        ranges = self._free.peek(count)
        if ranges is None:
            return None
        self._free.claim(ranges)
        return torch.tensor([r - 1 for a, b in ranges for r in range(a, b)], dtype=torch.int64)

    def free(self, rows):
        rows = sorted(int(r) + 1 for r in rows)
        if rows:
            self._free.release(rows)

    @property
    def free_rows(self):
        return self._free.count

    def layer(self, layer):
        """(K, V) pinned [rows, row_bytes] tensors of one layer."""
        return self.view[layer, 0], self.view[layer, 1]
