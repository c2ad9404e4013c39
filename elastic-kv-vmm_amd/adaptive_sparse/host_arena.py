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
