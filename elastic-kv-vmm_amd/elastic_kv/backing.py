"""HIP VMM backing with stable torch views and explicit residency control.

Drop-in for the reference's elastic_kv/backing.py (Backing :114-545,
_load_library :19-52, _BackingLifecycle :90-111). The native side is
libelastic_vmm.so built from csrc/vmm_backing.hip (same ev_* ABI, on
hipMemAddressReserve / hipMemCreate / hipMemMap / hipMemSetAccess). The raw
view is a DLPack capsule of device type kDLROCM built here instead of a CuPy
array. The cross-process SQLite capacity broker of the reference
(elastic_kv/global_broker.py) is not part of this build: asking for it through
the environment raises, and the broker query methods report "no broker".
"""

import ctypes as ct
import functools
import operator
import os
import time
import weakref
from pathlib import Path

import torch

from . import _dlpack

DEFAULT_CHUNK_BYTES = 2 << 20
_INVALID = (1 << 64) - 1
_PACKAGE_ROOT = Path(__file__).resolve().parents[1]
DEFAULT_LIBRARY = _PACKAGE_ROOT / "lib" / "libelastic_vmm.so"
BUILD_HINT = (
    "Build it with `python elastic-kv-vmm_amd/build_native.py` (the elastic-kv-build-vmm "
    "step of this build) or set ELASTIC_VMM_LIBRARY"
)
_BROKER_VARIABLES = ("EKV_GLOBAL_BROKER_PATH", "EKV_GLOBAL_BROKER_MIB", "EKV_GLOBAL_BROKER_FAIR_MODE")


@functools.lru_cache(maxsize=None)
def _load_library(path):
    """Load and type the native library; errors name the build step."""
    try:
        lib = ct.CDLL(path)
    except OSError as exc:
        raise RuntimeError(
            f"HIP VMM library could not be loaded. {BUILD_HINT}. "
            f"Library={path}; sources={_PACKAGE_ROOT / 'csrc'}"
        ) from exc
    lib.ev_create.argtypes = [ct.c_int, ct.c_uint64, ct.c_uint64]
    lib.ev_create.restype = ct.c_void_p
    for name in ("ev_ensure", "ev_precommit", "ev_drop"):
        fn = getattr(lib, name)
        fn.argtypes = [ct.c_void_p, ct.POINTER(ct.c_uint64), ct.c_size_t]
        fn.restype = ct.c_int
    try:
        for name in ("ev_base", "ev_backed", "ev_reserved", "ev_granularity"):
            fn = getattr(lib, name)
            fn.argtypes = [ct.c_void_p]
            fn.restype = ct.c_uint64
        lib.ev_poisoned.argtypes = [ct.c_void_p]
        lib.ev_poisoned.restype = ct.c_int
    except AttributeError as exc:
        raise RuntimeError(
            "HIP VMM library ABI is outdated; rebuild libelastic_vmm.so. " + BUILD_HINT
        ) from exc
    lib.ev_close.argtypes = [ct.c_void_p]
    lib.ev_close.restype = ct.c_int
    lib.ev_error.argtypes = []
    lib.ev_error.restype = ct.c_char_p
    return lib


def library_path(library=None):
    """Resolve the native library path (argument, ELASTIC_VMM_LIBRARY, default)."""
    if library is None:
        library = os.environ.get("ELASTIC_VMM_LIBRARY", DEFAULT_LIBRARY)
    return str(Path(library).expanduser().resolve())


class _BackingLifecycle:
    """Own native teardown without retaining the Backing object."""

    def __init__(self, library, handle):
        self.library = library
        self.handle = handle

    def close(self):
        if self.handle:
            if self.library.ev_close(self.handle):
                error = self.library.ev_error().decode("utf-8", errors="replace")
                return "native", error or "native VMM close failed"
            self.handle = None
        return "closed", None


class Backing:
    """Single scheduler-thread owner of one HIP virtual reservation.

    A tensor returned by raw can span unmapped addresses. Before reading or
    writing a tensor range, the caller must ensure every chunk it touches is
    mapped. reclaim() waits on the device by default, but the caller must also
    ensure no future work can access that chunk until it is ensured again.
    """

    def __init__(self, capacity_bytes, chunk_bytes=DEFAULT_CHUNK_BYTES, device=0, library=None):
        self.capacity_bytes = operator.index(capacity_bytes)
        self.chunk_bytes = operator.index(chunk_bytes)
        if not (0 < self.capacity_bytes < _INVALID and 0 < self.chunk_bytes < _INVALID):
            raise ValueError("capacity_bytes and chunk_bytes must be positive uint64 values")
        device = torch.device(f"cuda:{device}" if isinstance(device, int) else device)
        if device.type != "cuda":
            raise ValueError("VMM backing requires a GPU device")
        requested = [name for name in _BROKER_VARIABLES
                     if os.environ.get(name) not in (None, "", "0", "off")]
        if requested:
            raise ValueError(
                "the cross-process VMM capacity broker is not part of this build; unset "
                + ", ".join(requested)
            )
        self.device = torch.cuda.current_device() if device.index is None else device.index
        self._lib = _load_library(library_path(library))
        self._handle = self._lib.ev_create(self.device, self.capacity_bytes, self.chunk_bytes)
        if not self._handle:
            raise RuntimeError(self._error())
        self._lifecycle = _BackingLifecycle(self._lib, self._handle)
        self._finalizer = weakref.finalize(self, self._lifecycle.close)
        self._finalizer.atexit = False
        self.base = self._number("ev_base")
        self.reserved_bytes = self._number("ev_reserved")
        self.granularity = self._number("ev_granularity")
        self._mapped = set()
        self._precommitted = set()
        self._raw_ref = None
        self._poisoned = False
        self._metrics = dict.fromkeys((
            "ensure_calls", "ensure_chunks", "ensure_ns",
            "precommit_calls", "precommit_chunks", "precommit_ns",
            "reclaim_calls", "reclaim_chunks", "reclaim_ns", "reclaim_sync_ns",
            "peak_backed_bytes",
        ), 0)

    def _error(self):
        return self._lib.ev_error().decode("utf-8", errors="replace")

    def _number(self, name):
        if not self._handle:
            raise RuntimeError("VMM backing is closed")
        value = getattr(self._lib, name)(self._handle)
        if value == _INVALID:
            raise RuntimeError(self._error())
        return value

    def _check(self):
        if not self._handle or self._poisoned:
            raise RuntimeError("VMM backing is closed or has encountered a HIP error")

    @property
    def chunk_count(self):
        return self.reserved_bytes // self.chunk_bytes

    def _ids(self, indices):
        ids = {operator.index(index) for index in indices}
        limit = self.chunk_count
        if any(index < 0 or index >= limit for index in ids):
            raise ValueError("chunk index outside reserved range")
        return ids

    def _batch(self, name, indices):
        ids = (ct.c_uint64 * len(indices))(*sorted(indices))
        if getattr(self._lib, name)(self._handle, ids, len(indices)):
            error = self._error()
            try:
                poisoned = self._lib.ev_poisoned(self._handle)
            except Exception:
                poisoned = -1
            if poisoned != 0:
                self._poisoned = True
            raise RuntimeError(error)

    @property
    def mapped_chunks(self):
        return frozenset(self._mapped - self._precommitted)

    @property
    def backed_bytes(self):
        return self._number("ev_backed")

    @property
    def metrics(self):
        return {**self._metrics, "backed_bytes": self.backed_bytes,
                "reserved_bytes": self.reserved_bytes}

    # The reference's cross-process broker hooks; this build has no broker.
    @property
    def broker_available_bytes(self):
        return None

    @property
    def broker_snapshot(self):
        return None

    @property
    def has_global_broker(self):
        return False

    def claim_broker_capacity(self, key, byte_count, *, kind="prefill"):
        return None

    def release_broker_claim(self, key, *, kind="prefill"):
        return 0

    def shrink_broker_claim(self, key, maximum_bytes, *, kind="prefill"):
        return None

    @property
    def raw(self):
        """Borrow a contiguous uint8 view spanning the logical reservation."""
        self._check()
        if 0 not in self.mapped_chunks:
            raise RuntimeError("commit the sink chunk before building the tensor view")
        cached = self._raw_ref() if self._raw_ref else None
        if cached is not None:
            return cached
        raw = _dlpack.borrow_bytes(self.base, self.capacity_bytes, _dlpack.KDL_ROCM, self.device, self)
        if raw.data_ptr() != self.base:
            raise RuntimeError("DLPack did not preserve the reserved address")
        self._raw_ref = weakref.ref(raw)
        return raw

    def ensure(self, indices):
        """Commit and zero missing chunks, returning their count."""
        self._check()
        ids = self._ids(indices)
        pending = ids - self._mapped
        needs_initialization = pending or bool(ids & self._precommitted)
        if not needs_initialization:
            return 0
        start = time.perf_counter_ns()
        self._batch("ev_ensure", pending)
        self._mapped.update(pending)
        self._precommitted.clear()
        self._metrics["ensure_ns"] += time.perf_counter_ns() - start
        self._metrics["ensure_calls"] += 1
        self._metrics["ensure_chunks"] += len(pending)
        self._metrics["peak_backed_bytes"] = max(
            self._metrics["peak_backed_bytes"], len(self._mapped) * self.chunk_bytes
        )
        return len(pending)

    def precommit(self, indices):
        """Map missing chunks and start zeroing without blocking the caller.

        The chunks become usable only after a later ``ensure`` waits for the
        initialization stream. Callers must keep them out of kernel argument
        lists until then.
        """
        self._check()
        pending = self._ids(indices) - self._mapped
        if not pending:
            return 0
        start = time.perf_counter_ns()
        self._batch("ev_precommit", pending)
        self._mapped.update(pending)
        self._precommitted.update(pending)
        self._metrics["precommit_ns"] += time.perf_counter_ns() - start
        self._metrics["precommit_calls"] += 1
        self._metrics["precommit_chunks"] += len(pending)
        self._metrics["peak_backed_bytes"] = max(
            self._metrics["peak_backed_bytes"], len(self._mapped) * self.chunk_bytes
        )
        return len(pending)

    def reclaim(self, indices, *, synchronize=True):
        """Release idle chunks, returning their count.

        synchronize=False requires the caller to have already waited for all
        in-flight GPU accesses to the affected ranges.
        """
        self._check()
        pending = self._ids(indices) & self._mapped
        if not pending:
            return 0
        start = time.perf_counter_ns()
        if synchronize:
            torch.cuda.synchronize(self.device)
            self._metrics["reclaim_sync_ns"] += time.perf_counter_ns() - start
        self._batch("ev_drop", pending)
        self._mapped.difference_update(pending)
        self._precommitted.difference_update(pending)
        self._metrics["reclaim_ns"] += time.perf_counter_ns() - start
        self._metrics["reclaim_calls"] += 1
        self._metrics["reclaim_chunks"] += len(pending)
        return len(pending)

    def close(self):
        """Close once no tensor view, kernel, or transfer can access backing."""
        stage, message = self._lifecycle.close()
        if stage != "closed":
            self._poisoned = True
            raise RuntimeError(f"{stage} VMM teardown failed: {message}")
        self._handle = None
        self._finalizer.detach()
        self._mapped.clear()
        self._precommitted.clear()
