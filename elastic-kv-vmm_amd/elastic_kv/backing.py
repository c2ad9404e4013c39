"""Demand-backed HIP virtual KV range with a stable torch view.

Drop-in for the reference's elastic_kv/backing.py: the Backing class keeps
its constructor, properties, methods, metric names and error behaviour
(Backing :114-545, library loading :19-52, unreferenced teardown :90-111).
The native object is libelastic_vmm.so's ev_* ABI (csrc/vmm_backing.hip over
csrc/vmm_core.h: hipMemAddressReserve / hipMemCreate / hipMemMap /
hipMemSetAccess), and the raw view is a DLPack capsule of device type
kDLROCM built by _dlpack instead of a CuPy array.

How this module is organised:
  * _NativeObject owns one ev_* handle and turns every failing call into a
    _NativeFailure that carries the native message and whether the object is
    poisoned (a failed batch that could not be rolled back);
  * Backing keeps one dict of committed chunks, each either READY or ZEROING
    (precommitted: its zero fill may still run until the next ensure), and
    counts its calls, chunks and nanoseconds per operation;
  * teardown is a weakref finalizer over the _NativeObject, not the Backing,
    so an unreferenced Backing still releases its reservation.

The reference's cross-process capacity broker is not part of this library:
asking for it through the environment raises, and the broker queries answer
"no broker".
"""

import ctypes as ct
import functools
import operator
import os
import time
import weakref
from contextlib import contextmanager
from pathlib import Path

import torch

from . import _dlpack

DEFAULT_CHUNK_BYTES = 2 << 20
_INVALID = (1 << 64) - 1
_PACKAGE_ROOT = Path(__file__).resolve().parents[1]
DEFAULT_LIBRARY = _PACKAGE_ROOT / "lib" / "libelastic_vmm.so"
BUILD_HINT = (
    "Build it with `python elastic-kv-vmm_amd/build_native.py` (the counterpart of the reference's "
    "elastic-kv-build-vmm) or set ELASTIC_VMM_LIBRARY"
)
_BROKER_VARIABLES = ("EKV_GLOBAL_BROKER_PATH", "EKV_GLOBAL_BROKER_MIB", "EKV_GLOBAL_BROKER_FAIR_MODE")

_U64 = ct.c_uint64
_ID_LIST = ct.POINTER(ct.c_uint64)
# (ctypes argtypes, restype) of every ev_* symbol; the queries and ev_poisoned
# came last in the ABI's history, so their absence means an outdated build.
_CORE_SYMBOLS = {
    "ev_create": ([ct.c_int, _U64, _U64], ct.c_void_p),
    "ev_ensure": ([ct.c_void_p, _ID_LIST, ct.c_size_t], ct.c_int),
    "ev_precommit": ([ct.c_void_p, _ID_LIST, ct.c_size_t], ct.c_int),
    "ev_drop": ([ct.c_void_p, _ID_LIST, ct.c_size_t], ct.c_int),
    "ev_close": ([ct.c_void_p], ct.c_int),
    "ev_error": ([], ct.c_char_p),
}
_QUERY_SYMBOLS = {
    "ev_base": ([ct.c_void_p], _U64),
    "ev_backed": ([ct.c_void_p], _U64),
    "ev_reserved": ([ct.c_void_p], _U64),
    "ev_granularity": ([ct.c_void_p], _U64),
    "ev_poisoned": ([ct.c_void_p], ct.c_int),
}
# The spare pool (this library's extension of the ABI); a library without it
# serves Backings whose spare limit stays 0.
_SPARE_SYMBOLS = {
    "ev_set_spare": ([ct.c_void_p, _U64], ct.c_int),
    "ev_spare": ([ct.c_void_p], _U64),
}


def _declare(lib, symbols):
    for name, (argtypes, restype) in symbols.items():
        entry = getattr(lib, name)
        entry.argtypes = argtypes
        entry.restype = restype


@functools.lru_cache(maxsize=None)
def _load_library(path):
    """The native library at `path` with the ev_* signatures declared; errors name the build step."""
    try:
        lib = ct.CDLL(path)
    except OSError as exc:
        raise RuntimeError(
            f"HIP VMM library could not be loaded. {BUILD_HINT}. "
            f"Library={path}; sources={_PACKAGE_ROOT / 'csrc'}"
        ) from exc
    _declare(lib, _CORE_SYMBOLS)
    try:
        _declare(lib, _QUERY_SYMBOLS)
    except AttributeError as exc:
        raise RuntimeError("HIP VMM library ABI is outdated; rebuild libelastic_vmm.so. " + BUILD_HINT) from exc
    try:
        _declare(lib, _SPARE_SYMBOLS)
    except AttributeError:
        pass
    return lib


def library_path(library=None):
    """The native library to load: the argument, else ELASTIC_VMM_LIBRARY, else the in-tree build."""
    chosen = library if library is not None else os.environ.get("ELASTIC_VMM_LIBRARY", DEFAULT_LIBRARY)
    return str(Path(chosen).expanduser().resolve())


class _NativeFailure(RuntimeError):
    def __init__(self, message, poisoned):
        super().__init__(message)
        self.poisoned = poisoned


class _NativeObject:
    """One ev_* object. close() is idempotent; a failed close keeps the handle so it can be retried."""

    def __init__(self, lib, device, capacity_bytes, chunk_bytes):
        self.lib = lib
        self.handle = lib.ev_create(device, capacity_bytes, chunk_bytes)
        if not self.handle:
            raise RuntimeError(self.message())

    def message(self):
        return self.lib.ev_error().decode("utf-8", errors="replace")

    def query(self, name):
        if not self.handle:
            raise RuntimeError("VMM backing is closed")
        value = getattr(self.lib, name)(self.handle)
        if value == _INVALID:
            raise RuntimeError(self.message())
        return value

    def run(self, name, ids):
        """ev_ensure / ev_precommit / ev_drop over `ids` (sorted); raises _NativeFailure."""
        array = (ct.c_uint64 * len(ids))(*ids)
        if getattr(self.lib, name)(self.handle, array, len(ids)):
            message = self.message()
            try:
                state = self.lib.ev_poisoned(self.handle)
            except Exception:   # an unreadable state counts as poisoned
                state = -1
            raise _NativeFailure(message, state != 0)

    def close(self):
        """None once closed, else the native failure message."""
        if self.handle and self.lib.ev_close(self.handle):
            return self.message() or "native VMM close failed"
        self.handle = None
        return None


READY, ZEROING = "ready", "zeroing"
_METRIC_NAMES = ("ensure_calls", "ensure_chunks", "ensure_ns", "precommit_calls", "precommit_chunks",
                 "precommit_ns", "reclaim_calls", "reclaim_chunks", "reclaim_ns", "reclaim_sync_ns",
                 "peak_backed_bytes")


class Backing:
    """One stable HIP virtual reservation, owned by a single scheduler thread.

    A tensor returned by raw can span unmapped addresses: the caller must
    ensure every chunk a read or write touches. reclaim() waits for the device
    by default, and the caller must keep future work away from a reclaimed
    chunk until it is ensured again.
    """

    def __init__(self, capacity_bytes, chunk_bytes=DEFAULT_CHUNK_BYTES, device=0, library=None, spare_chunks=0):
        self.capacity_bytes = operator.index(capacity_bytes)
        self.chunk_bytes = operator.index(chunk_bytes)
        if not all(0 < value < _INVALID for value in (self.capacity_bytes, self.chunk_bytes)):
            raise ValueError("capacity_bytes and chunk_bytes must be positive uint64 values")
        target = torch.device(f"cuda:{device}" if isinstance(device, int) else device)
        if target.type != "cuda":
            raise ValueError("VMM backing requires a GPU device")
        asked = [name for name in _BROKER_VARIABLES if os.environ.get(name) not in (None, "", "0", "off")]
        if asked:
            raise ValueError("the cross-process VMM capacity broker is not part of this library; unset "
                             + ", ".join(asked))
        self.device = torch.cuda.current_device() if target.index is None else target.index
        self._native = _NativeObject(_load_library(library_path(library)), self.device, self.capacity_bytes,
                                     self.chunk_bytes)
        self._finalizer = weakref.finalize(self, self._native.close)
        self._finalizer.atexit = False
        self.base = self._native.query("ev_base")
        self.reserved_bytes = self._native.query("ev_reserved")
        self.granularity = self._native.query("ev_granularity")
        self._chunks = {}          # committed chunk id -> READY | ZEROING
        self._raw_ref = None
        self._poisoned = False
        self._metrics = dict.fromkeys(_METRIC_NAMES, 0)
        self.spare_chunks = 0
        if spare_chunks:
            self.set_spare_chunks(spare_chunks)

    # ---------------------------------------------------------------- state

    @property
    def chunk_count(self):
        return self.reserved_bytes // self.chunk_bytes

    @property
    def mapped_chunks(self):
        """Committed chunks whose zero fill is known to be complete."""
        return frozenset(chunk for chunk, state in self._chunks.items() if state == READY)

    @property
    def backed_bytes(self):
        return self._native.query("ev_backed")

    @property
    def spare_bytes(self):
        """Physical memory the spare pool holds (reclaimed chunks kept for the next commits)."""
        return self._native.query("ev_spare") if self.spare_chunks else 0

    @property
    def metrics(self):
        """Counters plus the memory picture: backed (mapped) bytes, the spare pool's bytes
        (unmapped but still held), their sum held_bytes, and the reservation."""
        backed, spare = self.backed_bytes, self.spare_bytes
        return {**self._metrics, "backed_bytes": backed, "spare_bytes": spare, "held_bytes": backed + spare,
                "reserved_bytes": self.reserved_bytes}

    def set_spare_chunks(self, count):
        """Keep up to `count` reclaimed chunks' physical memory for the next commits (0: release at once).

        An extension of the reference's Backing: a reclaim then unmaps without
        releasing, and an ensure or precommit maps a kept chunk (zero-filled
        as usual) instead of creating one, which saves two driver calls per
        recycled chunk. The memory stays held (spare_bytes) until a commit
        takes it, the limit is lowered or the backing closes.
        """
        count = operator.index(count)
        if not 0 <= count <= self.chunk_count:
            raise ValueError("spare_chunks must be between 0 and the reservation's chunk count")
        self._usable()
        if not hasattr(self._native.lib, "ev_set_spare"):
            if count:
                raise RuntimeError("this VMM library has no spare pool (ev_set_spare); " + BUILD_HINT)
            return
        if self._native.lib.ev_set_spare(self._native.handle, count):
            message = self._native.message()
            self._poisoned = self._poisoned or self._native.lib.ev_poisoned(self._native.handle) != 0
            raise RuntimeError(message)
        self.spare_chunks = count

    def _usable(self):
        if not self._native.handle or self._poisoned:
            raise RuntimeError("VMM backing is closed or has encountered a HIP error")

    def _chunk_ids(self, indices):
        ids = {operator.index(index) for index in indices}
        if ids and not (0 <= min(ids) and max(ids) < self.chunk_count):
            raise ValueError("chunk index outside reserved range")
        return ids

    @contextmanager
    def _timed(self, operation, chunks):
        """Count one call of `operation` over `chunks` chunks, if the body succeeds."""
        start = time.perf_counter_ns()
        yield start
        self._metrics[operation + "_ns"] += time.perf_counter_ns() - start
        self._metrics[operation + "_calls"] += 1
        self._metrics[operation + "_chunks"] += chunks

    def _native_batch(self, name, ids):
        try:
            self._native.run(name, ids)
        except _NativeFailure as failure:
            # A clean rollback leaves the object retryable; anything else is fail-stop.
            self._poisoned = self._poisoned or failure.poisoned
            raise RuntimeError(str(failure)) from None

    def _note_peak(self):
        backed = len(self._chunks) * self.chunk_bytes
        self._metrics["peak_backed_bytes"] = max(self._metrics["peak_backed_bytes"], backed)

    # ---------------------------------------------------------------- residency

    def ensure(self, indices):
        """Commit and zero the missing chunks (and wait for earlier precommits); returns how many were new."""
        self._usable()
        ids = self._chunk_ids(indices)
        missing = sorted(ids - self._chunks.keys())
        waits = any(self._chunks.get(chunk) == ZEROING for chunk in ids)
        if not missing and not waits:
            return 0
        with self._timed("ensure", len(missing)):
            self._native_batch("ev_ensure", missing)
            # The native ensure waited for every zero fill this object started.
            self._chunks = dict.fromkeys(self._chunks.keys() | set(missing), READY)
        self._note_peak()
        return len(missing)

    def precommit(self, indices):
        """Map the missing chunks and start their zero fill without waiting.

        They become usable only after a later ``ensure`` (of any chunks) has
        waited for the fill; keep them out of kernel arguments until then.
        """
        self._usable()
        missing = sorted(self._chunk_ids(indices) - self._chunks.keys())
        if not missing:
            return 0
        with self._timed("precommit", len(missing)):
            self._native_batch("ev_precommit", missing)
            self._chunks.update(dict.fromkeys(missing, ZEROING))
        self._note_peak()
        return len(missing)

    def reclaim(self, indices, *, synchronize=True):
        """Release committed chunks; returns how many.

        synchronize=False requires the caller to have waited for every GPU
        access to them already.
        """
        self._usable()
        held = sorted(self._chunk_ids(indices) & self._chunks.keys())
        if not held:
            return 0
        with self._timed("reclaim", len(held)) as start:
            if synchronize:
                torch.cuda.synchronize(self.device)
                self._metrics["reclaim_sync_ns"] += time.perf_counter_ns() - start
            self._native_batch("ev_drop", held)
            for chunk in held:
                del self._chunks[chunk]
        return len(held)

    # ---------------------------------------------------------------- view and teardown

    @property
    def raw(self):
        """A contiguous uint8 tensor over the whole reservation (borrowed; keeps this Backing alive)."""
        self._usable()
        if self._chunks.get(0) != READY:
            raise RuntimeError("commit the sink chunk before building the tensor view")
        view = self._raw_ref() if self._raw_ref is not None else None
        if view is None:
            view = _dlpack.borrow_bytes(self.base, self.capacity_bytes, _dlpack.KDL_ROCM, self.device, self)
            if view.data_ptr() != self.base:
                raise RuntimeError("DLPack did not preserve the reserved address")
            self._raw_ref = weakref.ref(view)
        return view

    def close(self):
        """Release everything; call once no view, kernel or transfer can touch the range."""
        message = self._native.close()
        if message is not None:
            self._poisoned = True
            raise RuntimeError(f"native VMM teardown failed: {message}")
        self._finalizer.detach()
        self._chunks.clear()

    # ---------------------------------------------------------------- no broker in this library
    # The reference's broker queries and claims (elastic_kv/backing.py); callers written
    # against them see a backing without a broker.

    @property
    def has_global_broker(self):
        return False

    @property
    def broker_available_bytes(self):
        return None

    @property
    def broker_snapshot(self):
        return None

    def claim_broker_capacity(self, key, byte_count, *, kind="prefill"):
        return None

    def release_broker_claim(self, key, *, kind="prefill"):
        return 0

    def shrink_broker_claim(self, key, maximum_bytes, *, kind="prefill"):
        return None
