"""A single-threaded VMM arena of per-request resident KV prefixes.

The interface of the reference's experimental/resident_arena.py:4-92 (the
sink chunk is committed at construction; reserve grows a prefix;
resize_quiescent shrinks one after a device synchronization; row_view borrows
rows; a backing failure makes the arena refuse further use). Here each request
keeps the set of chunks it holds, and every change commits or releases the
difference between that set and the one the new length needs.
"""

from contextlib import contextmanager

OPEN, FAILED, CLOSED = "open", "failed", "closed"


class VmmResidentArena:
    """Views are borrowed: retire tail views before a shrink and all views before close().

    Rows newly exposed by a grow must be written before they are read - a
    chunk kept across a shrink may still hold bytes of the discarded tail.
    """

    def __init__(self, layout, device=0, backing_factory=None, *, synchronize=None):
        if layout.chunk_bytes % layout.itemsize:
            raise ValueError("chunk size must align to the element size")
        if backing_factory is None:
            from elastic_kv.backing import Backing as backing_factory
        self.layout = layout
        self.backing = backing_factory(layout.capacity_bytes, chunk_bytes=layout.chunk_bytes, device=device)
        self._synchronize = synchronize or self._device_synchronize
        self._lengths = [0] * layout.max_requests
        self._held = [frozenset()] * layout.max_requests
        self._state = OPEN
        self.backing.ensure({0})                     # the sink

    def _device_synchronize(self):
        import torch

        torch.cuda.synchronize(self.backing.device)

    @contextmanager
    def _backing_call(self):
        """Any failure of the backing (or of a synchronization) makes the arena unusable."""
        try:
            yield
        except Exception:
            self._state = FAILED
            raise

    def _usable(self):
        if self._state != OPEN:
            raise RuntimeError("arena is closed or has encountered a backing error")

    def length(self, req):
        return self._lengths[req]

    def reserve(self, req, length):
        """Grow request `req`'s mapped prefix to `length` rows (no-op if it is already that long)."""
        self._usable()
        needed = self.layout.prefix_chunks(req, length)
        if length <= self._lengths[req]:
            return
        missing = needed - self._held[req]
        if missing:
            with self._backing_call():
                self.backing.ensure(missing)
        self._held[req], self._lengths[req] = needed, length

    def resize_quiescent(self, req, length):
        """Set request `req`'s prefix to `length` rows; a shrink discards the tail rows for good."""
        self._usable()
        needed = self.layout.prefix_chunks(req, length)
        if length >= self._lengths[req]:
            self.reserve(req, length)
            return
        surplus = self._held[req] - needed
        with self._backing_call():
            self._synchronize()
            if surplus:
                self.backing.reclaim(surplus, synchronize=False)
        self._held[req], self._lengths[req] = needed, length

    def row_view(self, req, length, dtype):
        """A borrowed (length, row_elements) tensor over request `req`'s committed prefix."""
        self._usable()
        self.layout.prefix_chunks(req, length)       # validates req and length
        if length > self._lengths[req]:
            raise ValueError(f"a view of {length} rows is longer than the {self._lengths[req]} rows "
                             f"request {req} has committed")
        if dtype.itemsize != self.layout.itemsize:
            raise ValueError(f"{dtype} has {dtype.itemsize}-byte elements; the layout's hold "
                             f"{self.layout.itemsize} bytes")
        window = self.backing.raw.narrow(0, self.layout.request_offset(req), length * self.layout.row_bytes)
        return window.view(dtype).reshape(length, self.layout.row_elements)

    def close(self):
        """Synchronize and release the reservation once every view is retired (idempotent)."""
        if self._state == CLOSED:
            return
        with self._backing_call():
            self._synchronize()
            self.backing.close()
        self._state = CLOSED
