"""Physical page ownership projected onto packed, chunk-aligned K/V planes.

PhysicalPages restates the reference's adaptive_sparse/minimax_vmm.py:20-98:
page p of every plane (plane_chunk, row_bytes) spans page_size rows starting
at plane_chunk * chunk_bytes + p * page_size * row_bytes; a chunk stays
mapped while any owned page touches it; page 0 is the permanent sink.
The SGLang pool installation of that module is serving-layer code outside
this path.
"""

from time import perf_counter_ns

CHUNK_BYTES = 2 << 20


class PhysicalPages:
    """Refcounted chunk ownership for the pages handed out by an allocator."""

    def __init__(self, backing, page_size, page_count, planes, synchronize,
                 chunk_bytes=CHUNK_BYTES, fast_decode=False):
        self.backing = backing
        self.page_size = page_size
        self.page_count = page_count
        self.planes = planes
        self.synchronize = synchronize
        self.chunk_bytes = chunk_bytes
        self.trim_sync_ns = 0
        self.fast_decode = fast_decode
        self.fast_no_new_page = 0
        self.decode_new_page = 0
        self._chunk_cache = {} if fast_decode else None
        self.pages = {0}
        self.refs = dict.fromkeys(self.chunks(0), 1)
        self.backing.ensure(set(self.refs))

    def chunks(self, page):
        """Chunk ids that page `page` touches in any plane."""
        if self._chunk_cache is not None:
            cached = self._chunk_cache.get(page)
            if cached is not None:
                return cached
        span = self.page_size
        touched = set()
        for plane_chunk, row_bytes in self.planes:
            first = page * span * row_bytes
            last = first + span * row_bytes - 1
            touched.update(range(plane_chunk + first // self.chunk_bytes,
                                 plane_chunk + last // self.chunk_bytes + 1))
        result = frozenset(touched)
        if self._chunk_cache is not None:
            self._chunk_cache[page] = result
        return result

    def acquire(self, pages):
        """Take ownership of pages, committing chunks no owned page uses yet."""
        pages = set(pages)
        if any(page <= 0 or page > self.page_count for page in pages):
            raise ValueError("invalid physical page")
        fresh = pages - self.pages
        footprints = [self.chunks(page) for page in fresh]
        if footprints:
            self.backing.ensure(set().union(*footprints))
        for footprint in footprints:
            for chunk in footprint:
                self.refs[chunk] = self.refs.get(chunk, 0) + 1
        self.pages.update(fresh)

    def validate_release(self, pages):
        if 0 in pages or not pages <= self.pages:
            raise RuntimeError("invalid or duplicate physical free")

    def release(self, pages):
        """Drop ownership; chunks reaching zero refs become reclaimable."""
        self.validate_release(pages)
        for page in pages:
            for chunk in self.chunks(page):
                remaining = self.refs[chunk] - 1
                if remaining:
                    self.refs[chunk] = remaining
                else:
                    del self.refs[chunk]
        self.pages.difference_update(pages)

    def clear(self):
        self.release(self.pages - {0})

    def reclaimable_chunks(self):
        return set(self.backing.mapped_chunks) - self.refs.keys()

    def stats(self):
        return {"backed_bytes": self.backing.backed_bytes,
                "reclaimable_bytes": len(self.reclaimable_chunks()) * self.chunk_bytes,
                "owned_pages": len(self.pages) - 1, "trim_sync_ns": self.trim_sync_ns,
                "fast_no_new_page": self.fast_no_new_page,
                "decode_new_page": self.decode_new_page}

    def trim_quiescent(self):
        """Unmap chunks no page owns. Call only with all device users idle."""
        pending = self.reclaimable_chunks()
        if not pending:
            return 0
        started = perf_counter_ns()
        self.synchronize()
        self.trim_sync_ns += perf_counter_ns() - started
        return self.backing.reclaim(pending, synchronize=False) * self.chunk_bytes
