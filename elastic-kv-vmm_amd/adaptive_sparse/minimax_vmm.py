"""Physical page ownership projected onto packed, chunk-aligned K/V planes.

The ownership contract of the reference's adaptive_sparse/minimax_vmm.py:20-98:
page p of a plane whose first chunk is c and whose rows are r bytes covers
bytes [p * page_size * r, (p + 1) * page_size * r) from chunk c on; a chunk
stays committed while any owned page covers it; page 0 is the permanent sink;
trimming releases the committed chunks no page covers. The SGLang pool
installation around it in the reference is serving-layer code outside this
path.

Two parts here: PageFootprints, the pure page -> chunk-set projection
(optionally memoized), and PhysicalPages, the owned-page set and per-chunk
reference counts kept over a Backing.
"""

from time import perf_counter_ns

CHUNK_BYTES = 2 << 20


class PageFootprints:
    """page -> frozenset of the chunk ids its rows cover in any plane."""

    def __init__(self, page_size, planes, chunk_bytes=CHUNK_BYTES, memoize=False):
        self.page_size = page_size
        self.planes = [tuple(plane) for plane in planes]   # (first chunk, row bytes) per plane
        self.chunk_bytes = chunk_bytes
        self._memo = {} if memoize else None

    def __call__(self, page):
        if self._memo is not None and page in self._memo:
            return self._memo[page]
        covered = set()
        for first_chunk, row_bytes in self.planes:
            page_bytes = self.page_size * row_bytes
            start, stop = page * page_bytes, (page + 1) * page_bytes        # [start, stop) in the plane
            covered.update(range(first_chunk + start // self.chunk_bytes,
                                 first_chunk + (stop - 1) // self.chunk_bytes + 1))
        footprint = frozenset(covered)
        if self._memo is not None:
            self._memo[page] = footprint
        return footprint


class PhysicalPages:
    """Refcounted chunk ownership of the pages an allocator hands out (pages 1..page_count).

    backing: ensure(ids), reclaim(ids, synchronize=False), mapped_chunks and
    backed_bytes, as elastic_kv.backing.Backing provides; synchronize: waits
    for every device user (called once per non-empty trim). fast_decode
    memoizes page footprints.
    """

    def __init__(self, backing, page_size, page_count, planes, synchronize,
                 chunk_bytes=CHUNK_BYTES, fast_decode=False):
        self.footprints = PageFootprints(page_size, planes, chunk_bytes, memoize=fast_decode)
        self.backing = backing
        self.page_count = page_count
        self.synchronize = synchronize
        self.trim_sync_ns = 0
        self.pages = {0}
        self.refs = dict.fromkeys(self.footprints(0), 1)
        backing.ensure(set(self.refs))

    page_size = property(lambda self: self.footprints.page_size)
    planes = property(lambda self: self.footprints.planes)
    chunk_bytes = property(lambda self: self.footprints.chunk_bytes)

    def chunks(self, page):
        return self.footprints(page)

    def acquire(self, pages):
        """Own `pages`, committing every chunk they cover first; ownership is unchanged if that fails."""
        wanted = set(pages)
        if not all(0 < page <= self.page_count for page in wanted):
            raise ValueError("invalid physical page")
        fresh = wanted - self.pages
        covers = [self.footprints(page) for page in fresh]
        if covers:
            self.backing.ensure(frozenset().union(*covers))
        for cover in covers:
            for chunk in cover:
                self.refs[chunk] = self.refs.get(chunk, 0) + 1
        self.pages |= fresh

    def validate_release(self, pages):
        if 0 in pages or not pages <= self.pages:
            raise RuntimeError("invalid or duplicate physical free")

    def release(self, pages):
        """Give up `pages`; chunks no remaining page covers become reclaimable."""
        self.validate_release(pages)
        for page in pages:
            for chunk in self.footprints(page):
                if self.refs[chunk] == 1:
                    del self.refs[chunk]
                else:
                    self.refs[chunk] -= 1
        self.pages -= pages

    def clear(self):
        self.release(self.pages - {0})

    def reclaimable_chunks(self):
        """Committed chunks that no owned page covers."""
        return set(self.backing.mapped_chunks).difference(self.refs)

    def stats(self):
        """backed (mapped) bytes, spare bytes (unmapped chunks the backing's spare pool still
        holds: a trim into the pool releases no device memory), reclaimable bytes, owned pages."""
        spare = getattr(self.backing, "spare_bytes", 0)
        return {"backed_bytes": self.backing.backed_bytes, "spare_bytes": spare,
                "reclaimable_bytes": len(self.reclaimable_chunks()) * self.chunk_bytes,
                "owned_pages": len(self.pages) - 1, "trim_sync_ns": self.trim_sync_ns}

    def trim_quiescent(self, only=None):
        """Release reclaimable chunks (those in `only`, if given); returns the bytes released.

        Call only with every device user idle: it synchronizes once, then
        unmaps without another wait.
        """
        idle = self.reclaimable_chunks()
        if only is not None:
            idle &= set(only)
        if not idle:
            return 0
        started = perf_counter_ns()
        self.synchronize()
        self.trim_sync_ns += perf_counter_ns() - started
        return self.backing.reclaim(idle, synchronize=False) * self.chunk_bytes
