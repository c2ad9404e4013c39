"""Demotion / promotion of request KV between the VMM pool and pinned host memory.

Mirrors the reference's adaptive_sparse/migration.py:
  * plan_demote_pages (:27-54) - which pages of a demoted request stay hot,
    in default (first pages) or chunk-aware mode (EKV_CHUNK_AWARE_RETENTION=1);
  * PreparedDemotion / PreparedPromotion (:14-24, :181-189) and the
    prepare / commit / abort transaction split.
The reference moves bytes through SGLang's host KV cache; here the byte
movement is this build's own: HIP pack/unpack kernels between scattered pool
pages and contiguous device staging, and hipMemcpyAsync between staging and
pinned host memory on a side stream (see migration_engine.py).
"""

import os
from collections import Counter


def plan_demote_pages(tracker, page_ids, keep_pages, *, chunk_aware=None):
    """Split a request's pages into (retained, released) tuples.

    Default: keep the first `keep_pages` pages. Chunk-aware: greedily keep
    the page whose not-yet-protected exclusive chunks are fewest, preferring
    chunk sets that more remaining pages share, then the lowest page id, so
    that the released pages free as many whole chunks as possible.
    """
    pages = tuple(page_ids)
    if not 0 < keep_pages <= len(pages) or len(set(pages)) != len(pages):
        raise ValueError("Invalid demotion page ownership")
    if chunk_aware is None:
        chunk_aware = os.environ.get("EKV_CHUNK_AWARE_RETENTION") == "1"
    if not chunk_aware:
        return pages[:keep_pages], pages[keep_pages:]
    if tracker is None:
        raise RuntimeError("Chunk-aware retention requires a physical page tracker")
    footprint = {page: frozenset(tracker.chunks(page)) for page in pages}
    users = Counter(chunk for chunks in footprint.values() for chunk in chunks)
    # Chunks whose every owner is a page of this request.
    exclusive = frozenset(chunk for chunk, count in users.items() if count == tracker.refs.get(chunk))
    own = {page: chunks & exclusive for page, chunks in footprint.items()}
    protected = set()
    candidates = set(pages)
    retained = []
    for _ in range(keep_pages):
        extra = {page: frozenset(own[page] - protected) for page in candidates}
        supply = Counter(extra.values())
        choice = min(candidates, key=lambda page: (len(extra[page]), -supply[extra[page]], page))
        retained.append(choice)
        protected |= own[choice]
        candidates.discard(choice)
    released = tuple(page for page in pages if page in candidates)
    return tuple(retained), released
