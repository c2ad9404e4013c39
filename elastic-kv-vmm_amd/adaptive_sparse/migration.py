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
from dataclasses import dataclass, field


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


# ---------------------------------------------------------------- transactions
#
# The reference's transactions (adaptive_sparse/migration.py:67-288) operate on
# SGLang's HiSparse coordinator. MigrationCoordinator holds the same state for
# this build's own paged pool: the logical->physical page mapping (0 = not
# resident), the pool, the byte mover, the per-request hot pages kept after a
# demotion and the pinned-host copies of demoted requests.


class MigrationCoordinator:
    def __init__(self, pool, engine, mapping, keep_pages):
        self.pool = pool
        self.engine = engine
        self.mapping = mapping          # int64 tensor: logical page -> physical page (0 = none)
        self.keep_pages = keep_pages    # hot pages retained per demoted request
        self.hot = {}                   # row -> retained physical pages
        self.host_backed = {}           # row -> HostPages


@dataclass
class MigrationRequest:
    row: int
    logical: object                     # int64 tensor of logical page ids, in request order


@dataclass
class PreparedDemotion:
    coordinator: object
    request: object
    row: int
    logical: object
    physical: object
    committed_len: int
    retained_rows: tuple
    released_rows: tuple
    status: str = "prepared"
    host: object = field(default=None, repr=False)


@dataclass
class PreparedPromotion:
    coordinator: object
    request: object
    row: int
    logical: object
    destination: object
    backed_before: int
    status: str = "prepared"


def prepare_demote(coordinator, req, synchronize):
    """Stage every committed page of `req` to pinned host; ownership unchanged."""
    logical = req.logical
    physical = coordinator.mapping[logical]
    if not bool((physical > 0).all()):
        raise RuntimeError("Resident request has missing physical locations")
    pages = [int(p) for p in physical.tolist()]
    if len(pages) != len(set(pages)):
        raise RuntimeError("Resident request reuses a physical page")
    retained, released = plan_demote_pages(coordinator.pool.pages, pages, min(coordinator.keep_pages, len(pages)))
    row_of = {page: i for i, page in enumerate(pages)}
    synchronize()
    host = None
    try:
        host = coordinator.engine.demote(pages)
        synchronize()
    except Exception:
        synchronize()
        if host is not None:
            coordinator.engine.release_host(host)
        raise
    return PreparedDemotion(coordinator, req, req.row, logical, physical, len(pages),
                            tuple(row_of[p] for p in retained), tuple(row_of[p] for p in released),
                            host=host)


def abort_demote(prepared):
    """Undo a prepared demotion (drop its host copy)."""
    if prepared.status != "prepared":
        raise RuntimeError("Only a prepared demotion can be aborted")
    prepared.coordinator.engine.release_host(prepared.host)
    prepared.status = "aborted"


def commit_demote(prepared, publish_host_backed, synchronize, trim_quiescent=None):
    """Unpublish the request, keep its retained pages hot, free the rest."""
    if prepared.status != "prepared":
        raise RuntimeError("Demotion has already been resolved")
    prepared.status = "committing"
    coordinator = prepared.coordinator
    pages = prepared.physical.tolist()
    coordinator.mapping[prepared.logical] = 0
    synchronize()
    coordinator.pool.release([pages[i] for i in prepared.released_rows])
    coordinator.hot[prepared.row] = tuple(pages[i] for i in prepared.retained_rows)
    coordinator.host_backed[prepared.row] = prepared.host
    synchronize()
    released_bytes = trim_quiescent() if trim_quiescent is not None else 0
    publish_host_backed(prepared.row)
    prepared.status = "committed"
    return released_bytes


def prepare_promote(coordinator, req, synchronize, destinations=None):
    """Copy a host-backed request into freshly committed pages, unpublished."""
    host = coordinator.host_backed.get(req.row)
    if host is None or len(host.pages) != len(req.logical):
        raise RuntimeError("Promotion source is missing committed host KV")
    pool = coordinator.pool
    backed_before = pool.backing.backed_bytes
    if destinations is None:
        ranges = pool.free.peek(len(host.pages))
        if ranges is None:
            raise MemoryError("No physical pages available for promotion")
        destinations = [p for a, b in ranges for p in range(a, b)]
    destinations = [int(p) for p in destinations]
    pool.allocate(destinations)
    try:
        coordinator.engine.promote(host, destinations)
        synchronize()
    except Exception:
        synchronize()
        pool.release(destinations)
        pool.trim()
        raise
    destination = torch_long(destinations, coordinator.mapping.device)
    return PreparedPromotion(coordinator, req, req.row, req.logical, destination, backed_before)


def abort_promote(prepared):
    """Release only the new destination after a rejected prepare."""
    if prepared.status != "prepared":
        raise RuntimeError("Only a prepared promotion can be aborted")
    pool = prepared.coordinator.pool
    pool.release(prepared.destination.tolist())
    pool.trim()
    prepared.status = "aborted"


def commit_promote(prepared, publish_gpu_resident, synchronize):
    """Release the host copy and hot pages, then publish the new mapping."""
    if prepared.status != "prepared":
        raise RuntimeError("Promotion has already been resolved")
    prepared.status = "committing"
    coordinator = prepared.coordinator
    host = coordinator.host_backed.pop(prepared.row)
    coordinator.engine.release_host(host)
    hot = coordinator.hot.pop(prepared.row, ())
    if hot:
        coordinator.pool.release(hot)
    coordinator.mapping[prepared.logical] = prepared.destination[:len(prepared.logical)]
    synchronize()
    coordinator.pool.trim()
    publish_gpu_resident(prepared.row)
    prepared.status = "committed"
    return max(0, coordinator.pool.backing.backed_bytes - prepared.backed_before)


def torch_long(values, device):
    import torch

    return torch.tensor(values, dtype=torch.int64, device=device)
