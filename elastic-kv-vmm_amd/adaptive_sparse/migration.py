"""Demotion / promotion of request KV between the VMM pool and pinned host memory.

Mirrors the reference's adaptive_sparse/migration.py:
  * plan_demote_pages (:27-54) - which pages of a demoted request stay hot,
    in default (first pages) or chunk-aware mode (EKV_CHUNK_AWARE_RETENTION=1);
  * PreparedDemotion / PreparedPromotion (:14-24, :181-189) and the
    prepare / commit / abort transactions (:67-288).
The reference's transactions act on SGLang's HiSparse coordinator, which is
not part of this path; HiSparseCoordinator holds the state they touch, under
SGLang's names: the request -> logical token table, the logical -> device slot
mapping (0 = not resident), the host token rows of host-backed requests, and
their hot buffers (device slots, the token each slot holds per layer, the LRU
order, the reserved slot of the newest token). Demotion leaves a request in
exactly the state ekv_hisparse_swap_in serves host-backed decode from, and
promotion restores it from there. The byte movement is this library's own:
ekv_move_kv copies scattered token rows of every plane between the pool and
device-mapped pinned host memory in one launch per direction.
"""

import os
from collections import Counter
from dataclasses import dataclass


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


class RowMover:
    """Token-row copies of every (layer, K|V) plane, on the current stream, timed by HIP events.

    Each call returns a Transfer; its seconds() is valid once the stream has
    passed its end event.
    """

    def __init__(self, pool, host):
        self.pool, self.host = pool, host

    def _move(self, src_planes, src_rows, dst_planes, dst_rows):
        import torch

        from .swap_in import move_kv

        layers, count = self.pool.layout.layers, len(src_rows)
        if count == 0:
            return Transfer(0)
        device = self.pool.device
        src = torch.as_tensor(src_rows).to(device, torch.int32).reshape(1, 1, count).expand(layers, 1, count)
        dst = torch.as_tensor(dst_rows).to(device, torch.int32).reshape(1, 1, count).expand(layers, 1, count)
        counts = torch.full((layers, 1), count, dtype=torch.int32, device=device)
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        move_kv(src_planes, src, dst_planes, dst, counts, zero_below=0)
        end.record()
        layout = self.pool.layout
        return Transfer(count * layout.layers * layout.kv * layout.row_bytes, start, end, (src, dst, counts))

    def pool_to_host(self, slots, host_rows):
        return self._move(self.pool.planes, slots, self.host.planes, host_rows)

    def host_to_pool(self, host_rows, slots):
        return self._move(self.host.planes, host_rows, self.pool.planes, slots)

    def pool_to_pool(self, src_slots, dst_slots):
        return self._move(self.pool.planes, src_slots, self.pool.planes, dst_slots)


@dataclass
class Transfer:
    bytes: int
    start: object = None
    end: object = None
    keep: object = None          # the row lists the queued copy reads

    def seconds(self):
        return self.start.elapsed_time(self.end) / 1e3 if self.start is not None else 0.0


class HiSparseCoordinator:
    """The HiSparse state the migration transactions act on (SGLang's names, this library's pool).

    pool: a PlanePagedPool (page_size token slots per page, slot 0 the sink);
    host: a HostKVCache; mover: the row copies (RowMover over both by
    default); rows / max_len: request rows and their longest length;
    logical_size: logical token locations; hot_capacity: H, the hot slots
    of a host-backed request. padded_buffer_size = the whole pages that hold
    H slots plus the reserved newest-token slot at index H. bandwidth: an
    optional MigrationBandwidthEstimator fed, per direction, with the copy
    bytes and time (HIP events) of every committed transaction.
    """

    def __init__(self, pool, host, *, rows, max_len, logical_size, hot_capacity, mover=None, bandwidth=None):
        import torch

        page = pool.page_size
        layers = pool.layout.layers
        device = pool.device
        self.pool, self.host = pool, host
        self.mover = mover if mover is not None else RowMover(pool, host)
        self.bandwidth = bandwidth
        self.device_buffer_size = int(hot_capacity)
        self.padded_buffer_size = -(-(self.device_buffer_size + 1) // page) * page
        self.req_to_token = torch.zeros((rows, max_len), dtype=torch.int64, device=device)
        self.mapping = torch.zeros(logical_size, dtype=torch.int64, device=device)   # logical loc -> device slot
        self.req_to_host_pool = torch.full((rows, max_len), -1, dtype=torch.int64, device=device)
        self.req_to_host_pool_allocated_len = [0] * rows
        self.req_to_device_buffer = torch.zeros((rows, self.padded_buffer_size), dtype=torch.int64, device=device)
        self.req_device_buffer_size = [0] * rows
        self.req_device_buffer_tokens = torch.full((layers, rows, self.padded_buffer_size), -1, dtype=torch.int32,
                                                   device=device)
        self._lru_init = torch.arange(self.device_buffer_size, dtype=torch.int16, device=device)
        self.lru_slots = self._lru_init.repeat(layers, rows, 1)
        self.skip_first_backup = [False] * rows
        self.hot_pages = {}      # row -> retained pages of a host-backed request

    def wait_for_pending_backup(self):
        """Backups are queued on the stream the transactions synchronize; nothing is pending apart."""

    def observe(self, direction, transfers):
        """Feed a committed migration's copy bytes and time to the bandwidth estimator.

        Only committed migrations count, as in adaptive_sparse/migration_budget.py:6-13.
        """
        if self.bandwidth is not None:
            moved = sum(t.bytes for t in transfers)
            return self.bandwidth.observe(direction, moved, sum(t.seconds() for t in transfers))
        return None

    def release_host(self, row):
        """Free a row's host token rows (the reference's _release_host)."""
        count = self.req_to_host_pool_allocated_len[row]
        if count:
            rows = self.req_to_host_pool[row, :count]
            self.host.free([r for r in rows.tolist() if r >= 0])
        self.req_to_host_pool[row].fill_(-1)
        self.req_to_host_pool_allocated_len[row] = 0

    def backup_previous_token(self, row, length):
        """Host-backed decode, before token `length` is written to the reserved slot.

        The reserved slot holds token length - 1 and it is copied to a new host
        row - unless this is the first step after a demotion, whose host copy
        already holds every committed token (the slot holds no token yet).
        """
        if self.skip_first_backup[row]:
            self.skip_first_backup[row] = False
            return None
        host_rows = self.host.alloc(1)
        if host_rows is None:
            raise MemoryError("the host KV cache is full")
        reserved = self.req_to_device_buffer[row, self.device_buffer_size:self.device_buffer_size + 1]
        transfer = self.mover.pool_to_host(reserved, host_rows)
        self.req_to_host_pool[row, length - 1] = int(host_rows[0])
        self.req_to_host_pool_allocated_len[row] = length
        return transfer

    def newest_slot(self, row):
        """The reserved device slot of a host-backed row's newest token."""
        return int(self.req_to_device_buffer[row, self.device_buffer_size])

    def swap_in(self, layer, req_pool_indices, seq_lens, top_k_blocks, top_k_device_locs, sparse_block_size,
                num_real_reqs=None):
        """One layer of host-backed decode: load_blocks_to_device_buffer_mha over this state."""
        from .hisparse_swap import load_blocks_to_device_buffer_mha

        host_k, host_v = self.host.layer(layer)
        load_blocks_to_device_buffer_mha(
            top_k_blocks=top_k_blocks, device_buffer_tokens=self.req_device_buffer_tokens[layer],
            host_cache_locs=self.req_to_host_pool, device_buffer_locs=self.req_to_device_buffer,
            host_cache_k=host_k, host_cache_v=host_v, device_buffer_k=self.pool.plane_rows(layer, 0),
            device_buffer_v=self.pool.plane_rows(layer, 1), top_k_device_locs=top_k_device_locs,
            req_pool_indices=req_pool_indices, seq_lens=seq_lens, lru_slots=self.lru_slots[layer],
            item_size_bytes=self.pool.layout.row_bytes, hot_buffer_size=self.device_buffer_size,
            sparse_block_size=sparse_block_size, num_real_reqs=num_real_reqs)


@dataclass
class MigrationRequest:
    row: int
    length: int             # committed tokens (kv_committed_len == kv_allocated_len)


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
    transfers: tuple = ()           # the host copy, timed; observed when the demotion commits


@dataclass
class PreparedPromotion:
    coordinator: object
    request: object
    row: int
    logical: object
    destination: object
    backed_before: int
    status: str = "prepared"
    transfers: tuple = ()           # the restoring copies, timed; observed when the promotion commits


def prepare_demote(coordinator, req, synchronize):
    """Copy every committed token of `req` to host rows in logical order; ownership unchanged.

    adaptive_sparse/migration.py:67-121.
    """
    row, length = req.row, req.length
    page = coordinator.pool.page_size
    if length < coordinator.padded_buffer_size:
        raise ValueError("Demotion requires a fully committed long resident request")
    if coordinator.req_device_buffer_size[row] or coordinator.req_to_host_pool_allocated_len[row]:
        raise RuntimeError("Resident request unexpectedly owns HiSparse cache state")
    logical = coordinator.req_to_token[row, :length].clone()
    physical = coordinator.mapping[logical]
    if not bool((physical > 0).all()):
        raise RuntimeError("Resident request has missing physical locations")
    page_starts = physical[::page].tolist()
    if any(slot % page for slot in page_starts):
        raise RuntimeError("Resident request page starts are misaligned")
    page_ids = [slot // page for slot in page_starts]
    if len(page_ids) != len(set(page_ids)):
        raise RuntimeError("Resident request reuses a physical page")
    retained, released = plan_demote_pages(coordinator.pool.pages, page_ids,
                                           coordinator.padded_buffer_size // page)
    index_of = {p: i for i, p in enumerate(page_ids)}
    coordinator.wait_for_pending_backup()
    synchronize()
    try:
        host_rows = coordinator.host.alloc(length)
        if host_rows is None:
            raise MemoryError("the host KV cache cannot hold the request")
        coordinator.req_to_host_pool[row, :length] = host_rows.to(coordinator.req_to_host_pool.device)
        coordinator.req_to_host_pool_allocated_len[row] = length
        transfer = coordinator.mover.pool_to_host(physical, host_rows)
        synchronize()
    except Exception:
        # Device work may still read the rows if the synchronization failed: wait before freeing them.
        synchronize()
        coordinator.release_host(row)
        raise
    return PreparedDemotion(coordinator, req, row, logical, physical, length,
                            tuple(index_of[p] for p in retained), tuple(index_of[p] for p in released),
                            transfers=(transfer,))


def abort_demote(prepared):
    """Undo a prepared demotion (free its host rows)."""
    if prepared.status != "prepared":
        raise RuntimeError("Only a prepared demotion can be aborted")
    prepared.coordinator.release_host(prepared.row)
    prepared.status = "aborted"


def commit_demote(prepared, publish_host_backed, synchronize, trim_quiescent=None):
    """Hand the retained pages to the row's hot buffer, unpublish the mapping, release the rest.

    adaptive_sparse/migration.py:131-178: the hot buffer's device slots are
    the retained pages' token slots (index H the reserved newest-token slot),
    no slot holds a token yet in any layer (every lookup starts as a miss),
    the LRU order restarts, and the host image is authoritative (it holds
    the latest committed token).
    """
    if prepared.status != "prepared":
        raise RuntimeError("Demotion has already been resolved")
    prepared.status = "committing"
    import torch

    coordinator = prepared.coordinator
    row = prepared.row
    capacity = coordinator.padded_buffer_size
    page = coordinator.pool.page_size
    page_starts = prepared.physical[::page]
    retained_rows = torch.tensor(prepared.retained_rows, dtype=torch.int64, device=page_starts.device)
    retained = (page_starts[retained_rows, None] + torch.arange(page, device=page_starts.device)).flatten()
    coordinator.req_to_device_buffer[row, :capacity] = retained
    coordinator.req_device_buffer_size[row] = capacity
    coordinator.req_device_buffer_tokens[:, row, :].fill_(-1)
    coordinator.lru_slots[:, row, :].copy_(coordinator._lru_init)
    coordinator.skip_first_backup[row] = True
    coordinator.mapping[prepared.logical] = 0
    synchronize()
    starts = page_starts.tolist()
    coordinator.pool.release([starts[i] // page for i in prepared.released_rows])
    coordinator.hot_pages[row] = tuple(starts[i] // page for i in prepared.retained_rows)
    synchronize()
    released_bytes = trim_quiescent() if trim_quiescent is not None else 0
    publish_host_backed(row)
    prepared.status = "committed"
    coordinator.observe("demotion", prepared.transfers)
    return released_bytes


def prepare_promote(coordinator, req, synchronize, destinations=None):
    """Restore a host-backed request into freshly committed pages, unpublished.

    adaptive_sparse/migration.py:192-257: the host holds tokens [0, host_len)
    - every committed token while the host image is authoritative (no decode
    step since the demotion), else all but the newest, which is copied from
    the reserved device slot in every layer. `destinations` optionally names
    the destination pages (default: the lowest free ones).
    """
    import torch

    row, length = req.row, req.length
    pool = coordinator.pool
    page = pool.page_size
    if length <= coordinator.device_buffer_size:
        raise ValueError("Promotion requires a fully committed long host-backed request")
    if coordinator.req_device_buffer_size[row] != coordinator.padded_buffer_size:
        raise RuntimeError("Unexpected source hot-buffer capacity")
    coordinator.wait_for_pending_backup()
    synchronize()
    logical = coordinator.req_to_token[row, :length].clone()
    host_authoritative = bool(coordinator.skip_first_backup[row])
    host_len = length if host_authoritative else length - 1
    host_rows = coordinator.req_to_host_pool[row, :host_len]
    if coordinator.req_to_host_pool_allocated_len[row] < host_len or not bool((host_rows >= 0).all()):
        raise RuntimeError("Promotion source is missing committed host KV")
    latest = None
    if not host_authoritative:
        latest = coordinator.req_to_device_buffer[row, coordinator.device_buffer_size:][:1]
        if not bool((latest > 0).all()):
            raise RuntimeError("Promotion source is missing the latest device token")
    backed_before = pool.backing.backed_bytes
    count = -(-length // page)
    if destinations is None:
        pages = pool.take(count)
        if pages is None:
            raise MemoryError("No physical pages available for promotion")
    else:
        pages = [int(p) for p in destinations]
        if len(pages) != count:
            raise ValueError(f"promotion of {length} tokens needs {count} destination pages")
        pool.allocate(pages)
    destination = pool.slots(pages)
    try:
        transfers = [coordinator.mover.host_to_pool(host_rows, destination[:host_len])]
        if latest is not None:
            transfers.append(coordinator.mover.pool_to_pool(latest, destination[host_len:host_len + 1]))
        synchronize()
    except Exception:
        synchronize()
        pool.release(pages)
        pool.trim()
        raise
    return PreparedPromotion(coordinator, req, row, logical, destination, backed_before, transfers=tuple(transfers))


def abort_promote(prepared):
    """Release only the new destination after a rejected prepare."""
    if prepared.status != "prepared":
        raise RuntimeError("Only a prepared promotion can be aborted")
    pool = prepared.coordinator.pool
    pool.release(sorted(set(s // pool.page_size for s in prepared.destination.tolist())))
    pool.trim()
    prepared.status = "aborted"


def commit_promote(prepared, publish_gpu_resident, synchronize):
    """Release the host rows and hot pages, then publish the new mapping.

    adaptive_sparse/migration.py:260-288.
    """
    if prepared.status != "prepared":
        raise RuntimeError("Promotion has already been resolved")
    prepared.status = "committing"
    coordinator = prepared.coordinator
    row = prepared.row
    coordinator.release_host(row)
    hot = coordinator.hot_pages.pop(row, ())
    if hot:
        coordinator.pool.release(hot)
    coordinator.req_device_buffer_size[row] = 0
    coordinator.req_device_buffer_tokens[:, row, :].fill_(-1)
    coordinator.req_to_device_buffer[row].zero_()
    coordinator.skip_first_backup[row] = False
    coordinator.mapping[prepared.logical] = prepared.destination[:len(prepared.logical)]
    synchronize()
    coordinator.pool.trim()
    publish_gpu_resident(row)
    prepared.status = "committed"
    coordinator.observe("promotion", prepared.transfers)
    return max(0, coordinator.pool.backing.backed_bytes - prepared.backed_before)
