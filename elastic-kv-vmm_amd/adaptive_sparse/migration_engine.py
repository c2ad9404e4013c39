"""Byte movement of page migration: HIP pack/unpack + pinned-host copies.

Replaces the third-party host-copy kernels the reference migrates through
(adaptive_sparse/migration.py:109-111 backup_from_device_all_layer and
:232-237 load_to_device_per_layer) with this library's own path:

  demote:  pool pages --pack (ekv_gather_kv)--> device staging
                      --hipMemcpyAsync D2H (side stream)--> pinned host
  promote: pinned host --hipMemcpyAsync H2D (side stream)--> device staging
                      --unpack (ekv_scatter_kv)--> freshly committed pool pages

The pages are packed in one launch, then copied in sub-batches so that the
two PCIe directions and the unpacks overlap; events order each sub-batch
across the three streams. (A pack that shares the GPU with the copy kernels
that carry the PCIe legs crawls: 64 pages of 2.25 MiB took 2.8-2.9 ms against
65 us alone, while the whole 512-page pack takes 0.49 ms.) All streams have
the default priority.
"""

from dataclasses import dataclass

import torch

from elastic_kv.backing import Backing
from elastic_kv.slots import FreeSlots

from .kv_pool import BlockMajorLayout, PlanePoolLayout
from .minimax_vmm import PhysicalPages
from .sparse_read import gather_kv, scatter_kv


class _PagedPool:
    """Page ownership over one VMM Backing: allocate / release / trim / close."""

    def _own(self, layout, device, backing_factory, page_size, page_count, planes):
        self.layout = layout
        self.device = torch.device("cuda", device) if isinstance(device, int) else torch.device(device)
        index = self.device.index or 0
        self.backing = backing_factory(layout.capacity_bytes, layout.chunk_bytes, index)
        self.pages = PhysicalPages(self.backing, page_size, page_count, planes,
                                   lambda: torch.cuda.synchronize(self.device), chunk_bytes=layout.chunk_bytes)
        self.free = FreeSlots(page_count)
        self.planes = layout.kv_planes(self.backing.base, index, owner=self.backing)

    def take(self, count):
        """Allocate the `count` lowest free page ids (committing their chunks); None when too few are free."""
        ranges = self.free.peek(count)
        if ranges is None:
            return None
        pages = [p for a, b in ranges for p in range(a, b)]
        self.allocate(pages)
        return pages

    def allocate(self, pages):
        """Take specific free page ids and commit their chunks (map + zero)."""
        ids = sorted(int(p) for p in pages)
        ranges = []
        for page in ids:
            if ranges and ranges[-1][1] == page:
                ranges[-1] = (ranges[-1][0], page + 1)
            else:
                ranges.append((page, page + 1))
        self.free.remove(ranges)
        try:
            self.pages.acquire(ids)
        except Exception:
            self.free.release(ids)
            raise

    def release(self, pages):
        ids = sorted(int(p) for p in pages)
        self.pages.release(set(ids))
        self.free.release(ids)

    def trim(self, after=None, pages=None):
        """Unmap chunks no page owns; returns the released bytes.

        By default the device is synchronized first and every such chunk is
        released. With `after`, an event after which no device work touches
        `pages` (pages just released, e.g. a round trip's sources with its
        `packed` event), the host waits for that event only and releases only
        the chunks those pages covered: the copies and kernels queued behind
        the event keep running, and chunks freed earlier, whose readers may
        still be queued on another stream, are left to a synchronized trim.
        """
        if after is None:
            return self.pages.trim_quiescent()
        if pages is None:
            raise ValueError("trim(after=...) needs the released pages whose chunks the event fences")
        covered = set().union(*(self.pages.chunks(int(page)) for page in pages)) if len(pages) else set()
        idle = self.pages.reclaimable_chunks() & covered
        if not idle:
            return 0
        after.synchronize()
        return self.backing.reclaim(idle, synchronize=False) * self.layout.chunk_bytes

    def close(self):
        torch.cuda.synchronize(self.device)
        self.backing.close()


class PagedKVPool(_PagedPool):
    """Block-major paged KV pool over one VMM Backing with refcounted chunks.

    Page p holds layers x kv plane rows of row_bytes contiguously; page 0 is
    the permanent sink. `pages` tracks ownership (PhysicalPages with one
    plane of block_bytes rows), `free` hands out page ids.
    """

    def __init__(self, layout, device=0, backing_factory=Backing):
        if not isinstance(layout, BlockMajorLayout):
            raise TypeError("layout must be a BlockMajorLayout")
        self._own(layout, device, backing_factory, 1, layout.blocks - 1, [(0, layout.block_bytes)])

    def page_view(self, page):
        """uint8 view of one page's bytes (its chunks must be mapped)."""
        return self.backing.raw.narrow(0, page * self.layout.block_bytes, self.layout.block_bytes)


class PlanePagedPool(_PagedPool):
    """Plane-major paged KV pool: the layout of the reference's MiniMax main pool.

    One plane per (layer, K|V), each padded to whole chunks
    (adaptive_sparse/minimax_vmm.py:220-243); page p holds token slots
    [p * page_size, (p + 1) * page_size) of every plane, slot s of a plane at
    s * row_bytes. Page 0 (and so slot 0) is the permanent sink. Ownership is
    PhysicalPages over the planes (adaptive_sparse/minimax_vmm.py:40-98).
    """

    def __init__(self, layers, kv, page_count, page_size, row_bytes, device=0, chunk_bytes=2 << 20,
                 backing_factory=Backing):
        layout = PlanePoolLayout(layers, kv, (page_count + 1) * page_size, row_bytes, chunk_bytes)
        planes = [(plane * layout.plane_chunks, row_bytes) for plane in range(layout.planes)]
        self.page_size = page_size
        self._own(layout, device, backing_factory, page_size, page_count, planes)

    def slots(self, pages):
        """int64 token slots of `pages`, page after page, on the pool's device."""
        pages = torch.as_tensor(list(pages), dtype=torch.int64).to(self.device)
        offsets = torch.arange(self.page_size, dtype=torch.int64, device=self.device)
        return (pages.view(-1, 1) * self.page_size + offsets).flatten()

    def plane_rows(self, layer, kv):
        """uint8 [slots, row_bytes] view of one plane (read only rows whose chunks are mapped)."""
        layout = self.layout
        return self.backing.raw.narrow(0, layout.plane_offset(layer, kv), layout.plane_bytes).view(
            layout.rows, layout.row_bytes)


@dataclass
class HostPages:
    """Rows of the engine's pinned host buffer holding demoted pages, in order."""

    rows: torch.Tensor      # int64 host-buffer rows, one per page
    pages: tuple            # the source pages, same order
    packed: object = None   # round_trip: event after the last read of the source pages


class MigrationEngine:
    """Pack/unpack kernels + pinned host staging for one PagedKVPool."""

    def __init__(self, pool, max_pages, *, sub_batch=64):
        layout = pool.layout
        self.pool = pool
        self.device = pool.device
        self.block_bytes = layout.block_bytes
        self.sub_batch = max(1, int(sub_batch))
        self.max_pages = int(max_pages)
        self.out_staging = torch.empty((self.max_pages, layout.block_bytes), dtype=torch.uint8, device=self.device)
        self.in_staging = torch.empty_like(self.out_staging)
        self.host = torch.empty((self.max_pages, layout.block_bytes), dtype=torch.uint8, pin_memory=True)
        self.host_free = FreeSlots(self.max_pages)
        self.d2h = torch.cuda.Stream(self.device)
        self.h2d = torch.cuda.Stream(self.device)
        # The latest queued copies of each direction: the next pack into the
        # device staging waits for the D2H reads of it, and the next D2H into
        # host rows waits for the H2D reads of them.
        self._d2h_done = None
        self._h2d_done = None

    # ------------------------------------------------------------ kernels

    def _dense(self, staging, start, count):
        """(1, L, KV, count, row) view of staging rows [start, start + count)."""
        layout = self.pool.layout
        block = staging.narrow(0, start, count).view(count, layout.layers, layout.kv, layout.row_bytes)
        return block.permute(1, 2, 0, 3).unsqueeze(0)

    def _slots(self, pages):
        layout = self.pool.layout
        if isinstance(pages, torch.Tensor):
            ids = pages.to(self.device, torch.int64)
        else:
            ids = torch.as_tensor(list(pages), dtype=torch.int64).to(self.device, non_blocking=True)
        return ids.view(1, 1, -1).expand(layout.layers, 1, len(ids))

    def pack(self, pages, staging, start=0):
        """staging[start + i] = bytes of page pages[i] (on the current stream).

        `pages` is a sequence of page ids or an int64 tensor of them (a device
        tensor saves the copy of the list)."""
        if len(pages):
            gather_kv(self.pool.planes, self._slots(pages), self._dense(staging, start, len(pages)), zero_below=1)

    def unpack(self, pages, staging, start=0):
        """Bytes of page pages[i] = staging[start + i] (on the current stream); `pages` as for pack()."""
        if len(pages):
            scatter_kv(self.pool.planes, self._slots(pages), self._dense(staging, start, len(pages)), zero_below=1)

    # ------------------------------------------------------------ host rows

    def reserve_host(self, count):
        ranges = self.host_free.peek(count)
        if ranges is None:
            raise MemoryError("pinned host staging is full")
        self.host_free.claim(ranges)
        return torch.tensor([r for a, b in ranges for r in range(a - 1, b - 1)], dtype=torch.int64)

    def release_host(self, host):
        self.host_free.release(sorted(int(r) + 1 for r in host.rows.tolist()))

    # ------------------------------------------------------------ transfers

    def _host_runs(self, rows):
        """Contiguous runs (host_start, offset_in_list, length) of host rows."""
        values = rows.tolist()
        runs = []
        for i, row in enumerate(values):
            if runs and runs[-1][0] + runs[-1][2] == row:
                runs[-1][2] += 1
            else:
                runs.append([row, i, 1])
        return runs

    def demote(self, pages, host_rows=None):
        """Copy pages to pinned host rows; returns HostPages when the D2H is queued.

        The pack kernel runs on the current stream and the D2H copies on a
        side stream; call wait() (or synchronize) before reading the host rows.
        """
        pages = tuple(int(p) for p in pages)
        if len(pages) > self.max_pages:
            raise ValueError("more pages than the staging holds")
        rows = self.reserve_host(len(pages)) if host_rows is None else host_rows
        compute = torch.cuda.current_stream(self.device)
        self._order_reuse(compute)
        self.d2h.wait_event(self._pack_all(pages, compute))
        for start in range(0, len(pages), self.sub_batch):
            with torch.cuda.stream(self.d2h):
                self._copy_rows(rows[start:start + self.sub_batch], self.out_staging, start, to_host=True)
        self._d2h_done = torch.cuda.Event()
        self._d2h_done.record(self.d2h)
        return HostPages(rows=rows, pages=pages)

    def _pack_all(self, pages, compute):
        """Pack every page into the device staging in one launch; returns the event after it."""
        self.pack(pages, self.out_staging)
        packed = torch.cuda.Event()
        packed.record(compute)
        return packed

    def _order_reuse(self, compute):
        """Order this call's writes after the previous calls' reads of the same buffers."""
        if self._d2h_done is not None:
            compute.wait_event(self._d2h_done)       # packing rewrites the device staging
        if self._h2d_done is not None:
            self.d2h.wait_event(self._h2d_done)      # D2H copies rewrite host rows

    def promote(self, host, destinations):
        """Copy demoted pages from pinned host into `destinations` (already allocated)."""
        destinations = tuple(int(p) for p in destinations)
        if len(destinations) != len(host.pages):
            raise ValueError("one destination per demoted page")
        compute = torch.cuda.current_stream(self.device)
        ready = torch.cuda.Event()
        ready.record(compute)
        self.h2d.wait_event(ready)                   # earlier unpacks read the same device staging
        if self._d2h_done is not None:
            self.h2d.wait_event(self._d2h_done)      # the host rows must have landed
        for start in range(0, len(destinations), self.sub_batch):
            chunk = destinations[start:start + self.sub_batch]
            with torch.cuda.stream(self.h2d):
                self._copy_rows(host.rows[start:start + len(chunk)], self.in_staging, start, to_host=False)
                landed = torch.cuda.Event()
                landed.record(self.h2d)
            compute.wait_event(landed)
            self.unpack(chunk, self.in_staging, start)
        self._h2d_done = landed if destinations else self._h2d_done

    def round_trip(self, pages, destinations):
        """Demote `pages` and promote them into `destinations`, pipelined per sub-batch."""
        pages = tuple(int(p) for p in pages)
        destinations = tuple(int(p) for p in destinations)
        if len(pages) != len(destinations) or len(pages) > self.max_pages:
            raise ValueError("pages and destinations must pair up within the staging size")
        rows = self.reserve_host(len(pages))
        compute = torch.cuda.current_stream(self.device)
        self._order_reuse(compute)
        ready = torch.cuda.Event()
        ready.record(compute)
        self.h2d.wait_event(ready)                   # earlier unpacks read the same device staging
        # One pack before any copy, so the source pages are free (`packed`)
        # about half a millisecond in; the unpacks follow on the compute
        # stream, each behind its own H2D copy.
        all_packed = self._pack_all(pages, compute)
        self.d2h.wait_event(all_packed)
        arrivals = []
        for start in range(0, len(pages), self.sub_batch):
            span = rows[start:start + self.sub_batch]
            with torch.cuda.stream(self.d2h):
                self._copy_rows(span, self.out_staging, start, to_host=True)
                copied = torch.cuda.Event()
                copied.record(self.d2h)
            self.h2d.wait_event(copied)
            with torch.cuda.stream(self.h2d):
                self._copy_rows(span, self.in_staging, start, to_host=False)
                landed = torch.cuda.Event()
                landed.record(self.h2d)
            arrivals.append((start, landed))
        for start, landed in arrivals:
            compute.wait_event(landed)
            self.unpack(destinations[start:start + self.sub_batch], self.in_staging, start)
        if pages:
            self._d2h_done, self._h2d_done = copied, landed
        return HostPages(rows=rows, pages=pages, packed=all_packed)

    def _copy_rows(self, rows, staging, start, *, to_host):
        for host_start, offset, length in self._host_runs(rows):
            device_part = staging.narrow(0, start + offset, length)
            host_part = self.host.narrow(0, host_start, length)
            if to_host:
                host_part.copy_(device_part, non_blocking=True)
            else:
                device_part.copy_(host_part, non_blocking=True)

    def wait(self):
        torch.cuda.synchronize(self.device)
