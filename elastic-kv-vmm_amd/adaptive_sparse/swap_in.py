"""Hot-buffer swap-in: LRU replacement of missed tokens, promoted from pinned host.

The single GPU replacement of the host-backed swap in the reference's decode
path (adaptive_sparse/request_residency.py:805-832, which calls SGLang's
load_blocks_to_device_buffer_mha): after the resident lookup has produced
slots and an ordered miss list, swap_in picks LRU victims in every
(layer, request) hot buffer, rewrites the token->slot table (and its
residency summary), patches the looked-up slots of the missed lanes and emits
(host row -> slot) promotion lists; move_kv then copies those rows from the
pinned host copy into the pool. The replacement policy is the reference's
batch-token LRU (benchmarks/hisparse_locality_replay.py:90-99). A token
repeated within a row (a Top-K block listed twice) is one access by its first
lane: the replay's rule applied to the selection with later repeats dropped.
"""

import torch

from elastic_kv import _native

from .kv_pool import KVPlanes
from .profile_ranges import profile_range

INT32_MIN = -(1 << 31)
STEP_STAMPS = 8192        # EKV_SWAP_STEP_STAMPS: recency stamps per LRU step, whatever the row width
SWAP_STAMP_OVERFLOW = 1   # EKV_SWAP_STAMP_OVERFLOW
SWAP_SHARED_REQUEST = 2   # EKV_SWAP_SHARED_REQUEST


class HotBuffers:
    """LRU hot buffers of `capacity` slots per (layer, request).

    table [L, R, T]: token -> global slot, int32 (0 = not resident), or with
    table_dtype=torch.int16 token -> local slot + 1 (0 = not resident; the
    lookup then takes slot_base=self.slot_base); bits: its residency summary,
    one bit per 2**bits_shift positions (the lookup takes
    bits_shift=self.bits_shift); slot_token [L, R, C]: token held by each
    slot (-1 = empty); stamps [L, R, C]: recency stamps; slot_base [R]:
    global slot of each request's local slot 0 (request r owns slots
    base .. base + C - 1; every base is at least 1, since global slot 0 is
    the sink that the lookup reports for a token that is not resident);
    status [1]: error bits of the swap-ins
    (check_status reads and clears them).
    table is a view into storage whose rows are padded to a multiple of 128
    positions, so every row starts 16-byte aligned and the lookup can stage
    its recent window with 16-byte loads; bits rows are whole 16-byte pieces.
    With bits_shift > 0, resident_counts [L, R, ceil(T / 2**bits_shift)]
    int32 holds the resident positions under each summary bit; the swap-in
    keeps it and the summary exact through evictions and insertions.
    """

    def __init__(self, layers, requests, context, capacity, device, *, slot_base=None, with_bits=True,
                 step_counter=False, table_dtype=torch.int32, bits_shift=0):
        self.layers, self.requests, self.context, self.capacity = layers, requests, context, capacity
        self.device = torch.device(device)
        if table_dtype not in (torch.int32, torch.int16):
            raise ValueError("table_dtype must be torch.int32 (global slots) or torch.int16 (local slots)")
        if table_dtype == torch.int16 and capacity >= 1 << 15:
            raise ValueError("an int16 table holds local slot + 1: capacity must be below 32768")
        kw = dict(dtype=torch.int32, device=self.device)
        padded = -(-context // 128) * 128
        self.table = torch.zeros((layers, requests, padded), dtype=table_dtype, device=self.device)[..., :context]
        self.bits_shift = int(bits_shift)
        # The summary keeps its padded width (whole 16-byte pieces, zero past the summary's words).
        from .resident_lookup import summary_words

        words = summary_words(context, self.bits_shift)
        self.bits = torch.zeros((layers, requests, words), **kw) if with_bits else None
        groups = -(-context // (1 << self.bits_shift))
        self.resident_counts = (torch.zeros((layers, requests, groups), **kw)
                                if with_bits and self.bits_shift > 0 else None)
        self.status = torch.zeros(1, **kw)
        self.slot_token = torch.full((layers, requests, capacity), -1, **kw)
        self.stamps = torch.full((layers, requests, capacity), INT32_MIN, **kw)
        if slot_base is None:
            slot_base = torch.arange(requests, dtype=torch.int64, device=self.device) * capacity + 1
        elif slot_base.numel() and int(slot_base.min()) < 1:
            raise ValueError("slot_base must be >= 1: global slot 0 is the sink that means 'not resident'")
        self.slot_base = slot_base
        self.step = 0
        # With a device step counter the swap-in reads and advances the step on
        # the GPU, so a captured HIP graph replays consecutive steps.
        self.step_counter = torch.zeros(1, dtype=torch.int64, device=self.device) if step_counter else None

    def install(self, tokens, local_slots):
        """Make `tokens` [L, R, n] resident in `local_slots` [L, R, n] (setup, not the hot path).

        Their recency follows their order along the last dimension (first =
        least recent), ahead of anything installed later.
        """
        L, R, n = tokens.shape
        tokens = tokens.to(self.device, torch.int64)
        local = local_slots.to(self.device, torch.int64)
        if self.table.dtype == torch.int16:
            entry = (local + 1).to(torch.int16)
        else:
            entry = (local + self.slot_base.view(1, R, 1)).to(torch.int32)
        self.table.scatter_(2, tokens, entry)
        self.slot_token.scatter_(2, local, tokens.to(torch.int32))
        rank = torch.arange(n, device=self.device, dtype=torch.int32).expand(L, R, n)
        self.stamps.scatter_(2, local, rank - n - 1)
        self.refresh_bits()

    def refresh_bits(self):
        """Rebuild the residency summary (and its group counts) exactly from the table.

        Needed after the table is edited outside the swap-in (install does it).
        """
        if self.bits is not None:
            from .resident_lookup import build_residency_bits

            build_residency_bits(self.table, out=self.bits, shift=self.bits_shift)
        if self.resident_counts is not None:
            self.resident_counts.copy_(residency_counts(self.table, self.bits_shift))

    def check_status(self):
        """Raise if a swap-in refused a row since the last check (a synchronizing read); clears the flags."""
        flags = int(self.status.item())
        if flags:
            self.status.zero_()
            reasons = []
            if flags & SWAP_STAMP_OVERFLOW:
                reasons.append("recency stamps would overflow (rebase() before the step counter runs out)")
            if flags & SWAP_SHARED_REQUEST:
                reasons.append("two selected rows named the same request")
            raise RuntimeError("swap_in refused rows: " + "; ".join(reasons))

    def rebase(self):
        """Renumber the recency stamps and restart the step counter.

        Every non-empty slot gets stamp rank - C, where rank orders the
        slots by (stamp, slot) as the LRU does. Empty slots stay INT32_MIN.
        The eviction order is unchanged, and later steps' stamps (>= 0) stay
        more recent than every renumbered one.
        """
        ranks = _ranks_from_stamps(self.stamps).to(torch.int32)
        empty = self.stamps == INT32_MIN
        self.stamps.copy_(torch.where(empty, torch.full_like(ranks, INT32_MIN), ranks - self.capacity))
        self.step = 0
        if self.step_counter is not None:
            self.step_counter.zero_()

    def steps_left(self):
        """Swap-in steps left before the stamps need a rebase (any width).

        Reads the device counter when there is one (a synchronizing read):
        graph replays advance it without the host seeing them.
        """
        step = int(self.step_counter.item()) if self.step_counter is not None else self.step
        # the last step that fits is the largest s with (s + 1) * STEP_STAMPS < 2**31
        return max(0, ((1 << 31) - 1) // STEP_STAMPS - step)


def residency_counts(table, shift):
    """Resident (non-zero) positions of `table` [.., T] per group of 2**shift positions, int32 [.., groups]."""
    size = 1 << shift
    groups = -(-table.shape[-1] // size)
    resident = table != 0
    if groups * size != table.shape[-1]:
        resident = torch.nn.functional.pad(resident, (0, groups * size - table.shape[-1]))
    return resident.reshape(*table.shape[:-1], groups, size).sum(-1, dtype=torch.int32)


def _ranks_from_stamps(stamps):
    """Per row, the rank of every slot's (stamp, slot) key, 0 = least recent."""
    order = torch.argsort(stamps.to(torch.int64), dim=-1, stable=True)
    ranks = torch.empty_like(order)
    ranks.scatter_(-1, order, torch.arange(stamps.shape[-1], device=stamps.device).expand_as(order))
    return ranks


@profile_range("native/swap")
def swap_in(topk, block_size, rows, selected, slots, misses, miss_count, buffers, host_table,
            promote_src, promote_dst, *, step=None, check=False):
    """Run one swap-in step (see module docstring); advances buffers.step.

    Rows the kernel refuses (selected rows sharing a request, stamps about
    to overflow) change nothing and set buffers.status; check=True reads it
    back after the call (a synchronization) and raises, otherwise call
    buffers.check_status() when convenient.

    Stamps are step * 8192 + lane (+ 4096 for a miss) in int32, so a step
    ranks above every earlier one whatever the width of each call; before
    they would overflow, the buffers' stamps are renumbered
    (HotBuffers.rebase) and the step restarts.
    With a device step counter (HotBuffers(step_counter=True)) the kernel
    reads the step from it and advances it, so the call can be captured in a
    HIP graph; graph users check steps_left() and rebase in time.
    """
    width = topk.shape[2] * block_size
    counted = buffers.step_counter is not None and step is None
    if step is None:
        if (buffers.step + 1) * STEP_STAMPS >= (1 << 31):
            buffers.rebase()
        step = buffers.step
    helper, entries = _native.launch_helper()
    status = helper.swap_in(
        entries["ekv_swap_in_counted" if counted else "ekv_swap_in"], int(counted), topk, int(block_size), rows,
        selected, slots, misses, miss_count, buffers.table, buffers.bits, int(buffers.bits_shift),
        buffers.resident_counts, buffers.slot_token, buffers.stamps, buffers.slot_base, host_table, promote_src,
        promote_dst, int(step), buffers.step_counter if counted else None, buffers.status)
    _native.launch_check(status, "swap_in")
    buffers.step = step + 1
    if check:
        buffers.check_status()


@profile_range("native/promote")
def move_kv(src_planes, src_rows, dst_planes, dst_rows, counts, *, zero_below=1):
    """dst(l, kv)[dst_rows[l, b, i]] = src(l, kv)[src_rows[l, b, i]] for i < counts[l, b]."""
    for planes in (src_planes, dst_planes):
        if not isinstance(planes, KVPlanes):
            raise TypeError("planes must be KVPlanes")
    helper, entries = _native.launch_helper()
    status = helper.move(entries["ekv_move_kv"], src_planes, src_rows, dst_planes, dst_rows, counts, int(zero_below))
    _native.launch_check(status, "move_kv")
