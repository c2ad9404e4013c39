"""Physical admission and lookahead precommit over VMM-backed arenas.

This bounds token admission by the bytes the VMM can still commit, and
precommits (maps and zero-fills asynchronously) the chunks just past newly
admitted ranges. Semantics follow the reference's Residency admission math
without its serving-engine coupling:
- fully backed chunks: elastic_kv/adapter.py:562-570;
- chunk budget from free device memory and prefill headroom: :572-647
  (the reference also caps it by its cross-process capacity broker, which
  is not part of this path);
- the admission walk over free slot ranges: :671-756;
- the request-affine preflight: :649-669;
- the lookahead precommit after admitted ranges: :806-831.

An arena is any object with `mapped_chunks` (a set of chunk ids), `planes`
(chunks committed per chunk id; default 1) and `precommit(ids)` returning
the number newly committed. This build's Backing and PhysicalPages have them.
"""

import time

__all__ = ["fully_backed_chunks", "chunk_budget", "available_tokens", "precommit_candidates",
           "PhysicalAdmission"]


def fully_backed_chunks(arenas, precommitted=()):
    """Chunk ids backed in every arena, plus the precommitted ones."""
    backed = set(precommitted)
    if arenas:
        backed.update(set.intersection(*(set(arena.mapped_chunks) for arena in arenas)))
    return backed


def chunk_budget(arenas, chunk_bytes, free_bytes, prefill_headroom, counters=None, reclaim=None):
    """(chunks that may still be committed, bytes per chunk id, headroom).

    Returns None when no arena commits anything. `free_bytes()` reports free
    device memory. When it is below headroom + one chunk id, `reclaim()` (for
    example the caching allocator's empty_cache) is called once and the
    memory is queried again.
    """
    counters = {} if counters is None else counters
    cost = sum(chunk_bytes * getattr(arena, "planes", 1) for arena in arenas)
    if cost <= 0:
        return None
    free = free_bytes()
    if free < prefill_headroom + cost and reclaim is not None:
        started = time.perf_counter_ns()
        reclaim()
        after = free_bytes()
        counters["physical_empty_cache_calls"] = counters.get("physical_empty_cache_calls", 0) + 1
        counters["physical_empty_cache_freed_bytes"] = (
            counters.get("physical_empty_cache_freed_bytes", 0) + max(0, after - free))
        counters["physical_empty_cache_ns"] = (
            counters.get("physical_empty_cache_ns", 0) + time.perf_counter_ns() - started)
        free = after
    usable = max(0, free - prefill_headroom)
    return usable // cost, cost, prefill_headroom


def _check_ranges(logical_free_tokens, ranges):
    if any(start < 1 or stop <= start for start, stop in ranges):
        raise ValueError("free_ranges must contain positive half-open ranges")
    if sum(stop - start for start, stop in ranges) != logical_free_tokens:
        raise ValueError("free_ranges length must match logical_free_tokens")
    if any(left[1] > right[0] for left, right in zip(ranges, ranges[1:])):
        raise ValueError("free_ranges must be sorted and disjoint")


def available_tokens(logical_free_tokens, free_ranges, slot_bytes, chunk_bytes, backed_chunks, budget):
    """Tokens admissible in `free_ranges` order before the chunk budget runs out.

    A slot whose chunks are all backed costs nothing. Otherwise the first
    touch of each missing chunk spends one unit of `budget`. The walk stops at
    the first slot that does not fit. It advances a whole chunk's slots at a
    time: every slot before the next chunk boundary uses only chunks already
    decided.
    """
    if logical_free_tokens < 0:
        raise ValueError("logical_free_tokens must be nonnegative")
    if logical_free_tokens == 0:
        return 0
    if slot_bytes <= 0 or slot_bytes > chunk_bytes:
        raise ValueError("physical admission requires 0 < slot_bytes <= chunk_bytes")
    ranges = tuple(free_ranges)
    _check_ranges(logical_free_tokens, ranges)
    backed = set(backed_chunks)
    admitted = 0
    for start, stop in ranges:
        position = start
        while position < stop:
            first = position * slot_bytes // chunk_bytes
            last = ((position + 1) * slot_bytes - 1) // chunk_bytes
            missing = [chunk for chunk in range(first, last + 1) if chunk not in backed]
            if len(missing) > budget:
                return admitted
            budget -= len(missing)
            backed.update(missing)
            boundary = max(position + 1, (last + 1) * chunk_bytes // slot_bytes)
            end = min(stop, boundary)
            admitted += end - position
            position = end
    return admitted


def precommit_candidates(ranges, slot_bytes, chunk_bytes, chunk_count, lookahead, idle, precommitted=()):
    """Chunk ids to precommit after admitting `ranges`, in ascending order.

    For each range these are the `lookahead` chunks starting at the chunk that
    holds the range's end, limited to chunks that `idle(chunk)` reports free
    of live slots and that are not already precommitted.
    """
    if lookahead <= 0:
        return []
    candidates = set()
    done = set(precommitted)
    for _, stop in ranges:
        first = stop * slot_bytes // chunk_bytes
        for chunk in range(first, min(chunk_count, first + lookahead)):
            if idle(chunk) and chunk not in done:
                candidates.add(chunk)
    return sorted(candidates)


class PhysicalAdmission:
    """Stateful admission over a set of arenas, with the reference's counters.

    `policy` is "physical" (bound by committable bytes) or "logical" (no
    bound). `free_bytes()` reports free device memory; it defaults to
    torch.cuda.mem_get_info on `device`, with torch.cuda.empty_cache as
    `reclaim`.
    """

    def __init__(self, arenas, slot_bytes, chunk_bytes, *, policy="physical", prefill_headroom_bytes=0,
                 precommit_lookahead=0, precommit_limit=0, device=0, free_bytes=None, reclaim=None):
        if policy not in ("physical", "logical"):
            raise ValueError("policy must be 'physical' or 'logical'")
        self.arenas = list(arenas)
        self.slot_bytes = slot_bytes
        self.chunk_bytes = chunk_bytes
        self.policy = policy
        self.prefill_headroom_bytes = prefill_headroom_bytes
        self.precommit_lookahead = precommit_lookahead
        self.precommit_limit = precommit_limit
        self.precommitted = set()
        self.counters = {}
        self._device = device
        self._free_bytes = free_bytes
        self._reclaim = reclaim

    def _memory(self):
        if self._free_bytes is not None:
            return self._free_bytes, self._reclaim
        import torch

        def free():
            return torch.cuda.mem_get_info(self._device)[0]

        def reclaim():
            with torch.cuda.device(self._device):
                torch.cuda.empty_cache()

        return free, reclaim

    def backed_chunks(self):
        return fully_backed_chunks(self.arenas, self.precommitted)

    def _budget(self):
        free, reclaim = self._memory()
        return chunk_budget(self.arenas, self.chunk_bytes, free, self.prefill_headroom_bytes, self.counters,
                            reclaim)

    def physical_available_tokens(self, logical_free_tokens, free_ranges):
        """Tokens of `free_ranges` whose backing fits the committable budget."""
        if logical_free_tokens < 0:
            raise ValueError("logical_free_tokens must be nonnegative")
        if self.policy == "logical":
            return logical_free_tokens
        if logical_free_tokens == 0:
            return 0
        if self.slot_bytes <= 0 or self.slot_bytes > self.chunk_bytes:
            raise ValueError("physical admission requires 0 < slot_bytes <= chunk_bytes")
        ranges = tuple(free_ranges)
        _check_ranges(logical_free_tokens, ranges)
        self.counters["physical_available_calls"] = self.counters.get("physical_available_calls", 0) + 1
        started = time.perf_counter_ns()
        budget = self._budget()
        if budget is None:
            return logical_free_tokens
        chunks, cost, headroom = budget
        admitted = available_tokens(logical_free_tokens, ranges, self.slot_bytes, self.chunk_bytes,
                                    self.backed_chunks(), chunks)
        self.counters["physical_configured_headroom_bytes"] = self.prefill_headroom_bytes
        self.counters["physical_headroom_bytes"] = headroom
        self.counters["physical_chunk_cost_bytes"] = cost
        self.counters["physical_available_tokens_min"] = min(
            self.counters.get("physical_available_tokens_min", admitted), admitted)
        self.counters["physical_available_tokens_last"] = admitted
        if admitted < logical_free_tokens:
            self.counters["physical_limited_calls"] = self.counters.get("physical_limited_calls", 0) + 1
        self.counters["physical_available_ns"] = (
            self.counters.get("physical_available_ns", 0) + time.perf_counter_ns() - started)
        return admitted

    def can_commit_chunks(self, chunks):
        """Whether the missing chunks among `chunks` fit the committable budget."""
        chunks = {int(chunk) for chunk in chunks}
        if self.policy == "logical" or not chunks:
            return True
        budget = self._budget()
        if budget is None:
            return True
        admitted = len(chunks - self.backed_chunks()) <= budget[0]
        self.counters["request_affine_physical_preflight_calls"] = (
            self.counters.get("request_affine_physical_preflight_calls", 0) + 1)
        if not admitted:
            self.counters["request_affine_physical_fallbacks"] = (
                self.counters.get("request_affine_physical_fallbacks", 0) + 1)
        return admitted

    def precommit_after(self, ranges, chunk_count, idle):
        """Precommit up to `precommit_limit` idle chunks past each admitted range.

        Returns the chunk ids added; each is precommitted in every arena
        (zero-filled on the arena's side stream, fenced by its next ensure).
        """
        candidates = precommit_candidates(ranges, self.slot_bytes, self.chunk_bytes, chunk_count,
                                          self.precommit_lookahead, idle, self.precommitted)
        added = []
        for chunk in candidates:
            if len(self.precommitted) >= self.precommit_limit:
                break
            if sum(arena.precommit([chunk]) for arena in self.arenas):
                self.precommitted.add(chunk)
                added.append(chunk)
        if added:
            self.counters["precommit_batches"] = self.counters.get("precommit_batches", 0) + 1
            self.counters["precommit_chunks"] = self.counters.get("precommit_chunks", 0) + len(added)
        return added

    def admitted(self, chunks):
        """Chunks that became live leave the precommitted set (now simply backed)."""
        self.precommitted.difference_update(int(chunk) for chunk in chunks)
