"""Which physical chunks a demotion of one or more requests would free.

Restates the release accounting of the reference's
adaptive_sparse/scheduler_budget.py:
  * per-page chunk counts and the release rule (:151-162);
  * pair and group release, exact when two requests name the same page
    (:165-189);
  * bounded enumeration of request groups under a byte cap and a search
    budget (:192-242);
  * the incremental page/chunk owner index (:245-297), the owner-closure
    group search (:299-385) and its exact fallback (:388-431).
The scheduler budget that ranks and runs demotions with these numbers is
serving policy and is not part of this package.

A tracker is anything with `chunks(page)` (the chunk ids a page touches),
`refs` (chunk -> number of live pages on it), `backing.mapped_chunks` and
`chunk_bytes`, such as `minimax_vmm.PhysicalPages`. Demoting a set of pages
frees a chunk when the chunk is mapped and every live page on it is in the
set. A request entry, as the reference's scheduler keeps it, is a tuple whose
item 1 is the request's page set and item 2 its per-chunk page counts.
"""

from collections import Counter, deque
from itertools import combinations, islice


def chunk_release_counts(tracker, pages):
    """Counter of chunk -> how many of `pages` touch it."""
    counts = Counter()
    for page in pages:
        counts.update(tracker.chunks(page))
    return counts


def releasable_counts(tracker, counts):
    """Chunks whose every live page is counted in `counts`, and that are mapped."""
    refs = tracker.refs
    mapped = tracker.backing.mapped_chunks
    return {chunk for chunk, held in counts.items() if chunk in mapped and refs.get(chunk) == held}


def releasable(tracker, pages):
    """Chunks freed by demoting the page set `pages` (duplicates count once)."""
    return releasable_counts(tracker, chunk_release_counts(tracker, set(pages)))


def releasable_group(tracker, candidates):
    """Chunks freed by demoting every (pages, counts) candidate together.

    Counts add up when the candidates own disjoint pages. A page named by two
    candidates would be counted twice, so then the union of the pages is
    recounted from the tracker.
    """
    union = set()
    total = Counter()
    shared = False
    for pages, counts in candidates:
        if not shared and not union.isdisjoint(pages):
            shared = True
        union.update(pages)
        total.update(counts)
    return releasable(tracker, union) if shared else releasable_counts(tracker, total)


def releasable_pair(tracker, left_pages, left_counts, right_pages, right_counts):
    """`releasable_group` of two candidates."""
    return releasable_group(tracker, ((left_pages, left_counts), (right_pages, right_counts)))


def _rotated(request_ids, rotation):
    ordered = sorted(request_ids)
    if not ordered:
        return ordered
    cut = rotation % len(ordered)
    return ordered[cut:] + ordered[:cut]


class _GroupScorer:
    """Prices and scores candidate groups; keeps the search's tallies."""

    def __init__(self, tracker, requests, cost, byte_cap, cap_observer):
        self.tracker = tracker
        self.requests = requests
        self.cost = cost
        self.byte_cap = byte_cap
        self.cap_observer = cap_observer
        self.groups = {}            # sorted group -> (released bytes, transfer bytes)
        self.chunks = {}            # sorted group -> released chunk ids
        self.examined = 0
        self.rejected = 0

    def score(self, group):
        self.examined += 1
        transfer = sum(self.cost(request_id) for request_id in group)
        if transfer > self.byte_cap:
            self.rejected += 1
            if self.cap_observer is not None:
                self.cap_observer(transfer)
            return
        entries = ((self.requests[request_id][1], self.requests[request_id][2]) for request_id in group)
        released = releasable_group(self.tracker, entries)
        if released:
            key = tuple(sorted(group))
            self.groups[key] = (len(released) * self.tracker.chunk_bytes, transfer)
            self.chunks[key] = released


def bounded_demotion_groups(tracker, requests, cost, *, max_group, byte_cap, search_limit, rotation=0,
                            cap_observer=None):
    """Score every group of 2..max_group requests, within a search budget.

    Request ids are sorted and rotated by `rotation` so that successive calls
    start their combinations at different requests. `search_limit` is split
    evenly over the group sizes (the smaller sizes get the remainder); a size
    whose combinations outlast its share sets `truncated`. Groups whose summed
    `cost` exceeds `byte_cap` are counted in `rejected` and reported to
    `cap_observer`.

    Returns (groups, chunks, examined, truncated, rejected): `groups` maps each
    sorted group that frees chunks to (freed bytes, transfer bytes), `chunks`
    to the freed chunk ids.
    """
    if search_limit < 1:
        raise ValueError("search_limit must be positive")
    order = _rotated(requests, rotation)
    sizes = range(2, min(max_group, len(order)) + 1)
    share, spare = divmod(search_limit, max(1, len(sizes)))
    scorer = _GroupScorer(tracker, requests, cost, byte_cap, cap_observer)
    truncated = False
    for rank, size in enumerate(sizes):
        pending = combinations(order, size)
        for group in islice(pending, share + (rank < spare)):
            scorer.score(group)
        if next(pending, None) is not None:
            truncated = True
    return scorer.groups, scorer.chunks, scorer.examined, truncated, scorer.rejected


class PhysicalDemandIndex:
    """Page and chunk owners of the candidate requests, updated per request.

    `records` maps request id -> (frozenset of pages, Counter of chunk counts
    without zero entries); `page_owners` maps page -> set of request ids;
    `chunk_owners` maps chunk -> {request id: pages of that request on it}.
    `sync` re-indexes only the requests whose entry changed.
    """

    def __init__(self):
        self.records = {}
        self.page_owners = {}
        self.chunk_owners = {}

    def sync(self, requests):
        """Bring the index to `requests`; return how many requests were added, changed or dropped."""
        changed = 0
        for request_id in [r for r in self.records if r not in requests]:
            self._drop(request_id)
            changed += 1
        for request_id, entry in requests.items():
            record = (frozenset(entry[1]), Counter({chunk: n for chunk, n in entry[2].items() if n}))
            current = self.records.get(request_id)
            if current == record:
                continue
            if current is not None:
                self._drop(request_id)
            self._index(request_id, record)
            changed += 1
        return changed

    def _index(self, request_id, record):
        pages, chunks = record
        self.records[request_id] = record
        for page in pages:
            self.page_owners.setdefault(page, set()).add(request_id)
        for chunk, held in chunks.items():
            self.chunk_owners.setdefault(chunk, {})[request_id] = held

    def _drop(self, request_id):
        pages, chunks = self.records.pop(request_id)
        for page in pages:
            owners = self.page_owners[page]
            owners.discard(request_id)
            if not owners:
                del self.page_owners[page]
        for chunk in chunks:
            owners = self.chunk_owners[chunk]
            del owners[request_id]
            if not owners:
                del self.chunk_owners[chunk]

    @property
    def has_page_overlap(self):
        """True when some page is named by more than one request."""
        return any(len(owners) > 1 for owners in self.page_owners.values())

    def candidate_groups(self, tracker, *, max_group, candidate_limit, rotation=0):
        """Groups closed over the owners of chunks they could free, breadth first.

        Starting from each request alone, a group grows by the owners of one of
        its chunks whose indexed pages are all of that chunk's live pages (only
        such chunks can ever be freed by indexed requests), as long as it stays
        within `max_group`. Every group of two or more requests reached is a
        candidate, ordered by the rotated request order. The walk stops, with
        `truncated` set, after a group below `max_group` is expanded once
        `candidate_limit` groups have been visited; full-size groups are
        collected without that check. The chunks of a group are followed in
        ascending id order, so a truncated walk visits the same groups on
        every call.
        """
        order = _rotated(self.records, rotation)
        position = {request_id: i for i, request_id in enumerate(order)}
        queue = deque((request_id,) for request_id in order)
        visited = set()
        found = set()
        truncated = False
        while queue:
            group = tuple(sorted(queue.popleft()))
            if group in visited:
                continue
            visited.add(group)
            if len(group) >= 2:
                found.add(group)
            if len(group) >= max_group:
                continue                        # full groups neither grow nor count toward the limit
            members = set(group)
            chunks = set()
            for request_id in group:
                chunks.update(self.records[request_id][1])
            for chunk in sorted(chunks):
                owners = self.chunk_owners.get(chunk, {})
                if sum(owners.values()) != tracker.refs.get(chunk):
                    continue
                grown = tuple(sorted(members | owners.keys()))
                if grown != group and len(grown) <= max_group:
                    queue.append(grown)
            if len(visited) >= candidate_limit:
                truncated = True
                break
        ordered = sorted(found, key=lambda group: [position[request_id] for request_id in group])
        return ordered, truncated


def indexed_demotion_groups(index, tracker, requests, cost, *, max_group, byte_cap, search_limit, rotation=0,
                            cap_observer=None):
    """Score the owner-closure candidates of `index`, at most `search_limit` of them.

    The closure walk may visit max(32, 4 * search_limit) groups. Returns
    (groups, chunks, examined, truncated, rejected) as `bounded_demotion_groups`.
    """
    if search_limit < 1:
        raise ValueError("search_limit must be positive")
    candidates, truncated = index.candidate_groups(tracker, max_group=max_group,
                                                   candidate_limit=max(32, 4 * search_limit), rotation=rotation)
    scorer = _GroupScorer(tracker, requests, cost, byte_cap, cap_observer)
    if len(candidates) > search_limit:
        truncated = True
    for group in candidates[:search_limit]:
        scorer.score(group)
    return scorer.groups, scorer.chunks, scorer.examined, truncated, scorer.rejected


def demand_index_demotion_groups(index, tracker, requests, cost, *, max_group, byte_cap, search_limit, rotation=0,
                                 cap_observer=None):
    """Owner-closure search, then exhaustive enumeration if it found nothing and pages overlap.

    Two requests that name the same page break the additive counts the closure
    walk relies on, so only then does an empty result fall back to
    `bounded_demotion_groups`. Returns (groups, chunks, indexed examined,
    fallback examined, indexed truncated, fallback truncated, rejected in
    both, whether the fallback ran).
    """
    groups, chunks, examined, truncated, rejected = indexed_demotion_groups(
        index, tracker, requests, cost, max_group=max_group, byte_cap=byte_cap, search_limit=search_limit,
        rotation=rotation, cap_observer=cap_observer)
    if groups or not index.has_page_overlap:
        return groups, chunks, examined, 0, truncated, False, rejected, False
    groups, chunks, fallback_examined, fallback_truncated, fallback_rejected = bounded_demotion_groups(
        tracker, requests, cost, max_group=max_group, byte_cap=byte_cap, search_limit=search_limit,
        rotation=rotation, cap_observer=cap_observer)
    return (groups, chunks, examined, fallback_examined, truncated, fallback_truncated,
            rejected + fallback_rejected, True)
