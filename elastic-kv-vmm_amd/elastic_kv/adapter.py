"""Logical KV chunks projected onto the equally padded K/V planes of one Backing.

Only the hot-path part of the reference's elastic_kv/adapter.py is rebuilt
here: PlaneProjection (:82-138), with its constructor, methods, properties and
metric key. The SGLang pool installation and residency policy of that module
are serving-layer code outside this path.

The projection: each of `planes` planes is padded to whole chunks
(plane_chunks of them), and logical chunk c of the KV is chunk
p * plane_chunks + c of the backing in plane p, so a logical chunk is
committed, precommitted or released in every plane at once. The projection
keeps the state of each logical chunk it committed: READY (ensured) or
ZEROING (precommitted; its zero fill may run until the next ensure of it).
"""

from .backing import Backing

READY, ZEROING = "ready", "zeroing"


class PlaneProjection:
    def __init__(self, plane_bytes, planes, chunk_bytes, device, backing_factory=Backing):
        self.plane_bytes = plane_bytes
        self.planes = planes
        self.plane_chunks = -(-plane_bytes // chunk_bytes)
        self.plane_stride = self.plane_chunks * chunk_bytes
        self.backing = backing_factory(self.plane_stride * planes, chunk_bytes, device)
        self._state = {}            # logical chunk -> READY | ZEROING

    def _in_every_plane(self, logical):
        """Backing chunk ids of the given logical chunks, plane by plane."""
        return [plane * self.plane_chunks + chunk for plane in range(self.planes) for chunk in logical]

    def ensure(self, indices):
        """Commit the logical chunks (waiting for any of them still zeroing) in every plane."""
        wanted = set(indices)
        if all(self._state.get(chunk) == READY for chunk in wanted):
            return
        self.backing.ensure(self._in_every_plane(wanted))
        self._state.update(dict.fromkeys(wanted, READY))

    def precommit(self, indices):
        """Start committing the logical chunks not yet held; returns how many."""
        fresh = set(indices).difference(self._state)
        if fresh:
            self.backing.precommit(self._in_every_plane(fresh))
            self._state.update(dict.fromkeys(fresh, ZEROING))
        return len(fresh)

    def reclaim(self, indices, *, synchronize=True):
        """Release the held logical chunks among `indices` in every plane."""
        held = set(indices).intersection(self._state)
        if held:
            self.backing.reclaim(self._in_every_plane(held), synchronize=synchronize)
            for chunk in held:
                del self._state[chunk]

    @property
    def mapped_chunks(self):
        return {chunk for chunk, state in self._state.items() if state == READY}

    @property
    def precommitted_chunks(self):
        return {chunk for chunk, state in self._state.items() if state == ZEROING}

    @property
    def allocated_chunks(self):
        return set(self._state)

    @property
    def backed_bytes(self):
        return self.backing.backed_bytes

    @property
    def metrics(self):
        return {**self.backing.metrics, "precommitted_chunks": len(self.precommitted_chunks)}

    def views(self, dtype, shape):
        """One borrowed tensor of `shape` per plane, over the plane's unpadded bytes."""
        raw = self.backing.raw
        return [raw.narrow(0, plane * self.plane_stride, self.plane_bytes).view(dtype).view(shape)
                for plane in range(self.planes)]
