"""Chunk projection of logical KV chunks onto the K/V planes of one Backing.

Only the hot-path part of the reference's elastic_kv/adapter.py is rebuilt
here: PlaneProjection (:82-138). The SGLang pool installation and residency
policy of that module are serving-layer code outside this path.
"""

from .backing import Backing


class PlaneProjection:
    """Project logical chunk ids onto equally padded, contiguous planes.

    Logical chunk c lives at chunk plane * plane_chunks + c of the backing in
    every plane, so committing a logical chunk commits it in all planes.
    """

    def __init__(self, plane_bytes, planes, chunk_bytes, device, backing_factory=Backing):
        self.plane_chunks = -(-plane_bytes // chunk_bytes)
        self.plane_stride = self.plane_chunks * chunk_bytes
        self.plane_bytes = plane_bytes
        self.planes = planes
        self.backing = backing_factory(self.plane_stride * planes, chunk_bytes, device)
        self.mapped_chunks = set()
        self.precommitted_chunks = set()

    def _physical_chunks(self, indices):
        return [plane * self.plane_chunks + index for plane in range(self.planes) for index in indices]

    def ensure(self, indices):
        indices = set(indices)
        if (indices - self.mapped_chunks) or (self.precommitted_chunks & indices):
            self.backing.ensure(self._physical_chunks(indices))
            self.mapped_chunks.update(indices)
            self.precommitted_chunks.difference_update(indices)

    def precommit(self, indices):
        pending = set(indices) - self.mapped_chunks - self.precommitted_chunks
        if not pending:
            return 0
        self.backing.precommit(self._physical_chunks(pending))
        self.precommitted_chunks.update(pending)
        return len(pending)

    def reclaim(self, indices, *, synchronize=True):
        pending = (self.mapped_chunks | self.precommitted_chunks) & set(indices)
        if pending:
            self.backing.reclaim(self._physical_chunks(pending), synchronize=synchronize)
            self.mapped_chunks.difference_update(pending)
            self.precommitted_chunks.difference_update(pending)

    @property
    def allocated_chunks(self):
        return self.mapped_chunks | self.precommitted_chunks

    @property
    def backed_bytes(self):
        return self.backing.backed_bytes

    @property
    def metrics(self):
        return {**self.backing.metrics, "precommitted_chunks": len(self.precommitted_chunks)}

    def views(self, dtype, shape):
        raw = self.backing.raw
        return [raw.narrow(0, plane * self.plane_stride, self.plane_bytes).view(dtype).view(shape)
                for plane in range(self.planes)]
