"""Byte layouts of KV pools over one VMM Backing, and their plane descriptors.

Two layouts cover the pools of this path:

* PlanePoolLayout - plane-major, the MiniMax main-pool layout of the
  reference (adaptive_sparse/minimax_vmm.py:220-243): one plane per
  (layer, K|V), each padded to whole chunks, slot s of a plane at
  s * row_bytes. Slot 0 of every plane is the sink row.
* BlockMajorLayout - every block (page) holds all of its planes contiguously,
  so committing a block commits about one chunk per block-MiB instead of one
  chunk per plane. Used by the migration pool.

KVPlanes is what the gather/scatter kernels consume: a base address plus the
strides of (layer, kv, slot).
"""

from dataclasses import dataclass, field


def _positive(name, value):
    if type(value) is not int or value < 1:
        raise ValueError(f"{name} must be a positive integer")


@dataclass(frozen=True)
class KVPlanes:
    """Planes (layer, kv) of slot rows inside a device address range."""

    base: int
    device: int
    layers: int
    kv: int
    layer_stride: int
    kv_stride: int
    row_stride: int
    row_bytes: int
    rows: int
    owner: object = field(default=None, compare=False, repr=False)

    def row_offset(self, layer, kv, slot):
        """Byte offset of a slot row from `base`."""
        return layer * self.layer_stride + kv * self.kv_stride + slot * self.row_stride


@dataclass(frozen=True)
class PlanePoolLayout:
    layers: int
    kv: int
    rows: int
    row_bytes: int
    chunk_bytes: int = 2 << 20

    def __post_init__(self):
        for name in ("layers", "kv", "rows", "row_bytes", "chunk_bytes"):
            _positive(name, getattr(self, name))
        if self.kv not in (1, 2):
            raise ValueError("kv must be 1 or 2")

    @property
    def planes(self):
        return self.layers * self.kv

    @property
    def plane_bytes(self):
        return self.rows * self.row_bytes

    @property
    def plane_chunks(self):
        return -(-self.plane_bytes // self.chunk_bytes)

    @property
    def plane_stride(self):
        return self.plane_chunks * self.chunk_bytes

    @property
    def capacity_bytes(self):
        return self.planes * self.plane_stride

    def plane_offset(self, layer, kv):
        return (layer * self.kv + kv) * self.plane_stride

    def chunks_for_slots(self, slots):
        """Chunk ids of every plane row of the given slots."""
        chunks = set()
        for slot in slots:
            if not 0 <= slot < self.rows:
                raise ValueError(f"slot {slot} outside the pool")
            begin = slot * self.row_bytes
            first, last = begin // self.chunk_bytes, (begin + self.row_bytes - 1) // self.chunk_bytes
            for plane in range(self.planes):
                base = plane * self.plane_chunks
                chunks.update(range(base + first, base + last + 1))
        return chunks

    def chunks_for_slot_range(self, start, stop):
        """Chunk ids covering slots [start, stop) in every plane."""
        if not 0 <= start <= stop <= self.rows:
            raise ValueError("slot range outside the pool")
        if start == stop:
            return set()
        first = start * self.row_bytes // self.chunk_bytes
        last = (stop * self.row_bytes - 1) // self.chunk_bytes
        return {plane * self.plane_chunks + c for plane in range(self.planes) for c in range(first, last + 1)}

    def kv_planes(self, base, device, owner=None):
        return KVPlanes(base=base, device=device, layers=self.layers, kv=self.kv,
                        layer_stride=self.kv * self.plane_stride, kv_stride=self.plane_stride,
                        row_stride=self.row_bytes, row_bytes=self.row_bytes, rows=self.rows, owner=owner)


@dataclass(frozen=True)
class BlockMajorLayout:
    """Blocks of `layers` x `kv` plane rows of `row_bytes`, block after block.

    A block's plane (layer, kv) row sits at block * block_bytes +
    (layer * kv_count + kv) * row_bytes. Block 0 is the sink.
    """

    blocks: int
    layers: int
    kv: int
    row_bytes: int
    chunk_bytes: int = 2 << 20

    def __post_init__(self):
        for name in ("blocks", "layers", "kv", "row_bytes", "chunk_bytes"):
            _positive(name, getattr(self, name))
        if self.kv not in (1, 2):
            raise ValueError("kv must be 1 or 2")

    @property
    def block_bytes(self):
        return self.layers * self.kv * self.row_bytes

    @property
    def capacity_bytes(self):
        return -(-self.blocks * self.block_bytes // self.chunk_bytes) * self.chunk_bytes

    def chunks_for_blocks(self, blocks):
        chunks = set()
        for block in blocks:
            if not 0 <= block < self.blocks:
                raise ValueError(f"block {block} outside the pool")
            begin = block * self.block_bytes
            chunks.update(range(begin // self.chunk_bytes, (begin + self.block_bytes - 1) // self.chunk_bytes + 1))
        return chunks

    def kv_planes(self, base, device, owner=None):
        return KVPlanes(base=base, device=device, layers=self.layers, kv=self.kv,
                        layer_stride=self.kv * self.row_bytes, kv_stride=self.row_bytes,
                        row_stride=self.block_bytes, row_bytes=self.row_bytes, rows=self.blocks,
                        owner=owner)


class BlockSegments:
    """Chunk projection of vLLM-style KV tensors sharing one backing allocation.

    Follows vllm_integration/adapter.py:31-64 (Residency): every layer tensor
    is a segment (start, block_stride) of the allocation, block b of a
    segment occupies [start + b * block_stride, + page_bytes), and a block's
    chunks are those every segment's page touches.
    """

    def __init__(self, segments, page_bytes, num_blocks, allocation_bytes, chunk_bytes=2 << 20):
        self.segments = [(int(start), int(stride)) for start, stride in segments]
        self.page_bytes = int(page_bytes)
        self.num_blocks = int(num_blocks)
        self.chunk_bytes = int(chunk_bytes)
        _positive("page_bytes", self.page_bytes)
        _positive("chunk_bytes", self.chunk_bytes)
        if self.num_blocks < 2:
            raise ValueError("a block layout needs at least two blocks (block 0 is the sink)")
        if any(start < 0 or stride <= 0 or start + (self.num_blocks - 1) * stride + self.page_bytes > allocation_bytes
               for start, stride in self.segments):
            raise ValueError("KV tensor segments exceed the allocation")

    def chunks(self, blocks):
        """Chunk ids holding any byte of the given blocks in any segment."""
        indices = set()
        for block in blocks:
            if not 0 <= block < self.num_blocks:
                raise ValueError(f"Invalid KV block {block}")
            for start, stride in self.segments:
                offset = start + block * stride
                indices.update(range(offset // self.chunk_bytes, (offset + self.page_bytes - 1) // self.chunk_bytes + 1))
        return indices

    def sink_chunks(self):
        """Chunks that stay mapped for the sink block 0 (and chunk 0)."""
        return self.chunks([0]) | {0}
