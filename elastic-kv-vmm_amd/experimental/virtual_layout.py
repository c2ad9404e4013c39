"""Byte layout of independent, chunk-aligned request KV regions.

Same layout as the reference's experimental/virtual_layout.py:14-61 (it is an
addressing contract shared with gather_rows' direct mode): chunk 0 is a sink,
request r owns a chunk-aligned region starting at chunk_bytes + r *
request_bytes, and token t of request r starts row_bytes * t into it.
"""

from dataclasses import dataclass, fields


def _require_int(name, value, low, high=None):
    if type(value) is not int:
        raise TypeError(f"{name} must be an integer")
    if value < low or (high is not None and value > high):
        raise ValueError(f"{name} outside supported range")


@dataclass(frozen=True)
class VirtualKVLayout:
    max_requests: int
    max_tokens: int
    row_elements: int
    itemsize: int = 2
    chunk_bytes: int = 2 << 20

    def __post_init__(self):
        for field in fields(self):
            _require_int(field.name, getattr(self, field.name), 1)

    @property
    def row_bytes(self):
        return self.row_elements * self.itemsize

    @property
    def request_bytes(self):
        """Bytes of one request region: its rows rounded up to whole chunks."""
        return -(-self.max_tokens * self.row_bytes // self.chunk_bytes) * self.chunk_bytes

    @property
    def capacity_bytes(self):
        return self.chunk_bytes + self.max_requests * self.request_bytes

    def request_offset(self, req):
        _require_int("request index", req, 0, self.max_requests - 1)
        return self.chunk_bytes + req * self.request_bytes

    def token_offset(self, req, token):
        _require_int("token position", token, 0, self.max_tokens - 1)
        return self.request_offset(req) + token * self.row_bytes

    def _chunks_covering(self, start, size):
        if not size:
            return range(0)
        return range(start // self.chunk_bytes, (start + size - 1) // self.chunk_bytes + 1)

    def prefix_chunks(self, req, length):
        """Chunks holding tokens [0, length) of request `req`."""
        _require_int("prefix length", length, 0, self.max_tokens)
        return frozenset(self._chunks_covering(self.request_offset(req), length * self.row_bytes))

    def selected_chunks(self, req, positions):
        """Chunks touched by the rows of the given token positions."""
        self.request_offset(req)
        chunks = set()
        for token in positions:
            chunks.update(self._chunks_covering(self.token_offset(req, token), self.row_bytes))
        return frozenset(chunks)
