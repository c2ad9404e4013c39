"""Chunk-aligned virtual regions of per-request KV rows.

The address map of the reference's experimental/virtual_layout.py:14-61, which
is the addressing contract of gather_rows' direct mode, so every number here
equals the reference's: the first chunk is a sink; request r owns
`chunks_per_request` chunks (the fewest that hold max_tokens rows) starting at
chunk 1 + r * chunks_per_request; token t's row starts t * row_bytes into the
request's region.
"""

from dataclasses import dataclass, fields


def _whole(name, value, low, high=None):
    """Check that value is an int (bool is not) within [low, high]."""
    if type(value) is not int:
        raise TypeError(f"{name} must be an integer, got {type(value).__name__}")
    if value < low or (high is not None and value > high):
        bound = f"[{low}, {high}]" if high is not None else f">= {low}"
        raise ValueError(f"{name} outside supported range: {value} not in {bound}")
    return value


@dataclass(frozen=True)
class VirtualKVLayout:
    max_requests: int
    max_tokens: int
    row_elements: int
    itemsize: int = 2
    chunk_bytes: int = 2 << 20

    def __post_init__(self):
        for spec in fields(self):
            _whole(spec.name, getattr(self, spec.name), 1)

    # ------------------------------------------------------------ sizes

    @property
    def row_bytes(self):
        return self.row_elements * self.itemsize

    @property
    def chunks_per_request(self):
        """Chunks of one request region: its max_tokens rows, rounded up."""
        return -(-(self.max_tokens * self.row_bytes) // self.chunk_bytes)

    @property
    def request_bytes(self):
        return self.chunks_per_request * self.chunk_bytes

    @property
    def capacity_bytes(self):
        return (1 + self.max_requests * self.chunks_per_request) * self.chunk_bytes

    # ------------------------------------------------------------ offsets

    def request_offset(self, req):
        _whole("request index", req, 0, self.max_requests - 1)
        return (1 + req * self.chunks_per_request) * self.chunk_bytes

    def token_offset(self, req, token):
        _whole("token position", token, 0, self.max_tokens - 1)
        return self.request_offset(req) + token * self.row_bytes

    # ------------------------------------------------------------ chunk sets

    def _span(self, first_byte, size):
        """Ids of the chunks that bytes [first_byte, first_byte + size) touch."""
        if size == 0:
            return range(0)
        last_byte = first_byte + size - 1
        return range(first_byte // self.chunk_bytes, last_byte // self.chunk_bytes + 1)

    def prefix_chunks(self, req, length):
        """Chunks holding the rows of tokens [0, length) of request `req`."""
        _whole("prefix length", length, 0, self.max_tokens)
        return frozenset(self._span(self.request_offset(req), length * self.row_bytes))

    def selected_chunks(self, req, positions):
        """Chunks holding the rows of the given token positions of request `req`."""
        base = self.request_offset(req)
        touched = set()
        for token in positions:
            _whole("token position", token, 0, self.max_tokens - 1)
            touched.update(self._span(base + token * self.row_bytes, self.row_bytes))
        return frozenset(touched)
