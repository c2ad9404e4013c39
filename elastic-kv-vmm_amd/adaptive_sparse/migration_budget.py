"""Migration bandwidth estimation and byte / time admission caps (pure CPU).

The interface of the reference's adaptive_sparse/migration_budget.py:6-107:
each direction (demotion, promotion) reports the configured rate until it has
seen a transfer of real size, then the exponentially weighted mean
rate <- alpha * sample + (1 - alpha) * rate of its successful transfers; a
time cap turns that rate into a byte cap, never above the configured one.
Here each direction's state is one small record, and the argument checks
are shared predicates.
"""

import math
from dataclasses import dataclass


def _integer(value):
    return isinstance(value, int) and not isinstance(value, bool)


def _real(value):
    return isinstance(value, (int, float)) and not isinstance(value, bool) and math.isfinite(value)


def _require(ok, message):
    if not ok:
        raise ValueError(message)


@dataclass
class _Direction:
    rate: float = None     # bytes/s; None until the first sample
    samples: int = 0

    def fold(self, sample, alpha):
        self.rate = sample if self.rate is None else alpha * sample + (1.0 - alpha) * self.rate
        self.samples += 1


class MigrationBandwidthEstimator:
    """Per-direction transfer throughput of committed migrations and the caps it implies."""

    DIRECTIONS = ("demotion", "promotion")

    def __init__(self, initial_bandwidth_bytes_per_s, ewma_alpha):
        _require(_integer(initial_bandwidth_bytes_per_s) and initial_bandwidth_bytes_per_s > 0,
                 "initial bandwidth must be a positive integer")
        _require(_real(ewma_alpha) and 0 < ewma_alpha <= 1, "EWMA alpha must be in (0, 1]")
        self.initial_bandwidth_bytes_per_s = initial_bandwidth_bytes_per_s
        self.ewma_alpha = float(ewma_alpha)
        self._state = {direction: _Direction() for direction in self.DIRECTIONS}

    def _direction(self, direction):
        state = self._state.get(direction)
        _require(state is not None, f"unknown migration direction: {direction}")
        return state

    def observe(self, direction, transfer_bytes, elapsed_seconds):
        """Fold one transfer into `direction`'s rate; returns its bandwidth, or None for an empty one."""
        state = self._direction(direction)
        _require(_integer(transfer_bytes) and transfer_bytes >= 0, "transfer bytes must be a nonnegative integer")
        _require(_real(elapsed_seconds), "elapsed seconds must be finite")
        if transfer_bytes == 0 or elapsed_seconds <= 0:
            return None
        sample = transfer_bytes / float(elapsed_seconds)
        state.fold(sample, self.ewma_alpha)
        return sample

    def bandwidth(self, direction):
        rate = self._direction(direction).rate
        return float(self.initial_bandwidth_bytes_per_s) if rate is None else rate

    def samples(self, direction):
        return self._direction(direction).samples

    def effective_byte_cap(self, byte_cap, time_cap_ms, direction="demotion"):
        """The most bytes both caps allow: byte_cap, lowered to what `direction` moves in time_cap_ms (0 = no time cap)."""
        rate = self.bandwidth(direction)
        _require(_integer(byte_cap) and byte_cap >= 1, "byte cap must be a positive integer")
        _require(_integer(time_cap_ms) and time_cap_ms >= 0, "time cap must be a nonnegative integer")
        if time_cap_ms == 0:
            return byte_cap
        return min(byte_cap, max(0, int(rate * time_cap_ms / 1000.0)))

    def snapshot(self):
        return {direction: self.bandwidth(direction) for direction in self.DIRECTIONS}

    def sample_counts(self):
        return {direction: state.samples for direction, state in self._state.items()}
