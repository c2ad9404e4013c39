"""Migration bandwidth estimation and byte/time admission caps (pure CPU).

Same API and arithmetic as the reference's adaptive_sparse/migration_budget.py:6-107:
a configured rate is used until a direction has a real sample, then an EWMA
(rate = alpha * sample + (1 - alpha) * rate) of successful transfers.
"""

import math

_DIRECTIONS = ("demotion", "promotion")


def _is_int(value):
    return isinstance(value, int) and not isinstance(value, bool)


class MigrationBandwidthEstimator:
    """Direction-specific transfer throughput from committed migrations."""

    DIRECTIONS = _DIRECTIONS

    def __init__(self, initial_bandwidth_bytes_per_s, ewma_alpha):
        if not _is_int(initial_bandwidth_bytes_per_s) or initial_bandwidth_bytes_per_s <= 0:
            raise ValueError("initial bandwidth must be a positive integer")
        if (isinstance(ewma_alpha, bool) or not isinstance(ewma_alpha, (int, float))
                or not math.isfinite(ewma_alpha) or not 0 < ewma_alpha <= 1):
            raise ValueError("EWMA alpha must be in (0, 1]")
        self.initial_bandwidth_bytes_per_s = initial_bandwidth_bytes_per_s
        self.ewma_alpha = float(ewma_alpha)
        self._rates = {}
        self._samples = dict.fromkeys(_DIRECTIONS, 0)

    @classmethod
    def _check_direction(cls, direction):
        if direction not in cls.DIRECTIONS:
            raise ValueError(f"unknown migration direction: {direction}")

    def observe(self, direction, transfer_bytes, elapsed_seconds):
        """Fold one transfer into the direction's rate; return its bandwidth or None."""
        self._check_direction(direction)
        if not _is_int(transfer_bytes) or transfer_bytes < 0:
            raise ValueError("transfer bytes must be a nonnegative integer")
        if (isinstance(elapsed_seconds, bool) or not isinstance(elapsed_seconds, (int, float))
                or not math.isfinite(elapsed_seconds)):
            raise ValueError("elapsed seconds must be finite")
        if transfer_bytes == 0 or elapsed_seconds <= 0:
            return None
        sample = transfer_bytes / float(elapsed_seconds)
        if direction in self._rates:
            alpha = self.ewma_alpha
            self._rates[direction] = alpha * sample + (1 - alpha) * self._rates[direction]
        else:
            self._rates[direction] = sample
        self._samples[direction] += 1
        return sample

    def bandwidth(self, direction):
        self._check_direction(direction)
        return self._rates.get(direction, float(self.initial_bandwidth_bytes_per_s))

    def samples(self, direction):
        self._check_direction(direction)
        return self._samples[direction]

    def effective_byte_cap(self, byte_cap, time_cap_ms, direction="demotion"):
        """Largest byte count allowed by both the byte cap and the time cap."""
        self._check_direction(direction)
        if not _is_int(byte_cap) or byte_cap < 1:
            raise ValueError("byte cap must be a positive integer")
        if not _is_int(time_cap_ms) or time_cap_ms < 0:
            raise ValueError("time cap must be a nonnegative integer")
        if time_cap_ms == 0:
            return byte_cap
        transferable = int(self.bandwidth(direction) * time_cap_ms / 1000.0)
        return min(byte_cap, max(0, transferable))

    def snapshot(self):
        return {direction: self.bandwidth(direction) for direction in self.DIRECTIONS}

    def sample_counts(self):
        return dict(self._samples)
