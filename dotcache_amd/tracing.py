"""Byte and call counters for the hip_mi355x backend.

The subset of reference ``dotcache/tracing.py:6-239`` that this backend
feeds: page bytes read (payload vs metadata), host-to-device bytes, and
per-entry-point call counts.  ``device_bytes_read`` counts compressed bytes
(codes, fp16 scales / biases, escape rows) for valid tokens -- the
algorithmic bytes of the roofline -- while ``metadata_bytes_read`` keeps
the reference's convention of including the JSON header length.
"""
from __future__ import annotations

from collections import Counter
from dataclasses import dataclass, field


@dataclass(slots=True)
class ExecutionTrace:
    payload_bytes_read: int = 0
    metadata_bytes_read: int = 0
    device_bytes_read: int = 0
    host_to_device_bytes: int = 0
    prepared_page_cache_hits: int = 0
    prepared_page_cache_misses: int = 0
    cache_resident_bytes: int = 0
    prepared_page_cache_evictions: int = 0
    cache_evicted_bytes: int = 0
    calls: Counter = field(default_factory=Counter)

    def record_page_read(self, payload_bytes: int, metadata_bytes: int) -> None:
        self.payload_bytes_read += int(payload_bytes)
        self.metadata_bytes_read += int(metadata_bytes)

    def record_device_read(self, nbytes: int) -> None:
        self.device_bytes_read += int(nbytes)

    def record_host_to_device(self, nbytes: int) -> None:
        self.host_to_device_bytes += int(nbytes)

    def record_call(self, name: str) -> None:
        self.calls[name] += 1

    # prepared-page cache counters (reference tracing.py:82-93)
    def record_cache_hit(self, count: int = 1) -> None:
        self.prepared_page_cache_hits += int(count)

    def record_cache_miss(self, count: int = 1) -> None:
        self.prepared_page_cache_misses += int(count)

    def observe_cache_resident_bytes(self, nbytes: int) -> None:
        self.cache_resident_bytes = max(self.cache_resident_bytes, int(nbytes))

    def record_cache_eviction(self, nbytes: int, count: int = 1) -> None:
        self.prepared_page_cache_evictions += int(count)
        self.cache_evicted_bytes += int(nbytes)

    @property
    def total_bytes_read(self) -> int:
        return self.payload_bytes_read + self.metadata_bytes_read

    def to_dict(self) -> dict:
        return {
            "payload_bytes_read": self.payload_bytes_read,
            "metadata_bytes_read": self.metadata_bytes_read,
            "device_bytes_read": self.device_bytes_read,
            "host_to_device_bytes": self.host_to_device_bytes,
            "prepared_page_cache_hits": self.prepared_page_cache_hits,
            "prepared_page_cache_misses": self.prepared_page_cache_misses,
            "cache_resident_bytes": self.cache_resident_bytes,
            "prepared_page_cache_evictions": self.prepared_page_cache_evictions,
            "cache_evicted_bytes": self.cache_evicted_bytes,
            "calls": dict(self.calls),
        }
