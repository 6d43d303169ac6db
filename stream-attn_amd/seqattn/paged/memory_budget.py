"""Operator-owned host memory accounting (reference paged/memory_budget.py:8-117).

Four categories, each with its own limit, under one total budget:
``pinned`` (page-locked staging the copy engines read), ``bounce`` (aligned
O_DIRECT buffers), ``cache`` (the DRAM page cache, limit = total minus the
other three reservations) and ``metadata`` (a fixed margin registered up
front).  ``register`` raises MemoryError before an allocation would exceed a
limit, so a run never allocates past its budget.
"""

from __future__ import annotations

import threading
from dataclasses import asdict, dataclass

CATEGORIES = ("pinned", "bounce", "cache", "metadata")


@dataclass(frozen=True)
class HostMemorySnapshot:
    operator_host_allocated_bytes: int
    operator_host_peak_bytes: int
    pinned_allocated_bytes: int
    pinned_peak_bytes: int
    direct_io_bounce_allocated_bytes: int
    direct_io_bounce_peak_bytes: int
    dram_cache_allocated_bytes: int
    dram_cache_peak_bytes: int
    metadata_allocated_bytes: int
    host_memory_budget_bytes: int

    def as_dict(self) -> dict[str, int]:
        return asdict(self)


class HostMemoryPlan:
    """Thread-safe ledger of every host allocation a paged run owns."""

    def __init__(
        self,
        *,
        total_budget_bytes: int,
        pinned_limit_bytes: int,
        bounce_limit_bytes: int,
        metadata_margin_bytes: int,
    ) -> None:
        if total_budget_bytes <= 0:
            raise ValueError("total_budget_bytes must be positive")
        if min(pinned_limit_bytes, bounce_limit_bytes, metadata_margin_bytes) < 0:
            raise ValueError("host memory limits must be non-negative")
        reserved = pinned_limit_bytes + bounce_limit_bytes + metadata_margin_bytes
        if reserved >= total_budget_bytes:
            raise ValueError("host reservations leave no room for the DRAM cache")
        self.total_budget_bytes = total_budget_bytes
        self.pinned_limit_bytes = pinned_limit_bytes
        self.bounce_limit_bytes = bounce_limit_bytes
        self.metadata_margin_bytes = metadata_margin_bytes
        self.cache_limit_bytes = total_budget_bytes - reserved
        self._limits = {
            "pinned": pinned_limit_bytes,
            "bounce": bounce_limit_bytes,
            "cache": self.cache_limit_bytes,
            "metadata": metadata_margin_bytes,
        }
        self._current = dict.fromkeys(CATEGORIES, 0)
        self._peak = dict.fromkeys(CATEGORIES, 0)
        self._peak_total = 0
        self._lock = threading.Lock()
        self.register("metadata", metadata_margin_bytes)

    def _check_category(self, category: str, size_bytes: int) -> None:
        if category not in self._limits:
            raise ValueError(f"unknown host allocation category: {category}")
        if size_bytes < 0:
            raise ValueError("allocation size must be non-negative")

    def register(self, category: str, size_bytes: int) -> None:
        self._check_category(category, size_bytes)
        with self._lock:
            after = self._current[category] + size_bytes
            if after > self._limits[category]:
                raise MemoryError(
                    f"{category} allocation exceeds its limit: {after} > {self._limits[category]} bytes"
                )
            total = sum(self._current.values()) + size_bytes
            if total > self.total_budget_bytes:
                raise MemoryError(
                    "operator-owned host allocation exceeds the configured budget: "
                    f"{total} > {self.total_budget_bytes} bytes"
                )
            self._current[category] = after
            self._peak[category] = max(self._peak[category], after)
            self._peak_total = max(self._peak_total, total)

    def release(self, category: str, size_bytes: int) -> None:
        self._check_category(category, size_bytes)
        with self._lock:
            if size_bytes > self._current[category]:
                raise RuntimeError(f"released more {category} memory than was registered")
            self._current[category] -= size_bytes

    def available(self, category: str) -> int:
        """Bytes ``category`` can still register under both of its limits."""
        self._check_category(category, 0)
        with self._lock:
            return max(0, min(self._limits[category] - self._current[category],
                              self.total_budget_bytes - sum(self._current.values())))

    @property
    def current_bytes(self) -> int:
        with self._lock:
            return sum(self._current.values())

    def snapshot(self) -> HostMemorySnapshot:
        with self._lock:
            return HostMemorySnapshot(
                operator_host_allocated_bytes=sum(self._current.values()),
                operator_host_peak_bytes=self._peak_total,
                pinned_allocated_bytes=self._current["pinned"],
                pinned_peak_bytes=self._peak["pinned"],
                direct_io_bounce_allocated_bytes=self._current["bounce"],
                direct_io_bounce_peak_bytes=self._peak["bounce"],
                dram_cache_allocated_bytes=self._current["cache"],
                dram_cache_peak_bytes=self._peak["cache"],
                metadata_allocated_bytes=self._current["metadata"],
                host_memory_budget_bytes=self.total_budget_bytes,
            )


__all__ = ["HostMemoryPlan", "HostMemorySnapshot"]
