"""Host-memory reservations of the expert tiers (the reference's MemoryBudget, src/vesper/resources.py:35-110).

A budget counts the bytes a component has explicitly reserved -- pinned staging, the RAM tier's copies,
direct-I/O buffers, digest tables -- against a cap, and refuses a reservation that would leave less than
`available_floor` bytes of the machine's available memory (/proc/meminfo MemAvailable). It does not track
process RSS. The reference's process-wide memory governor (src/vesper/memory.py) is outside this path: there is
no policy object, so reclaimer registration is a no-op.
"""

from __future__ import annotations

import threading
from dataclasses import dataclass, field
from pathlib import Path

GiB = 1 << 30
MiB = 1 << 20


def physical_memory() -> dict:
    """{"total", "available"} bytes of this machine (Linux /proc/meminfo)."""
    info = {}
    for line in Path("/proc/meminfo").read_text().splitlines():
        name, _, rest = line.partition(":")
        if name in ("MemTotal", "MemAvailable"):
            info[name] = int(rest.split()[0]) * 1024
    return {"total": info["MemTotal"], "available": info["MemAvailable"]}


@dataclass
class MemoryBudget:
    """Owned-allocation ledger: cap on reserved bytes plus a floor on the machine's available memory."""

    cap: int = 96 * GiB
    available_floor: int = 32 * GiB
    reserved: int = 0
    peak: int = 0
    owner: str = "expert_tiers"
    category: str = "admission"
    by_category: dict = field(default_factory=dict, compare=False, repr=False)
    _lock: object = field(default_factory=threading.RLock, compare=False, repr=False)
    _policy: object = field(default=None, compare=False, repr=False)

    def __post_init__(self):
        if self.cap <= 0 or self.available_floor < 0:
            raise ValueError("Invalid memory budget")

    def acquire(self, size: int, available: int | None = None, *, category: str | None = None) -> None:
        """Reserve `size` bytes; MemoryError when the cap or the available-memory floor would be crossed."""
        if size < 0:
            raise ValueError("Negative allocation")
        with self._lock:
            if size > self.cap - self.reserved:
                raise MemoryError("Allocation exceeds the owned-memory cap")
            free = physical_memory()["available"] if available is None else available
            if size > free - self.available_floor:
                raise MemoryError("Allocation would consume the system memory reserve")
            self.reserved += size
            self.peak = max(self.peak, self.reserved)
            name = category or self.category
            self.by_category[name] = self.by_category.get(name, 0) + size

    def release(self, size: int, *, category: str | None = None) -> None:
        with self._lock:
            if size < 0 or size > self.reserved:
                raise ValueError("Invalid release")
            self.reserved -= size
            name = category or self.category
            self.by_category[name] = self.by_category.get(name, 0) - size

    def register_reclaimer(self, callback):
        """No process-wide memory policy exists in this build: nothing calls reclaimers."""
        return None

    @staticmethod
    def unregister_reclaimer(handle):
        return None
