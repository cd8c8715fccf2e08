"""Non-overlapping wall-time stages (src/vesper/timing.py:7-31) with the reference's stage names."""

from __future__ import annotations

from contextlib import contextmanager
import time


class Timings:
    def __init__(self):
        self.totals: dict[str, float] = {}
        self.counts: dict[str, int] = {}
        self._active = None

    @contextmanager
    def section(self, name: str):
        if self._active is not None:
            raise RuntimeError(f"timing section {name!r} would overlap {self._active!r}")
        self._active = name
        start = time.perf_counter()
        try:
            yield
        finally:
            self.totals[name] = self.totals.get(name, 0.0) + (time.perf_counter() - start) * 1000.0
            self.counts[name] = self.counts.get(name, 0) + 1
            self._active = None

    def snapshot(self) -> dict:
        return {name: {"ms": self.totals[name], "count": self.counts[name]} for name in self.totals}
