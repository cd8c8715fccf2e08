"""Non-overlapping wall-time stages (src/vesper/timing.py:7-31) with the reference's stage names.

Timings(enabled) collects per-stage totals and call counts; a disabled collector never reads the clock.
snapshot() gives the totals, since(before) the per-stage change between two snapshots (the per-call
deltas the tiered runtime reports).
"""

from __future__ import annotations

from contextlib import contextmanager
import time


class Timings:
    def __init__(self, enabled: bool = True):
        self.enabled = bool(enabled)
        self.totals: dict[str, float] = {}
        self.counts: dict[str, int] = {}
        self._active = None

    @contextmanager
    def section(self, name: str):
        if not self.enabled:
            yield
            return
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
        return {name: {"calls": self.counts[name], "total_ms": self.totals[name]} for name in self.totals}

    def since(self, before: dict) -> dict:
        """Stages that ran since `before` (a snapshot): their call count and time in between."""
        out = {}
        for name, now in self.snapshot().items():
            then = before.get(name, {"calls": 0, "total_ms": 0.0})
            calls = now["calls"] - then["calls"]
            if calls:
                out[name] = {"calls": calls, "total_ms": now["total_ms"] - then["total_ms"]}
        return out
