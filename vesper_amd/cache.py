"""Exclusive expert tiers in front of the store (the reference's TieredCache, src/vesper/cache.py:19-287).

An expert lives in exactly one tier at a time: a compute-GPU slot, the RAM tier, or only in the store. A
request for an expert not in a GPU slot promotes it -- from RAM (dropping the RAM copy) or from the store
-- into a free slot; when no slot is free the least recently used slot is demoted to RAM first (its bytes
read back from the GPU), and the RAM tier in turn drops its least recently used copies to make room.
Requests are serialised; a slot handed out stays put until the request ends.

Integrity, as in the reference: every GPU upload is audited before the slot is published -- "readback"
reads the slot back to the host and checks its SHA-256 against the store manifest; "gpu-sha256" hashes it on
the GPU against the 4 KiB digest table taken from the verified store read, so host-side copies (RAM tier,
readbacks) skip their checks. A failed check raises ValueError and publishes nothing.

The tiers talk to a source (NativeStore: size, entries, read_into, validate) and a backend
(vesper_amd.tiered.HipCacheBackend: primary_slots, staging, read, write, verify); tests drive them with fakes.
The helper-GPU tier of the reference needs a second device and is not part of this single-GPU build: a
backend with helper slots is refused.
"""

from __future__ import annotations

import threading
from collections import OrderedDict
from contextlib import contextmanager

import numpy as np

from .resources import MemoryBudget, physical_memory
from .timing import Timings

COUNTERS = ("requests_started", "requests_completed", "requests_failed", "primary_hits", "helper_hits", "ram_hits",
            "store_read_attempts", "store_reads_completed", "store_bytes_requested", "primary_evictions",
            "helper_evictions", "ram_capacity_evictions", "ram_pressure_evictions", "ram_admission_refused",
            "pressure_refusals", "integrity_failures", "primary_h2d_bytes", "helper_h2d_bytes", "primary_d2h_bytes",
            "helper_d2h_bytes", "primary_audit_readback_bytes", "helper_audit_readback_bytes", "cpu_checks_deferred",
            "primary_gpu_audit_payload_bytes", "helper_gpu_audit_payload_bytes", "primary_gpu_audit_digest_d2h_bytes",
            "helper_gpu_audit_digest_d2h_bytes")


class SlotTable:
    """`capacity` numbered slots; keys in least-recently-used order."""

    def __init__(self, capacity: int):
        if capacity < 0:
            raise ValueError("Negative slot capacity")
        self.capacity = capacity
        self.by_key: OrderedDict = OrderedDict()

    @property
    def free(self) -> list:
        used = set(self.by_key.values())
        return [s for s in range(self.capacity) if s not in used]

    def touch(self, key):
        """The key's slot (now most recent), or None."""
        if key not in self.by_key:
            return None
        self.by_key.move_to_end(key)
        return self.by_key[key]

    def put(self, key, slot: int):
        if key in self.by_key or slot not in self.free:
            raise RuntimeError("Cache slot is already published")
        self.by_key[key] = slot

    def pop(self, key) -> int:
        return self.by_key.pop(key)

    def least_recent(self):
        return next(iter(self.by_key.items()))


class TieredCache:
    def __init__(self, source, backend, budget: MemoryBudget, ram_capacity_bytes: int, available=None, audit=True,
                 timings=None, gpu_verify=False):
        if ram_capacity_bytes < 0:
            raise ValueError("Negative RAM cache capacity")
        if gpu_verify and (not audit or not callable(getattr(backend, "verify", None))):
            raise ValueError("GPU verification requires a complete upload audit backend")
        if getattr(backend, "helper_slots", 0):
            raise ValueError("The helper-GPU tier needs a second device; this build runs on one GPU")
        self.source, self.backend, self.budget = source, backend, budget
        self.size, self.ram_capacity = source.size, ram_capacity_bytes
        self.available = available or (lambda: physical_memory()["available"])
        self.timings = timings or Timings()
        self.audit, self.gpu_verify = audit, gpu_verify
        self.primary = SlotTable(backend.primary_slots)
        if not self.primary.capacity:
            raise ValueError("A compute cache requires at least one primary slot")
        self.staging = backend.staging
        if len(self.staging) != 2 or any(a.dtype != np.uint8 or a.shape != (self.size,) or not a.flags.c_contiguous
                                          for a in self.staging):
            raise ValueError("Staging must contain two complete contiguous byte blocks")
        if np.shares_memory(self.staging[0], self.staging[1]):
            raise ValueError("Promotion and demotion need two distinct staging buffers")
        self.ram: OrderedDict = OrderedDict()
        self.stats = dict.fromkeys(COUNTERS, 0)
        self.lock, self.active, self.closed = threading.RLock(), False, False

    # -- RAM tier -------------------------------------------------------------------------------------
    def _forget_ram(self, key, counter=None):
        del self.ram[key]
        self.budget.release(self.size, category="cache")
        if counter:
            self.stats[counter] += 1

    def enforce_pressure(self):
        """Drop RAM copies while the machine is below the budget's floor; refuse if that is not enough."""
        while self.ram and self.available() < self.budget.available_floor:
            self._forget_ram(next(iter(self.ram)), "ram_pressure_evictions")
        if self.available() < self.budget.available_floor:
            self.stats["pressure_refusals"] += 1
            raise MemoryError("System memory remains below the reserve after releasing the RAM cache")

    def _room_for_one(self) -> bool:
        return ((len(self.ram) + 1) * self.size <= self.ram_capacity
                and self.budget.reserved + self.size <= self.budget.cap
                and self.available() - self.size >= self.budget.available_floor)

    def _keep_in_ram(self, key, data) -> bool:
        """Copy `data` into the RAM tier (LRU eviction to make room); False if it cannot be admitted."""
        if self.ram_capacity < self.size:
            self.stats["ram_admission_refused"] += 1
            return False
        self.enforce_pressure()
        while self.ram and not self._room_for_one():
            self._forget_ram(next(iter(self.ram)), "ram_capacity_evictions")
        if not self._room_for_one():
            self.stats["ram_admission_refused"] += 1
            return False
        self.budget.acquire(self.size, available=self.available(), category="cache")
        try:
            with self.timings.section("host.ram_copy"):
                copy = np.array(data, dtype=np.uint8, copy=True)
            self._check_host(key, copy)
        except BaseException:
            self.budget.release(self.size, category="cache")
            raise
        self.ram[key] = copy
        return True

    # -- checks -----------------------------------------------------------------------------------------
    def _check_host(self, key, data):
        """A host copy's SHA-256 against the store (deferred to the GPU audit in gpu-sha256 mode)."""
        if self.gpu_verify:
            self.stats["cpu_checks_deferred"] += 1
            return
        try:
            self.source.validate(key, data)
        except ValueError:
            self.stats["integrity_failures"] += 1
            raise

    def _upload(self, slot, key, data):
        """H2D into `slot`, then the audit of what the slot holds."""
        self.backend.write("primary", slot, data)
        self.stats["primary_h2d_bytes"] += self.size
        if not self.audit:
            return
        if self.gpu_verify:
            try:
                digest_bytes = self.backend.verify("primary", slot, key)
            except ValueError:
                self.stats["integrity_failures"] += 1
                raise
            self.stats["primary_gpu_audit_payload_bytes"] += self.size
            self.stats["primary_gpu_audit_digest_d2h_bytes"] += digest_bytes
        else:
            self.backend.read("primary", slot, self.staging[1])
            self.stats["primary_audit_readback_bytes"] += self.size
            self._check_host(key, self.staging[1])

    def _demote_least_recent(self):
        key, slot = self.primary.least_recent()
        if self.ram_capacity >= self.size:
            self.backend.read("primary", slot, self.staging[1])
            self.stats["primary_d2h_bytes"] += self.size
            self._check_host(key, self.staging[1])
            self._keep_in_ram(key, self.staging[1])
        self.primary.pop(key)
        self.stats["primary_evictions"] += 1

    def _fetch(self, key):
        """Bring `key` into staging[0]; returns the tier it came from."""
        if key in self.ram:
            with self.timings.section("host.ram_copy"):
                np.copyto(self.staging[0], self.ram[key])
            self._check_host(key, self.staging[0])
            self._forget_ram(key)
            self.stats["ram_hits"] += 1
            return "ram"
        self.stats["store_read_attempts"] += 1
        self.stats["store_bytes_requested"] += self.size
        try:
            self.source.read_into(key, self.staging[0])
        except ValueError:
            self.stats["integrity_failures"] += 1
            raise
        self.stats["store_reads_completed"] += 1
        return "store"

    def _ensure_primary(self, key):
        if key not in self.source.entries:
            raise KeyError("Requested expert is absent from the pinned native store")
        slot = self.primary.touch(key)
        if slot is not None:
            self.stats["primary_hits"] += 1
            return slot, "primary_gpu"
        origin = self._fetch(key)
        if not self.primary.free:
            self._demote_least_recent()
        slot = self.primary.free[0]
        self._upload(slot, key, self.staging[0])
        self.primary.put(key, slot)
        return slot, origin

    @contextmanager
    def acquire(self, key):
        """(slot, source tier) of `key`, held for the duration of the with-block."""
        with self.lock:
            if self.closed:
                raise RuntimeError("Cache is closed")
            if self.active:
                raise RuntimeError("Nested requests could replace a live compute slot")
            self.active = True
            self.stats["requests_started"] += 1
            try:
                self.enforce_pressure()
                slot, origin = self._ensure_primary(key)
                yield slot, origin
                self.enforce_pressure()
                self.stats["requests_completed"] += 1
            except BaseException:
                self.stats["requests_failed"] += 1
                raise
            finally:
                self.active = False

    def snapshot(self) -> dict:
        with self.lock:
            primary, ram = list(self.primary.by_key), list(self.ram)
            if set(primary) & set(ram):
                raise RuntimeError("Exclusive cache tiers contain duplicate expert identities")
            return {"primary_keys": primary, "helper_keys": [], "ram_keys": ram,
                    "ram_cache_bytes": len(ram) * self.size, "host_reserved_bytes": self.budget.reserved,
                    "host_peak_reserved_bytes": self.budget.peak,
                    "integrity_mode": "gpu-sha256" if self.gpu_verify else "readback", "counters": dict(self.stats)}

    def close(self):
        with self.lock:
            if self.active:
                raise RuntimeError("Cannot close a cache with a live compute slot")
            for key in list(self.ram):
                self._forget_ram(key)
            self.closed = True
