"""Exclusive expert tiers in front of the store, behind the interface of the reference's TieredCache
(src/vesper/cache.py:47-287: constructor, acquire, snapshot, close, enforce_pressure, the counter names, the
snapshot keys, the exception classes and their messages).

Design. Every expert the cache holds has one `_Home` in a single map: a compute-GPU slot or a host array of
the RAM tier. One map makes the tiers exclusive by construction (an expert cannot be in two places at once),
and recency is a logical clock stamped on a home at every use: a tier's least recent expert is its home
with the smallest stamp, so no per-tier ordered structure has to be kept in step with the map. Free GPU
slots sit in a min-heap, so an upload takes the lowest-numbered free slot.

A request for an expert brings it into a GPU slot: from the RAM tier (the host copy moves up and leaves RAM)
or from the store, through the backend's first staging buffer. When no slot is free the GPU's least recent
expert moves down first, read back through the second staging buffer into a new RAM copy (when the RAM tier
can hold one expert); the RAM tier makes room by dropping its least recent copies, and drops copies whenever
the machine's available memory falls below the budget's floor. Requests are serialised, and a slot handed
to a request stays put until the request ends.

Integrity: every upload is audited before its slot is published -- "readback" reads the slot back and
checks its SHA-256 against the store (source.validate); "gpu-sha256" hashes it on the GPU against the
digest table of the verified store read (backend.verify), which makes the host-side checks of RAM copies and
readbacks redundant, so they are counted as deferred. A failed check raises ValueError and publishes
nothing.

promote(keys) runs a batch of requests in order; with a NativeStore source the store reads and host checks
of the batch run ahead of the uploads on the store's prefetch pipeline (reading, hashing and uploading
different experts at once), with the same tier rules, counters and refusals as single requests.

The source is a NativeStore (size, entries, read_into, validate) and the backend a
vesper_amd.tiered.HipCacheBackend (primary_slots, staging, read, write, verify); the tests drive both with
fakes. The reference's helper-GPU tier needs a second device, which this single-GPU build does not use: a
backend with helper slots is refused, and the helper counters stay zero.
"""

from __future__ import annotations

import heapq
import itertools
import threading
from contextlib import contextmanager
from dataclasses import dataclass

import numpy as np

from .resources import MemoryBudget, physical_memory
from .timing import Timings

GPU, RAM = "primary_gpu", "ram"   # a home's tier, named as the request reports its origin

_COUNTER_GROUPS = (
    ("requests_started", "requests_completed", "requests_failed"),
    ("primary_hits", "helper_hits", "ram_hits"),
    ("store_read_attempts", "store_reads_completed", "store_bytes_requested"),
    ("primary_evictions", "helper_evictions", "ram_capacity_evictions", "ram_pressure_evictions",
     "ram_admission_refused", "pressure_refusals"),
    ("integrity_failures", "cpu_checks_deferred"),
    # per GPU tier: uploads, read-backs of demotions, audit read-backs, and the GPU audit's hashed payload and
    # digest download
    tuple(f"{tier}_{what}" for what in ("h2d_bytes", "d2h_bytes", "audit_readback_bytes",
                                        "gpu_audit_payload_bytes", "gpu_audit_digest_d2h_bytes")
          for tier in ("primary", "helper")),
)
COUNTERS = tuple(itertools.chain.from_iterable(_COUNTER_GROUPS))


@dataclass
class _Home:
    """Where one expert's bytes are: GPU slot `slot`, or the host array `data` of the RAM tier."""

    tier: str
    stamp: int
    slot: int = -1
    data: np.ndarray | None = None


class TieredCache:
    def __init__(self, source, backend, budget: MemoryBudget, ram_capacity_bytes: int, available=None, audit=True,
                 timings=None, gpu_verify=False):
        if ram_capacity_bytes < 0:
            raise ValueError("Negative RAM cache capacity")
        if gpu_verify and not (audit and callable(getattr(backend, "verify", None))):
            raise ValueError("GPU verification requires a complete upload audit backend")
        if getattr(backend, "helper_slots", 0):
            raise ValueError("The helper-GPU tier needs a second device; this build runs on one GPU")
        slots = int(backend.primary_slots)
        if slots < 0:
            raise ValueError("Negative slot capacity")
        if slots == 0:
            raise ValueError("A compute cache requires at least one primary slot")
        size = source.size
        staging = list(backend.staging)
        whole = [a.dtype == np.uint8 and a.shape == (size,) and a.flags.c_contiguous for a in staging]
        if len(staging) != 2 or not all(whole):
            raise ValueError("Staging must contain two complete contiguous byte blocks")
        if np.shares_memory(staging[0], staging[1]):
            raise ValueError("Promotion and demotion need two distinct staging buffers")
        self.source, self.backend, self.budget = source, backend, budget
        self.size, self.ram_capacity, self.slots = size, ram_capacity_bytes, slots
        self.incoming, self.outgoing = staging            # promotion and demotion/audit buffers
        self.available = available or (lambda: physical_memory()["available"])
        self.timings = timings or Timings()
        self.audit, self.gpu_verify = audit, gpu_verify
        self.stats = dict.fromkeys(COUNTERS, 0)
        self._homes: dict = {}
        self._free = list(range(slots))                   # a heap (already ordered)
        self._clock = itertools.count()
        self.lock, self.active, self.closed = threading.RLock(), False, False
        self._reclaimer = budget.register_reclaimer(self.reclaim)

    # -- the map ---------------------------------------------------------------------------------------------
    def _keys(self, tier: str) -> list:
        """Keys of one tier, least recent first."""
        return [k for k, h in sorted(self._homes.items(), key=lambda kv: kv[1].stamp) if h.tier == tier]

    def _least_recent(self, tier: str):
        found = None
        for key, home in self._homes.items():
            if home.tier == tier and (found is None or home.stamp < self._homes[found].stamp):
                found = key
        return found

    def _drop_copy(self, key, counter: str | None = None):
        """Free a RAM-tier copy and its budget reservation."""
        home = self._homes.pop(key)
        assert home.tier == RAM
        self.budget.release(self.size, category="cache")
        if counter is not None:
            self.stats[counter] += 1

    # -- host memory -----------------------------------------------------------------------------------------
    def _below_floor(self, extra: int = 0) -> bool:
        return self.available() - extra < self.budget.available_floor

    def enforce_pressure(self):
        """Drop RAM copies, least recent first, while the machine is below the budget's floor; MemoryError if
        it stays below with the RAM tier empty."""
        while self._below_floor():
            victim = self._least_recent(RAM)
            if victim is None:
                self.stats["pressure_refusals"] += 1
                raise MemoryError("System memory remains below the reserve after releasing the RAM cache")
            self._drop_copy(victim, "ram_pressure_evictions")

    def reclaim(self, requested: int) -> int:
        """Give back at least `requested` bytes of RAM copies if the cache is idle (a budget reclaimer); returns
        the bytes freed, 0 when a request holds the cache."""
        if not self.lock.acquire(blocking=False):
            return 0
        try:
            freed = 0
            while freed < requested and (victim := self._least_recent(RAM)) is not None:
                self._drop_copy(victim, "ram_pressure_evictions")
                freed += self.size
            return freed
        finally:
            self.lock.release()

    def _one_more_fits(self) -> bool:
        held = sum(h.tier == RAM for h in self._homes.values())
        return ((held + 1) * self.size <= self.ram_capacity and self.size <= self.budget.cap - self.budget.reserved
                and not self._below_floor(self.size))

    def _host_copy(self, key, data):
        """A verified RAM-tier array holding `data`, not yet placed in the map, or None when the tier cannot
        take it (counted as refused)."""
        if self.ram_capacity < self.size:
            self.stats["ram_admission_refused"] += 1
            return None
        self.enforce_pressure()
        while not self._one_more_fits():
            victim = self._least_recent(RAM)
            if victim is None:
                self.stats["ram_admission_refused"] += 1
                return None
            self._drop_copy(victim, "ram_capacity_evictions")
        self.budget.acquire(self.size, available=self.available(), category="cache")
        try:
            with self.timings.section("host.ram_allocate"):
                copy = np.empty(self.size, np.uint8)
            with self.timings.section("host.ram_copy"):
                np.copyto(copy, data)
            self._check_host_copy(key, copy)
        except BaseException:
            self.budget.release(self.size, category="cache")
            raise
        if self._below_floor():
            # the copy itself took the machine below its reserve: give it back and let the tier shrink
            del copy
            self.budget.release(self.size, category="cache")
            self.enforce_pressure()
            self.stats["ram_admission_refused"] += 1
            return None
        return copy

    # -- integrity -------------------------------------------------------------------------------------------
    def _check_host_copy(self, key, data):
        if self.gpu_verify:   # every upload is hashed on the GPU before use
            self.stats["cpu_checks_deferred"] += 1
            return
        try:
            self.source.validate(key, data)
        except Exception:
            self.stats["integrity_failures"] += 1
            raise

    def _audit_upload(self, slot: int, key):
        if not self.audit:
            return
        if not self.gpu_verify:
            self.backend.read("primary", slot, self.outgoing)
            self.stats["primary_audit_readback_bytes"] += self.size
            self._check_host_copy(key, self.outgoing)
            return
        try:
            digest_bytes = self.backend.verify("primary", slot, key)
        except ValueError:
            self.stats["integrity_failures"] += 1
            raise
        self.stats["primary_gpu_audit_payload_bytes"] += self.size
        self.stats["primary_gpu_audit_digest_d2h_bytes"] += digest_bytes

    # -- moves between tiers ---------------------------------------------------------------------------------
    def _stage_in(self, key, pipeline=None) -> str:
        """Put `key`'s bytes into the promotion buffer; returns the tier they came from. A store read comes
        from `pipeline` (already read and checked there) when one is given."""
        home = self._homes.get(key)
        if home is not None:   # a RAM copy (GPU residents never get here); it leaves RAM as it moves up
            with self.timings.section("host.ram_copy"):
                np.copyto(self.incoming, home.data)
            self._check_host_copy(key, self.incoming)
            self._drop_copy(key)
            self.stats["ram_hits"] += 1
            return RAM
        self.stats["store_read_attempts"] += 1
        self.stats["store_bytes_requested"] += self.size
        try:
            if pipeline is None or pipeline.next_key() != key:   # a key the batch itself moved out of its tier
                self.source.read_into(key, self.incoming)
            else:
                index, data, table = pipeline.get(key)
                try:
                    with self.timings.section("host.store_staging_copy"):
                        np.copyto(self.incoming, data)
                finally:
                    pipeline.release(index)
                if table is not None:
                    self.source.adopt_table(key, table)
        except ValueError:
            self.stats["integrity_failures"] += 1
            raise
        self.stats["store_reads_completed"] += 1
        return "store"

    def _move_down(self):
        """Free a GPU slot: its least recent expert goes to the RAM tier (if the tier can hold one) or is
        dropped."""
        key = self._least_recent(GPU)
        home = self._homes[key]
        copy = None
        if self.ram_capacity >= self.size:
            self.backend.read("primary", home.slot, self.outgoing)
            self.stats["primary_d2h_bytes"] += self.size
            self._check_host_copy(key, self.outgoing)
            copy = self._host_copy(key, self.outgoing)
        heapq.heappush(self._free, home.slot)
        if copy is None:
            del self._homes[key]
        else:
            self._homes[key] = _Home(RAM, next(self._clock), data=copy)
        self.stats["primary_evictions"] += 1

    def _resident(self, key, pipeline=None):
        """(slot, origin tier) of `key` in a GPU slot, promoting it if needed."""
        if key not in self.source.entries:
            raise KeyError("Requested expert is absent from the pinned native store")
        home = self._homes.get(key)
        if home is not None and home.tier == GPU:
            home.stamp = next(self._clock)
            self.stats["primary_hits"] += 1
            return home.slot, GPU
        origin = self._stage_in(key, pipeline)
        if not self._free:
            self._move_down()
        slot = self._free[0]
        self.backend.write("primary", slot, self.incoming)
        self.stats["primary_h2d_bytes"] += self.size
        self._audit_upload(slot, key)          # raises before anything is published
        heapq.heappop(self._free)
        self._homes[key] = _Home(GPU, next(self._clock), slot=slot)
        return slot, origin

    # -- requests --------------------------------------------------------------------------------------------
    def _begin(self):
        if self.closed:
            raise RuntimeError("Cache is closed")
        if self.active:
            raise RuntimeError("Nested requests could replace a live compute slot")
        self.active = True
        self.stats["requests_started"] += 1

    @contextmanager
    def acquire(self, key):
        """(slot, origin tier) of `key` -- "primary_gpu", "ram" or "store" -- for the with-block."""
        with self.lock:
            self._begin()
            try:
                self.enforce_pressure()
                yield self._resident(key)
                self.enforce_pressure()
            except BaseException:
                self.stats["requests_failed"] += 1
                raise
            else:
                self.stats["requests_completed"] += 1
            finally:
                self.active = False

    def promote(self, keys, *, depth: int = 6, readers: int = 3) -> list:
        """Bring `keys` into GPU slots in order, each as one request (the same tier rules, counters, checks
        and refusals as acquire), returning each key's origin tier. When the source offers a prefetch
        pipeline (NativeStore.prefetch), the store reads and host checks of the keys found in no tier run
        ahead on it -- reading later entries and hashing them while earlier ones upload -- with at most
        `depth` entries held in host buffers. A failed read or check fails the batch at that key; keys
        before it stay promoted. With more keys than slots, the batch's own earlier keys move down."""
        keys = list(keys)
        with self.lock:
            if self.closed:
                raise RuntimeError("Cache is closed")
            if self.active:
                raise RuntimeError("Nested requests could replace a live compute slot")
            for key in keys:
                if key not in self.source.entries:
                    raise KeyError("Requested expert is absent from the pinned native store")
            fetch = [k for k in dict.fromkeys(keys) if k not in self._homes]
            pipeline = None
            if fetch and callable(getattr(self.source, "prefetch", None)):
                pipeline = self.source.prefetch(fetch, depth=depth, readers=readers)
            origins = []
            try:
                for key in keys:
                    self._begin()
                    try:
                        self.enforce_pressure()
                        origins.append(self._resident(key, pipeline))
                        self.enforce_pressure()
                    except BaseException:
                        self.stats["requests_failed"] += 1
                        raise
                    else:
                        self.stats["requests_completed"] += 1
                    finally:
                        self.active = False
            finally:
                if pipeline is not None:
                    pipeline.close()
            return [origin for _, origin in origins]

    def snapshot(self) -> dict:
        with self.lock:
            ram = self._keys(RAM)
            return {"primary_keys": self._keys(GPU), "helper_keys": [], "ram_keys": ram,
                    "ram_cache_bytes": len(ram) * self.size, "host_reserved_bytes": self.budget.reserved,
                    "host_peak_reserved_bytes": self.budget.peak,
                    "integrity_mode": "gpu-sha256" if self.gpu_verify else "readback",
                    "counters": dict(self.stats)}

    def close(self):
        with self.lock:
            if self.active:
                raise RuntimeError("Cannot close a cache with a live compute slot")
            for key in self._keys(RAM):
                self._drop_copy(key)
            self.closed = True
            self.budget.unregister_reclaimer(self._reclaimer)
