"""Expert residency: the store-backed tiers and the asynchronous streaming cache (the reference's
TieredCache / CudaCacheBackend / TieredExpertRuntime, src/vesper/cache.py:19-287, src/vesper/tiered.py:21-216).

* CacheConfig, TieredExpertRuntime(store, config): the reference's constructor and single-expert call over
  the exclusive tiers of vesper_amd.cache (GPU slots, RAM, the on-disk store read with O_DIRECT), on the
  HipCacheBackend (pinned staging, tiled device slots, readback or GPU SHA-256 audit).
* ExpertCache: HBM slots over host-pinned expert bytes (mx_cache_*): LRU, misses copied with hipMemcpyAsync
  on a side stream, ordered by per-slot release events and a ready event instead of host waits.
* HostExpertPool: tiled experts in pinned host memory (a RAM tier for the streaming cache), filled from
  reference-layout arrays or from device-generated synthetic experts.
* PooledExpertRuntime: forward(key "layer:expert", x, w) through the streaming cache over a pool.
* OffloadDecode: several MoE layers whose routed experts live in the pool and are streamed into the cache
  per step; the shared experts stay resident.
"""

from __future__ import annotations

import ctypes as C
import threading
import time
from contextlib import ExitStack, contextmanager
from dataclasses import dataclass
from pathlib import Path

import numpy as np

from . import _lib
from .cache import TieredCache
from .config import MoEConfig
from .layer import TENSORS, ExpertBank, bf16_input, validate_expert_arrays
from .resources import GiB, MiB, MemoryBudget
from .store import REFERENCE_PROFILE, ModelProfile, NativeStore, tensor_layout
from .timing import Timings


def expert_key(layer: int, expert: int) -> int:
    """64-bit cache key of (layer, expert)."""
    if not (0 <= layer < 2 ** 31 and 0 <= expert < 2 ** 32):
        raise ValueError("layer or expert index outside the key range")
    return (int(layer) << 32) | int(expert)


def parse_key(key: str) -> tuple[int, int]:
    """The reference's "layer:expert" key (tiered.py:199)."""
    try:
        layer, expert = key.split(":")
        return int(layer), int(expert)
    except (AttributeError, ValueError):
        raise ValueError("Expert keys have the form 'layer:expert'") from None


class ExpertCache:
    """`slots` device slots of `slot_bytes` each, keyed by expert_key."""

    def __init__(self, ctx: _lib.Context, slot_bytes: int, slots: int):
        self.ctx, self.slot_bytes, self.slots = ctx, int(slot_bytes), int(slots)
        h = C.c_void_p()
        ctx.lib.cache_create(ctx._h(), self.slot_bytes, self.slots, C.byref(h))
        self.handle = h

    def register(self, key: int, host_ptr: int):
        self.ctx.lib.cache_register(self.handle, int(key), C.c_void_p(int(host_ptr)))

    def ensure(self, keys) -> tuple[list[int], np.ndarray]:
        keys = np.ascontiguousarray(keys, dtype=np.int64)
        ptrs = (C.c_void_p * max(len(keys), 1))()
        hits = np.zeros(max(len(keys), 1), np.int32)
        self.ctx.lib.cache_ensure(self.handle, keys.ctypes.data_as(C.c_void_p), len(keys), ptrs,
                                  hits.ctypes.data_as(C.c_void_p))
        return [int(p or 0) for p in ptrs[:len(keys)]], hits[:len(keys)]

    def ready_event(self) -> int:
        e = C.c_void_p()
        self.ctx.lib.cache_ready_event(self.handle, C.byref(e))
        return int(e.value)

    def wait_ready(self, stream=None):
        """Make `stream` wait for the copies of the last ensure()."""
        self.ctx.lib.stream_wait_event(self.ctx._h(), _lib._stream(stream), C.c_void_p(self.ready_event()))

    def forget(self, key: int):
        """Drop a key's slot (never served again until copied anew), e.g. after a failed audit."""
        self.ctx.lib.cache_forget(self.handle, int(key))

    def release(self, keys, stream=None):
        keys = np.ascontiguousarray(keys, dtype=np.int64)
        self.ctx.lib.cache_release(self.handle, keys.ctypes.data_as(C.c_void_p), len(keys), _lib._stream(stream))

    def set_timing(self, enable: bool):
        self.ctx.lib.cache_set_timing(self.handle, int(bool(enable)))

    def stats(self) -> dict:
        hits, misses, nbytes = C.c_uint64(), C.c_uint64(), C.c_uint64()
        ms, resident = C.c_double(), C.c_int32()
        self.ctx.lib.cache_stats(self.handle, C.byref(hits), C.byref(misses), C.byref(nbytes), C.byref(ms),
                                 C.byref(resident))
        return {"hits": hits.value, "misses": misses.value, "bytes_copied": nbytes.value, "copy_ms": ms.value,
                "resident": resident.value}

    def close(self):
        if self.handle:
            h, self.handle = self.handle, C.c_void_p()
            self.ctx.lib.cache_destroy(h)


class HostExpertPool:
    """`count` tiled experts in one pinned host allocation (the RAM tier of the reference's cache)."""

    def __init__(self, ctx: _lib.Context, config: MoEConfig, count: int):
        self.ctx, self.config, self.count = ctx, config, int(count)
        self.expert_bytes = int(ctx.lib.cdll.mx_tiled_expert_bytes(config.hidden, config.intermediate))
        self.base = ctx.host_alloc_pinned(self.expert_bytes * self.count)

    def ptr(self, index: int) -> int:
        if not 0 <= index < self.count:
            raise ValueError("pool index outside the pool")
        return self.base + index * self.expert_bytes

    def fill_from_bank(self, bank: ExpertBank, bank_index: int, index: int):
        """Copy one tiled expert of a device bank into pool entry `index` (D2H)."""
        self.ctx.lib.memcpy_d2h(self.ctx._h(), C.c_void_p(self.ptr(index)), C.c_void_p(bank.tiled_ptr(bank_index)),
                                self.expert_bytes, None)

    def upload_arrays(self, index: int, arrays: dict, staging: ExpertBank):
        """Reference-layout arrays -> tiled (on the device, via a one-expert staging bank) -> pool entry."""
        validate_expert_arrays(arrays, self.config)
        staging.upload(0, arrays)
        self.fill_from_bank(staging, 0, index)

    def close(self):
        if self.base:
            self.ctx.host_free_pinned(self.base)
            self.base = 0


INTEGRITY_MODES = ("readback", "gpu-sha256")


@dataclass(frozen=True)
class CacheConfig:
    """The expert tiers' configuration, with the reference's fields and defaults (src/vesper/tiered.py:21-47).

    host_cap_bytes / available_floor bound the host memory the tiers reserve; ram_cache_bytes is the RAM
    tier; primary_slots are the compute GPU's expert slots (device allocations capped at device_cap_bytes);
    integrity_mode "readback" (the default: each uploaded slot is read back and its SHA-256 checked on the
    host) or "gpu-sha256" (hashed on the GPU against the verified 4 KiB digest table). The helper-GPU tier
    (helper_device, helper_slots) needs a second device: with one GPU, set helper_device=None and
    helper_slots=0 -- the runtime refuses a helper it cannot open."""
    host_cap_bytes: int = 96 * GiB
    ram_cache_bytes: int = 80 * GiB
    available_floor: int = 32 * GiB
    primary_device: int = 0
    primary_slots: int = 1
    helper_device: int | None = 1
    helper_slots: int = 1
    device_cap_bytes: int = 64 * MiB
    metadata_allowance_bytes: int = MiB
    profile: bool = False
    integrity_mode: str = "readback"
    max_store_experts: int = 4

    def __post_init__(self):
        if type(self.max_store_experts) is not int or self.max_store_experts < 1:
            raise ValueError("Explicit native-store limit must be one to 48 experts")
        if self.integrity_mode not in INTEGRITY_MODES:
            raise ValueError("Unknown cache integrity mode")
        if self.primary_slots < 1 or self.helper_slots < 0 or self.ram_cache_bytes < 0:
            raise ValueError("Invalid expert cache capacity")
        if self.helper_device == self.primary_device:
            raise ValueError("The helper must be a distinct storage GPU")
        if self.helper_device is None and self.helper_slots:
            raise ValueError("Helper slots require a helper device")
        if self.metadata_allowance_bytes < MiB:
            raise ValueError("The bounded store requires at least 1 MiB metadata allowance")


class HipCacheBackend:
    """The compute GPU's side of the tiers (the reference's CudaCacheBackend, src/vesper/tiered.py:50-127).

    Two pinned staging buffers of one store-layout expert each (store reads are copied in from the direct
    reader's buffer), `primary_slots` device slots holding the tiled layout the expert kernels read, and one device
    staging expert in the store layout. A write copies staging -> device staging and tiles it into the slot;
    a read untiles the slot back and copies it to the host; the GPU audit untiles the slot and hashes it
    against the store's digest table -- so every check sees what the slot holds."""

    helper_slots = 0

    def __init__(self, ctx, profile, size: int, config: CacheConfig, budget: MemoryBudget, source=None,
                 timings: Timings | None = None):
        self.ctx, self.profile, self.size, self.config, self.budget = ctx, profile, size, config, budget
        self.primary_slots = config.primary_slots
        self.source, self.timings = source, timings or Timings(config.profile)
        self.tiled_bytes = int(ctx.lib.cdll.mx_tiled_expert_bytes(profile.hidden, profile.intermediate))
        self._pinned, self._device, self.verifier = [], [], None

    def __enter__(self):
        c, ctx = self.config, self.ctx
        self.budget.acquire(2 * self.size, category="staging")
        try:
            self._pinned = [ctx.host_alloc_pinned(self.size) for _ in range(2)]
            self.staging = [np.ctypeslib.as_array((C.c_uint8 * self.size).from_address(p)) for p in self._pinned]
            self.slots = [ctx.malloc(self.tiled_bytes) for _ in range(self.primary_slots)]
            self.device_staging = ctx.malloc(self.size)
            self._device = self.slots + [self.device_staging]
            at = {}
            for name, region in tensor_layout(self.profile).items():
                at[name] = self.device_staging + region["offset"]
            self.ref_ptrs = _lib.MxExpertPtrs(*[at[n] for n in TENSORS])
            if c.integrity_mode == "gpu-sha256":
                if self.source is None:
                    raise ValueError("GPU integrity requires original source digest tables")
                from .integrity import DeviceIntegrity
                self.verifier = DeviceIntegrity(ctx, self.size, self.timings)
            return self
        except BaseException:
            self.__exit__()
            raise

    def _tile(self, slot):
        self.ctx.lib.tile_expert(self.ctx._h(), C.byref(self.ref_ptrs), self.profile.hidden, self.profile.intermediate,
                                 C.c_void_p(self.slots[slot]), None)

    def _untile(self, slot):
        self.ctx.lib.untile_expert(self.ctx._h(), C.c_void_p(self.slots[slot]), self.profile.hidden,
                                   self.profile.intermediate, C.byref(self.ref_ptrs), None)

    def write(self, tier, slot, data):
        with self.timings.section(f"transfer.{tier}_h2d"):
            self.ctx.lib.memcpy_h2d(self.ctx._h(), C.c_void_p(self.device_staging), data.ctypes.data_as(C.c_void_p),
                                    self.size, None)
            self._tile(slot)
            self.ctx.sync()

    def read(self, tier, slot, target):
        with self.timings.section(f"transfer.{tier}_d2h"):
            self._untile(slot)
            self.ctx.lib.memcpy_d2h(self.ctx._h(), target.ctypes.data_as(C.c_void_p), C.c_void_p(self.device_staging),
                                    self.size, None)

    def verify(self, tier, slot, key):
        if key not in self.source.expected_chunks:
            raise ValueError("Original digest table must come from a fully verified store read")
        self._untile(slot)
        return self.verifier.verify(self.device_staging, self.source.expected_chunks[key])

    def slot_ptr(self, slot) -> int:
        return self.slots[slot]

    def __exit__(self, *_):
        if self.verifier is not None:
            self.verifier.close()
            self.verifier = None
        for p in self._device:
            self.ctx.free(p)
        self._device = []
        if self._pinned:
            for p in self._pinned:
                self.ctx.host_free_pinned(p)
            self._pinned = []
            self.budget.release(2 * self.size, category="staging")


def _stage_buffers(ctx, tokens, hidden, intermediate):
    t, h, i = tokens, hidden, intermediate
    return {"x": ctx.empty((t, h), np.uint16), "route": ctx.empty((t,), np.float32),
            "q": ctx.empty((t, h), np.uint8), "s": ctx.empty((t, h // 32), np.uint8),
            "w1": ctx.empty((t, i), np.uint16), "w3": ctx.empty((t, i), np.uint16),
            "down_input": ctx.empty((t, i), np.uint16), "trace": ctx.empty((t, i, 5), np.float32),
            "down_q": ctx.empty((t, i), np.uint8), "down_s": ctx.empty((t, i // 32), np.uint8),
            "w2": ctx.empty((t, h), np.uint16)}


def _run_tiled_expert(ctx, work, tiled_ptr, hidden, intermediate, limit, x, routing_weight):
    """One tiled expert over the BF16 rows of x (1-D: one token, results 1-D as the reference returns them);
    returns the reference's stage dict (src/vesper/expert.py:71-79)."""
    one = np.asarray(x).ndim == 1
    bits = bf16_input(x, hidden)
    t = bits.shape[0]
    if not 1 <= t <= work["x"].shape[0]:
        raise ValueError(f"One expert call accepts 1 to {work['x'].shape[0]} tokens")
    route = None
    if routing_weight is not None:
        route = np.broadcast_to(np.asarray(routing_weight, np.float32).reshape(-1), (t,)).copy()
        if not np.isfinite(route).all():
            raise ValueError("Routing weight must be finite")
    ctx.copy_h2d(work["x"].ptr, bits)
    if route is not None:
        ctx.copy_h2d(work["route"].ptr, route)
    stages = _lib.MxExpertStages(*[work[n].ptr for n in ("q", "s", "w1", "w3", "down_input", "trace", "down_q",
                                                        "down_s")])
    ctx.lib.expert_forward_tiled(ctx._h(), C.c_void_p(tiled_ptr), hidden, intermediate, C.c_void_p(work["x"].ptr), t,
                                 C.c_float(limit), None if route is None else C.c_void_p(work["route"].ptr),
                                 C.c_void_p(work["w2"].ptr), C.byref(stages), None)
    h, i = hidden, intermediate
    layout = {"q": ((t, h), np.uint8), "s": ((t, h // 32), np.uint8), "w1": ((t, i), np.uint16),
              "w3": ((t, i), np.uint16), "down_input": ((t, i), np.uint16), "trace": ((t, i, 5), np.float32),
              "down_q": ((t, i), np.uint8), "down_s": ((t, i // 32), np.uint8), "w2": ((t, h), np.uint16)}
    out = {n: ctx.download(work[n].ptr, shape, dt) for n, (shape, dt) in layout.items()}
    out["down_input"] = (out["down_input"].astype(np.uint32) << 16).view(np.float32)
    return {n: v[0] for n, v in out.items()} if one else out


class TieredExpertRuntime:
    """Single-expert execution over the exclusive tiers, behind the reference's constructor and call
    (src/vesper/tiered.py:130-216: TieredExpertRuntime(store, CacheConfig), forward(key, x, routing_weight),
    snapshot(), last_event, cleanup).

    Opening runs four steps, each leaving what it opened on one exit stack so that a failing step closes
    exactly what came before it: admit the metadata allowance in the host budget; open the store (a
    NativeStore over the directory, or source_factory(store, budget), which must charge the same budget) and
    check that the budget can hold its direct-I/O buffer and two pinned staging buffers; open the compute GPU
    (`primary_device`), the HipCacheBackend's slots and the stage buffers of the expert call; build the tiers.
    forward(key, x, w) holds expert "layer:expert" in a GPU slot -- served from the slot, the RAM tier or the
    store -- refuses to run when the device's free memory is below its floor, and runs the expert
    (mx_expert_forward_tiled) with the reference's stage dict as the result; last_event["source_tier"] names
    the tier. The model's shapes come from `model` (the reference's pinned checkpoint by default)."""

    DEVICE_FREE_FLOOR = GiB   # free device memory below which no expert call starts

    def __init__(self, store: Path, config: CacheConfig | None = None, *, source_factory=None,
                 model: ModelProfile = REFERENCE_PROFILE, max_tokens: int = 16):
        if source_factory is not None and not callable(source_factory):
            raise ValueError("Expected an explicit expert source factory")
        self.store_path, self.config, self.source_factory = Path(store), config or CacheConfig(), source_factory
        self.model, self.max_tokens = model, int(max_tokens)
        self.stack, self.cache, self.ctx = None, None, None

    # -- opening ---------------------------------------------------------------------------------------------
    def _admit_metadata(self, stack: ExitStack):
        allowance = self.config.metadata_allowance_bytes
        self.budget.acquire(allowance, category="metadata")
        stack.callback(self.budget.release, allowance, category="metadata")

    def _open_store(self, stack: ExitStack):
        c = self.config
        if self.source_factory is None:
            store = NativeStore(self.store_path, self.budget, max_experts=c.max_store_experts, profile=self.model)
        else:
            store = self.source_factory(self.store_path, self.budget)
        if store.budget is not self.budget:
            raise ValueError("Expert source must use the admitted cache budget")
        store.timings, store.gpu_integrity = self.timings, c.integrity_mode == "gpu-sha256"
        self.store = stack.enter_context(store)
        # the direct reader's aligned buffer and the two pinned staging experts, beside the metadata
        if 3 * self.store.size > c.host_cap_bytes - c.metadata_allowance_bytes:
            raise MemoryError("Host cap cannot fit direct-I/O scratch and two pinned staging buffers")

    def _open_device(self, stack: ExitStack):
        c = self.config
        self.ctx = stack.enter_context(_lib.Context(c.primary_device, c.device_cap_bytes))
        self.backend = stack.enter_context(HipCacheBackend(self.ctx, self.model, self.store.size, c, self.budget,
                                                           self.store, self.timings))
        work = _stage_buffers(self.ctx, self.max_tokens, self.model.hidden, self.model.intermediate)
        stack.callback(lambda: [buf.free() for buf in work.values()])
        self.work = work

    def _open_tiers(self, stack: ExitStack):
        c = self.config
        self.cache = TieredCache(self.store, self.backend, self.budget, c.ram_cache_bytes, timings=self.timings,
                                 gpu_verify=c.integrity_mode == "gpu-sha256")
        stack.callback(self.cache.close)

    def __enter__(self):
        if self.stack is not None:
            raise RuntimeError("Tiered runtime is already open")
        c = self.config
        if c.helper_device is not None and c.helper_slots:
            raise RuntimeError(f"The helper-GPU tier needs device {c.helper_device}; this build runs on one GPU "
                               "(set helper_device=None and helper_slots=0)")
        self.budget = MemoryBudget(c.host_cap_bytes, c.available_floor, owner="expert_tiers")
        self.timings = Timings(c.profile)
        stack = ExitStack()
        with stack:   # unwinds only if a step raises: pop_all() below takes the resources over
            for step in (self._admit_metadata, self._open_store, self._open_device, self._open_tiers):
                step(stack)
            self.stack = stack.pop_all()
        self.last_event = None
        return self

    # -- calls -----------------------------------------------------------------------------------------------
    @contextmanager
    def _recording(self, key: str):
        """Collects last_event for one call (published only when the call succeeds)."""
        started, mark = time.perf_counter(), self.timings.snapshot()
        event = {"key": key, "source_tier": None}
        yield event
        event["wall_ms"] = (time.perf_counter() - started) * 1000
        if self.timings.enabled:
            event["stage_timings"] = self.timings.since(mark)
        self.last_event = event

    def _check_headroom(self):
        if self.ctx.memory()["free"] < self.DEVICE_FREE_FLOOR:
            raise MemoryError("GPU headroom fell below the reserve; refusing further work")

    def forward(self, key: str, x, routing_weight=None) -> dict:
        if self.stack is None:
            raise RuntimeError("Use the tiered runtime as a context manager")
        with self._recording(key) as event, self.cache.acquire(key) as (slot, origin):
            event["source_tier"] = origin
            self._check_headroom()
            with self.timings.section("compute.kernels"):
                return _run_tiled_expert(self.ctx, self.work, self.backend.slot_ptr(slot), self.model.hidden,
                                         self.model.intermediate, self.model.swiglu_limit, x, routing_weight)

    def prefetch(self, keys, *, depth: int = 6, readers: int = 3) -> list:
        """Promote experts "layer:expert" into GPU slots as one pipelined batch (TieredCache.promote: store
        reads and host checks of later experts overlap the uploads and audits of earlier ones); returns each
        key's origin tier. Later forward() calls for them are GPU hits while they keep their slots."""
        if self.stack is None:
            raise RuntimeError("Use the tiered runtime as a context manager")
        return self.cache.promote(keys, depth=depth, readers=readers)

    def snapshot(self) -> dict:
        store, c = self.store, self.config
        footprint = {"primary_peak_explicit_bytes": self.ctx.owned_bytes()[1], "helper_peak_explicit_bytes": 0,
                     "store_direct_read_calls": store.read_calls, "store_direct_read_bytes": store.bytes_read,
                     "host_cap_bytes": c.host_cap_bytes, "host_available_floor_bytes": c.available_floor,
                     "ram_capacity_bytes": c.ram_cache_bytes,
                     "expected_digest_table_bytes": sum(t.nbytes for t in store.expected_chunks.values())}
        timings = {"stage_timings": self.timings.snapshot()} if self.timings.enabled else {}
        return {**self.cache.snapshot(), **timings, **footprint}

    def __exit__(self, *_):
        if self.stack is None:
            return
        live = self.ctx.owned_bytes()[0] if self.ctx is not None else 0
        stack, self.stack = self.stack, None
        stack.close()
        self.cleanup = {"host_buffer_reservations_bytes": self.budget.reserved,
                        "primary_explicit_live_bytes_before_close": live}


class PooledExpertRuntime:
    """Single-expert execution through the asynchronous device cache over a host-pinned pool of tiled experts
    (the pool is the RAM tier, filled from device banks or arrays): forward(key "layer:expert", x, w);
    last_event["source_tier"] is "primary_gpu" on a hit, "host_pinned" on a miss. audit=True checks every
    admitted slot on the GPU against the digest table of its pinned source before the expert runs (the
    reference's gpu-sha256 mode)."""

    def __init__(self, ctx: _lib.Context, config: MoEConfig, pool: HostExpertPool, index_of: dict, slots: int = 64,
                 audit: bool = False, swiglu_limit: float | None = None):
        self.ctx, self.config, self.pool, self.index_of = ctx, config, pool, dict(index_of)
        self.limit = config.swiglu_limit if swiglu_limit is None else float(swiglu_limit)
        self.cache = ExpertCache(ctx, pool.expert_bytes, slots)
        for key, index in self.index_of.items():
            self.cache.register(expert_key(*parse_key(key)), pool.ptr(index))
        self.audit = bool(audit)
        self.expected, self.slot_ptrs = {}, set()
        self.audit_stats = {"integrity_failures": 0, "gpu_audit_payload_bytes": 0, "gpu_audit_digest_d2h_bytes": 0}
        self.verifier = None
        if self.audit:
            from .integrity import DeviceIntegrity
            size = pool.expert_bytes
            self.verifier = DeviceIntegrity(ctx, size, allocation_size=lambda p: size if int(p) in self.slot_ptrs
                                            else ctx.owned_size(p))
        self.lock, self.active, self.last_event = threading.Lock(), False, None
        self.work = _stage_buffers(ctx, 16, config.hidden, config.intermediate)

    def forward(self, key: str, x, routing_weight=None) -> dict:
        if key not in self.index_of:
            raise KeyError("Requested expert is absent from the pinned native store")
        with self.lock:
            if self.active:
                raise RuntimeError("Nested requests could replace a live compute slot")
            self.active = True
            try:
                started = time.perf_counter()
                k = expert_key(*parse_key(key))
                (ptr,), (hit,) = self.cache.ensure([k])
                self.cache.wait_ready(None)
                if self.audit and not hit:
                    self._admit(key, k, ptr)
                out = _run_tiled_expert(self.ctx, self.work, ptr, self.config.hidden, self.config.intermediate,
                                        self.limit, x, routing_weight)
                self.cache.release([k], None)
                self.last_event = {"key": key, "source_tier": "primary_gpu" if hit else "host_pinned",
                                   "wall_ms": (time.perf_counter() - started) * 1000}
                return out
            finally:
                self.active = False

    def _admit(self, key, k, ptr):
        """Audit a freshly copied slot against its source's digest table; on a mismatch the slot is
        dropped before anything reads it and ValueError propagates."""
        from .integrity import digest_shape, hash_chunks
        if key not in self.expected:
            size = self.pool.expert_bytes
            src = np.ctypeslib.as_array((C.c_uint8 * size).from_address(self.pool.ptr(self.index_of[key])))
            table = np.empty(digest_shape(size), np.uint8)
            hash_chunks(src, table)
            self.expected[key] = table
        self.slot_ptrs.add(int(ptr))
        try:
            nbytes = self.verifier.verify(ptr, self.expected[key])
        except ValueError:
            self.cache.forget(k)
            self.audit_stats["integrity_failures"] += 1
            raise
        self.audit_stats["gpu_audit_payload_bytes"] += self.pool.expert_bytes
        self.audit_stats["gpu_audit_digest_d2h_bytes"] += nbytes

    def snapshot(self) -> dict:
        return dict(self.cache.stats(), integrity_mode="gpu-sha256" if self.audit else "none", **self.audit_stats)

    def close(self):
        if self.verifier is not None:
            self.verifier.close()
            self.verifier = None
        self.cache.close()
        for d in self.work.values():
            d.free()


class OffloadDecode:
    """`layers` MoE layers sharing one device cache; routed experts stream from host-pinned pools.

    pool_of(layer, expert) -> (pool, index) names each routed expert's host bytes; shared_ptrs[layer] is a
    resident tiled shared expert (or None). step(x, routing) runs every layer at T tokens with given
    routing: per layer, ensure its experts (copies on the cache stream), make the compute stream wait,
    re-point the layer's table (one launch), decode, release the slots -- all asynchronous, so the next
    layer's copies overlap this layer's compute.

    Routing is validated on the host when it is loaded (ids in range and distinct per token, weights finite:
    the reference's participation refusals, src/vesper/moe.py:18-30), and step_device runs what was loaded.

    audit=True is the reference's gpu-sha256 admission mode for this asynchronous path: every expert's
    digest table is taken once from its pinned source bytes (hashed on the device) and kept in HBM; the
    slots a layer admits are verified in one launch on an audit stream that waits for their copies, and
    the compute stream waits for the audit while the copy stream goes on with the next layer's copies;
    differing chunks accumulate in per-expert counters. After each layer an audit gate (mx_audit_gate)
    overwrites the layer's output with NaN when any expert it used -- admitted now or served as a hit of
    an earlier admission -- has a nonzero counter, so an output computed from bytes that failed their audit
    never passes as a number, and the NaN carries through every later layer. check_audit() (after a
    synchronisation) then refuses with ValueError, drops the failing slots from the cache and clears the
    counters; until it is called, a failing slot stays cached and every output that used it is NaN.
    """

    def __init__(self, ctx: _lib.Context, config: MoEConfig, layers: int, pool_of, shared_ptrs, cache: ExpertCache,
                 placeholder_ptr: int, audit: bool = False):
        self.ctx, self.config, self.layers, self.cache = ctx, config, int(layers), cache
        self.lib = ctx.lib
        self.handles = []
        self.stream = ctx.stream()
        self._owned = []
        cfg = _lib.MxMoeConfig(config.hidden, config.intermediate, config.experts, config.top_k,
                               _lib.MX_SCORE[config.score_func], config.route_scale, config.swiglu_limit,
                               _lib.MX_FMT_MXFP4 if config.shared else -1, config.max_tokens)
        rw = ctx.upload(np.zeros((config.experts, config.hidden), np.float32))   # router unused: routing is given
        self._owned.append(rw)
        for layer in range(self.layers):
            table = (C.c_void_p * config.experts)(*([placeholder_ptr] * config.experts))
            shared = C.c_void_p(shared_ptrs[layer]) if config.shared else None
            h = C.c_void_p()
            self.lib.layer_create(ctx._h(), C.byref(cfg), _lib.vp(rw), None, table, shared, C.byref(h))
            self.handles.append(h)
            for e in range(config.experts):
                pool, index = pool_of(layer, e)
                cache.register(expert_key(layer, e), pool.ptr(index))
        t, k = config.max_tokens, config.top_k
        self.routing = None
        self.ids = [ctx.empty((t, k), np.int32) for _ in range(self.layers)]
        self.wts = [ctx.empty((t, k), np.float32) for _ in range(self.layers)]
        self._owned += self.ids + self.wts
        self.audit = bool(audit)
        if self.audit:
            from .integrity import digest_shape
            self.slot_bytes = cache.slot_bytes
            self.table_bytes = digest_shape(self.slot_bytes)[0] * 32
            self.tables = ctx.empty((self.layers * config.experts, self.table_bytes), np.uint8)
            self.mismatch = ctx.upload(np.zeros((self.layers, config.experts), np.uint32))
            self._owned += [self.tables, self.mismatch]
            for layer in range(self.layers):
                for e in range(config.experts):
                    pool, index = pool_of(layer, e)
                    self.lib.sha256_chunks(ctx._h(), C.c_void_p(pool.ptr(index)), self.slot_bytes,
                                           C.c_void_p(self._table(layer, e)), _lib._stream(self.stream))
            ctx.sync(self.stream)
            self.audit_stream = ctx.stream()
            self.audit_done = ctx.event()
            self.audited_slots = 0

    def _table(self, layer: int, expert: int) -> int:
        return self.tables.ptr + (layer * self.config.experts + expert) * self.table_bytes

    def _checked_ids(self, ids) -> np.ndarray:
        cfg = self.config
        ids = np.ascontiguousarray(ids)
        if ids.dtype.kind not in "iu" or ids.ndim != 2 or ids.shape[1] != cfg.top_k or not 1 <= len(ids) <= cfg.max_tokens:
            raise ValueError(f"routing ids must be [T, {cfg.top_k}] integers with 1 <= T <= {cfg.max_tokens}")
        if ids.min() < 0 or ids.max() >= cfg.experts:
            raise ValueError("Expert ID is outside the pinned model")
        if cfg.top_k > 1 and np.any(np.diff(np.sort(ids, axis=1), axis=1) == 0):
            raise ValueError("Repeated expert IDs within a token are outside the unique-topk scope")
        return ids.astype(np.int32)

    def load_routing(self, routing):
        """routing[layer] = (ids [T, k] integers, weights [T, k] FP32): validated, kept on the host for the
        cache keys and copied to the device (synchronously). Raises ValueError before any copy."""
        if len(routing) != self.layers:
            raise ValueError(f"routing must give {self.layers} layers")
        checked = []
        for ids, w in routing:
            ids = self._checked_ids(ids)
            w = np.ascontiguousarray(w, np.float32)
            if w.shape != ids.shape or not np.isfinite(w).all():
                raise ValueError("route weights must be finite and shaped like the ids")
            checked.append((ids, w))
        for layer, (ids, w) in enumerate(checked):
            self.ctx.copy_h2d(self.ids[layer].ptr, ids)
            self.ctx.copy_h2d(self.wts[layer].ptr, w)
        self.routing = [ids for ids, _ in checked]

    def load_routing_device(self, host_ids, device_routing, stream=None):
        """Routing already on the device: device_routing[layer] = (ids, weights) device arrays of [T, k], copied
        into place on `stream` without a host wait; host_ids[layer] is the same ids on the host, validated and
        used for the cache keys. A device copy that differs from the host ids reaches the kernels' own
        validation: check_routes() after a synchronisation refuses the steps since the last check."""
        if len(host_ids) != self.layers or len(device_routing) != self.layers:
            raise ValueError(f"routing must give {self.layers} layers")
        checked = [self._checked_ids(ids) for ids in host_ids]
        for layer, (ids_dev, w_dev) in enumerate(device_routing):
            nbytes = checked[layer].nbytes
            if ids_dev.nbytes != nbytes or w_dev.nbytes != nbytes:
                raise ValueError("device routing must match the host ids' shape")
            self.ctx.copy_d2d(self.ids[layer].ptr, ids_dev.ptr, nbytes, stream)
            self.ctx.copy_d2d(self.wts[layer].ptr, w_dev.ptr, nbytes, stream)
        self.routing = checked

    def check_routes(self):
        """After a synchronisation: ValueError if any layer's kernels replaced a routing id since the last check
        (an id that the host validation did not see, e.g. a device copy that differs)."""
        replaced = {}
        for layer, h in enumerate(self.handles):
            count = C.c_uint32()
            self.lib.layer_route_errors(h, C.byref(count), 1, _lib._stream(self.stream))
            if count.value:
                replaced[layer] = int(count.value)
        if replaced:
            raise ValueError(f"routing ids outside the model or repeated within a token (per layer: {replaced})")

    def step_device(self, x_ptr: int, tokens: int, y_ptrs, routing_host=None):
        """Enqueue one step on self.stream over the routing of the last load_routing (routing_host, if given,
        must be that routing)."""
        if self.routing is None:
            raise RuntimeError("load_routing() must come before a step")
        if routing_host is not None and any(not np.array_equal(np.asarray(r)[:tokens], own[:tokens])
                                            for r, own in zip(routing_host, self.routing)):
            raise ValueError("step routing differs from the routing loaded on the device")
        if not 1 <= tokens <= min(len(r) for r in self.routing):
            raise ValueError("token count outside the loaded routing")
        for layer in range(self.layers):
            experts = np.unique(self.routing[layer][:tokens])
            keys = [expert_key(layer, int(e)) for e in experts]
            ptrs, hits = self.cache.ensure(keys)
            if self.audit:
                miss = [i for i in range(len(keys)) if not hits[i]]
                if miss:
                    n = len(miss)
                    slots = (C.c_void_p * n)(*[ptrs[i] for i in miss])
                    tables = (C.c_void_p * n)(*[self._table(layer, int(experts[i])) for i in miss])
                    counters = (C.c_int32 * n)(*[layer * self.config.experts + int(experts[i]) for i in miss])
                    self.cache.wait_ready(self.audit_stream)
                    self.lib.sha256_verify(self.ctx._h(), slots, tables, counters, n, self.slot_bytes,
                                           C.c_void_p(self.mismatch.ptr), _lib._stream(self.audit_stream))
                    self.ctx.record(self.audit_done, self.audit_stream)
                    self.lib.stream_wait_event(self.ctx._h(), _lib._stream(self.stream), C.c_void_p(self.audit_done))
                    self.audited_slots += n
            self.cache.wait_ready(self.stream)
            arr_e = (C.c_int32 * len(experts))(*[int(e) for e in experts])
            arr_p = (C.c_void_p * len(experts))(*ptrs)
            self.lib.layer_set_experts(self.handles[layer], len(experts), arr_e, arr_p, _lib._stream(self.stream))
            src = x_ptr if layer == 0 else y_ptrs[layer - 1]
            self.lib.moe_decode_routed(self.handles[layer], C.c_void_p(int(src)), int(tokens),
                                       C.c_void_p(self.ids[layer].ptr), C.c_void_p(self.wts[layer].ptr),
                                       C.c_void_p(int(y_ptrs[layer])), _lib._stream(self.stream))
            if self.audit:
                used = (C.c_int32 * len(experts))(*[layer * self.config.experts + int(e) for e in experts])
                self.lib.audit_gate(self.ctx._h(), C.c_void_p(self.mismatch.ptr), self.layers * self.config.experts,
                                    used, len(experts), C.c_void_p(int(y_ptrs[layer])),
                                    int(tokens) * self.config.hidden, _lib._stream(self.stream))
            self.cache.release(keys, self.stream)

    def check_audit(self):
        """After a synchronisation: raise ValueError if any slot admitted since the last check differed from
        its source's digests (those keys are dropped from the cache and the counters cleared)."""
        if not self.audit:
            return
        self.ctx.sync()
        counts = self.mismatch.download()
        bad = np.argwhere(counts > 0)
        if len(bad):
            for layer, e in bad:
                self.cache.forget(expert_key(int(layer), int(e)))
            self.mismatch.upload(np.zeros_like(counts))
            raise ValueError("GPU expert bytes differ from verified original SHA-256 chunks: "
                             + ", ".join(f"{int(l)}:{int(e)}" for l, e in bad))

    def close(self):
        if self.audit:
            self.ctx.sync(self.audit_stream)
            self.ctx.destroy_stream(self.audit_stream)
            self.ctx.destroy_event(self.audit_done)
            self.audit = False
        for h in self.handles:
            self.lib.layer_destroy(h)
        self.handles = []
        for d in self._owned:
            d.free()
        self._owned = []
        self.ctx.destroy_stream(self.stream)


def decode_routed(layer, x_ptr: int, tokens: int, ids_ptr: int, weights_ptr: int, y_ptr: int, stream=None):
    """mx_moe_decode_routed on a MoELayer (routing given on the device). Invalid ids are replaced in bounds and
    counted: read MoELayer.route_errors() after the call to refuse its output."""
    layer.lib.moe_decode_routed(layer.handle, C.c_void_p(int(x_ptr)), int(tokens), C.c_void_p(int(ids_ptr)),
                                C.c_void_p(int(weights_ptr)), C.c_void_p(int(y_ptr)), _lib._stream(stream))
