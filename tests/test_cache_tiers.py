"""The exclusive expert tiers (vesper_amd.cache.TieredCache) over a fake store and a fake GPU backend, no GPU.

Checks the tier an expert is served from across promotions and demotions, that an expert is in one tier at a
time, the RAM tier's LRU and capacity, both integrity modes (a corrupted upload is refused and nothing is
published; the GPU mode defers host checks to the upload audit), memory-pressure refusal, and that requests
cannot nest.
"""

import hashlib

import numpy as np
import pytest

from vesper_amd.cache import TieredCache
from vesper_amd.resources import MemoryBudget, MiB

SIZE = 4096


class FakeStore:
    def __init__(self, keys):
        self.size = SIZE
        self.entries = {k: None for k in keys}
        self.bytes = {k: np.random.default_rng(i).integers(0, 256, SIZE, dtype=np.uint8) for i, k in enumerate(keys)}
        self.digests = {k: hashlib.sha256(v.tobytes()).hexdigest() for k, v in self.bytes.items()}
        self.reads = []

    def read_into(self, key, target):
        self.reads.append(key)
        np.copyto(target, self.bytes[key])

    def validate(self, key, data, tensors=False):
        if hashlib.sha256(data.tobytes()).hexdigest() != self.digests[key]:
            raise ValueError("Native expert bytes differ from the store hash")


class FakeBackend:
    """GPU slots as host arrays; `corrupt_next` flips a byte of the next upload."""

    def __init__(self, slots, store, verify=True):
        self.primary_slots, self.helper_slots = slots, 0
        self.staging = [np.zeros(SIZE, np.uint8), np.zeros(SIZE, np.uint8)]
        self.slots = [np.zeros(SIZE, np.uint8) for _ in range(slots)]
        self.store, self.corrupt_next, self.audits = store, False, 0
        if not verify:
            self.verify = None

    def write(self, tier, slot, data):
        self.slots[slot][:] = data
        if self.corrupt_next:
            self.slots[slot][100] ^= 1
            self.corrupt_next = False

    def read(self, tier, slot, target):
        target[:] = self.slots[slot]

    def verify(self, tier, slot, key):
        self.audits += 1
        if hashlib.sha256(self.slots[slot].tobytes()).hexdigest() != self.store.digests[key]:
            raise ValueError("GPU expert bytes differ from verified original SHA-256 chunks")
        return 32


def make(slots=2, ram=2, gpu=False, available=None):
    store = FakeStore([f"0:{i}" for i in range(6)])
    backend = FakeBackend(slots, store)
    cache = TieredCache(store, backend, MemoryBudget(cap=64 * MiB, available_floor=0), ram * SIZE,
                        available=available or (lambda: 1 << 40), gpu_verify=gpu)
    return cache, store, backend


def serve(cache, key):
    with cache.acquire(key) as (slot, origin):
        np.testing.assert_array_equal(cache.backend.slots[slot], cache.source.bytes[key])
        return origin


@pytest.mark.parametrize("gpu", [False, True])
def test_promotion_demotion_and_exclusive_tiers(gpu):
    cache, store, backend = make(gpu=gpu)
    tiers = [serve(cache, k) for k in ("0:0", "0:1", "0:0", "0:2", "0:1", "0:3", "0:4", "0:0")]
    # 0:2 demotes 0:1 (least recent) to RAM; 0:1 comes back from RAM, demoting 0:0; 0:3 and 0:4 demote 0:2
    # and 0:1, and the RAM tier (2 experts) drops 0:0 to make room, so 0:0 comes from the store again and
    # demotes 0:3 (RAM drops 0:2)
    assert tiers == ["store", "store", "primary_gpu", "store", "ram", "store", "store", "store"]
    snap = cache.snapshot()
    assert snap["primary_keys"] == ["0:4", "0:0"] and snap["ram_keys"] == ["0:1", "0:3"]
    assert not set(snap["primary_keys"]) & set(snap["ram_keys"])
    c = snap["counters"]
    assert (c["primary_hits"], c["ram_hits"], c["store_reads_completed"]) == (1, 1, 6)
    assert c["primary_evictions"] == 5 and c["ram_capacity_evictions"] == 2
    assert store.reads == ["0:0", "0:1", "0:2", "0:3", "0:4", "0:0"]
    if gpu:
        assert backend.audits == 7 and c["cpu_checks_deferred"] > 0 and c["primary_audit_readback_bytes"] == 0
    else:
        assert c["primary_audit_readback_bytes"] == 7 * SIZE and c["cpu_checks_deferred"] == 0
    assert snap["integrity_mode"] == ("gpu-sha256" if gpu else "readback")


@pytest.mark.parametrize("gpu", [False, True])
def test_corrupted_upload_is_refused_and_not_published(gpu):
    cache, store, backend = make(gpu=gpu)
    serve(cache, "0:0")
    backend.corrupt_next = True
    with pytest.raises(ValueError, match="differ"):
        serve(cache, "0:1")
    snap = cache.snapshot()
    assert snap["primary_keys"] == ["0:0"] and snap["counters"]["integrity_failures"] == 1
    assert snap["counters"]["requests_failed"] == 1
    assert serve(cache, "0:1") == "store"                        # admitted afresh on the next request


def test_ram_tier_refusals_and_pressure():
    cache, _, _ = make(slots=1, ram=0)
    serve(cache, "0:0")
    serve(cache, "0:1")                                          # no RAM tier: 0:0 is simply dropped
    snap = cache.snapshot()
    assert snap["ram_keys"] == [] and snap["counters"]["primary_d2h_bytes"] == 0
    assert serve(cache, "0:0") == "store"
    free = {"bytes": 1 << 40}
    cache, _, _ = make(slots=1, ram=4, available=lambda: free["bytes"])
    cache.budget.available_floor = 1 << 30
    serve(cache, "0:0")
    serve(cache, "0:1")
    assert cache.snapshot()["ram_keys"] == ["0:0"]
    free["bytes"] = 1 << 29                                      # below the floor: RAM copies go first
    with pytest.raises(MemoryError, match="reserve"):
        serve(cache, "0:1")
    snap = cache.snapshot()
    assert snap["ram_keys"] == [] and snap["counters"]["ram_pressure_evictions"] == 1
    assert snap["counters"]["pressure_refusals"] == 1


def test_requests_do_not_nest_and_unknown_keys_fail():
    cache, _, _ = make()
    with cache.acquire("0:0"):
        with pytest.raises(RuntimeError, match="Nested"):
            with cache.acquire("0:1"):
                pass
    with pytest.raises(KeyError):
        with cache.acquire("9:9"):
            pass
    cache.close()
    with pytest.raises(RuntimeError, match="closed"):
        with cache.acquire("0:0"):
            pass


def test_construction_refusals():
    store = FakeStore(["0:0"])
    b = MemoryBudget(cap=64 * MiB, available_floor=0)
    with pytest.raises(ValueError, match="primary slot"):
        TieredCache(store, FakeBackend(0, store), b, 0)
    with pytest.raises(ValueError, match="audit backend"):
        TieredCache(store, FakeBackend(1, store, verify=False), b, 0, gpu_verify=True)
    helper = FakeBackend(1, store)
    helper.helper_slots = 1
    with pytest.raises(ValueError, match="second device"):
        TieredCache(store, helper, b, 0)
    shared = FakeBackend(1, store)
    shared.staging = [shared.staging[0], shared.staging[0]]
    with pytest.raises(ValueError, match="distinct staging"):
        TieredCache(store, shared, b, 0)
