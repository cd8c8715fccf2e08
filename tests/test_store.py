"""The on-disk expert store (vesper_amd.store) and the O_DIRECT reader (vesper_amd.disk), no GPU.

A store written by build_store reopens as a NativeStore whose reads return the written bytes, checked against
the manifest's SHA-256 (whole expert and each tensor); every refusal of the reference's reader is exercised
on a manifest or file damaged after writing, and expert fixtures round-trip through the reference's
fixture format.
"""

import hashlib
import json

import numpy as np
import pytest

from oracle.inputs import mxfp4_expert
from vesper_amd.disk import DirectReader
from vesper_amd.resources import MemoryBudget, MiB
from vesper_amd.store import (BASELINE_PROFILE, REFERENCE_PROFILE, ModelProfile, NativeStore, build_store,
                              expert_key, load_expert_fixture, tensor_layout, validate_store_limit,
                              write_expert_fixture)

TINY = ModelProfile("test/tiny-moe", "r1", 512, 256, 16, 3, 10.0, 48)


def experts(rng, keys, profile=TINY):
    return [(layer, expert, mxfp4_expert(rng, profile.hidden, profile.intermediate)) for layer, expert in keys]


def concat(arrays, profile=TINY):
    return np.concatenate([arrays[n].ravel() for n in profile.expert_layout()])


def budget():
    return MemoryBudget(cap=64 * MiB, available_floor=0)


def test_layouts_and_sizes():
    assert REFERENCE_PROFILE.expert_bytes == 18_800_640            # the reference's one expert
    assert BASELINE_PROFILE.expert_bytes == 23_396_352
    for profile in (REFERENCE_PROFILE, BASELINE_PROFILE, TINY):
        layout = tensor_layout(profile)
        assert list(layout) == ["w1_weight", "w1_scale", "w3_weight", "w3_scale", "w2_weight", "w2_scale"]
        ends = [r["offset"] + r["bytes"] for r in layout.values()]
        assert [r["offset"] for r in layout.values()][1:] == ends[:-1] and ends[-1] == profile.expert_bytes
        assert profile.expert_bytes % 4096 == 0
    assert expert_key(39, 383) == "39:383"
    for bad in ((40, 0), (0, 384), (-1, 0), (0, True)):
        with pytest.raises(ValueError, match="outside the pinned model"):
            expert_key(*bad)
    for bad in (0, 49, 4.0, True):
        with pytest.raises(ValueError, match="one to 48"):
            validate_store_limit(bad)


def test_written_store_reads_back_every_expert(direct_io_dir):
    rng = np.random.default_rng(5)
    items = experts(rng, [(0, 3), (2, 15), (1, 0)])
    report = build_store(items, direct_io_dir / "store", max_experts=3, profile=TINY)
    assert report["experts"] == 3 and report["file_bytes"] == 3 * TINY.expert_bytes
    manifest = json.loads((direct_io_dir / "store" / "manifest.json").read_text())
    assert [e["key"] for e in manifest["entries"]] == ["0:3", "2:15", "1:0"]
    with NativeStore(direct_io_dir / "store", budget(), max_experts=3, profile=TINY) as store:
        assert set(store.entries) == {"0:3", "2:15", "1:0"}
        target = np.empty(TINY.expert_bytes, np.uint8)
        for layer, expert, arrays in items:
            store.read_into(f"{layer}:{expert}", target)
            np.testing.assert_array_equal(target, concat(arrays))
        store.gpu_integrity = True
        store.read_into("2:15", target)
        table = store.expected_chunks["2:15"]
        assert table.shape == (TINY.expert_bytes // 4096, 32)
        assert table[1].tobytes() == hashlib.sha256(target[4096:8192].tobytes()).digest()
        assert store.read_calls == 4 and store.bytes_read == 4 * TINY.expert_bytes
    assert store.reader is None and store.expected_chunks == {}


def test_store_refusals(direct_io_dir):
    rng = np.random.default_rng(6)
    items = experts(rng, [(0, 1), (0, 2)])
    with pytest.raises(ValueError, match="limit"):
        build_store(items, direct_io_dir / "a", max_experts=1, profile=TINY)
    assert not (direct_io_dir / "a").exists()
    with pytest.raises(ValueError, match="different original experts"):
        build_store([items[0], items[0]], direct_io_dir / "b", max_experts=2, profile=TINY)
    assert not (direct_io_dir / "b").exists()                          # a failed build leaves nothing
    build_store(items, direct_io_dir / "s", max_experts=2, profile=TINY)
    with pytest.raises(FileExistsError):
        build_store(items, direct_io_dir / "s", max_experts=2, profile=TINY)
    with pytest.raises(ValueError, match="pinned format"):
        NativeStore(direct_io_dir / "s", budget(), max_experts=2)      # a TINY store is not the reference model
    with pytest.raises(ValueError, match="probe size"):
        NativeStore(direct_io_dir / "s", budget(), max_experts=1, profile=TINY)

    def damaged(edit):
        m = json.loads((direct_io_dir / "s" / "manifest.json").read_text())
        edit(m)
        (direct_io_dir / "s" / "manifest.json").write_text(json.dumps(m))

    original = (direct_io_dir / "s" / "manifest.json").read_text()
    for edit, message in ((lambda m: m["entries"][1].update(offset=0), "overlapping"),
                          (lambda m: m["entries"][1]["provenance"].update(layer=5), "outside the pinned model"),
                          (lambda m: m["entries"][0].update(sha256="xyz"), "overlapping"),
                          (lambda m: m.update(file_bytes=1), "file size"),
                          (lambda m: m["layout"]["w1_scale"].update(offset=1), "layout"),
                          (lambda m: m["entries"][0]["provenance"]["tensors"].pop(), "Incomplete")):
        damaged(edit)
        with pytest.raises(ValueError, match=message):
            NativeStore(direct_io_dir / "s", budget(), max_experts=2, profile=TINY)
        (direct_io_dir / "s" / "manifest.json").write_text(original)
    # a flipped byte in experts.bin: the whole-expert hash refuses the read
    data = bytearray((direct_io_dir / "s" / "experts.bin").read_bytes())
    data[TINY.expert_bytes + 77] ^= 1
    (direct_io_dir / "s" / "experts.bin").write_bytes(bytes(data))
    with NativeStore(direct_io_dir / "s", budget(), max_experts=2, profile=TINY) as store:
        target = np.empty(TINY.expert_bytes, np.uint8)
        store.read_into("0:1", target)
        with pytest.raises(ValueError, match="store hash"):
            store.read_into("0:2", target)
        with pytest.raises(KeyError):
            store.read_into("0:3", target)
    with pytest.raises(RuntimeError, match="closed"):
        store.read_into("0:1", target)


def test_direct_reader_alignment_and_budget(direct_io_dir):
    path = direct_io_dir / "blob.bin"
    payload = np.random.default_rng(7).integers(0, 256, 5 * 4096, dtype=np.uint8)
    path.write_bytes(payload.tobytes())
    b = budget()
    with DirectReader(path, 2 * 4096, b) as reader:
        assert b.reserved == 2 * 4096
        assert reader.read(4096, 8192) == payload[4096:8192].tobytes()
        np.testing.assert_array_equal(reader.array()[:8192], payload[4096:12288])
        for offset, size in ((1, 4096), (0, 100), (0, 3 * 4096), (-4096, 4096)):
            with pytest.raises(ValueError, match="aligned"):
                reader.read(offset, size)
        with pytest.raises(OSError, match="Short"):
            reader.read(4 * 4096, 8192)                           # past the end of the file
    assert b.reserved == 0
    with pytest.raises(RuntimeError, match="closed"):
        reader.read(0, 4096)


def test_budget_caps_reservations():
    b = MemoryBudget(cap=10 * MiB, available_floor=0)
    b.acquire(6 * MiB)
    with pytest.raises(MemoryError, match="cap"):
        b.acquire(5 * MiB)
    with pytest.raises(MemoryError, match="reserve"):
        MemoryBudget(cap=1 << 60, available_floor=1 << 59).acquire(1)
    b.release(6 * MiB)
    assert (b.reserved, b.peak) == (0, 6 * MiB)
    with pytest.raises(ValueError):
        b.release(1)


def test_expert_fixture_round_trip_and_store_from_fixtures(direct_io_dir):
    rng = np.random.default_rng(8)
    arrays = mxfp4_expert(rng, TINY.hidden, TINY.intermediate)
    path = write_expert_fixture(direct_io_dir / "fx", 1, 9, arrays, TINY)
    got, manifest = load_expert_fixture(path, TINY)
    assert manifest["layer"] == 1 and manifest["expert"] == 9
    for name in arrays:
        np.testing.assert_array_equal(got[name], arrays[name])
    build_store([path], direct_io_dir / "store", max_experts=1, profile=TINY)
    with NativeStore(direct_io_dir / "store", budget(), max_experts=1, profile=TINY) as store:
        target = np.empty(TINY.expert_bytes, np.uint8)
        store.read_into("1:9", target)
        np.testing.assert_array_equal(target, concat(arrays))
    m = json.loads((direct_io_dir / "fx" / "manifest.json").read_text())
    m["tensors"][0]["sha256"] = "0" * 64
    (direct_io_dir / "fx" / "manifest.json").write_text(json.dumps(m))
    with pytest.raises(ValueError, match="source hash"):
        load_expert_fixture(path, TINY)


class HostSlots:
    """A GPU backend stand-in whose slots are host arrays; verify() hashes the slot's 4 KiB chunks against the
    store's digest table of the verified read (what HipCacheBackend.verify does on the device)."""

    def __init__(self, store, slots):
        from vesper_amd.integrity import digest_shape, hash_chunks
        self.primary_slots, self.helper_slots, self.store = slots, 0, store
        self.staging = [np.zeros(store.size, np.uint8), np.zeros(store.size, np.uint8)]
        self.slots = [np.zeros(store.size, np.uint8) for _ in range(slots)]
        self._shape, self._hash = digest_shape, hash_chunks

    def write(self, tier, slot, data):
        self.slots[slot][:] = data

    def read(self, tier, slot, target):
        target[:] = self.slots[slot]

    def verify(self, tier, slot, key):
        table = np.empty(self._shape(self.store.size), np.uint8)
        self._hash(self.slots[slot], table)
        if not np.array_equal(table, self.store.expected_chunks[key]):
            raise ValueError("GPU expert bytes differ from verified original SHA-256 chunks")
        return table.nbytes


@pytest.mark.parametrize("gpu", [False, True])
def test_batch_promotion_reads_ahead_with_the_same_tiers_and_refusals(direct_io_dir, gpu):
    """TieredCache.promote over a real NativeStore: the store's prefetch pipeline reads and checks the batch's
    store entries ahead of their uploads (three reader threads, six host buffers); the slots hold the written
    bytes, the counters and tier walk are those of single requests, a damaged entry fails the batch at that
    key with nothing published for it (earlier keys stay promoted), and the pipeline's buffers leave the
    budget afterwards."""
    from vesper_amd.cache import TieredCache
    rng = np.random.default_rng(11)
    keys = [(0, e) for e in range(6)]
    items = experts(rng, keys)
    build_store(items, direct_io_dir / "store", max_experts=6, profile=TINY)
    b = MemoryBudget(cap=64 * MiB, available_floor=0)
    with NativeStore(direct_io_dir / "store", b, max_experts=6, profile=TINY) as store:
        store.gpu_integrity = gpu
        backend = HostSlots(store, 3)
        cache = TieredCache(store, backend, b, 0, available=lambda: 1 << 40, gpu_verify=gpu)
        held = b.reserved
        assert cache.promote(["0:0", "0:1", "0:2"]) == ["store"] * 3
        snap = cache.snapshot()
        assert snap["primary_keys"] == ["0:0", "0:1", "0:2"] and snap["counters"]["store_reads_completed"] == 3
        for key, (layer, expert, arrays) in zip(["0:0", "0:1", "0:2"], items):
            slot = snap["primary_keys"].index(key)
            np.testing.assert_array_equal(backend.slots[slot], concat(arrays))
        # a hit, then a store read that demotes the least recent expert (no RAM tier: dropped)
        assert cache.promote(["0:0", "0:3"]) == ["primary_gpu", "store"]
        assert cache.snapshot()["primary_keys"] == ["0:2", "0:0", "0:3"]
        tables = sum(t.nbytes for t in store.expected_chunks.values())   # kept for the GPU audit
        assert store.read_calls == 4 and b.reserved == held + tables and len(store.expected_chunks) == (4 if gpu else 0)
        # damage entry 0:5 on disk: the batch fails there, 0:4 stays promoted
        path = direct_io_dir / "store" / "experts.bin"
        data = bytearray(path.read_bytes())
        data[5 * TINY.expert_bytes + 100] ^= 1
        path.write_bytes(bytes(data))
        with pytest.raises(ValueError, match="differ"):
            cache.promote(["0:4", "0:5", "0:1"])
        snap = cache.snapshot()
        assert "0:4" in snap["primary_keys"] and "0:5" not in snap["primary_keys"]
        c = snap["counters"]
        assert c["integrity_failures"] == 1 and c["requests_failed"] == 1 and c["requests_completed"] == 6
        assert b.reserved == held + sum(t.nbytes for t in store.expected_chunks.values())
        cache.close()
