"""Host side of the SHA-256 admission audit (vesper_amd.integrity), no GPU.

The digest table is checked against hashlib chunk by chunk on payloads that straddle every SHA-256 padding
boundary and the 4 KiB chunk boundary, and against the FIPS 180-4 example digests. DeviceIntegrity's
argument refusals are checked on a recording stand-in for the device context: every refusal must happen
before a single library call.
"""

import hashlib

import numpy as np
import pytest

from vesper_amd.integrity import CHUNK_BYTES, DeviceIntegrity, digest_shape, hash_chunks

# FIPS 180-4 / NIST CSRC example messages and their SHA-256 digests
FIPS_EXAMPLES = {
    b"abc": "ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad",
    b"abcdbcdecdefdefgefghfghighijhijkijkljklmklmnlmnomnopnopq":
        "248d6a61d20638b8e5c026930c3e6039a33ce45964ff2167f6ecedd419db06c1",
}


def table_of(data: np.ndarray) -> np.ndarray:
    out = np.zeros(digest_shape(data.size), np.uint8)
    hash_chunks(data, out)
    return out


@pytest.mark.parametrize("message,digest", FIPS_EXAMPLES.items())
def test_single_chunk_payloads_give_the_fips_digests(message, digest):
    assert table_of(np.frombuffer(message, np.uint8)).tobytes().hex() == digest


@pytest.mark.parametrize("size", [1, 55, 56, 64, 119, 120, CHUNK_BYTES - 1, CHUNK_BYTES, CHUNK_BYTES + 1,
                                  3 * CHUNK_BYTES + 57])
def test_every_chunk_is_the_hashlib_digest_of_its_slice(size):
    data = np.random.default_rng(size).integers(0, 256, size, dtype=np.uint8)
    table = table_of(data)
    assert table.shape == ((size + CHUNK_BYTES - 1) // CHUNK_BYTES, 32)
    for row, start in enumerate(range(0, size, CHUNK_BYTES)):
        assert table[row].tobytes() == hashlib.sha256(data[start:start + CHUNK_BYTES].tobytes()).digest()


def test_one_flipped_byte_changes_exactly_its_chunk():
    data = np.zeros(5 * CHUNK_BYTES, np.uint8)
    clean = table_of(data)
    data[2 * CHUNK_BYTES + 100] ^= 1
    changed = np.flatnonzero((table_of(data) != clean).any(axis=1))
    assert changed.tolist() == [2]


def test_digest_shape_bounds():
    assert digest_shape(1) == (1, 32)
    assert digest_shape(CHUNK_BYTES) == (1, 32)
    assert digest_shape(CHUNK_BYTES + 1) == (2, 32)
    assert digest_shape(1 << 30) == (1 << 18, 32)
    for bad in (0, -4096, (1 << 30) + 1, True, 4096.0, "4096", None):
        with pytest.raises(ValueError, match="bounded integrity payload"):
            digest_shape(bad)


def test_hash_chunks_refuses_layouts_it_cannot_read_or_write():
    data = np.arange(2 * CHUNK_BYTES, dtype=np.int64).astype(np.uint8)
    good = np.zeros((2, 32), np.uint8)
    for source in (data[1::2], data.view(np.int8), data.reshape(4, -1), data.view(np.uint16)):
        with pytest.raises(ValueError, match="contiguous byte array"):
            hash_chunks(source, good)
    for target in (np.zeros((1, 32), np.uint8), np.zeros((2, 32), np.int8), np.zeros(64, np.uint8)):
        with pytest.raises(ValueError, match="wrong size"):
            hash_chunks(data, target)
    with pytest.raises(ValueError, match="overwrite source"):
        hash_chunks(data, data[CHUNK_BYTES:CHUNK_BYTES + 64].reshape(2, 32))


class RecordingLib:
    """Stands in for the library: records every call instead of touching a device."""

    def __init__(self):
        self.calls = []

    def __getattr__(self, name):
        return lambda *args: self.calls.append(name)


class StubContext:
    def __init__(self, owned):
        self.lib, self.owned = RecordingLib(), owned

    def _h(self):
        return 1

    def owned_size(self, pointer):
        return self.owned.get(int(pointer), 0)

    def empty(self, shape, dtype):
        from types import SimpleNamespace
        return SimpleNamespace(ptr=0xD16E57, free=lambda: None)


def checker(size=2 * CHUNK_BYTES, owned=None):
    ctx = StubContext(owned if owned is not None else {0x1000: 2 * CHUNK_BYTES})
    return DeviceIntegrity(ctx, size), ctx


def test_digests_refuses_reads_past_owned_bytes_or_capacity_before_any_call():
    audit, ctx = checker()
    with pytest.raises(ValueError, match="owned source"):
        audit.digests(0x1000 + 64, size=64)           # not an allocation base
    with pytest.raises(ValueError, match="fixed buffer scope"):
        audit.digests(0x1000, size=2 * CHUNK_BYTES + 1)
    audit.ctx.owned[0x2000] = 100
    with pytest.raises(ValueError, match="owned source"):
        audit.digests(0x2000, size=101)
    for bad in (np.zeros((1, 32), np.uint8), np.zeros((2, 32), np.uint16), np.zeros((2, 32), np.uint8)[:, ::-1]):
        with pytest.raises(ValueError, match="complete digest table"):
            audit.digests(0x1000, target=bad)
    readonly = np.zeros((2, 32), np.uint8)
    readonly.setflags(write=False)
    with pytest.raises(ValueError, match="complete digest table"):
        audit.digests(0x1000, target=readonly)
    assert ctx.lib.calls == []


def test_verify_refuses_aliasing_and_foreign_tables_before_any_call():
    audit, ctx = checker()
    expected = np.zeros((2, 32), np.uint8)
    with pytest.raises(ValueError, match="complete expert"):
        audit.verify(0x1000, np.zeros((3, 32), np.uint8))
    with pytest.raises(ValueError, match="complete expert"):
        audit.verify(0x1000, expected.view(np.int8))
    with pytest.raises(ValueError, match="original digest"):
        audit.verify(0x1000, expected, target=expected)
    scratch = np.zeros((2, 32), np.uint8)
    with pytest.raises(ValueError, match="comparison"):
        audit.verify(0x1000, expected, target=scratch, comparison=scratch.view(np.bool_))
    with pytest.raises(ValueError, match="comparison"):
        audit.verify(0x1000, expected, comparison=expected.view(np.bool_))
    with pytest.raises(ValueError, match="wrong layout"):
        audit.verify(0x1000, expected, comparison=np.zeros((2, 32), np.uint8))
    assert ctx.lib.calls == []


def test_closed_checker_refuses_work():
    audit, ctx = checker()
    audit.close()
    with pytest.raises(RuntimeError, match="closed"):
        audit.digests(0x1000)
    assert ctx.lib.calls == []


def test_verify_compares_the_table_the_device_returns():
    """With a stand-in device that 'returns' a given table, verify passes on equality and refuses one
    differing byte (the comparison scratch variant too)."""
    audit, ctx = checker()
    expected = np.random.default_rng(7).integers(0, 256, (2, 32), dtype=np.uint8)
    for returned, ok in ((expected.copy(), True), (expected ^ np.eye(2, 32, 5, dtype=np.uint8), False)):
        audit.digests = lambda pointer, target=None, returned=returned: returned
        for comparison in (None, np.zeros((2, 32), np.bool_)):
            if ok:
                assert audit.verify(0x1000, expected, comparison=comparison) == 64
            else:
                with pytest.raises(ValueError, match="differ from verified original"):
                    audit.verify(0x1000, expected, comparison=comparison)


def test_native_host_digest_table_equals_hashlib():
    """mx_host_sha256_chunks (the store's host digest tables, OpenSSL on host threads) against hashlib chunk by
    chunk, for a short last chunk, a single chunk and several thread counts; refusals as hash_chunks'."""
    import hashlib
    from vesper_amd.integrity import digest_shape, hash_chunks_native
    rng = np.random.default_rng(3)
    for size, threads in ((4096 * 37 + 123, 1), (4096 * 37 + 123, 5), (4096, 4), (1000, 2), (4096 * 64, 64)):
        data = rng.integers(0, 256, size, dtype=np.uint8)
        table = np.zeros(digest_shape(size), np.uint8)
        hash_chunks_native(data, table, threads)
        for c in range(table.shape[0]):
            assert table[c].tobytes() == hashlib.sha256(data[4096 * c:4096 * (c + 1)].tobytes()).digest(), (size, c)
    data = rng.integers(0, 256, 8192, dtype=np.uint8)
    with pytest.raises(ValueError):
        hash_chunks_native(data, np.zeros((3, 32), np.uint8))
    with pytest.raises(ValueError):
        hash_chunks_native(data.astype(np.int16), np.zeros((4, 32), np.uint8))
