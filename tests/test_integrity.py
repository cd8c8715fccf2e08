"""Host side of the SHA-256 admission audit (vesper_amd.integrity), no GPU: the reference's own cases
(tests/test_integrity.py:13-55) for digest_shape, hash_chunks and DeviceIntegrity's refusals before any
device work."""

import hashlib
from types import SimpleNamespace

import numpy as np
import pytest

from vesper_amd.integrity import DeviceIntegrity, digest_shape, hash_chunks


def test_known_sha256_and_every_chunk_boundary():
    abc = np.frombuffer(b"abc", np.uint8)
    actual = np.empty(digest_shape(3), np.uint8)
    hash_chunks(abc, actual)
    assert actual.tobytes().hex() == "ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad"
    for size in (1, 55, 56, 63, 64, 65, 4095, 4096, 4097, 8192):
        data = np.arange(size, dtype=np.int64).astype(np.uint8)
        actual = np.empty(digest_shape(size), np.uint8)
        hash_chunks(data, actual)
        for chunk, digest in enumerate(actual):
            assert digest.tobytes() == hashlib.sha256(data[chunk * 4096:(chunk + 1) * 4096]).digest()


def test_partial_or_excessive_buffers_are_rejected():
    for size in (0, -1, 2 ** 30 + 1, True, 4096.0):
        with pytest.raises(ValueError):
            digest_shape(size)
    assert digest_shape(2 ** 30) == (2 ** 18, 32)
    data = np.zeros(8192, np.uint8)
    for invalid in (data[::2], data.view(np.uint16), data.reshape(2, -1)):
        with pytest.raises(ValueError):
            hash_chunks(invalid, np.zeros((2, 32), np.uint8))
    with pytest.raises(ValueError):
        hash_chunks(data, np.zeros((1, 32), np.uint8))
    with pytest.raises(ValueError, match="overwrite"):
        hash_chunks(data, data[:64].reshape(2, 32))


def test_audit_readback_cannot_overwrite_its_own_expected_digest():
    checker = object.__new__(DeviceIntegrity)
    checker.shape = (2, 32)
    expected = np.zeros(checker.shape, np.uint8)
    with pytest.raises(ValueError, match="original digest"):
        checker.verify(0, expected, target=expected)
    with pytest.raises(ValueError, match="comparison"):
        checker.verify(0, expected, comparison=expected.view(np.bool_))
    with pytest.raises(ValueError, match="complete expert"):
        checker.verify(0, np.zeros((3, 32), np.uint8))


def test_closed_or_unowned_input_is_rejected_before_the_kernel():
    checker = object.__new__(DeviceIntegrity)
    checker.pointer, checker.size = None, 4096
    with pytest.raises(RuntimeError, match="closed"):
        checker.digests(123)
    checker.pointer = 456
    owned = {123: 32}
    checker.allocation_size = lambda p: owned.get(int(p), 0)
    with pytest.raises(ValueError, match="owned source"):
        checker.digests(123, size=33)
    with pytest.raises(ValueError, match="owned source"):
        checker.digests(999, size=1)
    with pytest.raises(ValueError, match="fixed buffer scope"):
        checker.digests(123, size=4097)
    with pytest.raises(ValueError, match="complete digest table"):
        checker.digests(123, size=32, target=np.zeros((2, 32), np.uint8))


def test_cache_config_accepts_only_the_supported_integrity_modes():
    from vesper_amd.tiered import CacheConfig
    assert CacheConfig().integrity_mode == "none"
    assert CacheConfig(integrity_mode="gpu-sha256").integrity_mode == "gpu-sha256"
    for bad in ("readback", "", "sha256", None):
        with pytest.raises(ValueError):
            CacheConfig(integrity_mode=bad)
