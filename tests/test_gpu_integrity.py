"""GPU parity of the SHA-256 admission audit (mx_sha256_chunks behind DeviceIntegrity): every digest byte
against the oracle for the reference's validation lengths and patterns (integrity_validation.py:27-75),
the FIPS "abc" answer, refusal of single-byte corruptions at the reference's offsets, and the 1 GiB
maximum payload with a short last chunk."""

import ctypes as C

import numpy as np
import pytest

from oracle.integrity import digest_table
from vesper_amd import _lib
from vesper_amd.integrity import DeviceIntegrity

pytestmark = pytest.mark.gpu

EXPERT_BYTES = 23_396_352
LENGTHS = (1, 3, 55, 56, 63, 64, 65, 119, 120, 127, 128, 4095, 4096, 4097, 8192, EXPERT_BYTES)


def test_lengths_and_patterns_match_the_oracle(gpu_ctx):
    original = np.random.default_rng(20261018).integers(0, 256, EXPERT_BYTES, dtype=np.uint8)
    src = gpu_ctx.upload(original)
    try:
        with DeviceIntegrity(gpu_ctx, EXPERT_BYTES) as checker:
            for pattern in ("random", "zeros", "ones"):
                work = original if pattern == "random" else np.full(EXPERT_BYTES, 0 if pattern == "zeros" else 255,
                                                                    np.uint8)
                src.upload(work)
                for size in LENGTHS:
                    got = checker.digests(src.ptr, size=size)
                    np.testing.assert_array_equal(got, digest_table(work[:size]), err_msg=f"{pattern} {size}")
            # a known message checks byte order and padding
            gpu_ctx.copy_h2d(src.ptr, np.frombuffer(b"abc", np.uint8))
            abc = checker.digests(src.ptr, size=3)
            assert abc.tobytes().hex() == "ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad"
    finally:
        src.free()


def test_verify_refuses_every_single_byte_corruption(gpu_ctx):
    original = np.random.default_rng(7).integers(0, 256, EXPERT_BYTES, dtype=np.uint8)
    expected = digest_table(original)
    src = gpu_ctx.upload(original)
    try:
        with DeviceIntegrity(gpu_ctx, EXPERT_BYTES) as checker:
            readback = np.empty_like(expected)
            comparison = np.empty(expected.shape, np.bool_)
            assert checker.verify(src.ptr, expected, readback, comparison) == expected.nbytes
            for offset in (0, 63, 4095, 4096, EXPERT_BYTES - 1):
                gpu_ctx.copy_h2d(src.ptr + offset, np.array([original[offset] ^ 1], np.uint8))
                with pytest.raises(ValueError, match="differ"):
                    checker.verify(src.ptr, expected, readback, comparison)
                assert np.flatnonzero(~comparison.all(axis=1)).tolist() == [offset // 4096], offset
                gpu_ctx.copy_h2d(src.ptr + offset, np.array([original[offset]], np.uint8))
                checker.verify(src.ptr, expected, readback, comparison)
            # unowned sources and interior pointers are refused before the kernel
            with pytest.raises(ValueError, match="owned source"):
                checker.digests(src.ptr + 4096, size=4096)
    finally:
        src.free()


def test_largest_payload_with_a_short_last_chunk(gpu_ctx):
    size = 2 ** 30
    ptr = gpu_ctx.malloc(size)
    try:
        gpu_ctx.fill_uniform_u8(ptr, size, 99, 0, 255)
        gpu_ctx.sync()
        data = gpu_ctx.download(ptr, (size,), np.uint8)
        with DeviceIntegrity(gpu_ctx, size) as checker:
            np.testing.assert_array_equal(checker.digests(ptr), digest_table(data))
            short = size - 4097              # last chunk 4095 bytes
            np.testing.assert_array_equal(checker.digests(ptr, size=short), digest_table(data[:short]))
    finally:
        gpu_ctx.free(ptr)


def test_entry_point_refusals(gpu_ctx):
    src = gpu_ctx.upload(np.zeros(8192, np.uint8))
    out = gpu_ctx.empty((2, 32), np.uint8)
    lib = gpu_ctx.lib
    try:
        for bad in ((src.ptr + 1, 4096, out.ptr), (src.ptr, 0, out.ptr), (src.ptr, 2 ** 30 + 1, out.ptr),
                    (src.ptr, 8192, src.ptr + 4096)):
            with pytest.raises(ValueError):
                lib.sha256_chunks(gpu_ctx._h(), C.c_void_p(bad[0]), bad[1], C.c_void_p(bad[2]), None)
        lib.sha256_chunks(gpu_ctx._h(), _lib.vp(src), 8192, _lib.vp(out), None)
        gpu_ctx.sync()
        np.testing.assert_array_equal(out.download(), digest_table(bytes(8192)))
    finally:
        src.free()
        out.free()


def test_batched_verify_counts_differing_chunks_per_slot(gpu_ctx):
    """mx_sha256_verify over 70 slots (two launches of up to 64): with counters NULL slot i adds its count of
    differing chunks to mismatches[i]; explicit counters map slots onto shared counters, which accumulate
    across calls (the call does not clear them)."""
    n, size = 70, 3 * 4096 + 100                               # three whole chunks and a short one
    rng = np.random.default_rng(70)
    data = rng.integers(0, 256, (n, size), dtype=np.uint8)
    tables = np.stack([digest_table(row) for row in data])       # [n, 4, 32]
    stride = (size + 255) // 256 * 256
    slots = gpu_ctx.empty((n, stride), np.uint8)
    exp = gpu_ctx.upload(tables)
    counts = gpu_ctx.upload(np.zeros(n, np.uint32))
    try:
        host = np.zeros((n, stride), np.uint8)
        host[:, :size] = data
        host[3, 5000] ^= 0x80                                   # slot 3, chunk 1
        host[67, 1] ^= 0x01                                     # slot 67 (second launch), chunk 0
        host[67, size - 1] ^= 0x01                              # and its short last chunk
        slots.upload(host)
        ptrs = (C.c_void_p * n)(*[slots.ptr + i * stride for i in range(n)])
        tabs = (C.c_void_p * n)(*[exp.ptr + i * tables[0].nbytes for i in range(n)])
        lib = gpu_ctx.lib
        lib.sha256_verify(gpu_ctx._h(), ptrs, tabs, None, n, size, _lib.vp(counts), None)
        gpu_ctx.sync()
        want = np.zeros(n, np.uint32)
        want[3], want[67] = 1, 2
        np.testing.assert_array_equal(counts.download(), want)
        to_zero = (C.c_int32 * n)(*([0] * n))
        lib.sha256_verify(gpu_ctx._h(), ptrs, tabs, to_zero, n, size, _lib.vp(counts), None)
        gpu_ctx.sync()
        want[0] += 3
        np.testing.assert_array_equal(counts.download(), want)
        with pytest.raises(ValueError):
            lib.sha256_verify(gpu_ctx._h(), ptrs, tabs, None, n, 0, _lib.vp(counts), None)
        bad = (C.c_int32 * n)(*([-1] + [0] * (n - 1)))
        with pytest.raises(ValueError):
            lib.sha256_verify(gpu_ctx._h(), ptrs, tabs, bad, n, size, _lib.vp(counts), None)
    finally:
        for d in (slots, exp, counts):
            d.free()
