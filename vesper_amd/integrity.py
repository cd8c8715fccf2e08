"""SHA-256 admission audit of expert bytes (mirrors src/vesper/integrity.py:1-112).

One digest per consecutive 4 KiB chunk. Source digests come from verified bytes on the host
(`hash_chunks`, the reference's host function); the device bytes are hashed by the HIP kernel behind
mx_sha256_chunks (`DeviceIntegrity.digests`), and `verify` refuses a slot whose digest table differs.
The device path has no host fallback: without the library nothing is hashed.
"""

from __future__ import annotations

import ctypes as C
import hashlib

import numpy as np

from . import _lib
from .timing import Timings

CHUNK_BYTES = 4096
DIGEST_BYTES = 32


def digest_shape(size):
    """(chunks, 32) for a payload of `size` bytes, 0 < size <= 2^30 (integrity.py:15-18)."""
    if type(size) is not int or not 0 < size <= 2 ** 30:
        raise ValueError("Invalid bounded integrity payload size")
    return ((size + CHUNK_BYTES - 1) // CHUNK_BYTES, DIGEST_BYTES)


def hash_chunks(data: np.ndarray, target: np.ndarray):
    """Host digests of verified source bytes into target (integrity.py:21-31)."""
    if data.dtype != np.uint8 or data.ndim != 1 or not data.flags.c_contiguous:
        raise ValueError("Integrity input must be a contiguous byte array")
    if target.dtype != np.uint8 or target.shape != digest_shape(data.size):
        raise ValueError("Integrity digest destination has the wrong size")
    if np.shares_memory(data, target):
        raise ValueError("Digest destination must not overwrite source bytes")
    view = memoryview(data)
    for i in range(target.shape[0]):
        target[i] = np.frombuffer(hashlib.sha256(view[i * CHUNK_BYTES:(i + 1) * CHUNK_BYTES]).digest(), np.uint8)


class DeviceIntegrity:
    """Owns one bounded device digest table (integrity.py:34-112); the caller owns the context."""

    def __init__(self, ctx: "_lib.Context", size, timings=None, allocation_size=None):
        """allocation_size(pointer) -> bytes owned at that base (default: the context's allocations; the
        tiered runtime adds its cache slots)."""
        self.shape = digest_shape(size)
        self.ctx, self.size = ctx, size
        self.allocation_size = allocation_size or ctx.owned_size
        self.timings = timings or Timings()
        self.table = ctx.empty(self.shape, np.uint8)
        self.pointer = self.table.ptr

    def digests(self, pointer, *, size=None, target=None, stream=None):
        """Digest table of the `size` device bytes at `pointer` (an allocation base this context owns)."""
        if self.pointer is None:
            raise RuntimeError("Integrity checker is closed")
        size = self.size if size is None else size
        shape = digest_shape(size)
        if size > self.size:
            raise ValueError("Integrity payload exceeds the fixed buffer scope")
        if self.allocation_size(pointer) < size:
            raise ValueError("Integrity read exceeds an owned source allocation")
        if target is not None and (target.dtype != np.uint8 or target.shape != shape
                                   or not target.flags.c_contiguous or not target.flags.writeable):
            raise ValueError("Integrity readback must fit the complete digest table")
        with self.timings.section("integrity.gpu_sha256"):
            self.ctx.lib.sha256_chunks(self.ctx._h(), C.c_void_p(int(pointer)), int(size), C.c_void_p(self.pointer),
                                       _lib._stream(stream))
        with self.timings.section("integrity.gpu_digest_d2h"):
            out = np.empty(shape, np.uint8) if target is None else target
            self.ctx.lib.memcpy_d2h(self.ctx._h(), out.ctypes.data_as(C.c_void_p), C.c_void_p(self.pointer),
                                    out.nbytes, _lib._stream(stream))
            self.ctx.sync(stream)
            return out

    def verify(self, pointer, expected, target=None, comparison=None):
        """Refuse (ValueError) device bytes whose digests differ from the verified table; returns the
        digest bytes compared."""
        if expected.dtype != np.uint8 or expected.shape != self.shape:
            raise ValueError("Original digest table does not identify one complete expert")
        if target is not None and np.shares_memory(expected, target):
            raise ValueError("Audit readback must not overwrite the original digest table")
        if comparison is not None and (np.shares_memory(expected, comparison)
                                        or (target is not None and np.shares_memory(target, comparison))):
            raise ValueError("Audit comparison must not overwrite source or readback digests")
        actual = self.digests(pointer, target=target)
        if comparison is None:
            match = np.array_equal(actual, expected)
        else:
            if comparison.dtype != np.bool_ or comparison.shape != self.shape:
                raise ValueError("Integrity comparison scratch has the wrong layout")
            np.equal(actual, expected, out=comparison)
            match = bool(comparison.all())
        if not match:
            raise ValueError("GPU expert bytes differ from verified original SHA-256 chunks")
        return actual.nbytes

    def close(self):
        if self.pointer is not None:
            self.table.free()
            self.pointer = None

    def __enter__(self):
        return self

    def __exit__(self, *_):
        self.close()
