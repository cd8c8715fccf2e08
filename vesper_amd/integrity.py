"""SHA-256 admission audit of expert bytes behind the reference's interface (src/vesper/integrity.py:1-112).

The audit's unit is a digest table: one SHA-256 per consecutive 4 KiB chunk of a payload, the last chunk
possibly short. Trusted tables come from verified host bytes (`hash_chunks`); device bytes are hashed by
the HIP kernel behind mx_sha256_chunks, one lane per chunk (`DeviceIntegrity.digests`), and
`DeviceIntegrity.verify` refuses a slot whose table differs from the trusted one. The device path has no
host fallback: without the library nothing is hashed. Names, messages and exception classes are the
reference's; argument checks run before any device call.
"""

from __future__ import annotations

import ctypes as C
import hashlib
from concurrent.futures import ThreadPoolExecutor

import numpy as np

from . import _lib
from .timing import Timings

CHUNK_BYTES = 4096
DIGEST_BYTES = 32
MAX_PAYLOAD = 1 << 30

# Host hashing threads: hashlib releases the GIL while it hashes a buffer of more than 2 KiB, so independent
# large digests (the whole expert and its tensors) run on separate cores.
# host hashing threads: the digests of one read run beside each other, and a batch promotion hashes several
# experts at once (the GPU box's host share is 16 cores)
HASHERS = ThreadPoolExecutor(max_workers=8, thread_name_prefix="vesper-sha256")


def digest_shape(size):
    """(chunk count, 32) for a payload of 0 < size <= 2^30 bytes."""
    if type(size) is not int or size <= 0 or size > MAX_PAYLOAD:
        raise ValueError("Invalid bounded integrity payload size")
    whole, tail = divmod(size, CHUNK_BYTES)
    return (whole + (1 if tail else 0), DIGEST_BYTES)


def _is_byte_vector(array) -> bool:
    return array.dtype == np.uint8 and array.ndim == 1 and array.flags.c_contiguous


def hash_chunks(data: np.ndarray, target: np.ndarray):
    """Write the digest table of host bytes `data` into `target` (chunks x 32 bytes)."""
    if not _is_byte_vector(data):
        raise ValueError("Integrity input must be a contiguous byte array")
    if target.dtype != np.uint8 or target.shape != digest_shape(data.size):
        raise ValueError("Integrity digest destination has the wrong size")
    if np.shares_memory(data, target):
        raise ValueError("Digest destination must not overwrite source bytes")
    _hash_range(memoryview(data), target, 0, target.shape[0])


def _hash_range(payload, target: np.ndarray, first: int, last: int):
    """Digests of chunks [first, last) of `payload` into rows [first, last) of `target`."""
    table = b"".join(hashlib.sha256(payload[i * CHUNK_BYTES:(i + 1) * CHUNK_BYTES]).digest()
                     for i in range(first, last))
    target[first:last] = np.frombuffer(table, np.uint8).reshape(last - first, DIGEST_BYTES)


def hash_chunks_native(data: np.ndarray, target: np.ndarray, threads: int = 4):
    """hash_chunks computed by the library on `threads` host threads (mx_host_sha256_chunks: OpenSSL's
    SHA-256 per chunk, no per-chunk interpreter work, the interpreter lock released for the whole call)."""
    import ctypes as C
    from . import _lib
    if not _is_byte_vector(data):
        raise ValueError("Integrity input must be a contiguous byte array")
    if target.dtype != np.uint8 or target.shape != digest_shape(data.size) or not target.flags.c_contiguous:
        raise ValueError("Integrity digest destination has the wrong size")
    if np.shares_memory(data, target):
        raise ValueError("Digest destination must not overwrite source bytes")
    _lib.load().host_sha256_chunks(C.c_void_p(data.ctypes.data), data.size, C.c_void_p(target.ctypes.data),
                                   int(threads))


def _overlapping(*arrays) -> bool:
    present = [a for a in arrays if a is not None]
    return any(np.shares_memory(a, b) for i, a in enumerate(present) for b in present[i + 1:])


class DeviceIntegrity:
    """A device digest table of fixed capacity for payloads of up to `size` bytes; the caller owns the
    context. `allocation_size(pointer)` gives the bytes owned at an allocation base (default: the
    context's allocations; the tiered runtime adds its cache slots), so reads past an owned region are
    refused before the kernel runs."""

    def __init__(self, ctx: "_lib.Context", size, timings=None, allocation_size=None):
        self.shape = digest_shape(size)
        self.ctx, self.size = ctx, size
        self.allocation_size = allocation_size if allocation_size is not None else ctx.owned_size
        self.timings = timings if timings is not None else Timings()
        self.table = ctx.empty(self.shape, np.uint8)
        self.pointer = self.table.ptr

    def _check_read(self, pointer, size, target):
        if self.pointer is None:
            raise RuntimeError("Integrity checker is closed")
        shape = digest_shape(size)
        if size > self.size:
            raise ValueError("Integrity payload exceeds the fixed buffer scope")
        if self.allocation_size(pointer) < size:
            raise ValueError("Integrity read exceeds an owned source allocation")
        if target is not None:
            writable = target.flags.c_contiguous and target.flags.writeable
            if target.dtype != np.uint8 or target.shape != shape or not writable:
                raise ValueError("Integrity readback must fit the complete digest table")
        return shape

    def digests(self, pointer, *, size=None, target=None, stream=None):
        """Digest table of `size` (default: the capacity) device bytes at `pointer`, read back to the host."""
        size = self.size if size is None else size
        shape = self._check_read(pointer, size, target)
        lib, handle = self.ctx.lib, self.ctx._h()
        with self.timings.section("integrity.gpu_sha256"):
            lib.sha256_chunks(handle, C.c_void_p(int(pointer)), int(size), C.c_void_p(self.pointer),
                              _lib._stream(stream))
        table = target if target is not None else np.empty(shape, np.uint8)
        with self.timings.section("integrity.gpu_digest_d2h"):
            lib.memcpy_d2h(handle, table.ctypes.data_as(C.c_void_p), C.c_void_p(self.pointer), table.nbytes,
                           _lib._stream(stream))
            self.ctx.sync(stream)
        return table

    def verify(self, pointer, expected, target=None, comparison=None):
        """Refuse (ValueError) device bytes whose digest table differs from `expected`; returns the number
        of digest bytes read back."""
        if expected.dtype != np.uint8 or expected.shape != self.shape:
            raise ValueError("Original digest table does not identify one complete expert")
        if _overlapping(expected, target):
            raise ValueError("Audit readback must not overwrite the original digest table")
        if comparison is not None and _overlapping(comparison, expected) | _overlapping(comparison, target):
            raise ValueError("Audit comparison must not overwrite source or readback digests")
        if comparison is not None and (comparison.dtype != np.bool_ or comparison.shape != self.shape):
            raise ValueError("Integrity comparison scratch has the wrong layout")
        actual = self.digests(pointer, target=target)
        if comparison is None:
            equal = bool((actual == expected).all())
        else:
            np.equal(actual, expected, out=comparison)
            equal = bool(comparison.all())
        if not equal:
            raise ValueError("GPU expert bytes differ from verified original SHA-256 chunks")
        return actual.nbytes

    def close(self):
        table, self.pointer = self.table, None
        if table is not None and table.ptr:
            table.free()

    def __enter__(self):
        return self

    def __exit__(self, *_):
        self.close()
