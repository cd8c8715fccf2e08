"""Per-chunk SHA-256 digest tables (CPU oracle, test infrastructure only).

Restates ``src/vesper/integrity.py`` of the reference:
  digest_table   integrity.py:21-31   SHA-256 of every consecutive 4 KiB chunk (the last one may be short),
                                      32 digest bytes per chunk in chunk order

SHA-256 is hashlib's (FIPS 180-4), the routine the reference's own host path calls. Tests pin it with the
FIPS 180-4 example messages and the reference's "abc" vector (tests/test_integrity.py:13-17), and pin the
chunking against whole-message digests of single-chunk payloads.
"""

from __future__ import annotations

import hashlib

import numpy as np

CHUNK_BYTES = 4096


def digest_table(data) -> np.ndarray:
    """[ceil(len / 4096), 32] uint8: row c = SHA-256 of bytes [4096 c, 4096 (c + 1))."""
    view = memoryview(np.ascontiguousarray(np.frombuffer(bytes(data), np.uint8) if isinstance(data, (bytes, bytearray))
                                           else np.asarray(data, np.uint8).reshape(-1)))
    n = (len(view) + CHUNK_BYTES - 1) // CHUNK_BYTES
    out = np.empty((n, 32), np.uint8)
    for c in range(n):
        out[c] = np.frombuffer(hashlib.sha256(view[c * CHUNK_BYTES:(c + 1) * CHUNK_BYTES]).digest(), np.uint8)
    return out
