"""Direct (O_DIRECT) reads of the expert store (the reference's DirectReader, src/vesper/disk.py:23-131).

One page-aligned buffer of `capacity` bytes, reserved in the caller's MemoryBudget, receives aligned reads
that bypass the page cache; callers copy from it. (Memory from hipHostMalloc cannot be the target of an
O_DIRECT read on ROCm -- the kernel refuses its mapping with EFAULT -- so pinned staging is filled by a
copy from this buffer.) There is no buffered fallback: a filesystem that refuses O_DIRECT makes the open fail.
"""

from __future__ import annotations

import mmap
import os
from pathlib import Path

import numpy as np

PAGE = 4096


def _aligned_request(offset: int, size: int, capacity: int) -> None:
    if offset < 0 or offset % PAGE or size <= 0 or size % PAGE or size > capacity:
        raise ValueError("Direct read is not aligned or exceeds the buffer")


class DirectReader:
    def __init__(self, path: Path, capacity: int, budget):
        if not hasattr(os, "O_DIRECT") or not hasattr(os, "preadv"):
            raise RuntimeError("Direct I/O is unavailable; buffered fallback is intentionally disabled")
        self.capacity, self.budget = int(capacity), budget
        self.handle, self.buffer = None, None
        budget.acquire(self.capacity, category="scratch")
        try:
            self.handle = os.open(path, os.O_RDONLY | os.O_DIRECT)
            self.buffer = mmap.mmap(-1, self.capacity)        # anonymous mappings are page-aligned
        except BaseException:
            self.close()
            raise

    def _open(self):
        if self.handle is None or self.buffer is None:
            raise RuntimeError("Direct reader is closed")

    def _read_exact(self, views, offset: int, size: int) -> None:
        done = os.preadv(self.handle, views, offset)
        if done != size:
            raise OSError("Short direct read")

    def read(self, offset: int, size: int) -> bytes:
        """Read `size` bytes at `offset` into the buffer; returns the first page (for spot checks)."""
        self._open()
        _aligned_request(offset, size, self.capacity)
        view = memoryview(self.buffer)[:size]
        try:
            self._read_exact([view], offset, size)
            return bytes(view[:PAGE])
        finally:
            view.release()

    def switch_file(self, path: Path) -> None:
        """Point the reader at another file, keeping the buffer; the old handle stays valid if the open fails."""
        self._open()
        replacement = os.open(path, os.O_RDONLY | os.O_DIRECT)
        old, self.handle = self.handle, replacement
        os.close(old)

    def array(self) -> np.ndarray:
        """The aligned buffer as bytes (borrowed: not valid after close)."""
        self._open()
        return np.frombuffer(self.buffer, dtype=np.uint8, count=self.capacity)

    def close(self) -> None:
        buffer, handle, budget = self.buffer, self.handle, self.budget
        self.buffer, self.handle, self.budget = None, None, None
        if buffer is not None:
            buffer.close()
        if handle is not None:
            os.close(handle)
        if budget is not None:
            budget.release(self.capacity, category="scratch")

    def __enter__(self):
        return self

    def __exit__(self, *_):
        self.close()
