"""Timing workload for the SHA-256 admission audit (mx_sha256_chunks), used by bench.py and for counter runs.

  python -m vesper_amd.integrity_workload --iters 20

Times the digest kernel with HIP events on (a) one expert slot at the BASELINE shapes (23,396,352 bytes,
5,712 chunks), rotating over 12 device-generated slots (280 MB, more than the 256 MB Infinity Cache) as
consecutive cache admissions would, and (b) the largest payload the audit accepts (1 GiB, 262,144 chunks).
Beside them, the host path the reference uses for source digests (hash_chunks: hashlib, one core) on
the same expert bytes. Work per payload: every byte hashed once, 65 SHA-256 compressions per full chunk.
"""

from __future__ import annotations

import argparse
import ctypes as C
import json
import sys
import time

import numpy as np

EXPERT_BYTES = 23_396_352
SLOTS = 12
GIB = 1 << 30


def run(iters=20, ctx=None):
    from . import _lib
    from .integrity import digest_shape, hash_chunks
    own = ctx is None
    ctx = ctx or _lib.Context(0)
    lib = ctx.lib
    slots = [ctx.malloc(EXPERT_BYTES) for _ in range(SLOTS)]
    big = ctx.malloc(GIB)
    table = ctx.empty(digest_shape(GIB), np.uint8)
    start, stop = ctx.event(), ctx.event()
    out = {}
    try:
        for i, p in enumerate(slots):
            ctx.fill_uniform_u8(p, EXPERT_BYTES, 1000 + i, 0, 255)
        ctx.fill_uniform_u8(big, GIB, 77, 0, 255)
        ctx.sync()

        def launch(ptr, size):
            lib.sha256_chunks(ctx._h(), C.c_void_p(ptr), size, _lib.vp(table), None)

        for i in range(3):
            launch(slots[i % SLOTS], EXPERT_BYTES)
        ctx.sync()
        ctx.record(start)
        for i in range(iters):
            launch(slots[(3 + i) % SLOTS], EXPERT_BYTES)
        ctx.record(stop)
        us = ctx.elapsed_ms(start, stop) * 1000 / iters
        out["expert"] = {"bytes": EXPERT_BYTES, "chunks": digest_shape(EXPERT_BYTES)[0], "us": round(us, 2),
                         "GB_per_s": round(EXPERT_BYTES / us / 1e3, 1)}
        launch(big, GIB)
        ctx.sync()
        reps = max(2, iters // 4)
        ctx.record(start)
        for _ in range(reps):
            launch(big, GIB)
        ctx.record(stop)
        us = ctx.elapsed_ms(start, stop) * 1000 / reps
        out["max_payload"] = {"bytes": GIB, "chunks": digest_shape(GIB)[0], "us": round(us, 1),
                              "GB_per_s": round(GIB / us / 1e3, 1)}
        host = ctx.download(slots[0], (EXPERT_BYTES,), np.uint8)
        target = np.empty(digest_shape(EXPERT_BYTES), np.uint8)
        times = []
        for _ in range(3):
            t0 = time.perf_counter()
            hash_chunks(host, target)
            times.append(time.perf_counter() - t0)
        sec = sorted(times)[1]
        out["host_hash_chunks"] = {"bytes": EXPERT_BYTES, "us": round(sec * 1e6, 1),
                                   "GB_per_s": round(EXPERT_BYTES / sec / 1e9, 3), "cores": 1}
    finally:
        for p in slots:
            ctx.free(p)
        ctx.free(big)
        table.free()
        if own:
            ctx.close()
    return out


def main():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--iters", type=int, default=20)
    args = p.parse_args()
    print(json.dumps(run(args.iters)), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
