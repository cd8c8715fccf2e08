"""Timing workload for the FP8 projections, used by bench.py and for counter runs.

  python -m vesper_amd.fp8_workload --tokens 1 16 2048 --iters 20

Builds the four configuration-3 projections (q_a 7168->1536, q_b 1536->24576, kv_a 7168->576,
o 16384->7168; E4M3 weights with FP32 128 x 128 block scales, log-uniform in [2^-8, 2^-2]; synthetic,
generated in HBM) and times each projection call (quantizer + product) with HIP events over `iters`
back-to-back calls. q_a and kv_a, which read the same input, run as one call over their stacked 2112 rows
(FUSED_LAYOUT; `layout=LAYOUT` times them separately). Algorithmic work per call: weight bytes N*K +
scales, x and y; FLOP 2*T*N*K.

Each projection is held in as many copies as take at least ROTATE_BYTES together, and consecutive
calls use consecutive copies, as consecutive layers of a model would: a call never finds its weights
in the GPU's caches (4 MB L2 per XCD, 256 MB Infinity Cache) from the call before.
"""

from __future__ import annotations

import argparse
import ctypes as C
import json
import sys

import numpy as np

LAYOUT = {"q_a": (1536, 7168), "q_b": (24576, 1536), "kv_a": (576, 7168), "o": (7168, 16384)}
# q_a and kv_a read the same input: as one projection of their stacked rows (q_a's rows, then kv_a's), one
# quantization of x and one launch serve both; every output is the same dot product as in the separate calls.
FUSED_LAYOUT = {"q_kv_a": (1536 + 576, 7168), "q_b": (24576, 1536), "o": (7168, 16384)}
ROTATE_BYTES = 512 << 20


def run(tokens=(1, 16, 2048), iters=20, seed=20261018, ctx=None, layout=None):
    from . import _lib
    own = ctx is None
    ctx = ctx or _lib.Context(0)
    lib = ctx.lib
    rng = np.random.default_rng(seed)
    layout = layout or FUSED_LAYOUT
    blobs = {}
    for i, (name, (n, k)) in enumerate(layout.items()):
        size = int(lib.cdll.mx_fp8_tiled_bytes(n, k, 128))
        w = ctx.malloc(n * k)
        ctx.fill_uniform_u8(w, n * k, seed * 31 + i, 0, 126)      # finite E4M3 codes (no 0x7F / 0xFF)
        sw = np.exp2(rng.uniform(-8.0, -2.0, ((n + 127) // 128, k // 128))).astype(np.float32)
        swd = ctx.upload(sw)
        blob = ctx.malloc(size)
        lib.fp8_tile(ctx._h(), C.c_void_p(w), _lib.vp(swd), n, k, 128, C.c_void_p(blob), None)
        copies = [blob]
        for _ in range(max(2, -(-ROTATE_BYTES // size)) - 1):
            c = ctx.malloc(size)
            ctx.copy_d2d(c, blob, size)
            copies.append(c)
        ctx.sync()
        ctx.free(w)
        swd.free()
        blobs[name] = copies
    tmax = max(tokens)
    kmax = max(k for _, k in layout.values())
    nmax = max(n for n, _ in layout.values())
    x = rng.standard_normal((tmax, kmax)).astype(np.float32)
    b = x.view(np.uint32).astype(np.uint64)
    xd = ctx.upload(((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16))
    yd = ctx.empty((tmax, nmax), np.uint16)
    start, stop = ctx.event(), ctx.event()
    out = {}
    for t in tokens:
        per = {}
        total_us, total_bytes, total_flop = 0.0, 0, 0
        for name, (n, k) in layout.items():
            # the input is the first T rows of a [T, k] view of the buffer; call i uses copy i
            copies = blobs[name]
            calls = [(ctx._h(), C.c_void_p(c), n, k, 128, _lib.vp(xd), t, _lib.vp(yd), None, None, None, None)
                     for c in copies]
            for i in range(3):
                lib.fp8_projection(*calls[i % len(calls)])
            ctx.sync()
            ctx.record(start)
            for i in range(iters):
                lib.fp8_projection(*calls[(3 + i) % len(calls)])
            ctx.record(stop)
            us = ctx.elapsed_ms(start, stop) * 1000 / iters
            nbytes = n * k + ((n + 127) // 128) * (k // 128) * 4 + t * k * 2 + t * n * 2
            flop = 2 * t * n * k
            per[name] = {"us": round(us, 2), "GB_per_s": round(nbytes / us / 1e3, 1),
                         "TFLOP_per_s": round(flop / us / 1e6, 2)}
            total_us += us
            total_bytes += nbytes
            total_flop += flop
        out[t] = {"projections": per, "us": round(total_us, 2), "bytes": total_bytes, "flop": total_flop,
                  "GB_per_s": round(total_bytes / total_us / 1e3, 1),
                  "TFLOP_per_s": round(total_flop / total_us / 1e6, 2)}
    for copies in blobs.values():
        for c in copies:
            ctx.free(c)
    xd.free()
    yd.free()
    if own:
        ctx.close()
    return out


def run_grouped(tokens=(1, 8), iters=20, seed=20261018, ctx=None):
    """The grouped output projection wo_a (8 groups x 1024 rows over 4096, block-32 E4M3, the reference's
    own shapes) per call: mx_kv_round32 of the [T, 8, 4096] input, then mx_fp8_grouped_projection, with
    weights rotated over at least ROTATE_BYTES of copies. Bytes: E4M3 weights + E8M0 scales, the BF16 input
    read once, rounded / codes / scales written, and the BF16 output."""
    from . import _lib
    own = ctx is None
    ctx = ctx or _lib.Context(0)
    lib = ctx.lib
    rows, width, groups = 8192, 4096, 8
    rng = np.random.default_rng(seed)
    size = int(lib.cdll.mx_fp8_tiled_bytes(rows, width, 32))
    w = ctx.malloc(rows * width)
    ctx.fill_uniform_u8(w, rows * width, seed * 7, 0, 126)
    swd = ctx.upload(rng.integers(118, 127, (rows // 32, width // 32), dtype=np.uint8))
    copies = [ctx.malloc(size) for _ in range(max(2, -(-ROTATE_BYTES // size)))]
    lib.fp8_tile(ctx._h(), C.c_void_p(w), _lib.vp(swd), rows, width, 32, C.c_void_p(copies[0]), None)
    for c in copies[1:]:
        ctx.copy_d2d(c, copies[0], size)
    ctx.sync()
    ctx.free(w)
    swd.free()
    tmax = max(tokens)
    x = rng.standard_normal((tmax, groups, width)).astype(np.float32)
    b = x.view(np.uint32).astype(np.uint64)
    xd = ctx.upload(((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16))
    rd = ctx.empty((tmax, groups, width), np.uint16)
    qd = ctx.empty((tmax, groups, width), np.uint8)
    sd = ctx.empty((tmax, groups, width // 32), np.uint8)
    yd = ctx.empty((tmax, rows), np.uint16)
    start, stop = ctx.event(), ctx.event()
    out = {}
    try:
        for t in tokens:
            def call(i):
                lib.kv_round32(ctx._h(), _lib.vp(xd), t * groups * width, _lib.vp(rd), _lib.vp(qd), _lib.vp(sd), None)
                lib.fp8_grouped_projection(ctx._h(), C.c_void_p(copies[i % len(copies)]), groups, rows // groups,
                                           width, _lib.vp(qd), _lib.vp(sd), t, _lib.vp(yd), None, None)
            for i in range(3):
                call(i)
            ctx.sync()
            ctx.record(start)
            for i in range(iters):
                call(3 + i)
            ctx.record(stop)
            us = ctx.elapsed_ms(start, stop) * 1000 / iters
            nbytes = rows * width + (rows // 32) * (width // 32) + t * groups * width * (2 + 2 + 1) + t * groups * 128 \
                + t * rows * 2
            out[t] = {"us": round(us, 2), "GB_per_s": round(nbytes / us / 1e3, 1),
                      "TFLOP_per_s": round(2 * t * rows * width / us / 1e6, 3), "bytes": nbytes,
                      "bf16_weight_bytes_avoided": rows * width}
    finally:
        for c in copies:
            ctx.free(c)
        for d in (xd, rd, qd, sd, yd):
            d.free()
        if own:
            ctx.close()
    return out


def main():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--tokens", type=int, nargs="+", default=[1, 16, 2048])
    p.add_argument("--iters", type=int, default=20)
    args = p.parse_args()
    print(json.dumps(run(tuple(args.tokens), args.iters)), flush=True)
    print(json.dumps({"wo_a_grouped": run_grouped(iters=args.iters)}), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
