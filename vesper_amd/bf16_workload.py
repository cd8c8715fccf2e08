"""Timing workload for the configuration-0 expert (BF16 activations; mx_expert_forward_bf16), used by bench.py.

  python -m vesper_amd.bf16_workload --tokens 1 4 16 --iters 50

BASELINE configuration 0's expert: 7168 x 2048 MXFP4 (uniform packed bytes, E8M0 codes in [118, 126];
synthetic, generated in HBM and tiled), held in as many copies as take at least ROTATE_BYTES, consecutive
calls using consecutive copies so that no call finds its weights in the GPU's caches from the call before.
Each call (gate/up with SwiGLU, down: two launches) is timed with HIP events over `iters` back-to-back calls.
Algorithmic bytes per call: the expert's weight and scale bytes, x and y (BF16); FLOP 2 x 3 x T x H x I.
"""

from __future__ import annotations

import argparse
import ctypes as C
import json
import sys

import numpy as np

ROTATE_BYTES = 512 << 20


def run(tokens=(1, 4, 16), iters=50, seed=20261018, ctx=None, hidden=7168, intermediate=2048):
    from . import _lib
    from .config import MoEConfig
    from .layer import ExpertBank
    own = ctx is None
    ctx = ctx or _lib.Context(0)
    lib = ctx.lib
    h, i = hidden, intermediate
    cfg = MoEConfig(hidden=h, intermediate=i)
    per_expert = int(lib.cdll.mx_tiled_expert_bytes(h, i))
    count = max(2, -(-ROTATE_BYTES // per_expert))
    bank = ExpertBank(ctx, cfg, count)
    try:
        bank.fill_synthetic(seed)
        rng = np.random.default_rng(seed)
        tmax = max(tokens)
        x = rng.standard_normal((tmax, h)).astype(np.float32)
        b = x.view(np.uint32).astype(np.uint64)
        xd = ctx.upload(((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16))
        gu = ctx.empty((tmax, 2 * i), np.float32)
        hd = ctx.empty((tmax, i), np.float32)
        yd = ctx.empty((tmax, h), np.uint16)
        ctx.sync()
        start, stop = ctx.event(), ctx.event()
        out = {}
        for t in tokens:
            def call(n):
                lib.expert_forward_bf16(ctx._h(), C.c_void_p(bank.tiled_ptr(n % count)), h, i, _lib.vp(xd), t,
                                        None, _lib.vp(hd), _lib.vp(gu), _lib.vp(yd), None)
            for n in range(3):
                call(n)
            ctx.sync()
            ctx.record(start)
            for n in range(iters):
                call(3 + n)
            ctx.record(stop)
            us = ctx.elapsed_ms(start, stop) * 1e3 / iters
            nbytes = per_expert + 2 * 2 * t * h
            out[str(t)] = {"us": round(us, 2), "bytes": nbytes, "GB_per_s": round(nbytes / (us * 1e-6) / 1e9, 1),
                           "TFLOP_per_s": round(2 * 3 * t * h * i / (us * 1e-6) / 1e12, 3)}
        xd.free(), gu.free(), hd.free(), yd.free()
        return {"expert": f"{h} x {i} MXFP4, BF16 activations", "copies_rotated": count, "per_tokens": out}
    finally:
        bank.free()
        if own:
            ctx.close()


def main(argv=None) -> int:
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--tokens", type=int, nargs="+", default=[1, 4, 16])
    p.add_argument("--iters", type=int, default=50)
    args = p.parse_args(argv)
    print(json.dumps(run(tuple(args.tokens), args.iters)), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
