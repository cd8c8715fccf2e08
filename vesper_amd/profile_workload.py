"""Fixed workloads for hardware-counter runs (rocprofv3 --kernel-trace / --pmc).

  python -m vesper_amd.profile_workload --tokens 16 --iters 20
      builds the BASELINE decode layer (synthetic weights generated in HBM), runs one decode at
      T tokens, then re-launches every stage `iters` times back to back (router, route_plan,
      gateup, down, combine), so per-dispatch counters of each kernel can be read in isolation.
  python -m vesper_amd.profile_workload --copy-mib 1024 --iters 5
      copies a buffer of known size with the plain copy kernel: the calibration run for
      FETCH_SIZE / WRITE_SIZE (algorithmic bytes = size read + size written).
"""

from __future__ import annotations

import argparse
import sys

import numpy as np


def main() -> int:
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--tokens", type=int, default=16)
    p.add_argument("--iters", type=int, default=20)
    p.add_argument("--seed", type=int, default=20261018)
    p.add_argument("--copy-mib", type=int, default=0)
    args = p.parse_args()
    from . import _lib
    ctx = _lib.Context(0)
    if args.copy_mib:
        n = args.copy_mib << 20
        src, dst = ctx.malloc(n), ctx.malloc(n)
        ctx.fill_uniform_u8(src, n, 1, 0, 255)
        for _ in range(args.iters):
            ctx.lib.copy_kernel(ctx._h(), _lib.vp(dst), _lib.vp(src), n, None)
        ctx.sync()
        print(f"copy kernel: {args.iters} x {n} bytes", flush=True)
        ctx.free(src)
        ctx.free(dst)
        ctx.close()
        return 0
    from .config import BASELINE as cfg
    from .layer import ExpertBank, MoELayer, bf16_input
    rng = np.random.default_rng(args.seed)
    bank = ExpertBank(ctx, cfg, cfg.experts + 1)
    bank.fill_synthetic(args.seed)
    w = (rng.standard_normal((cfg.experts, cfg.hidden)) * 0.02).astype(np.float32)
    layer = MoELayer(ctx, cfg, w, bank)
    x = ctx.upload(bf16_input(rng.standard_normal((args.tokens, cfg.hidden)).astype(np.float32), cfg.hidden))
    y = ctx.empty((args.tokens, cfg.hidden), np.uint16)
    layer.decode_device(x.ptr, args.tokens, y.ptr)
    ctx.sync()
    plan = layer.plan()
    print(f"decode T={args.tokens}: {plan['n_routed']} distinct routed experts + shared", flush=True)
    for stage in MoELayer.STAGES:
        us = layer.time_stage(stage, args.iters)
        print(f"{stage:10s} {us:8.2f} us/launch over {args.iters} launches", flush=True)
    layer.close()
    bank.free()
    ctx.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
