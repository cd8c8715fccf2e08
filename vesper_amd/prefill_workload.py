"""Timing workload for the MoE prefill, used by bench.py and for counter runs.

  python -m vesper_amd.prefill_workload --tokens 4096 --iters 5

The BASELINE layer (256 MXFP4 experts of 7168 x 2048 + shared, synthetic weights generated in HBM),
T tokens of x ~ N(0, 1) BF16 and Zipf(1.1) routing over a random permutation of the experts, timed with
HIP events over `iters` back-to-back mx_moe_prefill calls (plan + grouped gate/up + grouped down +
combine). Work per call: 2 * (T * k + T) * 3 * I * H FLOP (every routed pair and the shared expert),
and every expert with a routed token streamed at least once.
"""

from __future__ import annotations

import argparse
import json
import sys

import numpy as np


HBM_PEAK = 8.0e12        # B/s
FP8_MFMA_PEAK = 5.0e15   # FLOP/s, dense


def seeded_inputs(tokens, seed, cfg):
    """(router weight [E, H], x [T, H] FP32, ids [T, k], weights [T, k]) of the workload's seeded stream (the
    experts themselves are generated in HBM from the same seed)."""
    from .workloads import zipf_routing
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((cfg.experts, cfg.hidden)) * 0.02).astype(np.float32)
    x = rng.standard_normal((tokens, cfg.hidden)).astype(np.float32)
    ids, wts = zipf_routing(rng, tokens, cfg.experts, cfg.top_k)
    return w, x, ids, wts


def per_expert_roofline(ids, tokens, cfg, has_shared=True):
    """Sum over the experts with rows (the shared expert with all T) of max(weight bytes / HBM peak,
    2 rows 3 I H / dense FP8 MFMA peak), in microseconds: each expert's weights stream once while its rows'
    products run at the MFMA peak, experts back to back."""
    counts = np.bincount(np.asarray(ids).ravel(), minlength=cfg.experts)
    rows = [int(c) for c in counts if c] + ([tokens] if has_shared else [])
    return sum(max(cfg.expert_bytes / HBM_PEAK, 2.0 * r * 3 * cfg.intermediate * cfg.hidden / FP8_MFMA_PEAK)
               for r in rows) * 1e6


def run(tokens=4096, iters=5, seed=20261018, ctx=None):
    from . import _lib
    from .config import BASELINE as cfg
    from .layer import ExpertBank, MoELayer, bf16_input
    own = ctx is None
    ctx = ctx or _lib.Context(0)
    bank = ExpertBank(ctx, cfg, cfg.experts + 1)
    bank.fill_synthetic(seed)
    w, xv, ids, wts = seeded_inputs(tokens, seed, cfg)
    layer = MoELayer(ctx, cfg, w, bank)
    x = ctx.upload(bf16_input(xv, cfg.hidden))
    idd, wd = ctx.upload(ids), ctx.upload(wts)
    y = ctx.empty((tokens, cfg.hidden), np.uint16)
    nbytes = layer.workspace_bytes(tokens)
    ws = ctx.malloc(nbytes)
    layer.prefill_device(x.ptr, tokens, y.ptr, ws, nbytes, idd, wd)
    ctx.sync()
    start, stop = ctx.event(), ctx.event()
    ctx.record(start)
    for _ in range(iters):
        layer.prefill_device(x.ptr, tokens, y.ptr, ws, nbytes, idd, wd)
    ctx.record(stop)
    us = ctx.elapsed_ms(start, stop) * 1000 / iters
    pairs = tokens * cfg.top_k + tokens
    flop = 2 * pairs * 3 * cfg.intermediate * cfg.hidden
    used = len(np.unique(ids)) + 1
    counts = np.bincount(ids.ravel(), minlength=cfg.experts)
    out = {"tokens": tokens, "us": round(us, 1), "flop": flop, "TFLOP_per_s": round(flop / us / 1e6, 1),
           "experts_used": used, "weight_bytes": used * cfg.expert_bytes,
           "weight_GB_per_s": round(used * cfg.expert_bytes / us / 1e3, 1),
           "max_tokens_per_expert": int(counts.max()), "median_tokens_per_expert": float(np.median(counts))}
    roof = per_expert_roofline(ids, tokens, cfg)
    out.update(roofline_us=round(roof, 1), roofline_frac=round(roof / us, 4),
               roofline_rule="sum over experts of max(weight bytes / 8 TB/s, 6 rows I H / 5 PFLOP/s)")
    ctx.free(ws)
    for d in (x, idd, wd, y):
        d.free()
    layer.close()
    bank.free()
    if own:
        ctx.close()
    return out


def main():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--tokens", type=int, default=4096)
    p.add_argument("--iters", type=int, default=5)
    args = p.parse_args()
    print(json.dumps(run(args.tokens, args.iters)), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
