"""Benchmark: routed MoE decode layer on one MI355X.

One step = one MoE decode layer (router over 256 experts, top-8, 8 routed + 1 shared MXFP4
SwiGLU experts of 7168 x 2048, ordered combine) at each batch size T in {1, 4, 16}, inputs
resident in HBM. Expert weights are synthetic (uniform nibbles, E8M0 codes uniform in
[118, 126]) generated in HBM; W_r ~ N(0, 0.02); x ~ N(0, 1) rounded to BF16.

Consecutive decode calls go to consecutive layers of LAYERS independently generated ones (own 257
experts and router each, 6 GB per layer), as in a model: no call finds the weights of the call before
in the GPU's caches (256 MB Infinity Cache), which a single layer re-run with one routing would allow.

value = whole-step weight-stream throughput: algorithmic bytes (distinct selected experts + shared
+ router + activations, counted from each call's seeded routing) / step time. Prints one JSON line.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0
TOKENS = (1, 4, 16)
LAYERS = 4
ROOT = os.path.dirname(os.path.abspath(__file__))
TRAFFIC = os.path.join(ROOT, "profiles", "gateup_T16_traffic.json")


def parse():
    p = argparse.ArgumentParser(description=__doc__)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--seed", type=int, default=20261018)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--profile-iters", type=int, default=20)
    p.add_argument("--no-secondary", action="store_true",
                   help="skip the other BASELINE configurations (prefill, FP8 projections, offload)")
    return p.parse_args()


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def algorithmic_bytes(cfg, plan, tokens):
    """Bytes a decode layer must move: every distinct selected expert + shared once, the FP32 router,
    x, and the BF16 output."""
    experts = plan["n_slots"]
    router = cfg.experts * cfg.hidden * 4
    act = tokens * cfg.hidden * 2 * 2
    return experts * cfg.expert_bytes + router + act


def gateup_bytes(cfg, plan, tokens):
    """Algorithmic bytes of one gate/up launch: W1+W3 (+ scales) of every slot, quantized x, written
    down-input codes and scales."""
    per_slot = 2 * cfg.intermediate * (cfg.hidden // 2 + cfg.hidden // 32)
    rows = plan["total_rows"]
    return (plan["n_slots"] * per_slot + tokens * (cfg.hidden + cfg.hidden // 32)
            + rows * (cfg.intermediate + cfg.intermediate // 32))


def measured_traffic(algorithmic):
    """HBM bytes per gate/up launch at T=16 from the committed counter runs (FETCH_SIZE + WRITE_SIZE per
    dispatch, each divided by the copy-kernel calibration factor), or None when they do not describe this
    workload (different algorithmic byte count)."""
    try:
        with open(TRAFFIC) as f:
            rec = json.load(f)
    except (OSError, ValueError):
        return None
    if rec.get("algorithmic_bytes") != algorithmic:
        return None
    return rec.get("traffic_bytes")


def read_ceiling(ctx, stream, nbytes=2 << 30, reps=7):
    """HBM read rate of the fastest plain read kernel measured on this part (mx_read_kernel: 4096
    workgroups over contiguous ranges, non-temporal 16-byte loads), median of `reps` launches of
    `nbytes`, HIP events on the launch stream."""
    from vesper_amd import _lib
    import ctypes as C
    src = ctx.malloc(nbytes)
    out = ctx.empty((4 * 4096,), np.uint32)
    start, stop = ctx.event(), ctx.event()
    times = []
    for i in range(reps + 2):
        ctx.record(start, stream)
        ctx.lib.read_kernel(ctx._h(), C.c_void_p(src), nbytes, _lib.vp(out), _lib._stream(stream))
        ctx.record(stop, stream)
        ms = ctx.elapsed_ms(start, stop)
        if i >= 2:
            times.append(ms)
    ctx.free(src)
    out.free()
    gbs = nbytes / (float(np.median(times)) * 1e-3) / 1e9
    return {"GB_per_s": round(gbs, 1), "frac_of_peak": round(gbs / HBM_PEAK_GBS, 4), "bytes": nbytes,
            "kernel": "read_ceiling_kernel (mx_read_kernel): 4096 workgroups over contiguous ranges, "
                      "non-temporal 16-byte loads, 3 x 4 KB in flight per wave; median of "
                      f"{reps} launches"}


CPU_RUNS = 5
CPU_SAMPLE_EXPERTS = 2
CPU_FP8_SAMPLE_ROWS = 64
CPU_PREFILL_SAMPLE_ROWS = (32, 64)


def _median_s(fn, runs=CPU_RUNS):
    """One untimed warm-up call, then the median of `runs` timed calls (perf_counter_ns), in seconds."""
    fn()
    times = []
    for _ in range(runs):
        t0 = time.perf_counter_ns()
        fn()
        times.append((time.perf_counter_ns() - t0) * 1e-9)
    return float(np.median(times))


def cpu_prefill_leg(bank, cfg, tokens=4096, seed=20261018):
    """Configuration 2 (prefill, T = 4096, the prefill workload's own seeded Zipf routing) on the NumPy oracle,
    as a declared subset: the busiest expert through expert_forward on its first 32 and first 64 rows gives a
    per-expert cost (dequantising the weights, independent of the rows) and a per-row cost; the linear model
    is summed over every expert with rows and the shared expert's T rows. The combine's per-token sums are
    not included (a few milliseconds)."""
    from oracle.expert import expert_forward
    from oracle.formats import bf16_round
    from vesper_amd.prefill_workload import seeded_inputs
    _, x, ids, wts = seeded_inputs(tokens, seed, cfg)
    counts = np.bincount(ids.ravel(), minlength=cfg.experts)
    busiest = int(np.argmax(counts))
    rows = np.flatnonzero((ids == busiest).any(axis=1))
    route = wts[rows, (ids[rows] == busiest).argmax(axis=1)]
    xr = bf16_round(x[rows[:max(CPU_PREFILL_SAMPLE_ROWS)]])
    arrays = bank.download(busiest)
    lo, hi = CPU_PREFILL_SAMPLE_ROWS
    t_lo = _median_s(lambda: expert_forward(xr[:lo], arrays, route[:lo], cfg.swiglu_limit), 1)
    t_hi = _median_s(lambda: expert_forward(xr[:hi], arrays, route[:hi], cfg.swiglu_limit), 1)
    per_row = max(t_hi - t_lo, 0.0) / (hi - lo)
    fixed = t_lo - lo * per_row
    slots = [int(c) for c in counts if c] + [tokens]
    total = sum(fixed + per_row * r for r in slots)
    flop = 2 * sum(slots) * 3 * cfg.intermediate * cfg.hidden
    return {"us": total * 1e6, "TFLOP_per_s": flop / total / 1e12, "us_per_expert_fixed": fixed * 1e6,
            "us_per_row": per_row * 1e6, "expert_slots": len(slots), "rows": sum(slots),
            "sample": f"declared subset: the busiest expert ({counts[busiest]} rows) on its first {lo} and {hi} "
                      "rows in full (one warm-up, one timed call each), a linear per-expert + per-row model summed "
                      "over the routing's experts and the shared expert"}


def cpu_baseline(bank, w, x_rows, cfg, plans):
    """The NumPy oracle on the host cores, bounded samples of the benchmark's own inputs (one warm-up, median
    of 5 per leg):

    * config 0: one MXFP4 expert at T = 1 in configuration 0's own formula (BF16 activations, FP32
      accumulation, no activation quantization);
    * config 1 at T = 1, 4, 16: the router in full, the shared expert on all T rows, and the first
      CPU_SAMPLE_EXPERTS routed experts (ascending ID) on their own token rows; the routed time is
      extrapolated linearly to every distinct selected expert (the per-expert cost is dominated by
      dequantising its weights, which does not depend on its row count at these T);
    * config 2 at T = 4096 (declared subset, cpu_prefill_leg): one expert at 32 and 64 rows, extrapolated;
    * config 3 at T = 1, 16: all four FP8 projections in full (synthetic weights of the same shapes), and
      T = 2048 as a declared subset (T = 64 in full, extrapolated linearly in rows).

    value = config 1's bytes of one bench step (T = 1, 4 and 16) / the summed CPU time of the three legs."""
    import threadpoolctl
    sys.path.insert(0, ROOT)
    from oracle.expert import expert_forward, expert_reference_fp32
    from oracle.moe import participation
    from oracle.projections import fp8_projection, fp8_weights
    from oracle.router import gate_logits, route
    from vesper_amd.fp8_workload import LAYOUT

    threads = min(16, len(os.sched_getaffinity(0)))      # the GPU box's CPU share is 16 cores
    legs, step_bytes, step_s = {}, 0, 0.0
    with threadpoolctl.threadpool_limits(threads):
        blas = [f"{m.get('internal_api')} {m.get('version')} x{m.get('num_threads')}"
                for m in threadpoolctl.threadpool_info()]
        shared = bank.download(cfg.experts)
        x1 = x_rows[:1]
        sec = _median_s(lambda: expert_reference_fp32(x1, shared))
        legs["config0_T1"] = {"us": sec * 1e6, "GB_per_s": cfg.expert_bytes / sec / 1e9,
                              "sample": "one expert in full, BF16 activations (configuration 0's formula)"}
        log(f"cpu config 0: {sec:.2f} s")
        for t in TOKENS:
            x = x_rows[:t]
            r = route(gate_logits(w, x), cfg.top_k, cfg.route_scale, cfg.score_func)
            selected = participation(r["indices"], cfg.experts, cfg.top_k)
            sample = sorted(selected)[:CPU_SAMPLE_EXPERTS]
            arrays = {e: bank.download(e) for e in sample}
            weight = {e: np.array([r["weights"][row, list(r["indices"][row]).index(e)] for row in selected[e]],
                                  np.float32) for e in sample}
            router_s = _median_s(lambda: route(gate_logits(w, x), cfg.top_k, cfg.route_scale, cfg.score_func))
            shared_s = _median_s(lambda: expert_forward(x, shared, None, cfg.swiglu_limit))
            routed_s = _median_s(lambda: [expert_forward(x[selected[e]], arrays[e], weight[e], cfg.swiglu_limit)
                                          for e in sample]) / len(sample)
            total = router_s + shared_s + routed_s * len(selected)
            nbytes = algorithmic_bytes(cfg, plans[0, t], t)
            step_bytes += nbytes
            step_s += total
            legs[f"config1_T{t}"] = {"us": total * 1e6, "GB_per_s": nbytes / total / 1e9,
                                     "router_us": router_s * 1e6, "shared_us": shared_s * 1e6,
                                     "routed_us_per_expert": routed_s * 1e6, "distinct_experts": len(selected),
                                     "sample": f"router + shared in full; {len(sample)} of {len(selected)} routed "
                                               "experts timed, extrapolated linearly"}
            log(f"cpu config 1 T={t}: {total:.2f} s (extrapolated)")
        legs["config2_T4096"] = cpu_prefill_leg(bank, cfg)
        log(f"cpu config 2 T=4096: {legs['config2_T4096']['us'] * 1e-6:.2f} s (extrapolated)")
        rng = np.random.default_rng(20261018)
        weights = {name: fp8_weights(rng, n, k, 128) for name, (n, k) in LAYOUT.items()}
        c3 = {}
        for t in (1, 16, CPU_FP8_SAMPLE_ROWS):
            xs = {name: rng.standard_normal((t, k)).astype(np.float32) for name, (n, k) in LAYOUT.items()}
            runs = CPU_RUNS if t <= 16 else 1
            c3[t] = _median_s(lambda: [fp8_projection(xs[name], *weights[name], 128) for name in LAYOUT], runs)
            log(f"cpu config 3 T={t}: {c3[t]:.2f} s")

        def fp8_bytes(t):
            return sum(n * k + ((n + 127) // 128) * (k // 128) * 4 + t * (n + k) * 2 for n, k in LAYOUT.values())
        for t in (1, 16):
            legs[f"config3_T{t}"] = {"us": c3[t] * 1e6, "GB_per_s": fp8_bytes(t) / c3[t] / 1e9,
                                     "sample": "q_a, q_b, kv_a and o in full"}
        # T = 2048: token rows are independent, so the T = 16 and T = 128 times give a per-call and a per-row
        # cost, extrapolated linearly
        s0 = CPU_FP8_SAMPLE_ROWS
        per_row = (c3[s0] - c3[16]) / (s0 - 16)
        sec = c3[16] + per_row * (2048 - 16)
        flop = 2 * 2048 * sum(n * k for n, k in LAYOUT.values())
        legs["config3_T2048"] = {"us": sec * 1e6, "GB_per_s": fp8_bytes(2048) / sec / 1e9,
                                 "TFLOP_per_s": flop / sec / 1e12, "us_per_row": per_row * 1e6,
                                 "sample": f"declared subset: all four projections at T = 16 and T = {s0} in full (one warm-up, "
                                           f"one timed call at T = {s0}), extrapolated linearly in rows to T = 2048"}
        log(f"cpu config 3 T=2048: {sec:.2f} s (extrapolated)")
    legs = {name: {k: (round(v, 3) if isinstance(v, float) else v) for k, v in leg.items()} for name, leg in legs.items()}
    return {"value": round(step_bytes / step_s / 1e9, 5), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"NumPy oracle; config 1 step (T = 1, 4, 16) with {CPU_SAMPLE_EXPERTS} routed experts per T "
                      f"timed and extrapolated ({step_s:.1f} s per step); one warm-up, median of {CPU_RUNS} per leg",
            "legs": legs, "threads": {"blas": blas, "numpy_elementwise": 1},
            "cpu": platform.processor() or platform.machine(), "numpy": np.__version__,
            "os_cpu_count": os.cpu_count(), "affinity_cores": threads}


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only: the MoE path is single-GPU here "
                                   "(expert-parallel sharding is designed, not run)",
                          "n_gpus": args.gpus}))
        return 2
    from vesper_amd import _lib
    from vesper_amd.config import BASELINE
    from vesper_amd.layer import ExpertBank, MoELayer

    cfg = BASELINE
    ctx = _lib.Context(0)
    name, arch = ctx.device_name()
    log(f"device {name} {arch}")
    # layer 0 (and x) as in vesper_amd.profile_workload, so their counter runs describe its kernels
    rng = np.random.default_rng(args.seed)
    banks, routers, layers = [], [], []
    for li in range(LAYERS):
        bank = ExpertBank(ctx, cfg, cfg.experts + 1)
        bank.fill_synthetic(args.seed + li)
        r = rng if li == 0 else np.random.default_rng(args.seed + li)
        w = (r.standard_normal((cfg.experts, cfg.hidden)) * 0.02).astype(np.float32)
        banks.append(bank)
        routers.append(w)
        layers.append(MoELayer(ctx, cfg, w, bank))
        if li == 0:
            x_rows = rng.standard_normal((max(TOKENS), cfg.hidden)).astype(np.float32)
    bits = x_rows.view(np.uint32).astype(np.uint64)
    bits = ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16).astype(np.uint16)
    xs = {t: ctx.upload(bits[:t].copy()) for t in TOKENS}
    ys = {t: ctx.empty((t, cfg.hidden), np.uint16) for t in TOKENS}
    stream = ctx.stream()
    ctx.sync()
    log(f"weights of {LAYERS} layers resident; warming up")

    plans, per_t = {}, {}
    for li, layer in enumerate(layers):
        for t in TOKENS:
            layer.decode_device(xs[t].ptr, t, ys[t].ptr, stream)
            ctx.sync(stream)
            plans[li, t] = layer.plan()
    calls = 0
    for _ in range(args.warmup):
        for t in TOKENS:
            layers[calls % LAYERS].decode_device(xs[t].ptr, t, ys[t].ptr, stream)
            calls += 1
    ctx.sync(stream)

    # timed region: K steps, each a decode layer at T = 1, 4, 16, consecutive calls on consecutive layers
    start, stop = ctx.event(), ctx.event()
    ctx.sync()
    timed_bytes = 0
    ctx.record(start, stream)
    for _ in range(args.steps):
        for t in TOKENS:
            li = calls % LAYERS
            layers[li].decode_device(xs[t].ptr, t, ys[t].ptr, stream)
            timed_bytes += algorithmic_bytes(cfg, plans[li, t], t)
            calls += 1
    ctx.record(stop, stream)
    total_ms = ctx.elapsed_ms(start, stop)
    ctx.sync()
    ms_per_step = total_ms / args.steps
    log(f"timed {args.steps} steps: {ms_per_step * 1000:.1f} us/step")

    # per-T latency (calls rotating over the layers) and per-kernel timing of layer 0 (each stage
    # re-launched back to back on the launch stream, HIP events around the loop)
    for t in TOKENS:
        t_bytes = 0
        ctx.record(start, stream)
        for i in range(args.steps):
            layers[i % LAYERS].decode_device(xs[t].ptr, t, ys[t].ptr, stream)
            t_bytes += algorithmic_bytes(cfg, plans[i % LAYERS, t], t)
        ctx.record(stop, stream)
        us = ctx.elapsed_ms(start, stop) / args.steps * 1000
        b = t_bytes / args.steps
        layers[0].decode_device(xs[t].ptr, t, ys[t].ptr, stream)
        kernel_us = {stage: layers[0].time_stage(stage, args.profile_iters, stream) for stage in MoELayer.STAGES}
        distinct = [plans[li, t]["n_routed"] for li in range(LAYERS)]
        per_t[t] = {"us_per_layer": us, "distinct_experts": float(np.mean(distinct)),
                    "distinct_experts_per_layer": distinct, "bytes": b,
                    "GB_per_s": b / (us * 1e-6) / 1e9, "hbm_frac": b / (us * 1e-6) / 1e9 / HBM_PEAK_GBS,
                    "kernel_us_layer0": kernel_us, "gateup_bytes_layer0": gateup_bytes(cfg, plans[0, t], t)}
        log(f"T={t}: {us:.1f} us/layer, {per_t[t]['GB_per_s']:.0f} GB/s, layer-0 kernels {kernel_us}")

    ceiling = read_ceiling(ctx, stream)
    log(f"read ceiling: {ceiling['GB_per_s']} GB/s")
    value = timed_bytes / (total_ms * 1e-3) / 1e9
    head = per_t[16]
    gu_us = head["kernel_us_layer0"]["gateup"]
    achieved = head["gateup_bytes_layer0"] / (gu_us * 1e-6) / 1e9
    result = {
        "metric": "MoE decode-layer us + MXFP4 weight-stream GB/s (% HBM peak), top-8 of 256",
        "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "mxfp4xe4m3->f32", "data": "synthetic (seeded; weights generated in HBM)",
        "config": {"workload": "BASELINE config 1: routed MoE decode layer, T in {1,4,16} per step",
                   "layers_rotated": LAYERS,
                   "hidden": cfg.hidden, "intermediate": cfg.intermediate, "experts": cfg.experts,
                   "top_k": cfg.top_k, "shared": cfg.shared, "score_func": cfg.score_func,
                   "route_scale": cfg.route_scale, "tokens_per_step": list(TOKENS)},
        "hbm_frac": round(value / HBM_PEAK_GBS, 4),
        "per_batch": {str(t): {k: (round(v, 3) if isinstance(v, float) else v) for k, v in d.items()}
                      for t, d in per_t.items()},
        "roofline": {"kernel": "gateup_kernel<false> (T=16)", "bound": "hbm", "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(head["gateup_bytes_layer0"]), "launch_us": round(gu_us, 2),
                     "algorithmic_bytes": head["gateup_bytes_layer0"],
                     "read_ceiling_GB_s": ceiling["GB_per_s"],
                     "frac_of_read_ceiling": round(achieved / ceiling["GB_per_s"], 4)},
        "hbm_read_ceiling": ceiling,
        "device": {"name": name, "arch": arch},
    }
    if not args.no_cpu_baseline:
        log("cpu baseline (oracle, bounded sample)")
        x_bf16 = (bits.astype(np.uint32) << 16).view(np.float32)
        result["cpu_baseline"] = cpu_baseline(banks[0], routers[0], x_bf16, cfg, plans)
    for layer, bank in zip(layers, banks):
        layer.close()
        bank.free()
    if not args.no_secondary:
        result["secondary"] = secondary(ctx)
    print(json.dumps(result), flush=True)
    ctx.close()
    return 0


def secondary(ctx):
    """The other BASELINE configurations, measured on the same GPU (each a few seconds): 2 = MoE prefill
    (T = 4096, Zipf(1.1) routing), 3 = FP8 block-128 projections at T = 1, 16, 2048, 4 = 8-layer offload
    decode at T = 4 with 25 % of the routed experts resident; the SHA-256 admission audit of expert
    slots (one expert, and the 1 GiB maximum payload); the promotion of single experts from the on-disk
    store into HBM slots; and configuration 0's expert with BF16 activations at T = 1, 4, 16."""
    from vesper_amd import (bf16_workload, fp8_workload, integrity_workload, offload_workload, prefill_workload,
                            store_workload)
    out = {}
    log("configuration 0: one expert, BF16 activations")
    c0 = bf16_workload.run((1, 4, 16), 50, ctx=ctx)
    for v in c0["per_tokens"].values():
        v["hbm_frac"] = round(v["GB_per_s"] / HBM_PEAK_GBS, 4)
    out["config0_bf16_expert"] = c0
    log(f"config 0: {c0}")
    log("configuration 2: prefill")
    p = prefill_workload.run(4096, 5, ctx=ctx)
    out["prefill_T4096"] = dict(p, mfma_peak_TFLOP_per_s=5000.0, mfma_frac=round(p["TFLOP_per_s"] / 5000.0, 4))
    log(f"prefill: {p}")
    log("configuration 3: FP8 projections")
    f = fp8_workload.run((1, 16, 2048), 20, ctx=ctx)
    out["fp8_projections"] = {str(t): {"us": v["us"], "GB_per_s": v["GB_per_s"], "TFLOP_per_s": v["TFLOP_per_s"],
                                       "hbm_frac": round(v["GB_per_s"] / HBM_PEAK_GBS, 4),
                                       "mfma_frac": round(v["TFLOP_per_s"] / 5000.0, 4),
                                       "per_projection_us": {k: p2["us"] for k, p2 in v["projections"].items()}}
                              for t, v in f.items()}
    log(f"fp8: {out['fp8_projections']}")
    g = fp8_workload.run_grouped((1, 8), 20, ctx=ctx)
    out["wo_a_grouped"] = {str(t): dict(v, hbm_frac=round(v["GB_per_s"] / HBM_PEAK_GBS, 4)) for t, v in g.items()}
    log(f"wo_a grouped: {out['wo_a_grouped']}")
    log("configuration 4: offload decode")
    o = offload_workload.run(10, 4, ctx=ctx)
    out["offload_8layers_T4"] = o
    log(f"offload: {o}")
    log("cache admission audit: SHA-256 per 4 KiB chunk")
    out["integrity_sha256"] = integrity_workload.run(20, ctx=ctx)
    log(f"integrity: {out['integrity_sha256']}")
    log("store -> HBM promotion of single experts (O_DIRECT read, pinned staging, tiled slot, audit)")
    out["store_to_hbm"] = store_workload.run(8)
    log(f"store: {out['store_to_hbm']}")
    return out


if __name__ == "__main__":
    sys.exit(main())
