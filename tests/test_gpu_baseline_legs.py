"""GPU parity of the benchmark's own workloads at their full shapes.

* Routing end to end: for the benchmark's four seeded layers at T = 1, 4 and 16,
  the top-8 indices the decode kernels choose equal the oracle's routing of the oracle's own FP32 gate
  logits (float64 GEMV rounded once). The route weights are within 4 FP32 ulps: the kernel's logits are
  FP32 sums in its own order, an ulp or so from the correctly rounded ones, and the weights follow them
  (on the kernel's own logits they are bit-exact, tests/test_gpu_moe.py). The smallest gap between the
  8th and 9th selection score is printed: it bounds how far the logits could move before the selection
  changes.
* Configuration 4 at its shapes: 8 layers, T = 4, a cache of 25 % of the routed experts, the benchmark's
  60 %-repeat trace, two steps through OffloadDecode. Every layer's output is finite and bit-identical to
  the same routing decoded with every expert resident (decode_routed), and sampled tokens of the first and
  last layer match the oracle's routed layer on the same layer input within the north-star bar. The
  experts' E8M0 codes are drawn from [118, 120] as in the benchmark's offload workload: with config 0's
  [118, 126] each synthetic layer scales its input up about a million-fold and a chain of 8 overflows.
"""

import ctypes as C

import numpy as np
import pytest

from oracle.formats import bf16_values
from oracle.moe import moe_layer_routed
from oracle.router import gate_logits, route, scores
from tests.helpers import assert_close
from vesper_amd.config import BASELINE
from vesper_amd.layer import ExpertBank, MoELayer, bf16_input

pytestmark = pytest.mark.gpu
SEED = 20261018      # bench.py's default seed
LAYERS = 4           # bench.py rotates over this many layers


def bench_inputs():
    """Router weights and activations exactly as bench.py draws them."""
    cfg = BASELINE
    rng = np.random.default_rng(SEED)
    routers = []
    for li in range(LAYERS):
        r = rng if li == 0 else np.random.default_rng(SEED + li)
        routers.append((r.standard_normal((cfg.experts, cfg.hidden)) * 0.02).astype(np.float32))
        if li == 0:
            x = rng.standard_normal((16, cfg.hidden)).astype(np.float32)
    return routers, bf16_input(x, cfg.hidden)


def test_routing_indices_from_the_oracles_own_logits(gpu_ctx):
    cfg = BASELINE
    routers, bits = bench_inputs()
    bank = ExpertBank(gpu_ctx, cfg, cfg.experts + 1)
    bank.fill_synthetic(SEED)
    x = gpu_ctx.upload(bits)
    y = gpu_ctx.empty((16, cfg.hidden), np.uint16)
    min_gap = np.inf
    try:
        for li, w in enumerate(routers):
            with MoELayer(gpu_ctx, cfg, w, bank) as layer:
                for t in (1, 4, 16):
                    layer.decode_device(x.ptr, t, y.ptr, diagnostics=True)
                    gpu_ctx.sync()
                    got_ids = layer.read("indices", (t, cfg.top_k), np.int32)
                    got_w = layer.read("weights", (t, cfg.top_k), np.float32)
                    logits = gate_logits(w, bf16_values(bits[:t]))
                    ref = route(logits, cfg.top_k, cfg.route_scale, cfg.score_func)
                    np.testing.assert_array_equal(got_ids, ref["indices"], err_msg=f"layer {li} T={t}")
                    ulps = np.abs(got_w.view(np.int32).astype(np.int64) - ref["weights"].view(np.int32))
                    assert ulps.max() <= 4, f"layer {li} T={t}: weights {ulps.max()} ulps apart"
                    s = np.sort(scores(logits, cfg.score_func), axis=1)[:, ::-1]
                    min_gap = min(min_gap, float(np.min(s[:, cfg.top_k - 1] - s[:, cfg.top_k])))
    finally:
        x.free()
        y.free()
        bank.free()
    print(f"smallest gap between the 8th and 9th selection score: {min_gap:.3e}")
    assert min_gap > 0


@pytest.mark.timeout(400)
def test_offload_baseline_shapes_equal_resident_and_oracle(gpu_ctx):
    from vesper_amd.offload_workload import trace
    from vesper_amd.tiered import ExpertCache, HostExpertPool, OffloadDecode, decode_routed
    cfg = BASELINE
    layers, tokens, steps = 8, 4, 2
    rng = np.random.default_rng(SEED)
    bank = ExpertBank(gpu_ctx, cfg, cfg.experts + 1)          # routed experts 0..255 and the shared one
    bank.fill_synthetic(SEED, scale_lo=118, scale_hi=120)
    pool = HostExpertPool(gpu_ctx, cfg, cfg.experts)
    for e in range(cfg.experts):
        pool.fill_from_bank(bank, e, e)
    gpu_ctx.sync()
    cache = ExpertCache(gpu_ctx, pool.expert_bytes, layers * cfg.experts // 4)
    off = OffloadDecode(gpu_ctx, cfg, layers, lambda l, e: (pool, e), [bank.tiled_ptr(cfg.experts)] * layers, cache,
                        bank.tiled_ptr(0))
    resident = MoELayer(gpu_ctx, cfg, np.zeros((cfg.experts, cfg.hidden), np.float32), bank)
    tr = trace(rng, steps, layers, tokens, cfg.experts, cfg.top_k)
    x = gpu_ctx.upload(bf16_input(rng.standard_normal((tokens, cfg.hidden)).astype(np.float32), cfg.hidden))
    ys = [gpu_ctx.empty((tokens, cfg.hidden), np.uint16) for _ in range(layers)]
    refs = [gpu_ctx.empty((tokens, cfg.hidden), np.uint16) for _ in range(layers)]
    try:
        for s in range(steps):
            off.load_routing(tr[s])
            off.step_device(x.ptr, tokens, [y.ptr for y in ys])
            gpu_ctx.sync()
            off.check_routes()
            for l in range(layers):
                src = x.ptr if l == 0 else refs[l - 1].ptr
                decode_routed(resident, src, tokens, off.ids[l].ptr, off.wts[l].ptr, refs[l].ptr)
            gpu_ctx.sync()
            assert resident.route_errors() == 0
            outs = [y.download() for y in ys]
            for l in range(layers):
                assert not np.any((outs[l] & 0x7F80) == 0x7F80), f"step {s} layer {l}: non-finite output"
                np.testing.assert_array_equal(outs[l], refs[l].download(), err_msg=f"step {s} layer {l}")
            print(f"step {s}: 8 layers bit-identical to the resident decode; cache {cache.stats()}")
        st = cache.stats()
        assert st["misses"] > 0 and st["hits"] > 0
        # the last step's first and last layer against the oracle, on the layer's own input
        inputs = [x.download()] + outs[:-1]
        shared = bank.download(cfg.experts)
        for l, toks in ((0, [0, 3]), (layers - 1, [1])):
            ids, w = tr[steps - 1][l]
            needed = {int(e): bank.download(int(e)) for e in np.unique(ids[toks])}
            ref = moe_layer_routed(bf16_values(inputs[l]), ids, w, needed, shared, num_experts=cfg.experts,
                                   swiglu_limit=cfg.swiglu_limit, tokens=toks)
            assert_close(outs[l][toks], ref["output_bf16"], f"layer {l} tokens {toks}")
    finally:
        off.close()
        resident.close()
        cache.close()
        for d in [x] + ys + refs:
            d.free()
        pool.close()
        bank.free()
