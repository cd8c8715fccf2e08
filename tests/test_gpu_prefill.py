"""GPU parity of the MoE prefill (mx_moe_prefill: token-sorted grouped GEMMs).

Per token the prefill is the decode layer's arithmetic (the oracle's per-token layer). The gate/up GEMM
follows the block spec bit for bit (every 32-block dot rounded once, blocks added in ascending order), so
every routed pair's and the shared expert's down-input codes and scales -- which W1 and W3 determine
through the SwiGLU and the per-32 quantizer -- must equal the oracle's (mx_prefill_stage_offsets reads them
from the workspace); the layer output is compared within the north-star tolerance (the down GEMM sums K in
its own order). Cases: Zipf-skewed routing (experts with several 128-row tiles, experts with none, ragged
tails), narrow shapes, the layer's own router, the BASELINE and reference-model shapes on sampled tokens,
and the three configurations a one-off randomized sweep found outside the bar while gate/up summed four
blocks per rounding. The routed rows' plan is checked through the combine: a wrong row, order or token
would move whole outputs, far outside the tolerance.
"""

import numpy as np
import pytest

from oracle.expert import expert_forward
from oracle.inputs import activations, mxfp4_expert, router_weight
from vesper_amd.workloads import zipf_routing
from oracle.moe import moe_layer, moe_layer_routed
from tests.helpers import assert_close, assert_gemv_close, max_rel_err
from vesper_amd import _lib
from vesper_amd.config import MoEConfig
from vesper_amd.layer import ExpertBank, MoELayer, bf16_input
from vesper_amd.tiered import decode_routed

pytestmark = pytest.mark.gpu


def small_layer(ctx, rng, cfg):
    bank = ExpertBank(ctx, cfg, cfg.experts + (1 if cfg.shared else 0))
    arrays = {}
    for e in range(bank.count):
        arrays[e] = mxfp4_expert(rng, cfg.hidden, cfg.intermediate)
        bank.upload(e, arrays[e])
    w = router_weight(rng, cfg.experts, cfg.hidden) * np.float32(8.0)
    return MoELayer(ctx, cfg, w, bank), bank, w, arrays


def check_down_codes(stages, ids, ref_experts, tokens=None, shared=None, what=""):
    """The prefill's down-input codes and scales of every routed pair (and of the shared expert's rows, when
    `shared` is the oracle's stage dict for it) equal the oracle's. ref_experts: the oracle's per-expert
    stage dicts over `tokens` (all tokens if None), rows in ascending token order."""
    tokens = np.arange(ids.shape[0]) if tokens is None else np.asarray(tokens)
    for e, out in ref_experts.items():
        toks = tokens[(ids[tokens] == e).any(axis=1)]
        ranks = (ids[toks] == e).argmax(axis=1)
        rows = stages["pair_row"][toks, ranks]
        np.testing.assert_array_equal(stages["down_q"][rows], out["down_q"], err_msg=f"{what} expert {e} codes")
        np.testing.assert_array_equal(stages["down_s"][rows], out["down_s"], err_msg=f"{what} expert {e} scales")
    if shared is not None:
        rows = stages["row0"][-1] + tokens
        np.testing.assert_array_equal(stages["down_q"][rows], shared["down_q"], err_msg=f"{what} shared codes")
        np.testing.assert_array_equal(stages["down_s"][rows], shared["down_s"], err_msg=f"{what} shared scales")


@pytest.mark.parametrize("tokens,shared", [(300, True), (129, False), (7, True)])
def test_prefill_zipf_routing_matches_oracle(gpu_ctx, tokens, shared):
    cfg = MoEConfig(hidden=512, intermediate=256, experts=32, top_k=4, swiglu_limit=10.0,
                    shared="mxfp4" if shared else None, max_tokens=16)
    rng = np.random.default_rng(tokens)
    layer, bank, w, arrays = small_layer(gpu_ctx, rng, cfg)
    try:
        x = activations(rng, tokens, cfg.hidden)
        # Zipf over 28 of the 32 experts: four experts get no token (empty slots in the plan)
        used = np.sort(rng.choice(cfg.experts, 28, replace=False)).astype(np.int32)
        ids, wts = zipf_routing(rng, tokens, 28, cfg.top_k)
        ids = used[ids]
        counts = np.bincount(ids.ravel(), minlength=cfg.experts)
        if tokens == 300:
            assert counts.max() > 128 and (counts == 0).any()      # multi-tile experts and idle ones
        got, stages = layer.prefill(x, ids, wts, stages=True)
        ref = moe_layer_routed(x, ids, wts, {e: arrays[e] for e in range(cfg.experts)},
                               arrays[cfg.experts] if shared else None, num_experts=cfg.experts,
                               swiglu_limit=cfg.swiglu_limit)
        sh = expert_forward(x, arrays[cfg.experts], None, cfg.swiglu_limit) if shared else None
        check_down_codes(stages, ids, ref["experts"], shared=sh, what="prefill")
        assert_close(got, ref["output_bf16"], "prefill")
        for t in range(tokens):                                     # every token, not just the aggregate
            assert max_rel_err(got[t], ref["output_bf16"][t]) <= 2e-2, t
    finally:
        layer.close()
        bank.free()


def test_prefill_narrow_shapes_take_the_smaller_tiles(gpu_ctx):
    """I % 256 != 0 and H % 512 != 0: gate/up with one 64-row group per wave, down on 8-wave tiles."""
    cfg = MoEConfig(hidden=768, intermediate=384, experts=16, top_k=4, swiglu_limit=7.0, shared="mxfp4",
                    max_tokens=16)
    rng = np.random.default_rng(384)
    layer, bank, w, arrays = small_layer(gpu_ctx, rng, cfg)
    try:
        x = activations(rng, 200, cfg.hidden)
        ids, wts = zipf_routing(rng, 200, cfg.experts, cfg.top_k)
        got, stages = layer.prefill(x, ids, wts, stages=True)
        ref = moe_layer_routed(x, ids, wts, {e: arrays[e] for e in range(cfg.experts)}, arrays[cfg.experts],
                               num_experts=cfg.experts, swiglu_limit=cfg.swiglu_limit)
        check_down_codes(stages, ids, ref["experts"], shared=expert_forward(x, arrays[cfg.experts], None,
                                                                           cfg.swiglu_limit), what="narrow")
        assert_close(got, ref["output_bf16"], "prefill narrow")
        for t in range(200):
            assert max_rel_err(got[t], ref["output_bf16"][t]) <= 2e-2, t
    finally:
        layer.close()
        bank.free()


def test_prefill_through_the_layer_router(gpu_ctx):
    cfg = MoEConfig(hidden=512, intermediate=256, experts=32, top_k=4, swiglu_limit=0.0, shared="mxfp4",
                    max_tokens=16)
    rng = np.random.default_rng(77)
    layer, bank, w, arrays = small_layer(gpu_ctx, rng, cfg)
    try:
        x = activations(rng, 40, cfg.hidden)
        got = layer.prefill(x)
        logits = np.stack([GateProjection_logits(gpu_ctx, w, row) for row in x])
        ref = moe_layer(x, w, {e: arrays[e] for e in range(cfg.experts)}, arrays[cfg.experts], top_k=cfg.top_k,
                        route_scale=cfg.route_scale, score_func=cfg.score_func, swiglu_limit=cfg.swiglu_limit,
                        logits=logits)
        assert_close(got, ref["output_bf16"], "prefill via router")
        # the decode layer on the first 16 tokens routes identically; outputs agree within tolerance
        dec = layer.decode(x[:16])
        assert_close(got[:16], dec, "prefill vs decode")
    finally:
        layer.close()
        bank.free()


def GateProjection_logits(ctx, w, row):
    from oracle.formats import bf16_bits
    wd = ctx.upload(np.ascontiguousarray(w, np.float32))
    xd = ctx.upload(bf16_bits(row.reshape(1, -1)))
    out = ctx.empty((1, w.shape[0]), np.float32)
    try:
        ctx.lib.gate_project(ctx._h(), _lib.vp(wd), _lib.vp(xd), 1, w.shape[1], w.shape[0], _lib.vp(out), None)
        return out.download()[0]
    finally:
        for d in (wd, xd, out):
            d.free()


def test_prefill_baseline_shapes_sampled_tokens(gpu_ctx):
    """BASELINE configuration 2 shapes: 256 experts x (7168 x 2048) + shared, T = 4096, Zipf(1.1) routing;
    five tokens (first, last, and three in between) against the oracle."""
    cfg = MoEConfig()
    rng = np.random.default_rng(20261018)
    bank = ExpertBank(gpu_ctx, cfg, cfg.experts + 1)
    bank.fill_synthetic(seed=5)
    w = router_weight(rng, cfg.experts, cfg.hidden)
    layer = MoELayer(gpu_ctx, cfg, w, bank)
    try:
        T = 4096
        x = activations(rng, T, cfg.hidden)
        ids, wts = zipf_routing(rng, T, cfg.experts, cfg.top_k)
        got, stages = layer.prefill(x, ids, wts, stages=True)
        sample = np.array([0, 1234, 2048, 3001, T - 1])
        needed = sorted({int(e) for e in ids[sample].ravel()})
        experts = {e: bank.download(e) for e in needed}
        shared = bank.download(cfg.experts)
        ref = moe_layer_routed(x, ids, wts, experts, shared, num_experts=cfg.experts,
                               swiglu_limit=cfg.swiglu_limit, tokens=sample)
        check_down_codes(stages, ids, ref["experts"], tokens=sample,
                         shared=expert_forward(x[sample], shared, None, cfg.swiglu_limit), what="T=4096")
        assert_close(got[sample], ref["output_bf16"], "prefill T=4096 sample")
    finally:
        layer.close()
        bank.free()


def test_prefill_reference_shapes_sampled_tokens(gpu_ctx):
    """The reference model's shapes (384 experts x (5120 x 2304), top-6, clamp 10, shared expert): K runs
    of 40 and 18 chunks (not multiples of the weight ring's depth), 9 gate/up and 10 down row blocks;
    Zipf routing over 600 tokens, four tokens against the oracle."""
    from vesper_amd.config import REFERENCE as cfg
    rng = np.random.default_rng(5120)
    bank = ExpertBank(gpu_ctx, cfg, cfg.experts + 1)
    bank.fill_synthetic(seed=11)
    w = router_weight(rng, cfg.experts, cfg.hidden)
    layer = MoELayer(gpu_ctx, cfg, w, bank)
    try:
        T = 600
        x = activations(rng, T, cfg.hidden)
        ids, wts = zipf_routing(rng, T, cfg.experts, cfg.top_k)
        assert np.bincount(ids.ravel()).max() > 128                # a multi-tile expert
        got = layer.prefill(x, ids, wts)
        sample = np.array([0, 233, 417, T - 1])
        needed = sorted({int(e) for e in ids[sample].ravel()})
        experts = {e: bank.download(e) for e in needed}
        ref = moe_layer_routed(x, ids, wts, experts, bank.download(cfg.experts), num_experts=cfg.experts,
                               swiglu_limit=cfg.swiglu_limit, tokens=sample)
        assert_close(got[sample], ref["output_bf16"], "prefill reference shapes")
    finally:
        layer.close()
        bank.free()


def test_prefill_refuses_bad_routing(gpu_ctx):
    cfg = MoEConfig(hidden=512, intermediate=256, experts=16, top_k=2, shared=None, max_tokens=16)
    rng = np.random.default_rng(3)
    layer, bank, w, arrays = small_layer(gpu_ctx, rng, cfg)
    try:
        x = activations(rng, 4, cfg.hidden)
        with pytest.raises(ValueError):
            layer.prefill(x, np.array([[0, 0]] * 4, np.int32), np.ones((4, 2), np.float32))
        with pytest.raises(ValueError):
            layer.prefill(x, np.array([[0, 16]] * 4, np.int32), np.ones((4, 2), np.float32))
        with pytest.raises(ValueError):
            layer.prefill(x, np.array([[0, 1]] * 4, np.int32), None)
    finally:
        layer.close()
        bank.free()


def sweep_case(ctx, seed):
    """Configuration `seed` of the one-off randomized prefill sweep (rng = default_rng(5000 + seed)): the
    layer, T, x and a Zipf routing over a random subset of the experts, drawn in the sweep's order."""
    rng = np.random.default_rng(5000 + seed)
    experts = int(rng.choice([8, 16, 32, 64]))
    top_k = min(int(rng.choice([1, 2, 4, 8])), experts)
    cfg = MoEConfig(hidden=int(rng.choice([256, 512, 1024])), intermediate=int(rng.choice([128, 256, 512])),
                    experts=experts, top_k=top_k, swiglu_limit=float(rng.choice([0.0, 10.0])),
                    shared="mxfp4" if rng.integers(2) else None, max_tokens=16)
    layer, bank, w, arrays = small_layer(ctx, rng, cfg)
    T = int(rng.choice([1, 2, 5, 17, 64, 127, 128, 129, 255, 300, 513]))
    x = activations(rng, T, cfg.hidden)
    used_n = int(rng.integers(max(top_k, 1), experts + 1))
    used = np.sort(rng.choice(experts, used_n, replace=False)).astype(np.int32)
    ids, wts = zipf_routing(rng, T, used_n, top_k)
    return cfg, layer, bank, arrays, x, used[ids], wts


@pytest.mark.parametrize("seed,tokens", [(131, 127), (133, 128), (396, 513)])
def test_prefill_sweep_misses_are_bit_exact_in_gate_up(gpu_ctx, seed, tokens):
    """The sweep's three misses (max relative error 1.36e-2, 1.08e-2, 1.08e-2 while gate/up summed four
    blocks per rounding; sigmoid scores, no shared expert): one BF16 ulp of a W1 output moved one E4M3 code
    of the down input. With the in-order block sums the codes equal the oracle's and the output meets the
    bar, every token included."""
    cfg, layer, bank, arrays, x, ids, wts = sweep_case(gpu_ctx, seed)
    try:
        assert x.shape[0] == tokens
        print(f"prefill sweep seed {seed}: T={tokens} {cfg}", flush=True)
        got, stages = layer.prefill(x, ids, wts, stages=True)
        ref = moe_layer_routed(x, ids, wts, {e: arrays[e] for e in range(cfg.experts)},
                               arrays[cfg.experts] if cfg.shared else None, num_experts=cfg.experts,
                               swiglu_limit=cfg.swiglu_limit)
        sh = expert_forward(x, arrays[cfg.experts], None, cfg.swiglu_limit) if cfg.shared else None
        check_down_codes(stages, ids, ref["experts"], shared=sh, what=f"seed {seed}")
        assert_close(got, ref["output_bf16"], f"seed {seed}")
        for t in range(tokens):
            assert max_rel_err(got[t], ref["output_bf16"][t]) <= 2e-2, t
    finally:
        layer.close()
        bank.free()


def test_prefill_T4096_in_full_against_routed_decode_and_tile_edges(gpu_ctx):
    """BASELINE configuration 2 in full (T = 4096, Zipf(1.1) routing): every one of the 4096 prefill outputs
    against mx_moe_decode_routed on the same ids and weights (256 calls of 16 tokens) within the north-star
    bar -- per token, not only in aggregate; and the busiest expert (28 tiles of 128 rows): the first and
    last row of every tile through the oracle's expert -- down-input codes and scales bit-exact (they come
    from the exact gate/up), the expert's W2 output rows GEMV-close (the down GEMM sums K in its own order)."""
    cfg = MoEConfig()
    rng = np.random.default_rng(20261018)
    bank = ExpertBank(gpu_ctx, cfg, cfg.experts + 1)
    bank.fill_synthetic(seed=5)
    w = router_weight(rng, cfg.experts, cfg.hidden)
    layer = MoELayer(gpu_ctx, cfg, w, bank)
    T, k, h = 4096, cfg.top_k, cfg.hidden
    bufs = []
    try:
        x = activations(rng, T, h)
        ids, wts = zipf_routing(rng, T, cfg.experts, k)
        got, stages = layer.prefill(x, ids, wts, stages=True)
        xd, idd, wd = gpu_ctx.upload(bf16_input(x, h)), gpu_ctx.upload(ids), gpu_ctx.upload(wts)
        yd = gpu_ctx.empty((T, h), np.uint16)
        bufs = [xd, idd, wd, yd]
        for t0 in range(0, T, 16):
            decode_routed(layer, xd.ptr + 2 * h * t0, 16, idd.ptr + 4 * k * t0, wd.ptr + 4 * k * t0,
                          yd.ptr + 2 * h * t0)
        dec = yd.download()
        assert_close(got, dec, "prefill vs routed decode, all 4096 tokens")
        worst = max(max_rel_err(got[t], dec[t]) for t in range(T))
        assert worst <= 2e-2, worst

        counts = np.bincount(ids.ravel(), minlength=cfg.experts)
        e = int(np.argmax(counts))
        toks = np.flatnonzero((ids == e).any(axis=1))             # the expert's rows, ascending token
        tiles = (len(toks) + 127) // 128
        assert tiles == 28
        edges = sorted({i for tl in range(tiles) for i in (128 * tl, min(128 * tl + 127, len(toks) - 1))})
        sample = toks[edges]
        rank = (ids[sample] == e).argmax(axis=1)
        ref = expert_forward(x[sample], bank.download(e), wts[sample, rank], cfg.swiglu_limit)
        rows = stages["pair_row"][sample, rank]
        np.testing.assert_array_equal(stages["down_q"][rows], ref["down_q"], err_msg="busiest expert codes")
        np.testing.assert_array_equal(stages["down_s"][rows], ref["down_s"], err_msg="busiest expert scales")
        place = (np.sort(ids[sample], axis=1) == e).argmax(axis=1)  # the expert's place among the token's
        assert_gemv_close(stages["expert_out"][sample, place], ref["w2"], "busiest expert W2 rows")
    finally:
        for d in bufs:
            d.free()
        layer.close()
        bank.free()
