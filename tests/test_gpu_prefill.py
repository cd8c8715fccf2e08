"""GPU parity of the MoE prefill (mx_moe_prefill: token-sorted grouped GEMMs on scaled MXFP4 MFMA).

Per token the prefill is the decode layer's arithmetic (the oracle's per-token layer): compared within the
north-star tolerance on Zipf-skewed routing (experts with several 128-row tiles, experts with none, ragged
tails), through the layer's own router (identical logits to mx_gate_project), and at the BASELINE shapes
on a sample of tokens. The routed rows' plan is checked bit-exactly through the combine: a wrong row,
order or token would move whole outputs, far outside the tolerance.
"""

import numpy as np
import pytest

from oracle.inputs import activations, mxfp4_expert, router_weight
from vesper_amd.workloads import zipf_routing
from oracle.moe import moe_layer, moe_layer_routed
from tests.helpers import assert_close, max_rel_err
from vesper_amd import _lib
from vesper_amd.config import MoEConfig
from vesper_amd.layer import ExpertBank, MoELayer

pytestmark = pytest.mark.gpu


def small_layer(ctx, rng, cfg):
    bank = ExpertBank(ctx, cfg, cfg.experts + (1 if cfg.shared else 0))
    arrays = {}
    for e in range(bank.count):
        arrays[e] = mxfp4_expert(rng, cfg.hidden, cfg.intermediate)
        bank.upload(e, arrays[e])
    w = router_weight(rng, cfg.experts, cfg.hidden) * np.float32(8.0)
    return MoELayer(ctx, cfg, w, bank), bank, w, arrays


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
        got = layer.prefill(x, ids, wts)
        ref = moe_layer_routed(x, ids, wts, {e: arrays[e] for e in range(cfg.experts)},
                               arrays[cfg.experts] if shared else None, num_experts=cfg.experts,
                               swiglu_limit=cfg.swiglu_limit)
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
        got = layer.prefill(x, ids, wts)
        ref = moe_layer_routed(x, ids, wts, {e: arrays[e] for e in range(cfg.experts)}, arrays[cfg.experts],
                               num_experts=cfg.experts, swiglu_limit=cfg.swiglu_limit)
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
        got = layer.prefill(x, ids, wts)
        sample = np.array([0, 1234, 2048, 3001, T - 1])
        needed = sorted({int(e) for e in ids[sample].ravel()})
        experts = {e: bank.download(e) for e in needed}
        ref = moe_layer_routed(x, ids, wts, experts, bank.download(cfg.experts), num_experts=cfg.experts,
                               swiglu_limit=cfg.swiglu_limit, tokens=sample)
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
