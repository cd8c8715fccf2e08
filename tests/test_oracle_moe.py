"""Pins the oracle's participation, ordered combine and layer composition (CPU only).

The 38 aggregation cases recorded from the official DeepSeek MoE.forward
(results/2026-10-18-moe-arithmetic/moe-aggregation.json) are regenerated from
their seeds; inputs are checked by hash and every FP32 stage and the BF16
output must reproduce the recorded SHA-256. Negative controls restate
src/vesper/moe_reference.py:177-197 and must be detected.
"""

import hashlib
import json
from pathlib import Path

import numpy as np
import pytest

from oracle.expert import expert_forward, expert_reference_fp32, expert_reference_stages, swiglu
from oracle.formats import bf16_bits, bf16_values
from oracle.inputs import activations, aggregation_cases, mxfp4_expert, router_weight
from oracle.moe import combine, moe_layer, participation

GOLDEN = Path(__file__).resolve().parent / "golden" / "moe_aggregation.json"


def digest(array):
    return hashlib.sha256(np.ascontiguousarray(array).tobytes()).hexdigest()


def test_sparse_participation_uses_expert_id_order_and_token_order():
    ids = np.array([[383, 1, 4, 2, 0, 3], [5, 4, 3, 2, 1, 0]], np.int64)
    rows = participation(ids, 384, 6, 32)
    assert list(rows) == [0, 1, 2, 3, 4, 5, 383]
    assert rows[0].tolist() == [0, 1] and rows[5].tolist() == [1] and rows[383].tolist() == [0]
    assert participation(np.empty((0, 6), np.int64), 384, 6, 32) == {}


def test_invalid_routes_and_overlapping_same_expert_writes_are_rejected():
    valid = np.arange(6, dtype=np.int64).reshape(1, 6)
    for ids in (valid.astype(np.float32), valid[:, :5], np.tile(valid, (33, 1)),
                np.array([[-1, 1, 2, 3, 4, 5]], np.int64), np.array([[0, 1, 2, 3, 4, 384]], np.int64),
                np.array([[0, 0, 2, 3, 4, 5]], np.int64)):
        with pytest.raises(ValueError):
            participation(ids, 384, 6, 32)


def _negative_controls(indices, contributions, shared):
    values = {e: bf16_values(b) for e, b in contributions.items()}
    wrong = {}
    total = np.zeros_like(bf16_values(shared))
    for expert in indices[0]:
        total = (total + values[int(expert)]).astype(np.float32)
    wrong["route_rank_order"] = bf16_bits(total + bf16_values(shared))
    total = np.zeros_like(total)
    for expert in sorted(values):
        total = bf16_values(bf16_bits(total + values[expert]))
    wrong["BF16_after_each_expert"] = bf16_bits(total + bf16_values(shared))
    total = bf16_values(shared).copy()
    for expert in sorted(values):
        total = (total + values[expert]).astype(np.float32)
    wrong["shared_first"] = bf16_bits(total)
    return wrong


def test_recorded_official_aggregation_hashes():
    golden = json.loads(GOLDEN.read_text())
    detected = {"route_rank_order": False, "BF16_after_each_expert": False, "shared_first": False}
    cases = list(aggregation_cases())
    assert len(cases) == len(golden["cases"]) == 38
    for record, case in zip(golden["cases"], cases):
        assert record["input"] == case["input"]
        assert record["indices"] == case["indices"].tolist()
        assert record["shared_sha256"] == digest(case["shared"])
        assert record["contribution_sha256"] == {str(e): digest(a) for e, a in case["contributions"].items()}
        stages = combine(case["indices"], case["contributions"], case["shared"], 384, 6)
        assert set(stages) == set(record["expected_sha256"])
        for name, array in stages.items():
            assert digest(array) == record["expected_sha256"][name], (case["input"], name)
        if case["input"].startswith("cancellation_rank_"):
            for name, bits in _negative_controls(case["indices"], case["contributions"], case["shared"]).items():
                detected[name] |= bool(np.count_nonzero(bits != stages["output_bf16"]))
    assert all(detected.values()), detected


def test_swiglu_clamp_order_and_route_before_down():
    w1 = bf16_bits(np.array([[12.0, -30.0, 0.5, 9.0]], np.float32))
    w3 = bf16_bits(np.array([[-11.0, 3.0, 20.0, 2.0]], np.float32))
    down, trace = swiglu(w1, w3, 10.0, [0.25])
    np.testing.assert_array_equal(trace[0, :, 0], [10.0, -30.0, 0.5, 9.0])      # gate clamped above only
    np.testing.assert_array_equal(trace[0, :, 1], [-10.0, 3.0, 10.0, 2.0])      # up clamped both sides
    g = trace[0, :, 0].astype(np.float64)
    np.testing.assert_allclose(trace[0, :, 2], g / (1 + np.exp(-g)), rtol=2 ** -22)
    np.testing.assert_array_equal(trace[0, :, 4], (np.float32(0.25) * trace[0, :, 3]).astype(np.float32))
    np.testing.assert_array_equal(down, bf16_values(bf16_bits(trace[0, :, 4]))[None])
    _, unclamped = swiglu(w1, w3, 0.0, None)
    assert unclamped[0, 0, 0] == 12.0 and unclamped[0, 2, 1] == 20.0


def test_quantized_expert_tracks_the_fp32_formula():
    rng = np.random.default_rng(20261018)
    arrays = mxfp4_expert(rng, 512, 256)
    x = activations(rng, 3, 512)
    w = np.array([0.3, 0.7, 1.1], np.float32)
    out = expert_forward(x, arrays, w, limit=0.0)
    ref = expert_reference_fp32(x, arrays, w)
    y = bf16_values(out["w2"]).astype(np.float64)
    cos = (y * ref).sum() / np.linalg.norm(y) / np.linalg.norm(ref)
    assert cos > 0.999, cos      # W4A8 quantization error against the unquantized formula
    assert out["q"].shape == (3, 512) and out["down_q"].shape == (3, 256) and out["trace"].shape == (3, 256, 5)


def test_layer_routes_weights_before_w2_and_combines_in_id_order():
    rng = np.random.default_rng(5)
    hidden, inter, experts = 256, 128, 16
    bank = {e: mxfp4_expert(rng, hidden, inter) for e in range(experts)}
    shared = mxfp4_expert(rng, hidden, inter)
    wr = router_weight(rng, experts, hidden) * 20
    x = activations(rng, 4, hidden)
    out = moe_layer(x, wr, bank, shared, top_k=4, route_scale=2.5)
    ids, weights = out["routing"]["indices"], out["routing"]["weights"]
    for t in range(4):
        for rank, e in enumerate(ids[t]):
            rows = participation(ids, experts, 4)[int(e)]
            position = int(np.flatnonzero(rows == t)[0])
            alone = expert_forward(x[t], bank[int(e)], [weights[t, rank]], 0.0)
            np.testing.assert_array_equal(out["experts"][int(e)]["w2"][position], alone["w2"][0])
    # weighting after W2 instead of before is a different (wrong) arithmetic
    e0 = int(ids[0, 0])
    unweighted = expert_forward(x[0], bank[e0], None, 0.0)["w2"]
    post = bf16_bits(bf16_values(unweighted) * weights[0, 0])
    assert np.count_nonzero(post != out["experts"][e0]["w2"][0]) > 0


def _brute_dequant(packed, scales):
    """E2M1 byte pairs (low nibble = even K) times 2^(E8M0 - 127) per 32 K, written out per element."""
    magnitude = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]
    rows, half = packed.shape
    out = np.zeros((rows, 2 * half))
    for r in range(rows):
        for b in range(half):
            for j, code in enumerate((int(packed[r, b]) & 0xF, int(packed[r, b]) >> 4)):
                k = 2 * b + j
                value = magnitude[code & 7] * (-1.0 if code & 8 else 1.0)
                out[r, k] = value * 2.0 ** (int(scales[r, k // 32]) - 127)
    return out


def test_configuration0_formula_against_brute_force():
    """expert_reference_stages (BASELINE configuration 0's formula) against an element-by-element
    restatement on a tiny expert: W1 and W3 kept apart, W2 applied to h (not to g or u), K and rows not
    transposed, the route weight on h."""
    rng = np.random.default_rng(11)
    hidden, inter = 64, 32
    arrays = mxfp4_expert(rng, hidden, inter, scale_lo=124, scale_hi=129)
    x = activations(rng, 2, hidden)
    route = np.array([0.5, 2.0], np.float32)
    ref = expert_reference_stages(x, arrays, route)
    xv = bf16_values(bf16_bits(x)).astype(np.float64)
    w1 = _brute_dequant(arrays["w1_weight"], arrays["w1_scale"])
    w3 = _brute_dequant(arrays["w3_weight"], arrays["w3_scale"])
    w2 = _brute_dequant(arrays["w2_weight"], arrays["w2_scale"])
    for t in range(2):
        g = [sum(w1[i, k] * xv[t, k] for k in range(hidden)) for i in range(inter)]
        u = [sum(w3[i, k] * xv[t, k] for k in range(hidden)) for i in range(inter)]
        h = [g[i] / (1.0 + np.exp(-g[i])) * u[i] * float(route[t]) for i in range(inter)]
        y = [sum(w2[o, i] * h[i] for i in range(inter)) for o in range(hidden)]
        np.testing.assert_allclose(ref["g"][t], g, rtol=1e-12, atol=1e-12)
        np.testing.assert_allclose(ref["u"][t], u, rtol=1e-12, atol=1e-12)
        np.testing.assert_allclose(ref["h"][t], h, rtol=1e-12, atol=1e-12)
        np.testing.assert_allclose(ref["y"][t], y, rtol=1e-10, atol=1e-12)
