"""Pins the oracle's router (CPU only).

Goldens: tests/test_router.py:28-76 of the reference, and the 232 recorded
PyTorch-CUDA selection cases of results/2026-10-18-routing-ties (E=384, k=6),
regenerated from their seeds and checked by input hash.
"""

import hashlib
import json
from pathlib import Path

import numpy as np
import pytest

from oracle.inputs import selection_cases
from oracle.router import (gate_logits, ordered_keys, route, route_weights, scores, select_scores,
                           tie_flag, topk_indices, tree_sum)

GOLDEN = Path(__file__).resolve().parent / "golden" / "router_selection.json"


def test_pinned_cuda_tie_order_goldens_and_padding():
    for level in (0, -1, 1):
        assert topk_indices(np.full(384, level, np.float32), 6).tolist() == [1, 0, 4, 5, 2, 3]
    signed = np.resize(np.array([-0.0, 0.0], np.float32), 384)
    assert topk_indices(signed, 6).tolist() == [3, 1, 9, 11, 5, 7]
    for invalid in (np.full(384, np.nan, np.float32), np.full(384, np.inf, np.float32)):
        with pytest.raises(ValueError):
            topk_indices(invalid, 6)


def test_bias_selects_experts_without_scaling_their_raw_weights():
    s = np.linspace(1, 2, 384, dtype=np.float32)
    bias = np.zeros(384, np.float32)
    bias[0] = 100
    weights, indices = select_scores(s, bias, 6, 1.5)
    assert indices.tolist() == [0, 383, 382, 381, 380, 379]
    assert weights[0] < weights[1]
    assert abs(float(weights.sum()) - 1.5) < 1e-6
    assert float(weights[0]) < 0.2


def test_selected_and_boundary_ties_keep_the_selected_expert_set():
    s = np.arange(384, dtype=np.float32)
    bias = np.zeros(384, np.float32)
    for positions in ((382, 383), (377, 378)):
        changed = s.copy()
        changed[positions[0]] = changed[positions[1]]
        weights, indices = select_scores(changed, bias, 6, 1.5)
        expected = set(range(378, 384)) if positions[0] == 382 else {377, 379, 380, 381, 382, 383}
        assert set(indices.tolist()) == expected
        assert abs(float(weights.sum()) - 1.5) < 1e-6
    s[0] = s[1]
    _, indices = select_scores(s, bias, 6, 1.5)
    assert indices.tolist() == [383, 382, 381, 380, 379, 378]
    for bad in (np.ones(383, np.float32), np.full(384, np.inf, np.float32), np.full(384, -1, np.float32)):
        with pytest.raises(ValueError):
            select_scores(bad, bias, 6, 1.5)


def test_recorded_cuda_selection_cases():
    golden = json.loads(GOLDEN.read_text())["cases"]
    regenerated = list(selection_cases())
    assert len(regenerated) == len(golden) == 232
    for record, (meta, s, selection) in zip(golden, regenerated):
        assert record["kind"] == meta["kind"]
        assert hashlib.sha256(memoryview(s)).hexdigest() == record["input_scores_sha256"]
        assert hashlib.sha256(memoryview(selection)).hexdigest() == record["input_selection_sha256"]
        ids = topk_indices(selection, 6)
        assert ids.tolist() == record["reference_indices"], meta
        _, _, w = route_weights(s, ids, 1.5)
        assert w.view(np.uint32).tolist() == record["reference_weight_bits"], meta
        assert tie_flag(selection, 6) == record["candidate_tie_flag"], meta


@pytest.mark.parametrize("experts,k", [(256, 8), (384, 6), (64, 4), (32, 32)])
def test_untied_selection_is_a_descending_sort(experts, k):
    rng = np.random.default_rng(experts * 100 + k)
    for _ in range(20):
        selection = rng.permutation(experts).astype(np.float32) - experts / 2
        ids = topk_indices(selection, k)
        np.testing.assert_array_equal(ids, np.argsort(-selection, kind="stable")[:k])


def test_tied_selection_takes_lowest_ids_at_the_threshold():
    selection = np.zeros(256, np.float32)
    selection[[200, 100]] = 1.0
    ids = topk_indices(selection, 8)
    assert set(ids.tolist()) == {100, 200, 0, 1, 2, 3, 4, 5}
    assert set(ids[:2].tolist()) == {100, 200}


def test_ordered_keys_follow_float_order():
    values = np.array([-np.inf, -3e38, -1.0, -1e-45, -0.0, 0.0, 1e-45, 1.0, 3e38, np.inf], np.float32)
    keys = ordered_keys(values)
    assert (np.diff(keys.astype(np.int64)) > 0).all()


def test_tree_sum_order_for_six_and_eight_terms():
    r = np.array([2.0 ** 24, 1.0, 1.0, 1.0, 1.0, 1.0, 1.0, 1.0], np.float32)
    # k=6: ((r0+r4)+r2) + ((r1+r5)+r3): r0+r4 rounds to 2^24, +r2 rounds again; right side 3
    assert tree_sum(r[:6]) == np.float32(np.float32(np.float32(r[0] + r[4]) + r[2]) + np.float32(3))
    assert tree_sum(r) == np.float32(np.float32(np.float32(r[0] + r[4]) + np.float32(r[2] + r[6]))
                                     + np.float32(np.float32(r[1] + r[5]) + np.float32(r[3] + r[7])))
    assert tree_sum(np.array([5.0], np.float32)) == 5.0


def test_sigmoid_and_sqrtsoftplus_scores():
    z = np.array([-200, -20, -1, 0, 1, 20, 20.5, 200], np.float32)
    sig = scores(z, "sigmoid")
    np.testing.assert_allclose(sig, (1 / (1 + np.exp(-z.astype(np.float64)))).astype(np.float32), rtol=2 ** -22)
    assert sig[0] == 0.0 and sig[-1] == 1.0 and sig[3] == 0.5
    ssp = scores(z, "sqrtsoftplus")
    softplus = np.where(z > 20, z, np.log1p(np.exp(z.astype(np.float64)))).astype(np.float32)
    ref = np.sqrt(softplus.astype(np.float64)).astype(np.float32)
    np.testing.assert_allclose(ssp, ref, rtol=2 ** -22)


def test_gate_logits_and_route_shapes():
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((256, 512)) * 0.02).astype(np.float32)
    x = rng.standard_normal((4, 512)).astype(np.float32)
    logits = gate_logits(w, x)
    np.testing.assert_allclose(logits, x.astype(np.float64) @ w.astype(np.float64).T, rtol=1e-6, atol=1e-7)
    r = route(logits, 8, 2.5)
    assert r["indices"].shape == (4, 8) and r["weights"].shape == (4, 8)
    np.testing.assert_allclose(r["weights"].sum(1), 2.5, rtol=1e-6)
    for row in range(4):
        assert len(set(r["indices"][row].tolist())) == 8
