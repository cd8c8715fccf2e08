"""GPU parity of the router: recorded PyTorch-CUDA selection goldens, tie goldens, sigmoid top-8 of 256."""

import hashlib
import json
from pathlib import Path

import numpy as np
import pytest

from oracle.inputs import router_weight, selection_cases
from oracle.router import gate_logits, route, scores as oracle_scores, tie_flag
from oracle.formats import bf16_bits, bf16_values
from tests.helpers import max_rel_err
from vesper_amd.router import GateProjection, RouterProbe

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden" / "router_selection.json"


def test_recorded_cuda_selection_goldens_on_device():
    golden = json.loads(GOLDEN.read_text())["cases"]
    cases = list(selection_cases())
    scores = np.stack([c[1] for c in cases])
    selection = np.stack([c[2] for c in cases])
    for record, (meta, s, sel) in zip(golden, cases):
        assert hashlib.sha256(memoryview(sel)).hexdigest() == record["input_selection_sha256"]
    with RouterProbe(experts=384, top_k=6, score_func="sqrtsoftplus", route_scale=1.5) as probe:
        got = probe.inspect_selection(scores, selection)
    for row, record in enumerate(golden):
        assert got["indices"][row].tolist() == record["reference_indices"], row
        assert got["weights"][row].view(np.uint32).tolist() == record["reference_weight_bits"], row
        assert bool(got["tied"][row]) == record["candidate_tie_flag"], row


def test_pinned_tie_order_goldens_on_device():
    with RouterProbe(experts=384, top_k=6, score_func="sqrtsoftplus", route_scale=1.5) as probe:
        s = np.linspace(0.0001, 30, 384, dtype=np.float32)
        for level in (0, -1, 1):
            got = probe.inspect_selection(s, np.full(384, level, np.float32))
            assert got["indices"].tolist() == [1, 0, 4, 5, 2, 3]
        got = probe.inspect_selection(s, np.resize(np.array([-0.0, 0.0], np.float32), 384))
        assert got["indices"].tolist() == [3, 1, 9, 11, 5, 7]


@pytest.mark.parametrize("score_func,experts,k,scale", [("sigmoid", 256, 8, 2.5), ("sqrtsoftplus", 384, 6, 1.5),
                                                        ("sigmoid", 64, 4, 1.0)])
def test_postprocess_matches_oracle_bit_exactly(score_func, experts, k, scale):
    rng = np.random.default_rng(experts + k)
    logits = (rng.standard_normal((40, experts)) * np.array([[0.5], [4.0], [16.0], [64.0]] * 10)).astype(np.float32)
    logits[0] = 0.0                               # all tied
    logits[1, ::2] = logits[1, 1::2]              # pairwise ties
    bias = (rng.standard_normal(experts) * 0.01).astype(np.float32)
    with RouterProbe({"bias": bias}, experts=experts, top_k=k, score_func=score_func, route_scale=scale) as probe:
        got = probe.inspect(logits)
    ref = route(logits, k, scale, score_func, bias)
    for name in ("scores", "selection", "raw", "denominator", "weights"):
        np.testing.assert_array_equal(got[name].view(np.uint32), ref[name].view(np.uint32), err_msg=name)
    np.testing.assert_array_equal(got["indices"], ref["indices"])
    assert [bool(v) for v in got["tied"]] == [tie_flag(ref["selection"][t], k) for t in range(40)]


def test_gate_projection_matches_float64_oracle():
    rng = np.random.default_rng(9)
    w = router_weight(rng, 256, 7168)
    x = bf16_values(bf16_bits(rng.standard_normal((5, 7168)).astype(np.float32)))
    with GateProjection(w) as gate:
        got = gate.project(x)
        single = gate.project(x[0])
    ref = gate_logits(w, x)
    assert max_rel_err(got, ref) < 1e-5
    np.testing.assert_array_equal(single, got[0])
    # BF16 gate weights are promoted exactly (gate.py:133)
    wb = bf16_bits(w)
    with GateProjection(wb) as gate:
        got = gate.project(x)
    assert max_rel_err(got, gate_logits(bf16_values(wb), x)) < 1e-5
