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


def test_untied_and_edge_selections_against_the_oracle():
    """Untied selections are ranked by the threshold rounds themselves; a zero among the winners (where
    +0 and -0 are distinct keys but equal floats, so the sorting network decides their order), ties,
    negative values, subnormals and winners one ULP apart are covered too: indices, weights and the tie
    flag bit-exact against the oracle in every case."""
    from oracle.router import route_weights, topk_indices
    rng = np.random.default_rng(3131)
    k, scale = 8, 2.5
    rows = []
    for case in range(12):
        sel = rng.standard_normal(256).astype(np.float32)
        if case in (1, 2, 3):
            sel = -np.abs(sel)
            lo, hi = (4, 9) if case != 2 else (9, 4)
            sel[lo] = np.float32(0.0)              # +0 and -0 both win; by key +0 ranks first
            sel[hi] = np.float32(-0.0)
            if case == 3:
                sel[hi] = sel[lo]                  # a single zero among the winners
        elif case == 4:
            sel = -np.abs(sel)                     # all negative
        elif case == 5:
            sel = (sel * np.float32(1e-39)).astype(np.float32)    # subnormals of both signs
        elif case == 6:
            top = np.argsort(sel)[::-1][:9]
            v = np.float32(0.75)
            for e in top:                          # nine winners one ULP apart, descending by ID order
                sel[e] = v
                v = np.nextafter(v, np.float32(0.0), dtype=np.float32)
        elif case == 7:
            top = np.argsort(sel)[::-1]
            sel[top[8]] = sel[top[7]]              # the k-th value shared with an unselected expert
        elif case == 8:
            top = np.argsort(sel)[::-1]
            sel[top[3]] = sel[top[1]]              # a tie inside the winners
        rows.append(sel)
    selection = np.stack(rows)
    scores = rng.uniform(0.01, 1.0, selection.shape).astype(np.float32)
    with RouterProbe(experts=256, top_k=k, score_func="sigmoid", route_scale=scale) as probe:
        got = probe.inspect_selection(scores, selection)
    for row in range(len(rows)):
        ids = topk_indices(selection[row], k)
        _, _, weights = route_weights(scores[row], ids, scale)
        assert got["indices"][row].tolist() == ids.tolist(), row
        np.testing.assert_array_equal(got["weights"][row].view(np.uint32), weights.view(np.uint32), err_msg=str(row))
        assert bool(got["tied"][row]) == tie_flag(selection[row], k), row


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


def test_selection_handover_at_every_round():
    """The device ranks untied winners over each lane's sorted keys (4 experts per lane at E = 256) and
    hands over to the threshold search from the start at the first round whose value is tied, a zero or
    below every winner. Every hand-over position is covered: the values at places r and r + 1 of the
    ranking (from 0; r = 7: the k-th winner and the first loser; r = 8 and 9: below the cut, no hand-over)
    are a tie between two lanes, a tie inside one lane, a +0 / -0 pair, or a +0 above a negative value.
    Indices, weights and the tie flag bit-exact against the oracle in every row."""
    from oracle.router import route_weights, topk_indices
    rng = np.random.default_rng(4242)
    k, scale, experts = 8, 2.5, 256
    rows = []
    for r in range(10):
        for pattern in ("two lanes", "one lane", "signed zeros", "zero above negative"):
            perm = rng.permutation(experts)
            partner = (perm[r] + 4) % experts if pattern == "two lanes" else perm[r] ^ 1
            if pattern in ("two lanes", "one lane"):
                j = int(np.flatnonzero(perm == partner)[0])
                perm[[r + 1, j]] = perm[[j, r + 1]]
                assert (perm[r] // 4 == perm[r + 1] // 4) == (pattern == "one lane")
            sel = np.empty(experts, np.float32)
            if pattern in ("two lanes", "one lane"):
                sel[perm] = (1.0 - np.arange(experts) / 512.0).astype(np.float32)
                sel[perm[r + 1]] = sel[perm[r]]
            else:
                pos = np.arange(experts)
                vals = np.where(pos < r, 0.5 - pos / 1024.0, -(pos + 1) / 1024.0).astype(np.float32)
                vals[r] = np.float32(0.0)
                if pattern == "signed zeros":
                    vals[r + 1] = np.float32(-0.0)
                sel[perm] = vals
            rows.append(sel)
    selection = np.stack(rows)
    scores = rng.uniform(0.01, 1.0, selection.shape).astype(np.float32)
    with RouterProbe(experts=experts, top_k=k, score_func="sigmoid", route_scale=scale) as probe:
        got = probe.inspect_selection(scores, selection)
    for row in range(len(rows)):
        ids = topk_indices(selection[row], k)
        _, _, weights = route_weights(scores[row], ids, scale)
        assert got["indices"][row].tolist() == ids.tolist(), row
        np.testing.assert_array_equal(got["weights"][row].view(np.uint32), weights.view(np.uint32), err_msg=str(row))
        assert bool(got["tied"][row]) == tie_flag(selection[row], k), row
