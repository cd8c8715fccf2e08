"""Host side of the MoE participation and accumulator interface (vesper_amd.moe), no GPU.

participation() is called exactly as the reference's callers call it -- `participation(ids.reshape(1, 6),
max_tokens=1)` (src/vesper/connected.py:148) and `participation(ids, self.max_tokens)`
(src/vesper/moe.py:99,138) -- and compared with a brute-force grouping. The accumulator's refusals are
checked on a recording stand-in for the device: each must come before any library call.
"""

import itertools

import numpy as np
import pytest

from vesper_amd import moe
from vesper_amd.moe import MoEAccumulator, participation


def brute_force(ids):
    out = {}
    for e in sorted({int(v) for v in np.asarray(ids).ravel()}):
        out[e] = [t for t in range(len(ids)) if e in set(int(v) for v in ids[t])]
    return out


def as_lists(groups):
    return {e: rows.tolist() for e, rows in groups.items()}


def test_reference_call_forms_use_the_pinned_model():
    rng = np.random.default_rng(20261018)
    one = rng.choice(384, 6, replace=False).astype(np.int64)
    got = participation(one.reshape(1, 6), max_tokens=1)                 # connected.py:148
    assert list(got) == sorted(one.tolist()) and all(r.tolist() == [0] for r in got.values())
    assert all(r.dtype == np.int32 for r in got.values())
    ids = np.stack([rng.choice(384, 6, replace=False) for _ in range(32)]).astype(np.int32)
    assert as_lists(participation(ids, 32)) == brute_force(ids)         # moe.py:99,138
    with pytest.raises(ValueError, match="at most 1 tokens with six"):
        participation(ids[:2], max_tokens=1)
    with pytest.raises(ValueError, match="outside the pinned model"):
        participation(np.array([[0, 1, 2, 3, 4, 384]]), 1)


@pytest.mark.parametrize("experts,k,tokens", [(16, 4, 9), (256, 8, 16), (8, 8, 5), (3, 1, 7)])
def test_grouping_matches_brute_force_for_other_models(experts, k, tokens):
    rng = np.random.default_rng(experts * 100 + k)
    ids = np.stack([rng.choice(experts, k, replace=False) for _ in range(tokens)]).astype(np.int64)
    got = participation(ids, tokens, experts=experts, top_k=k)
    assert list(got) == sorted(got)
    assert as_lists(got) == brute_force(ids)
    assert sum(len(r) for r in got.values()) == tokens * k


def test_empty_routing_gives_no_experts():
    assert participation(np.empty((0, 6), np.int64)) == {}


def test_refusals_in_the_reference_order():
    good = np.array([[5, 1, 9, 2, 7, 3]], np.int64)
    for bad in (good.astype(np.float32), good.astype(np.uint32), good[0], good[:, :5], np.tile(good, (33, 1))):
        with pytest.raises(ValueError, match="integer expert IDs"):
            participation(bad)
    with pytest.raises(ValueError, match="outside the pinned model"):
        participation(np.array([[5, 1, 9, 2, 7, -1]]))
    for i, j in itertools.combinations(range(6), 2):
        dup = good.copy()
        dup[0, j] = dup[0, i]
        with pytest.raises(ValueError, match="Repeated expert IDs"):
            participation(dup)
    # a repeated id across tokens is fine
    assert participation(np.array([[1, 2, 3, 4, 5, 6], [6, 5, 4, 3, 2, 1]]))[6].tolist() == [0, 1]


class RecordingLib:
    def __init__(self):
        self.calls = []

    def __getattr__(self, name):
        return lambda *args: self.calls.append(name)


class StubArray:
    def __init__(self, ptr):
        self.ptr = ptr

    def __int__(self):
        return self.ptr


class StubContext:
    """Device context stand-in: allocations are addresses, transfers and launches are recorded."""

    def __init__(self, ordinal=0):
        self.lib, self.next = RecordingLib(), 0x10000

    def _h(self):
        return 1

    def empty(self, shape, dtype):
        self.next += 1 << 24
        return StubArray(self.next)

    def copy_h2d(self, dst, array, stream=None):
        self.lib.calls.append("h2d")

    def download(self, src, shape, dtype, stream=None):
        self.lib.calls.append("d2h")
        return np.zeros(shape, dtype)

    def close(self):
        pass


@pytest.fixture
def accumulator(monkeypatch):
    monkeypatch.setattr(moe._lib, "Context", StubContext)
    with MoEAccumulator(0, 4) as acc:
        yield acc


def test_accumulator_enforces_ascending_order_and_shared_last(accumulator):
    acc, lib = accumulator, accumulator.ctx.lib
    ids = np.array([[10, 3, 7, 1, 2, 4], [3, 8, 1, 2, 11, 5]], np.int64)
    acc.begin(ids)
    assert acc.state == "routed"
    rows = lambda n: np.zeros((n, 5120), np.uint16)
    with pytest.raises(ValueError, match="ascending expert-ID order"):
        acc.add(2, rows(2))                      # expert 1 comes first
    with pytest.raises(ValueError, match="ascending expert-ID order"):
        acc.add(np.int64(1), rows(2))            # ids are Python ints
    with pytest.raises(ValueError, match="precede the shared expert"):
        acc.finish(rows(2))
    before = len(lib.calls)
    with pytest.raises(ValueError, match=r"participating_tokens, 5120"):
        acc.add(1, rows(1))                      # expert 1 has two rows
    with pytest.raises(ValueError, match="finite"):
        acc.add(1, np.full((2, 5120), 0x7F80, np.uint16))
    assert len(lib.calls) == before
    for e in (1, 2, 3, 4, 5, 7, 8, 10, 11):
        acc.add(e, rows(len(participation(ids)[e])))
    with pytest.raises(ValueError, match="ascending expert-ID order"):
        acc.add(12, rows(1))
    stages = acc.finish(rows(2))
    assert set(stages) == {"before_shared_fp32", "after_shared_fp32", "output_bf16"}
    assert acc.state == "finished"
    with pytest.raises(ValueError, match="ascending expert-ID order"):
        acc.add(1, rows(2))


def test_run_validates_the_whole_call_before_the_device(accumulator):
    acc, lib = accumulator, accumulator.ctx.lib
    ids = np.array([[1, 2, 3, 4, 5, 6]], np.int64)
    contributions = {e: np.zeros((1, 5120), np.uint16) for e in range(1, 7)}
    before = len(lib.calls)
    with pytest.raises(ValueError, match="exactly the selected"):
        acc.run(ids, {e: v for e, v in contributions.items() if e != 6}, np.zeros((1, 5120), np.uint16))
    with pytest.raises(ValueError, match="exactly the selected"):
        acc.run(ids, {np.int64(e): v for e, v in contributions.items()}, np.zeros((1, 5120), np.uint16))
    bad = dict(contributions)
    bad[6] = np.zeros((2, 5120), np.uint16)
    with pytest.raises(ValueError, match="participating_tokens"):
        acc.run(ids, bad, np.zeros((1, 5120), np.uint16))
    with pytest.raises(ValueError, match="participating_tokens"):
        acc.run(ids, contributions, np.zeros((1, 5119), np.uint16))
    assert len(lib.calls) == before
    stages = acc.run(ids, contributions, np.zeros((1, 5120), np.uint16))
    assert list(stages)[:6] == [f"after_expert_{e}_fp32" for e in range(1, 7)]


def test_accumulator_lifecycle():
    acc = MoEAccumulator()
    assert acc.state == "closed"
    with pytest.raises(RuntimeError, match="context manager"):
        acc.begin(np.array([[1, 2, 3, 4, 5, 6]]))
    for bad in (0, 4097, 2.0, True):
        with pytest.raises(ValueError, match="workspace supports"):
            MoEAccumulator(0, bad)


def test_offload_trace_repeats_each_slot_with_probability_0_6():
    """BASELINE configuration 4's routing: a token keeps each of its previous 8 experts with probability 0.6
    (independently per slot), every step's experts are distinct, and the replacements are experts it did not
    use at the previous step. 200 steps x 4 tokens x 2 layers: the mean repeat fraction is within 3 standard
    errors of 0.6, and a repeat of exactly 5 of 8 is not forced."""
    from vesper_amd.offload_workload import trace

    tr = trace(np.random.default_rng(7), 200, 2, 4, 256, 8)
    kept = []
    for s in range(1, 200):
        for layer in range(2):
            for t in range(4):
                now, before = tr[s][layer][0][t], tr[s - 1][layer][0][t]
                assert len(set(now.tolist())) == 8
                kept.append(len(set(now.tolist()) & set(before.tolist())))
    kept = np.asarray(kept)
    se = np.sqrt(0.6 * 0.4 / (8 * kept.size))
    assert abs(kept.mean() / 8 - 0.6) < 3 * se
    assert len(np.unique(kept)) > 3          # binomial spread, not a fixed count
