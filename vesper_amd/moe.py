"""Participation and ordered accumulation behind the reference's MoE interface (src/vesper/moe.py:18-160).

`participation(indices, max_tokens)` turns a [T, k] routing table into {expert: ascending token rows} with
the experts ascending -- the same plan the decode and prefill kernels build on the device (expert-major
rows, tokens ascending within an expert). Here it is made by one stable sort of the T k (expert, token)
pairs; the refusals are the reference's (same exception classes and messages).

`MoEAccumulator` is the stepwise form of the device combine. `begin` fixes the plan and uploads every
expert's token rows at once as one expert-major row table; each `add` then uploads one BF16 contribution
and adds it into the FP32 sum at its slice of that table; `finish` adds the shared rows and rounds once to
BF16. The order is enforced by a cursor over the plan, so contributions arrive in ascending expert ID and
the shared expert last, as the reference requires. All validation happens before any device call.

The model shape defaults to the reference's pinned model (hidden 5120, 384 experts, top-6: the
constants of src/vesper/moe.py:13-15); other shapes are passed explicitly.
"""

from __future__ import annotations

import numpy as np

from . import _lib
from .config import REFERENCE

PINNED_HIDDEN, PINNED_EXPERTS, PINNED_TOP_K = REFERENCE.hidden, REFERENCE.experts, REFERENCE.top_k
_COUNT_WORDS = {1: "one", 2: "two", 3: "three", 4: "four", 5: "five", 6: "six", 7: "seven", 8: "eight"}


def _routing_table(indices, max_tokens: int, experts: int, top_k: int) -> np.ndarray:
    """The [T, k] id table as int64 after the reference's three refusals (moe.py:18-27)."""
    table = np.asarray(indices)
    integral = table.dtype in (np.dtype(np.int32), np.dtype(np.int64))
    if not integral or table.ndim != 2 or table.shape[1] != top_k or table.shape[0] > max_tokens:
        count = _COUNT_WORDS.get(top_k, str(top_k))
        raise ValueError(f"Expected at most {max_tokens} tokens with {count} integer expert IDs each")
    table = table.astype(np.int64, copy=False)
    if table.size and (int(table.min()) < 0 or int(table.max()) >= experts):
        raise ValueError("Expert ID is outside the pinned model")
    return table


def participation(indices, max_tokens=32, *, experts: int = PINNED_EXPERTS, top_k: int = PINNED_TOP_K) -> dict:
    """{expert id: int32 token rows ascending}, expert ids ascending (src/vesper/moe.py:18-30).

    Positional arguments are the reference's (`participation(ids, max_tokens)`); the model's expert count
    and k are keyword-only and default to the reference's pinned model."""
    table = _routing_table(indices, max_tokens, experts, top_k)
    tokens, k = table.shape
    expert_of_pair = table.reshape(-1)
    token_of_pair = np.repeat(np.arange(tokens, dtype=np.int64), k)
    # one sort key per pair: expert-major, token-minor (tokens < 2^32 and ids < 2^31 fit in 63 bits)
    order = np.argsort((expert_of_pair << 32) | token_of_pair, kind="stable")
    by_expert, by_token = expert_of_pair[order], token_of_pair[order]
    if by_expert.size > 1 and np.any((by_expert[1:] == by_expert[:-1]) & (by_token[1:] == by_token[:-1])):
        # a token naming one expert twice (the unique top-k returns distinct ids)
        raise ValueError("Repeated expert IDs within a token are outside the unique-topk scope")
    starts = np.flatnonzero(np.r_[True, by_expert[1:] != by_expert[:-1]]) if by_expert.size else np.empty(0, int)
    ends = np.r_[starts[1:], by_expert.size]
    return {int(by_expert[s]): by_token[s:e].astype(np.int32) for s, e in zip(starts, ends)}


def _expert_rows(array, tokens: int, hidden: int) -> np.ndarray:
    """A contribution as contiguous BF16 bits [tokens, hidden], finite (moe.py:33-38)."""
    rows = np.asarray(array)
    if rows.dtype != np.uint16 or rows.shape != (tokens, hidden):
        raise ValueError(f"Expected BF16 storage bits with shape (participating_tokens, {hidden})")
    exponent_all_ones = (rows & np.uint16(0x7F80)) == np.uint16(0x7F80)
    if exponent_all_ones.any():
        raise ValueError("Expert output must be finite in this probe")
    return np.ascontiguousarray(rows)


class _Plan:
    """One accumulation's routing: experts ascending, their row slices in one expert-major table."""

    def __init__(self, selected: dict, tokens: int):
        self.tokens = tokens
        self.experts = list(selected)
        sizes = [len(selected[e]) for e in self.experts]
        self.first = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64)
        self.table = (np.concatenate([selected[e] for e in self.experts]).astype(np.int32)
                      if self.experts else np.empty(0, np.int32))
        self.cursor = 0

    def expect(self, expert_id) -> tuple[int, int]:
        """(first row, row count) of the next contribution if it is `expert_id`; ValueError otherwise."""
        if (self.cursor >= len(self.experts) or type(expert_id) is not int
                or expert_id != self.experts[self.cursor]):
            raise ValueError("Contributions must follow the selected ascending expert-ID order")
        return int(self.first[self.cursor]), int(self.first[self.cursor + 1] - self.first[self.cursor])

    @property
    def complete(self) -> bool:
        return self.cursor == len(self.experts)


class MoEAccumulator:
    """FP32 device sum of BF16 expert outputs in ascending expert ID, shared output last, one BF16 rounding
    (src/vesper/moe.py:42-160). It never weights a contribution: route weights act before W2."""

    def __init__(self, ordinal=0, max_tokens=32, *, hidden: int = PINNED_HIDDEN, experts: int = PINNED_EXPERTS,
                 top_k: int = PINNED_TOP_K):
        if type(max_tokens) is not int or not 1 <= max_tokens <= 4096:
            raise ValueError("Aggregation workspace supports one to 4096 tokens")
        self.ordinal, self.max_tokens = ordinal, max_tokens
        self.hidden, self.experts, self.top_k = hidden, experts, top_k
        self.ctx, self.plan, self.buffers = None, None, {}

    # -- lifetime -----------------------------------------------------------------------------
    def __enter__(self):
        if self.ctx is not None:
            raise RuntimeError("Accumulator is already open")
        ctx = _lib.Context(self.ordinal)
        try:
            elements = self.max_tokens * self.hidden
            self.buffers = {"sum": ctx.empty((elements,), np.float32),
                            "rows_in": ctx.empty((elements,), np.uint16),
                            "row_table": ctx.empty((self.max_tokens * self.top_k,), np.int32),
                            "out": ctx.empty((elements,), np.uint16)}
        except BaseException:
            ctx.close()
            raise
        self.ctx = ctx
        return self

    def close(self):
        ctx, self.ctx, self.plan, self.buffers = self.ctx, None, None, {}
        if ctx is not None:
            ctx.close()

    def __exit__(self, *_):
        self.close()

    @property
    def state(self) -> str:
        if self.ctx is None:
            return "closed"
        if self.plan is None:
            return "ready"
        return "finished" if self.plan.cursor < 0 else "routed"

    def _device(self) -> _lib.Context:
        if self.ctx is None:
            raise RuntimeError("Use the accumulator as a context manager")
        return self.ctx

    def _sum_rows(self) -> np.ndarray:
        tokens = self.plan.tokens
        if tokens == 0:
            return np.empty((0, self.hidden), np.float32)
        return self.ctx.download(self.buffers["sum"].ptr, (tokens, self.hidden), np.float32)

    def _select(self, indices) -> dict:
        return participation(indices, self.max_tokens, experts=self.experts, top_k=self.top_k)

    # -- the reference's stepwise interface ----------------------------------------------------
    def begin(self, indices):
        """Fix the routing of one call and zero its FP32 rows."""
        ctx = self._device()
        selected = self._select(indices)
        plan = _Plan(selected, np.asarray(indices).shape[0])
        if plan.table.size:
            ctx.copy_h2d(self.buffers["row_table"].ptr, plan.table)
        ctx.lib.acc_zero(ctx._h(), _lib.vp(self.buffers["sum"]), plan.tokens * self.hidden, None)
        self.plan = plan

    def add(self, expert_id, output) -> np.ndarray:
        """Add the next expert's BF16 rows (ascending ID); returns the FP32 sum after it."""
        ctx = self._device()
        if self.plan is None or self.plan.cursor < 0:
            raise ValueError("Contributions must follow the selected ascending expert-ID order")
        first, count = self.plan.expect(expert_id)
        rows = _expert_rows(output, count, self.hidden)
        ctx.copy_h2d(self.buffers["rows_in"].ptr, rows)
        row_table = self.buffers["row_table"].ptr + 4 * first
        ctx.lib.acc_add_rows(ctx._h(), _lib.vp(self.buffers["sum"]), _lib.vp(self.buffers["rows_in"]),
                             _lib.vp(row_table), count, self.hidden, None)
        self.plan.cursor += 1
        return self._sum_rows()

    def finish(self, shared) -> dict:
        """Add the shared expert's rows last and round the sum to BF16 once."""
        ctx = self._device()
        if self.plan is None or self.plan.cursor < 0 or not self.plan.complete:
            raise ValueError("All selected expert contributions must precede the shared expert")
        tokens = self.plan.tokens
        shared = _expert_rows(shared, tokens, self.hidden)
        stages = {"before_shared_fp32": self._sum_rows()}
        elements = tokens * self.hidden
        ctx.copy_h2d(self.buffers["rows_in"].ptr, shared)
        ctx.lib.acc_add(ctx._h(), _lib.vp(self.buffers["sum"]), _lib.vp(self.buffers["rows_in"]), elements, None)
        stages["after_shared_fp32"] = self._sum_rows()
        ctx.lib.acc_finish(ctx._h(), _lib.vp(self.buffers["sum"]), _lib.vp(self.buffers["out"]), elements, None)
        stages["output_bf16"] = (ctx.download(self.buffers["out"].ptr, (tokens, self.hidden), np.uint16)
                                 if tokens else np.empty((0, self.hidden), np.uint16))
        self.plan.cursor = -1
        return stages

    def run(self, indices, contributions: dict, shared) -> dict:
        """The whole call at once; every argument is checked before the device is touched."""
        selected = self._select(indices)
        if set(contributions) != set(selected) or not all(type(e) is int for e in contributions):
            raise ValueError("Supply exactly the selected expert contributions")
        _expert_rows(shared, np.asarray(indices).shape[0], self.hidden)
        for expert, token_rows in selected.items():
            _expert_rows(contributions[expert], len(token_rows), self.hidden)
        self.begin(indices)
        stages = {}
        for expert in self.plan.experts:
            stages[f"after_expert_{expert}_fp32"] = self.add(expert, contributions[expert])
        stages.update(self.finish(shared))
        return stages
