"""Participation and ordered accumulation (mirrors src/vesper/moe.py:18-160).

participation(indices) -> {expert: ascending token rows}, experts ascending,
with the reference's refusals. MoEAccumulator(ordinal, max_tokens) runs
begin / add (ascending expert order only) / finish / run on the device with
the acc_* kernels: FP32 zero, FP32 adds of BF16 contributions, shared last,
one BF16 rounding. All validation happens before any device call.
"""

from __future__ import annotations

import numpy as np

from . import _lib

MiB = 1 << 20


def participation(indices, experts: int = 256, top_k: int = 8, max_tokens: int = 32) -> dict:
    indices = np.asarray(indices)
    if (indices.dtype not in (np.dtype(np.int32), np.dtype(np.int64)) or indices.ndim != 2
            or indices.shape[1] != top_k or indices.shape[0] > max_tokens):
        raise ValueError(f"Expected at most {max_tokens} tokens with {top_k} integer expert IDs each")
    if np.any(indices < 0) or np.any(indices >= experts):
        raise ValueError("Expert ID is outside the model")
    if top_k > 1 and np.any(np.diff(np.sort(indices, axis=1), axis=1) == 0):
        raise ValueError("Repeated expert IDs within a token are outside the unique-topk scope")
    selected = {}
    for expert in np.unique(indices):
        selected[int(expert)] = np.flatnonzero((indices == expert).any(axis=1)).astype(np.int32)
    return selected


def _bf16_output(array, tokens: int, hidden: int):
    array = np.asarray(array)
    if array.dtype != np.uint16 or array.shape != (tokens, hidden):
        raise ValueError(f"Expected BF16 storage bits with shape (participating_tokens, {hidden})")
    if np.any((array & np.uint16(0x7F80)) == np.uint16(0x7F80)):
        raise ValueError("Expert output must be finite in this probe")
    return np.ascontiguousarray(array)


class MoEAccumulator:
    """Add BF16 expert outputs in ID order and the shared output last; never weights them."""

    def __init__(self, ordinal=0, max_tokens=32, *, hidden=7168, experts=256, top_k=8):
        if type(max_tokens) is not int or not 1 <= max_tokens <= 4096:
            raise ValueError("Aggregation workspace supports one to 4096 tokens")
        self.ordinal, self.max_tokens = ordinal, max_tokens
        self.hidden, self.experts, self.top_k = hidden, experts, top_k
        self.ctx, self.state = None, "closed"

    def __enter__(self):
        if self.ctx is not None:
            raise RuntimeError("Accumulator is already open")
        self.ctx = _lib.Context(self.ordinal)
        try:
            count = self.max_tokens * self.hidden
            self.work = {"sum": self.ctx.empty((count,), np.float32), "input": self.ctx.empty((count,), np.uint16),
                         "rows": self.ctx.empty((self.max_tokens,), np.int32),
                         "output": self.ctx.empty((count,), np.uint16)}
            self.state = "ready"
            return self
        except BaseException:
            self.close()
            raise

    def _open(self):
        if self.ctx is None:
            raise RuntimeError("Use the accumulator as a context manager")

    def _snapshot(self):
        if not self.tokens:
            return np.empty((0, self.hidden), np.float32)
        return self.ctx.download(self.work["sum"].ptr, (self.tokens, self.hidden), np.float32)

    def begin(self, indices):
        self._open()
        selected = participation(indices, self.experts, self.top_k, self.max_tokens)
        self.tokens = np.asarray(indices).shape[0]
        self.selected, self.order, self.position = selected, list(selected), 0
        self.ctx.lib.acc_zero(self.ctx._h(), _lib.vp(self.work["sum"]), self.tokens * self.hidden, None)
        self.state = "routed"

    def add(self, expert_id, output):
        self._open()
        if (self.state != "routed" or self.position >= len(self.order)
                or type(expert_id) is not int or expert_id != self.order[self.position]):
            raise ValueError("Contributions must follow the selected ascending expert-ID order")
        rows = self.selected[expert_id]
        output = _bf16_output(output, len(rows), self.hidden)
        self.ctx.copy_h2d(self.work["input"].ptr, output)
        self.ctx.copy_h2d(self.work["rows"].ptr, rows.astype(np.int32))
        self.ctx.lib.acc_add_rows(self.ctx._h(), _lib.vp(self.work["sum"]), _lib.vp(self.work["input"]),
                                  _lib.vp(self.work["rows"]), len(rows), self.hidden, None)
        self.position += 1
        return self._snapshot()

    def finish(self, shared):
        self._open()
        if self.state != "routed" or self.position != len(self.order):
            raise ValueError("All selected expert contributions must precede the shared expert")
        shared = _bf16_output(shared, self.tokens, self.hidden)
        before = self._snapshot()
        count = self.tokens * self.hidden
        self.ctx.copy_h2d(self.work["input"].ptr, shared)
        self.ctx.lib.acc_add(self.ctx._h(), _lib.vp(self.work["sum"]), _lib.vp(self.work["input"]), count, None)
        after = self._snapshot()
        self.ctx.lib.acc_finish(self.ctx._h(), _lib.vp(self.work["sum"]), _lib.vp(self.work["output"]), count, None)
        output = (self.ctx.download(self.work["output"].ptr, (self.tokens, self.hidden), np.uint16)
                  if self.tokens else np.empty((0, self.hidden), np.uint16))
        self.state = "finished"
        return {"before_shared_fp32": before, "after_shared_fp32": after, "output_bf16": output}

    def run(self, indices, contributions: dict, shared) -> dict:
        selected = participation(indices, self.experts, self.top_k, self.max_tokens)
        if set(contributions) != set(selected) or any(type(k) is not int for k in contributions):
            raise ValueError("Supply exactly the selected expert contributions")
        shared = _bf16_output(shared, np.asarray(indices).shape[0], self.hidden)
        for expert, rows in selected.items():
            _bf16_output(contributions[expert], len(rows), self.hidden)
        self.begin(indices)
        stages = {f"after_expert_{e}_fp32": self.add(e, contributions[e]) for e in self.order}
        stages.update(self.finish(shared))
        return stages

    def close(self):
        try:
            if self.ctx is not None:
                self.ctx.close()
        finally:
            self.ctx, self.state = None, "closed"

    def __exit__(self, *_):
        self.close()
