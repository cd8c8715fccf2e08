"""Participation, ordered combine, and the whole routed MoE layer (CPU oracle, test infrastructure only).

  participation  src/vesper/moe.py:18-30   {expert: ascending token rows}, experts ascending;
                                           refuses bad dtype/shape, out-of-range and repeated IDs
  combine        src/vesper/moe.py:42-148, src/vesper/kernels/aggregation_probe.cu:1-25
                 FP32 zero; per expert in ascending ID: sum[rows] += FP32(BF16 output);
                 then += FP32(BF16 shared); one final BF16 rounding
  moe_layer      src/vesper/connected.py:125-186 order: gate -> router -> participation ->
                 routed experts (weight applied before W2) -> shared expert -> combine
  moe_layer_routed  the same after the router, on given indices and route weights (prefill workloads
                 whose routing is drawn, e.g. Zipf-skewed)
"""

from __future__ import annotations

import numpy as np

from .expert import expert_forward
from .formats import bf16_bits, bf16_round, bf16_values
from .router import gate_logits, route


def participation(indices, experts: int, top_k: int, max_tokens: int = 4096) -> dict:
    indices = np.asarray(indices)
    if (indices.dtype not in (np.dtype(np.int32), np.dtype(np.int64)) or indices.ndim != 2
            or indices.shape[1] != top_k or indices.shape[0] > max_tokens):
        raise ValueError(f"Expected at most {max_tokens} tokens with {top_k} integer expert IDs each")
    if np.any(indices < 0) or np.any(indices >= experts):
        raise ValueError("Expert ID is outside the model")
    if np.any(np.diff(np.sort(indices, axis=1), axis=1) == 0):
        raise ValueError("Repeated expert IDs within a token are outside the unique-topk scope")
    return {int(e): np.flatnonzero(np.any(indices == e, axis=1)).astype(np.int32) for e in np.unique(indices)}


def combine(indices, contributions: dict, shared, experts: int, top_k: int) -> dict:
    """Every FP32 stage of the ordered combine, keyed like MoEAccumulator.run (moe.py:137-148)."""
    selected = participation(indices, experts, top_k)
    shared = np.asarray(shared, dtype=np.uint16)
    tokens = np.asarray(indices).shape[0]
    hidden = shared.shape[-1]
    total = np.zeros((tokens, hidden), np.float32)
    stages = {}
    for expert, rows in selected.items():
        total[rows] = (total[rows] + bf16_values(contributions[expert])).astype(np.float32)
        stages[f"after_expert_{expert}_fp32"] = total.copy()
    stages["before_shared_fp32"] = total.copy()
    total = (total + bf16_values(shared)).astype(np.float32)
    stages["after_shared_fp32"] = total.copy()
    stages["output_bf16"] = bf16_bits(total)
    return stages


def moe_layer(x, router_weight, experts: dict, shared: dict | None, *, top_k: int, route_scale: float,
              score_func: str = "sigmoid", bias=None, swiglu_limit: float = 0.0,
              shared_format: str = "mxfp4", logits=None) -> dict:
    """One routed MoE layer over T tokens. `experts` maps expert ID -> six tensors.

    `logits` may be supplied (e.g. the kernel's own) so that selection parity is
    checked on identical inputs, as RouterProbe.inspect does (router.py:227-241).
    """
    x = bf16_round(np.atleast_2d(np.asarray(x, dtype=np.float32)))
    n_experts = np.asarray(router_weight).shape[0]
    if logits is None:
        logits = gate_logits(router_weight, x)
    routing = route(logits, top_k, route_scale, score_func, bias)
    selected = participation(routing["indices"], n_experts, top_k)
    outputs = {}
    for expert, rows in selected.items():
        ranks = [int(np.flatnonzero(routing["indices"][r] == expert)[0]) for r in rows]
        weights = routing["weights"][rows, ranks]
        outputs[expert] = expert_forward(x[rows], experts[expert], weights, swiglu_limit)
    tokens, hidden = x.shape
    if shared is not None:
        shared_out = expert_forward(x, shared, None, swiglu_limit, shared_format)
        shared_bits = shared_out["w2"]
    else:
        shared_out, shared_bits = None, np.zeros((tokens, hidden), np.uint16)
    aggregation = combine(routing["indices"], {e: o["w2"] for e, o in outputs.items()}, shared_bits,
                          n_experts, top_k)
    return {"input_bf16": bf16_bits(x), "logits": routing["logits"], "routing": routing, "experts": outputs,
            "shared": shared_out, "aggregation": aggregation, "output_bf16": aggregation["output_bf16"]}


def moe_layer_routed(x, indices, weights, experts: dict, shared: dict | None, *, num_experts: int,
                     swiglu_limit: float = 0.0, shared_format: str = "mxfp4", tokens=None) -> dict:
    """The layer after routing, on given `indices` [T, k] and `weights` [T, k]; `tokens` (optional) limits the
    work to those tokens' rows (the result then covers only them, in that order). `experts` maps the
    needed expert IDs to their six tensors."""
    x = bf16_round(np.atleast_2d(np.asarray(x, dtype=np.float32)))
    sel = np.arange(x.shape[0]) if tokens is None else np.asarray(tokens)
    idx = np.asarray(indices)[sel]
    wts = np.asarray(weights, dtype=np.float32)[sel]
    xs = x[sel]
    selected = participation(idx, num_experts, idx.shape[1], max_tokens=max(len(sel), 1))
    outputs = {}
    for expert, rows in selected.items():
        ranks = [int(np.flatnonzero(idx[r] == expert)[0]) for r in rows]
        outputs[expert] = expert_forward(xs[rows], experts[expert], wts[rows, ranks], swiglu_limit)
    if shared is not None:
        shared_bits = expert_forward(xs, shared, None, swiglu_limit, shared_format)["w2"]
    else:
        shared_bits = np.zeros(xs.shape, np.uint16)
    aggregation = combine(idx, {e: o["w2"] for e, o in outputs.items()}, shared_bits, num_experts, idx.shape[1])
    return {"experts": outputs, "aggregation": aggregation, "output_bf16": aggregation["output_bf16"]}
