"""Synthetic workload generators (inputs only; nothing here checks results)."""

from __future__ import annotations

import numpy as np


def zipf_routing(rng, tokens: int, experts: int, top_k: int, s: float = 1.1, route_scale: float = 2.5):
    """Prefill routing with Zipf(s) skew over a random permutation of the experts:
    expert perm[r] is drawn with probability proportional to 1 / (r + 1)^s; each token takes top_k distinct
    experts. Route weights: uniform positive scores normalized per token, times route_scale (the shape of
    the sigmoid router's weights). Returns int32 indices [T, k] and FP32 weights [T, k]."""
    perm = rng.permutation(experts)
    p = 1.0 / np.arange(1, experts + 1, dtype=np.float64) ** s
    p /= p.sum()
    prob = np.empty(experts)
    prob[perm] = p
    idx = np.empty((tokens, top_k), np.int32)
    for t in range(tokens):
        idx[t] = rng.choice(experts, size=top_k, replace=False, p=prob)
    raw = rng.uniform(0.05, 1.0, (tokens, top_k)).astype(np.float32)
    w = (raw / raw.sum(axis=1, keepdims=True) * np.float32(route_scale)).astype(np.float32)
    return idx, w
