"""Gate projection, scores, top-k selection and route weights (CPU oracle, test infrastructure only).

Restates, generalised from the reference's fixed E=384 / k=6 / sqrtsoftplus / x1.5:
  gate_logits    gate.py:133-147, blas.py:70-73   FP32 W_r . FP32(x)   (textbook GEMV, float64 then FP32)
  scores         routing_probe.cu:5-15             sqrtsoftplus (softplus threshold 20) or sigmoid
  topk_indices   router.py:23-61, routing_probe.cu:17-86
                 order-preserving u32 keys; threshold = k-th largest; gather keys above the
                 threshold by ID, then keys equal to it by ID; then the 32-slot bitonic network
  route_weights  router.py:174-192, routing_probe.cu:78-84
                 raw = score[ids]; den = tree_sum(raw) + 1e-20; w = (raw / den) * route_scale

The denominator tree: pad k to the next power of two P, then for stride P/2 .. 1
add s[i+stride] into s[i] when it exists. For k = 6 this is the reference's
((r0+r4)+r2) + ((r1+r5)+r3). For k = 8 it is this build's rule: parity unpinned
against PyTorch (no recorded k = 8 golden exists), pinned by the k = 6 restriction.

Transcendentals are evaluated in float64 and rounded once to FP32, as the HIP
kernels do.
"""

from __future__ import annotations

import numpy as np

NORMALIZATION_EPSILON = np.float32(1e-20)
SCORE_FUNCS = ("sigmoid", "sqrtsoftplus")


def gate_logits(weight, x) -> np.ndarray:
    """[T, E] FP32 logits of W_r [E, H] (FP32) applied to BF16-valued x [T, H]."""
    w = np.asarray(weight, dtype=np.float32).astype(np.float64)
    x = np.atleast_2d(np.asarray(x, dtype=np.float32)).astype(np.float64)
    return (x @ w.T).astype(np.float32)


def scores(logits, score_func: str = "sigmoid") -> np.ndarray:
    z = np.asarray(logits, dtype=np.float32)
    with np.errstate(over="ignore"):
        if score_func == "sigmoid":
            e = np.exp(-z.astype(np.float64)).astype(np.float32)
            return (np.float32(1) / (np.float32(1) + e)).astype(np.float32)
        if score_func == "sqrtsoftplus":
            softplus = np.where(z > np.float32(20), z,
                                np.log1p(np.exp(z.astype(np.float64))).astype(np.float32)).astype(np.float32)
            return np.sqrt(softplus).astype(np.float32)
    raise ValueError(f"Unknown score function {score_func!r}")


def ordered_keys(values) -> np.ndarray:
    """FP32 -> u32 keys whose unsigned order is the float order (-0 below +0)."""
    bits = np.asarray(values, dtype=np.float32).view(np.uint32)
    flip = np.where((bits & np.uint32(0x80000000)) != 0, np.uint32(0xFFFFFFFF), np.uint32(0x80000000))
    return (bits ^ flip).astype(np.uint32)


def bitonic32(keys, ids, count: int):
    """The 32-slot descending bitonic network over `count` valid leading entries.

    Pairs of each stage are disjoint, so evaluating them in order reproduces the
    parallel network. direction: (lane & size/2) != 0 for sizes 2..16, false for
    the final 32-wide merge; an entry moves up when its key is larger and valid,
    or when its partner is padding (routing_probe.cu:60-73).
    """
    keys = np.array(keys, dtype=np.float32)
    ids = np.array(ids, dtype=np.int32)
    valid = np.arange(32) < count
    size = 2
    while size <= 32:
        stride = size // 2
        while stride:
            for lane in range(16):
                pos = 2 * lane - (lane & (stride - 1))
                other = pos + stride
                descending_block = False if size == 32 else bool(lane & (size // 2))
                promote = bool((keys[pos] > keys[other] and valid[pos]) or not valid[other])
                if promote == descending_block:
                    keys[pos], keys[other] = keys[other], keys[pos]
                    ids[pos], ids[other] = ids[other], ids[pos]
                    valid[pos], valid[other] = valid[other], valid[pos]
            stride //= 2
        size *= 2
    return keys, ids


def topk_indices(selection, k: int) -> np.ndarray:
    """Expert IDs of one token's k largest selection scores, in the reference's output order."""
    selection = np.asarray(selection, dtype=np.float32).reshape(-1)
    e = selection.size
    if not 1 <= k <= min(32, e):
        raise ValueError("top-k needs 1 <= k <= min(32, experts)")
    if not np.isfinite(selection).all():
        raise ValueError("Top-k selection requires finite FP32 values")
    keys = ordered_keys(selection)
    threshold = np.partition(keys, e - k)[e - k]
    order = np.concatenate((np.flatnonzero(keys > threshold), np.flatnonzero(keys == threshold)))[:k]
    slot_keys = np.zeros(32, np.float32)
    slot_ids = np.zeros(32, np.int32)
    slot_keys[:k] = selection[order]
    slot_ids[:k] = order
    _, sorted_ids = bitonic32(slot_keys, slot_ids, k)
    return sorted_ids[:k].copy()


def tie_flag(selection, k: int) -> bool:
    """True when the k-th largest value is shared with an unselected expert or among the top
    (routing_probe.cu:24-38 reports ties met during the serial arg-max passes)."""
    keys = ordered_keys(selection)
    ranked = np.sort(keys)[::-1]
    return bool(len(np.unique(ranked[:k])) < k or (ranked.size > k and ranked[k] == ranked[k - 1]))


def tree_sum(values) -> np.float32:
    """FP32 halving-tree sum (see module docstring)."""
    v = [np.float32(x) for x in np.asarray(values, dtype=np.float32)]
    width = 1
    while width < len(v):
        width *= 2
    slots = v + [None] * (width - len(v))
    stride = width // 2
    while stride:
        for i in range(stride):
            if slots[i + stride] is not None:
                slots[i] = np.float32(slots[i] + slots[i + stride]) if slots[i] is not None else slots[i + stride]
        stride //= 2
    return np.float32(slots[0])


def route_weights(scores_row, ids, route_scale: float):
    """raw, denominator, weights of one token (router.py:174-192)."""
    scores_row = np.asarray(scores_row, dtype=np.float32)
    raw = scores_row[np.asarray(ids)]
    with np.errstate(over="ignore"):
        denominator = np.float32(tree_sum(raw) + NORMALIZATION_EPSILON)
        weights = ((raw / denominator) * np.float32(route_scale)).astype(np.float32)
    return raw.astype(np.float32), denominator, weights


def select_scores(scores_row, bias, k: int, route_scale: float):
    """CPU selection spec of router.py:174-192 generalised to (E, k): returns (weights, indices)."""
    scores_row, bias = np.asarray(scores_row, dtype=np.float32), np.asarray(bias, dtype=np.float32)
    if (scores_row.shape != bias.shape or not np.isfinite(scores_row).all() or not np.isfinite(bias).all()
            or np.any(scores_row < 0)):
        raise ValueError("Selection requires finite nonnegative scores and finite biases")
    with np.errstate(over="ignore"):
        selection = (scores_row + bias).astype(np.float32)
    if not np.isfinite(selection).all():
        raise ValueError("Selection score overflow")
    indices = topk_indices(selection, k)
    _, denominator, weights = route_weights(scores_row, indices, route_scale)
    if not np.isfinite(denominator):
        raise ValueError("Routing normalization overflows the finite probe scope")
    return weights, indices


def route(logits, k: int, route_scale: float, score_func: str = "sigmoid", bias=None) -> dict:
    """Full router postprocessing for [T, E] logits; every stage kept."""
    logits = np.atleast_2d(np.asarray(logits, dtype=np.float32))
    s = scores(logits, score_func)
    b = np.zeros(logits.shape[1], np.float32) if bias is None else np.asarray(bias, dtype=np.float32)
    with np.errstate(over="ignore"):
        selection = (s + b[None, :]).astype(np.float32)
    t = logits.shape[0]
    ids = np.zeros((t, k), np.int32)
    raw = np.zeros((t, k), np.float32)
    den = np.zeros(t, np.float32)
    weights = np.zeros((t, k), np.float32)
    for row in range(t):
        ids[row] = topk_indices(selection[row], k)
        raw[row], den[row], weights[row] = route_weights(s[row], ids[row], route_scale)
    return {"logits": logits, "scores": s, "selection": selection, "indices": ids,
            "raw": raw, "denominator": den, "weights": weights}
