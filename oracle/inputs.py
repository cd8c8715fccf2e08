"""Seeded synthetic inputs (CPU oracle, test infrastructure only).

Two kinds:
  * Regenerations of the reference's own input generators, so that the recorded
    SHA-256 goldens in its results/ files pin the oracle:
      aggregation_cases  src/vesper/moe_reference.py:25-62 (E=384, k=6, hidden 5120)
      selection_cases    src/vesper/router_reference.py:105-130
    These must draw from numpy's Generator in the same order as the reference,
    or the recorded input hashes would not match.
  * BASELINE.json configuration generators (uniform nibble bytes, E8M0 scale
    codes uniform in [118, 126], x ~ N(0,1) rounded to BF16, W_r ~ N(0, 0.02)).
"""

from __future__ import annotations

import numpy as np

from .expert import expert_layout
from .formats import bf16_bits, bf16_round
from .moe import participation

SEEDS = (20261018, 0, 1, 42, 127, 512, 4096, 65535)
REFERENCE_HIDDEN = 5120


def aggregation_cases(hidden: int = REFERENCE_HIDDEN):
    pool = np.array([0, 1, 3, 31, 32, 95, 96, 127, 128, 255, 256, 383], np.int64)
    for seed in SEEDS:
        rng = np.random.default_rng(seed)
        for tokens in (1, 2, 8, 32):
            indices = np.stack([rng.choice(pool, 6, replace=False) for _ in range(tokens)])
            contributions = {}
            for expert, rows in participation(indices, 384, 6, 32).items():
                normal = rng.standard_normal((len(rows), hidden)).astype(np.float32)
                exponents = rng.integers(-24, 25, (len(rows), hidden))
                contributions[expert] = bf16_bits(np.ldexp(normal, exponents))
            shared = bf16_bits(rng.standard_normal((tokens, hidden)).astype(np.float32))
            yield {"input": f"random_seed{seed}_tokens{tokens}", "indices": indices,
                   "contributions": contributions, "shared": shared}
    ids = np.array([[0, 1, 2, 3, 4, 383]], np.int64)
    values = {int(e): np.zeros((1, hidden), np.float32) for e in ids[0]}
    big = np.float32(2.0 ** 26)
    values[0][:, 0::3], values[1][:, 0::3], values[2][:, 0::3] = big, 1.0, -big
    values[0][:, 1::3], values[1][:, 1::3], values[2][:, 1::3] = 1.0, 2.0 ** -8, 2.0 ** -8
    values[0][:, 2::3], values[1][:, 2::3] = big, -big
    cancellation = {e: bf16_bits(v) for e, v in values.items()}
    shared = np.zeros((1, hidden), np.float32)
    shared[:, 2::3] = 1.0
    for order in ((0, 1, 2, 3, 4, 383), (0, 2, 1, 383, 4, 3), (383, 4, 3, 2, 1, 0)):
        yield {"input": "cancellation_rank_" + "_".join(map(str, order)),
               "indices": np.array([order], np.int64), "contributions": cancellation,
               "shared": bf16_bits(shared)}
    signed = np.resize(np.array([0, 0x8000, 1, 0x8001, 0x007F, 0x807F, 0x0080, 0x8080], np.uint16), (2, hidden))
    two = np.tile(ids, (2, 1))
    yield {"input": "signed_zero_and_BF16_subnormals", "indices": two,
           "contributions": {int(e): signed.copy() for e in two[0]}, "shared": signed.copy()}
    yield {"input": "zero_contributions", "indices": two,
           "contributions": {int(e): np.zeros((2, hidden), np.uint16) for e in two[0]},
           "shared": np.zeros((2, hidden), np.uint16)}
    yield {"input": "empty_token_batch", "indices": np.empty((0, 6), np.int64),
           "contributions": {}, "shared": np.empty((0, hidden), np.uint16)}


def selection_cases():
    for seed in range(32):
        rng = np.random.default_rng(seed + 10000)
        for bins in (1, 2, 4, 8, 32, 384):
            selection = rng.integers(-bins, bins + 1, 384).astype(np.float32) / np.float32(16)
            scores = np.ldexp(rng.uniform(0.5, 1, 384).astype(np.float32), rng.integers(-60, 61, 384))
            yield {"kind": "discrete_selection", "seed": seed + 10000, "bins": bins}, scores, selection
    rng = np.random.default_rng(38906)
    for higher in range(6):
        for equal in sorted({7 - higher, 16, 64, 384 - higher}):
            ids = rng.permutation(384)
            selection = np.full(384, -10, np.float32)
            selection[ids[:higher]] = np.arange(30, 30 - higher, -1, dtype=np.float32)
            selection[ids[higher:higher + equal]] = 10
            scores = rng.uniform(0.001, 20, 384).astype(np.float32)
            yield {"kind": "boundary_tie", "strictly_higher": higher, "equal_to_boundary": equal}, scores, selection
    tiny = np.nextafter(np.float32(0), np.float32(1))
    for name, selection in (
        ("all_equal", np.zeros(384, np.float32)),
        ("signed_zero", np.resize(np.array([-0.0, 0.0], np.float32), 384)),
        ("subnormal_selection", np.arange(-192, 192, dtype=np.float32) * tiny),
        ("finite_extreme_selection", np.linspace(-3e38, 3e38, 384, dtype=np.float64).astype(np.float32)),
    ):
        for repeat in range(4):
            yield {"kind": name, "repeat": repeat}, np.linspace(0.0001, 30, 384, dtype=np.float32), selection.copy()


# --- BASELINE.json configurations -------------------------------------------------------------

def mxfp4_expert(rng, hidden: int, intermediate: int, scale_lo: int = 118, scale_hi: int = 126) -> dict:
    """Packed E2M1 bytes uniform over 0..255 (both nibbles uniform over 16 codes), E8M0 codes in [lo, hi]."""
    arrays = {}
    for name, shape in expert_layout(hidden, intermediate).items():
        if name.endswith("weight"):
            arrays[name] = rng.integers(0, 256, shape, dtype=np.uint8)
        else:
            arrays[name] = rng.integers(scale_lo, scale_hi + 1, shape, dtype=np.uint8)
    return arrays


def fp8_block32_expert(rng, hidden: int, intermediate: int, scale_lo: int = 118, scale_hi: int = 124) -> dict:
    """E4M3 weight codes uniform over the 254 finite codes, one E8M0 code per 32x32 block."""
    finite = np.array([c for c in range(256) if (c & 0x7F) != 0x7F], np.uint8)
    arrays = {}
    for name, shape in expert_layout(hidden, intermediate, "fp8_block32").items():
        if name.endswith("weight"):
            arrays[name] = finite[rng.integers(0, finite.size, shape)]
        else:
            arrays[name] = rng.integers(scale_lo, scale_hi + 1, shape, dtype=np.uint8)
    return arrays


def fp8_block32_expert_normal(rng, hidden: int, intermediate: int, sigma: float = 0.02) -> dict:
    """Checkpoint-like FP8 block-32 weights: N(0, sigma) values quantized per 32 x 32 block with a
    power-of-two E8M0 scale 2^ceil(log2(amax / 448)) (no code saturates), E4M3 codes of value / scale."""
    from .formats import encode_e4m3
    arrays = {}
    for name, shape in expert_layout(hidden, intermediate, "fp8_block32").items():
        if not name.endswith("weight"):
            continue
        rows, width = shape
        w = (rng.standard_normal((rows, width)) * sigma).astype(np.float32)
        blocks = np.abs(w).reshape(rows // 32, 32, width // 32, 32).max(axis=(1, 3))
        e = np.ceil(np.log2(np.maximum(blocks, 1e-30) / 448.0)).astype(np.int32)
        scale = np.exp2(e).astype(np.float32)
        arrays[name] = encode_e4m3(w / np.repeat(np.repeat(scale, 32, 0), 32, 1))
        arrays[name.replace("weight", "scale")] = (e + 127).astype(np.uint8)
    return {n: arrays[n] for n in expert_layout(hidden, intermediate, "fp8_block32")}


def activations(rng, tokens: int, hidden: int) -> np.ndarray:
    return bf16_round(rng.standard_normal((tokens, hidden)).astype(np.float32))


def router_weight(rng, experts: int, hidden: int) -> np.ndarray:
    return (rng.standard_normal((experts, hidden)) * 0.02).astype(np.float32)

