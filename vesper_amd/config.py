"""MoE layer configuration (replaces the reference's module constants).

The reference hard-codes HIDDEN/TOP_K/EXPERTS (src/vesper/moe.py:13-15), ROUTER_CONFIG
(src/vesper/router.py:16-17) and EXPERT_SHAPES (src/vesper/checkpoint.py:139-141); one
frozen dataclass carries them here so both the reference model's shapes and the
BASELINE (DeepSeek-V3 style) shapes run through the same kernels.
"""

from __future__ import annotations

from dataclasses import dataclass

import math

SCORE_FUNCS = ("sigmoid", "sqrtsoftplus")
MAX_DECODE_TOKENS = 16


@dataclass(frozen=True)
class MoEConfig:
    hidden: int = 7168
    intermediate: int = 2048
    experts: int = 256
    top_k: int = 8
    score_func: str = "sigmoid"
    route_scale: float = 2.5
    swiglu_limit: float = 0.0          # 0 disables the clamp (BASELINE formula has none)
    shared: str | None = "mxfp4"       # None, "mxfp4"
    max_tokens: int = MAX_DECODE_TOKENS

    def __post_init__(self):
        if self.hidden <= 0 or self.hidden % 128 or self.intermediate <= 0 or self.intermediate % 128:
            raise ValueError("hidden and intermediate sizes must be positive multiples of 128")
        if not 1 <= self.experts <= 1024:
            raise ValueError("experts must be in [1, 1024]")
        if not 1 <= self.top_k <= min(32, self.experts):
            raise ValueError("top_k must be in [1, min(32, experts)]")
        if self.score_func not in SCORE_FUNCS:
            raise ValueError(f"score_func must be one of {SCORE_FUNCS}")
        if not math.isfinite(self.route_scale):
            raise ValueError("route_scale must be finite")
        if not math.isfinite(self.swiglu_limit) or self.swiglu_limit < 0:
            raise ValueError("Invalid SwiGLU limit")
        if self.shared not in (None, "mxfp4"):
            raise ValueError("shared expert format must be None or 'mxfp4'")
        if not 1 <= self.max_tokens <= MAX_DECODE_TOKENS:
            raise ValueError(f"max_tokens must be in [1, {MAX_DECODE_TOKENS}]")

    def expert_layout(self) -> dict:
        """Per-expert tensor shapes in on-disk order (checkpoint.py:139-149, storage.py:33-41)."""
        h, i = self.hidden, self.intermediate
        return {"w1_weight": (i, h // 2), "w1_scale": (i, h // 32),
                "w3_weight": (i, h // 2), "w3_scale": (i, h // 32),
                "w2_weight": (h, i // 2), "w2_scale": (h, i // 32)}

    @property
    def expert_bytes(self) -> int:
        return sum(r * c for r, c in self.expert_layout().values())


# BASELINE.json configuration 1 (DeepSeek-V3 style) and the reference model's own shapes.
BASELINE = MoEConfig()
REFERENCE = MoEConfig(hidden=5120, intermediate=2304, experts=384, top_k=6, score_func="sqrtsoftplus",
                      route_scale=1.5, swiglu_limit=10.0, shared="mxfp4", max_tokens=MAX_DECODE_TOKENS)
