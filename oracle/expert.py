"""One SwiGLU expert over a batch of tokens, stage by stage (CPU oracle, test infrastructure only).

Restates the stage order of ``ExpertExecutor.execute`` (src/vesper/expert.py:51-79)
and the FP32 epilogue of ``expert_swiglu`` (src/vesper/kernels/expert_probe.cu:4-26):

  x -> BF16 -> per-32 E4M3/E8M0 (q, s) -> W1 (gate), W3 (up) block GEMV -> BF16
    -> FP32 clamp (gate <= L; -L <= up <= L; L = 0 disables)
    -> silu = gate / (1 + exp(-gate)) -> product = silu * up -> routed = w * product (routed experts)
    -> BF16 (down_input) -> per-32 E4M3/E8M0 (down_q, down_s) -> W2 block GEMV -> BF16 (w2)

The routing weight multiplies the FP32 product before W2 (docs/moe-arithmetic-validation.md:48-51).

exp is evaluated in float64 and rounded once to FP32; the HIP kernel does the
same, so both agree bit for bit except where two float64 exp results straddle
an FP32 rounding boundary (probability ~2^-28 per element). The reference's
CUDA expf is not correctly rounded, which is why these stages are compared with
a tolerance against the reference itself.
"""

from __future__ import annotations

import numpy as np

from .formats import (bf16_bits, bf16_round, bf16_values, fp8_block32_gemv_fp32, mxfp4_gemv_fp32,
                      quantize_activation)

EXPERT_TENSORS = ("w1_weight", "w1_scale", "w3_weight", "w3_scale", "w2_weight", "w2_scale")


def expert_layout(hidden: int, intermediate: int, fmt: str = "mxfp4") -> dict:
    """Tensor shapes per expert; order = on-disk order (checkpoint.py:139-149, storage.py:33-41)."""
    shapes = {"w1": (intermediate, hidden), "w3": (intermediate, hidden), "w2": (hidden, intermediate)}
    layout = {}
    for name, (rows, width) in shapes.items():
        if fmt == "mxfp4":
            layout[f"{name}_weight"] = (rows, width // 2)
            layout[f"{name}_scale"] = (rows, width // 32)
        elif fmt == "fp8_block32":          # shared.py:20-24
            layout[f"{name}_weight"] = (rows, width)
            layout[f"{name}_scale"] = (rows // 32, width // 32)
        else:
            raise ValueError(f"Unknown expert format {fmt!r}")
    return layout


def exp_f32(values) -> np.ndarray:
    """FP32 exp rounded once from float64."""
    with np.errstate(over="ignore"):
        return np.exp(np.asarray(values, dtype=np.float32).astype(np.float64)).astype(np.float32)


def swiglu(w1_bits, w3_bits, limit: float, routing_weight=None):
    """FP32 epilogue of expert_probe.cu:10-25; returns (down_input f32 BF16-valued, trace [...,5])."""
    gate = bf16_values(w1_bits).copy()
    up = bf16_values(w3_bits).copy()
    limit = np.float32(limit)
    if limit > 0:
        gate = np.where(gate > limit, limit, gate).astype(np.float32)
        up = np.where(up > limit, limit, up).astype(np.float32)
        up = np.where(up < -limit, -limit, up).astype(np.float32)
    with np.errstate(over="ignore", invalid="ignore", divide="ignore"):
        silu = (gate / (np.float32(1) + exp_f32(-gate))).astype(np.float32)
        product = (silu * up).astype(np.float32)
        if routing_weight is None:
            routed = product
        else:
            w = np.asarray(routing_weight, dtype=np.float32).reshape(-1, *([1] * (product.ndim - 1)))
            routed = (w * product).astype(np.float32)
    trace = np.stack([gate, up, silu, product, routed], axis=-1).astype(np.float32)
    return bf16_round(routed), trace


def _gemv(fmt, q, s, arrays, name):
    if fmt == "mxfp4":
        return mxfp4_gemv_fp32(q, s, arrays[f"{name}_weight"], arrays[f"{name}_scale"])
    return fp8_block32_gemv_fp32(q, s, arrays[f"{name}_weight"], arrays[f"{name}_scale"])


def expert_forward(x, arrays: dict, routing_weight=None, limit: float = 10.0, fmt: str = "mxfp4") -> dict:
    """All stage outputs for T tokens through one expert (expert.py:51-79, batched).

    x: [T, H] or [H] FP32 (BF16-rounded here). routing_weight: None (shared
    expert) or one FP32 weight per token. Returns q, s, w1, w3, down_input,
    trace, down_q, down_s, w2 with a leading token axis.
    """
    x = np.atleast_2d(np.asarray(x, dtype=np.float32))
    q, s = quantize_activation(bf16_round(x))
    w1 = bf16_bits(_gemv(fmt, q, s, arrays, "w1"))
    w3 = bf16_bits(_gemv(fmt, q, s, arrays, "w3"))
    down_input, trace = swiglu(w1, w3, limit, routing_weight)
    down_q, down_s = quantize_activation(down_input)
    w2 = bf16_bits(_gemv(fmt, down_q, down_s, arrays, "w2"))
    return {"q": q, "s": s, "w1": w1, "w3": w3, "down_input": down_input, "trace": trace,
            "down_q": down_q, "down_s": down_s, "w2": w2}


def expert_reference_stages(x, arrays: dict, routing_weight=None) -> dict:
    """Every stage of BASELINE config 0's formula y = W2(silu(W1 x) * W3 x) in float64: g = W1 x, u = W3 x,
    h = silu(g) u (times the route weight), y = W2 h, from the exactly dequantized MXFP4 weights and the
    BF16-rounded activations (no activation quantization, no clamp)."""
    from .formats import unpack_fp4
    x = np.atleast_2d(bf16_round(x)).astype(np.float64)
    w1 = unpack_fp4(arrays["w1_weight"], arrays["w1_scale"]).astype(np.float64)
    w3 = unpack_fp4(arrays["w3_weight"], arrays["w3_scale"]).astype(np.float64)
    w2 = unpack_fp4(arrays["w2_weight"], arrays["w2_scale"]).astype(np.float64)
    g = x @ w1.T
    u = x @ w3.T
    h = g / (1.0 + np.exp(-g)) * u
    if routing_weight is not None:
        h = h * np.asarray(routing_weight, dtype=np.float64).reshape(-1, 1)
    return {"g": g, "u": u, "h": h, "y": h @ w2.T}


def expert_reference_fp32(x, arrays: dict, routing_weight=None) -> np.ndarray:
    """Unquantized-activation reference y = W2(silu(W1 x) * W3 x) with dequantized weights.

    This is BASELINE config 0's formula (no activation quantization, no clamp),
    evaluated in float64 from FP32-dequantized MXFP4 weights. The W4A8 pipeline
    above is compared to it only through the tolerance metrics.
    """
    return expert_reference_stages(x, arrays, routing_weight)["y"]
