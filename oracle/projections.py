"""FP8 E4M3 block-scaled projections (CPU oracle, test infrastructure only).

Two scale profiles of the same arithmetic:

* block 32 (the reference's own projection path): NativeProjections.fp8
  (src/vesper/projections.py:135-154) quantizes the BF16 input per 32 with the
  activation32 quantizer (formats.quantize_activation) and runs projection_fp8
  (src/vesper/kernels/projection_probe.cu:9-51): per 32-wide K group, d = the
  exact E4M3 x E4M3 dot, then sum = sum + (d * sa) * sw in FP32 with
  sw = E8M0 of the weight's 32 x 32 block (row / 32, group); BF16 output and the
  FP32 sum as the trace. This is formats.fp8_block32_gemv_fp32.
* block 128 (DeepSeek-style FP8): FP32 weight scales
  per 128 x 128 block ([ceil(N/128), K/128]) and per-token per-128 FP32
  activation scales s = f32(max(amax, 1e-4)) / 448, codes E4M3(clip(x / s)).
  Per 128-wide K group d = exact dot rounded once to FP32, then
  sum = fma(d, f32(sa * sw), sum): one rounding per output and group (the
  kernels' fused multiply-add; formats.fma_f32 restates it exactly). The
  reference has no block-128 path (its only FP8 projection has power-of-two
  block-32 scales, where every order of the scaling gives the same sums); this
  profile restates the configuration with the reference's amax floor and this
  build's accumulation order. Parity unpinned beyond its closed form: pinned by
  exact-arithmetic checks (designed representable inputs), an exact-rational
  check of the per-group scaling, and the exact-rational pin of fma_f32.

E4M3 x E4M3 products are multiples of 2^-18 below 2^18, so a 128-term dot is
exact in float64 and is rounded once to FP32.
"""

from __future__ import annotations

import numpy as np

from .formats import (AMAX_FLOOR, bf16_bits, bf16_values, e4m3_values, encode_e4m3, fma_f32,
                      fp8_block32_gemv_fp32, quantize_activation)

# Projection shapes [rows, width] (DeepSeek low-rank attention).
CONFIG3_LAYOUT = {"q_a": (1536, 7168), "q_b": (24576, 1536), "kv_a": (576, 7168), "o": (7168, 16384)}
# The reference's registered shapes (projections.py:16).
REFERENCE_LAYOUT = {"wq_a": (1280, 5120), "wq_b": (32768, 1280), "wkv": (512, 5120), "wo_b": (5120, 8192)}
STAGES = ("input_fp8", "scale", "output_fp32", "output_bf16")


def quantize_activation_128(values) -> tuple[np.ndarray, np.ndarray]:
    """Per-token per-128 E4M3 codes and FP32 scales of BF16-valued input [T, K]."""
    x = np.atleast_2d(np.asarray(values, dtype=np.float32))
    t, k = x.shape
    if k % 128:
        raise ValueError("width must be a multiple of 128")
    blocks = x.reshape(t, k // 128, 128)
    amax = np.maximum(np.max(np.abs(blocks), axis=2), AMAX_FLOOR).astype(np.float32)
    scale = (amax / np.float32(448.0)).astype(np.float32)                         # one IEEE division
    y = (blocks / scale[..., None]).astype(np.float32)
    y = np.clip(y, np.float32(-448.0), np.float32(448.0))
    return encode_e4m3(y).reshape(t, k), scale


def fp8_block128_gemm_fp32(act_codes, act_scales, weight_codes, weight_scales) -> np.ndarray:
    """[T, K] E4M3 codes with FP32 scales [T, K/128] times [N, K] E4M3 with FP32 scales [ceil(N/128), K/128]."""
    q = np.atleast_2d(np.asarray(act_codes, dtype=np.uint8))
    sa = np.atleast_2d(np.asarray(act_scales, dtype=np.float32))
    w = np.asarray(weight_codes, dtype=np.uint8)
    sw = np.asarray(weight_scales, dtype=np.float32)
    n, k = w.shape
    t = q.shape[0]
    g = k // 128
    if q.shape[1] != k or sa.shape != (t, g) or sw.shape != ((n + 127) // 128, g):
        raise ValueError("Mismatched FP8 block-128 dimensions")
    lut = e4m3_values(np.arange(256, dtype=np.uint8)).astype(np.float64)
    row_scale = sw[np.arange(n) // 128]                                          # [N, G]
    acc = np.zeros((t, n), np.float32)
    for j in range(g):
        cols = slice(128 * j, 128 * (j + 1))
        # the block dot: 128 products, each a multiple of 2^-18 below 2^18, so the float64 sum is exact in
        # any order (BLAS is free to reorder) and is rounded once to FP32
        d = (lut[q[:, cols]] @ lut[w[:, cols]].T).astype(np.float32)
        scale = (sa[:, j:j + 1] * row_scale[None, :, j]).astype(np.float32)    # f32(sa * sw)
        acc = fma_f32(d, scale, acc)                                             # acc = f32(d * scale + acc)
    return acc


def fp8_projection(x, weight_codes, weight_scales, block: int) -> dict:
    """Stage dict of one projection (projections.py:135-154 stage names, with `scale` holding the
    E8M0 codes for block 32 or the FP32 scales for block 128)."""
    xb = bf16_values(bf16_bits(np.atleast_2d(np.asarray(x, dtype=np.float32))))
    if block == 32:
        q, s = quantize_activation(xb)
        acc = fp8_block32_gemv_fp32(q, s, weight_codes, weight_scales)
    elif block == 128:
        q, s = quantize_activation_128(xb)
        acc = fp8_block128_gemm_fp32(q, s, weight_codes, weight_scales)
    else:
        raise ValueError("block must be 32 or 128")
    return dict(zip(STAGES, (q, s, acc, bf16_bits(acc))))


def fp8_reference_fp32(x, weight_codes, weight_scales, block: int) -> np.ndarray:
    """Unquantized-activation FP32 reference: BF16 x times the dequantized weights (float64 sum)."""
    xb = bf16_values(bf16_bits(np.atleast_2d(np.asarray(x, dtype=np.float32)))).astype(np.float64)
    w = e4m3_values(np.asarray(weight_codes, np.uint8)).astype(np.float64)
    n, k = w.shape
    sw = np.asarray(weight_scales)
    if block == 32:
        from .formats import e8m0_values
        scale = np.repeat(np.repeat(e8m0_values(sw).astype(np.float64), 32, 0), 32, 1)[:n, :k]
    else:
        scale = np.repeat(np.repeat(sw.astype(np.float64), 128, 0), 128, 1)[:n, :k]
    return (xb @ (w * scale).T).astype(np.float32)


def fp8_weights(rng, rows, width, block: int):
    """Synthetic weights: E4M3 codes uniform over the finite codes; block-128 FP32 scales
    log-uniform in [2^-8, 2^-2] (configuration 3), block-32 E8M0 codes uniform in [118, 126]."""
    codes = rng.integers(0, 256, (rows, width), dtype=np.uint8)
    codes = np.where((codes & 0x7F) == 0x7F, codes ^ 1, codes).astype(np.uint8)
    if block == 128:
        scales = np.exp2(rng.uniform(-8.0, -2.0, ((rows + 127) // 128, width // 128))).astype(np.float32)
    else:
        scales = rng.integers(118, 127, (rows // 32, width // 32), dtype=np.uint8)
    return codes, scales


def kv_round32(values_bits):
    """kv_round32 (kv_probe.cu:4-25): per-32 E4M3 codes and E8M0 scales of the BF16 values (the
    activation32 quantizer, formats.quantize_activation) and the round trip
    rounded = BF16(E4M3(code) x 2^(scale - 127)), exact in FP32 and in BF16.
    Returns (rounded BF16 bits, codes, scales)."""
    from .formats import bf16_bits, bf16_values, e4m3_values, e8m0_values, quantize_activation
    codes, scales = quantize_activation(bf16_values(np.asarray(values_bits, np.uint16)))
    vals = e4m3_values(codes).astype(np.float32).reshape(*codes.shape[:-1], -1, 32) * e8m0_values(scales)[..., None]
    return bf16_bits(vals.reshape(codes.shape).astype(np.float32)), codes, scales


def dequant_block32(weight_codes, weight_scales) -> np.ndarray:
    """E4M3 codes x E8M0 of their 32 x 32 block, as float64 (projection_dequant_wo_a; every value is exact
    in BF16, so the reference's BF16 conversion keeps it)."""
    from .formats import e4m3_values, e8m0_values
    s = np.repeat(np.repeat(e8m0_values(weight_scales).astype(np.float64), 32, axis=0), 32, axis=1)
    return e4m3_values(weight_codes).astype(np.float64) * s


def wo_a_grouped(values_bits, weight_codes, weight_scales, groups: int = 8) -> dict:
    """NativeProjections.grouped (projections.py:60-67,156-171): kv_round32 of the [T, groups, K] input,
    then per group g out[t, g, r] = BF16(sum_k W[g R + r, k] x rounded[t, g, k]) with R = rows / groups,
    W the exactly dequantized weight. The reference runs a batched BF16 GEMM with FP32 accumulation in
    an order the library does not specify; the sum here is evaluated in float64 (exact products) and
    rounded once to FP32."""
    from .formats import bf16_bits, bf16_values
    values_bits = np.asarray(values_bits, np.uint16)
    t = int(np.prod(values_bits.shape[:-2]))
    rounded, codes, scales = kv_round32(values_bits)
    x = bf16_values(rounded).astype(np.float64).reshape(t, groups, -1)
    w = dequant_block32(weight_codes, weight_scales).reshape(groups, -1, x.shape[-1])
    out = np.einsum("grk,tgk->tgr", w, x).astype(np.float32)
    return {"rounded_bf16": rounded, "input_fp8": codes, "scale_e8m0": scales, "output_fp32": out,
            "output_bf16": bf16_bits(out).reshape(*values_bits.shape[:-1], -1)}
