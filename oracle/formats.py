"""Format codecs and the MX block GEMV specification (CPU oracle, test infrastructure only).

Restates ``src/vesper/formats.py`` of the reference:
  fp4_values          formats.py:11-21   E2M1 code -> FP32, sign in bit 3, -0 kept
  e8m0_values         formats.py:24-29   code c -> 2^(c-127); 0 -> 2^-127; 255 -> NaN
  unpack_fp4          formats.py:32-42   packed byte -> (low nibble = even K, high = odd K) x block scale
  e4m3_values         formats.py:45-52   OCP E4M3FN decode
  encode_e4m3         formats.py:55-66   FP32 -> E4M3, round-to-nearest-even, saturate to +-448, NaN -> 0x7F
  bf16_bits/values    formats.py:69-77   FP32 -> BF16 RNE (NaN quieted), BF16 -> FP32
  quantize_activation formats.py:80-94   per-block amax (floor 1e-4) -> E8M0 -> E4M3 codes
  mxfp4_gemv_spec     formats.py:97-118  per-block exact dot -> FP32 -> (dot*sa)*sw -> in-order FP32 sum

The encoders here are written with exponent/mantissa arithmetic; the reference
searches a value table. Tests check each against an independent method.
"""

from __future__ import annotations

import numpy as np

# np.float32(1/448): FP32 nearest to 1/448, the reciprocal the block quantizer multiplies by.
INV_448_BITS = 0x3B124925
E4M3_MAX = 448.0
AMAX_FLOOR = np.float32(1e-4)


def _fp4_formula(codes) -> np.ndarray:
    """E2M1: bit3 sign, bits 2-1 exponent (bias 1), bit 0 mantissa (formats.py:11-21)."""
    exponent = ((codes >> 1) & 3).astype(np.int32)
    mantissa = (codes & 1).astype(np.float64)
    magnitude = np.where(exponent == 0, mantissa * 0.5,
                         np.ldexp(1.0 + mantissa * 0.5, exponent - 1)).astype(np.float32)
    return np.where((codes & 8) != 0, -magnitude, magnitude).astype(np.float32)


# the formula evaluated once for each of the 16 codes; fp4_values indexes it (the same values, without
# evaluating ldexp per weight)
_FP4_TABLE = _fp4_formula(np.arange(16, dtype=np.uint8))


def fp4_values(codes) -> np.ndarray:
    """E2M1 code -> FP32 value (formats.py:11-21)."""
    codes = np.asarray(codes, dtype=np.uint8)
    if np.any(codes > 15):
        raise ValueError("An E2M1 code occupies four bits")
    return _FP4_TABLE[codes]


def e8m0_values(codes) -> np.ndarray:
    """E8M0 scale byte -> FP32 power of two (formats.py:24-29)."""
    codes = np.asarray(codes, dtype=np.uint8)
    with np.errstate(over="ignore"):
        values = np.ldexp(np.float32(1.0), codes.astype(np.int32) - 127).astype(np.float32)
    return np.where(codes == 255, np.float32(np.nan), values).astype(np.float32)


def split_nibbles(packed) -> np.ndarray:
    """[..., K/2] bytes -> [..., K] E2M1 codes; the low nibble holds the even K index."""
    packed = np.asarray(packed, dtype=np.uint8)
    codes = np.empty((*packed.shape[:-1], packed.shape[-1] * 2), dtype=np.uint8)
    codes[..., 0::2] = packed & 0x0F
    codes[..., 1::2] = packed >> 4
    return codes


def unpack_fp4(packed, scales, block: int = 32) -> np.ndarray:
    """Dequantize packed MXFP4 [..., K/2] with E8M0 scales [..., K/32] to FP32 (formats.py:32-42)."""
    packed = np.asarray(packed, dtype=np.uint8)
    if block != 32 or (packed.shape[-1] * 2) % block:
        raise ValueError("Native expert blocks contain 32 values")
    codes = split_nibbles(packed)
    scales = np.asarray(scales, dtype=np.uint8)
    if scales.shape != (*codes.shape[:-1], codes.shape[-1] // block):
        raise ValueError("Scale shape does not match packed FP4 weights")
    with np.errstate(over="ignore", invalid="ignore"):
        return (fp4_values(codes) * np.repeat(e8m0_values(scales), block, axis=-1)).astype(np.float32)


def e4m3_values(codes) -> np.ndarray:
    """OCP E4M3FN: bias 7, subnormals m/512, 0x7F/0xFF NaN, max 448 (formats.py:45-52)."""
    codes = np.asarray(codes, dtype=np.uint8)
    exponent = ((codes >> 3) & 15).astype(np.int32)
    mantissa = (codes & 7).astype(np.float64)
    magnitude = np.where(exponent == 0, np.ldexp(mantissa, -9),
                         np.ldexp(1.0 + mantissa / 8.0, exponent - 7))
    magnitude = np.where((exponent == 15) & ((codes & 7) == 7), np.nan, magnitude).astype(np.float32)
    return np.where((codes & 0x80) != 0, -magnitude, magnitude).astype(np.float32)


def encode_e4m3(values) -> np.ndarray:
    """FP32 -> E4M3FN code, RNE, saturating to +-448, NaN -> 0x7F (formats.py:55-66).

    With the magnitude clipped to 448, the code is (E+6)*8 + M where E is the
    binade (floored at -6, the subnormal binade) and M = rint(|v| / 2^(E-3)) in
    [0, 16]; M = 16 carries into the next binade, and rint's ties-to-even on M is
    ties-to-even on the code because 8 is even.
    """
    v = np.asarray(values, dtype=np.float32)
    nan = np.isnan(v)
    magnitude = np.minimum(np.abs(np.where(nan, np.float32(0), v)), np.float32(E4M3_MAX)).astype(np.float64)
    _, binade = np.frexp(magnitude)
    exponent = np.where(magnitude < 2.0 ** -6, -6, binade - 1)
    steps = np.rint(np.ldexp(magnitude, 3 - exponent)).astype(np.int64)
    code = ((exponent + 6) * 8 + steps).astype(np.uint8)
    code = code | np.where(np.signbit(v), np.uint8(0x80), np.uint8(0)).astype(np.uint8)
    return np.where(nan, np.uint8(0x7F), code).astype(np.uint8)


def bf16_bits(values) -> np.ndarray:
    """FP32 -> BF16 storage bits, round-to-nearest-even, NaN quieted (formats.py:69-73)."""
    bits = np.asarray(values, dtype=np.float32).view(np.uint32).astype(np.uint64)
    is_nan = ((bits & 0x7F800000) == 0x7F800000) & ((bits & 0x007FFFFF) != 0)
    rounded = (bits + 0x7FFF + ((bits >> 16) & 1)) >> 16
    return np.where(is_nan, (bits >> 16) | 0x40, rounded).astype(np.uint16)


def bf16_values(bits) -> np.ndarray:
    """BF16 storage bits -> FP32 (formats.py:76-77)."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_round(values) -> np.ndarray:
    return bf16_values(bf16_bits(values))


def fma_f32(a, b, c) -> np.ndarray:
    """f32(a * b + c) with one rounding (an IEEE fused multiply-add in FP32), for finite FP32 arrays whose
    results are normal. a * b is exact in float64 (24 + 24 bits); the float64 sum s = a b + c is rounded,
    and its rounding error e is recovered exactly (Knuth's two-sum). Rounding s to FP32 is then the correct
    rounding of the exact value except when s lies exactly halfway between two FP32 values and e != 0: the
    exact value is then on e's side of the halfway point, and the result moves one FP32 step that way."""
    a, b, c = (np.asarray(v, dtype=np.float32) for v in (a, b, c))
    p = a.astype(np.float64) * b.astype(np.float64)
    c64 = c.astype(np.float64)
    s = p + c64
    bb = s - p
    e = (p - (s - bb)) + (c64 - bb)
    r = s.astype(np.float32)
    halfway = (s.view(np.uint64) & np.uint64((1 << 29) - 1)) == np.uint64(1 << 28)
    r64 = r.astype(np.float64)
    up = halfway & (e > 0) & (r64 < s)
    down = halfway & (e < 0) & (r64 > s)
    r = np.where(up, np.nextafter(r, np.float32(np.inf)), r)
    return np.where(down, np.nextafter(r, np.float32(-np.inf)), r).astype(np.float32)


def quantize_activation(values, block: int = 32) -> tuple[np.ndarray, np.ndarray]:
    """BF16-round, then per-block E4M3 codes with E8M0 scales (formats.py:80-94).

    scale exponent e = ceil(log2(f32(amax * f32(1/448)))) taken from the FP32
    bits (unbiased exponent + 1 when the mantissa is nonzero); amax is floored at
    1e-4 so an all-zero block gets code 105.
    """
    x = bf16_round(values)
    if x.shape[-1] % block or not np.isfinite(x).all():
        raise ValueError("Activation must be finite with a width divisible by 32")
    grouped = x.reshape(*x.shape[:-1], -1, block)
    amax = np.maximum(np.abs(grouped).max(axis=-1), AMAX_FLOOR).astype(np.float32)
    scaled = (amax * np.uint32(INV_448_BITS).view(np.float32)).astype(np.float32)
    bits = scaled.view(np.uint32)
    exponents = ((bits >> 23) & 0xFF).astype(np.int32) - 127 + ((bits & 0x7FFFFF) != 0)
    if np.any((exponents < -126) | (exponents > 127)):
        raise ValueError("Activation scale outside this probe's finite normal range")
    scales = (exponents + 127).astype(np.uint8)
    normalized = (grouped / e8m0_values(scales)[..., None]).astype(np.float32)
    codes = encode_e4m3(np.clip(normalized, np.float32(-E4M3_MAX), np.float32(E4M3_MAX)))
    return codes.reshape(x.shape), scales


def block_dots(act_codes, weight_values_f64, block: int = 32) -> np.ndarray:
    """Exact per-block dots [T, N, G] as FP32 (float64 products/sums are exact here).

    E4M3 x E2M1 products are multiples of 2^-10 below 2^12, so a 32-term sum
    needs at most 27 significant bits and float64 holds it exactly in any order.
    """
    a = e4m3_values(act_codes).astype(np.float64)
    t = a.shape[0]
    groups = a.shape[1] // block
    a = a.reshape(t, groups, block).transpose(1, 0, 2)             # [G, T, 32]
    w = weight_values_f64.reshape(weight_values_f64.shape[0], groups, block).transpose(1, 2, 0)  # [G, 32, N]
    dots = np.matmul(a, w)                                          # [G, T, N]
    return dots.transpose(1, 2, 0).astype(np.float32)               # [T, N, G]


def scaled_group_sum(dots, act_scales, weight_scales_f32) -> np.ndarray:
    """sum_g ((dot_g * sa_g) * sw_g) in FP32, g ascending (formats.py:115-118)."""
    sa = e8m0_values(act_scales)                                    # [T, G]
    t, n, groups = dots.shape
    result = np.zeros((t, n), dtype=np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        for g in range(groups):
            result = result + (dots[:, :, g] * sa[:, g:g + 1]) * weight_scales_f32[None, :, g]
    return result.astype(np.float32)


def mxfp4_gemv_fp32(act_codes, act_scales, packed_weight, weight_scales) -> np.ndarray:
    """E4M3 [T,K] (E8M0 per 32) x MXFP4 [N,K] -> FP32 [T,N] before the BF16 output rounding."""
    act_codes = np.atleast_2d(np.asarray(act_codes, dtype=np.uint8))
    act_scales = np.atleast_2d(np.asarray(act_scales, dtype=np.uint8))
    packed_weight = np.asarray(packed_weight, dtype=np.uint8)
    n, packed_k = packed_weight.shape
    k = packed_k * 2
    if act_codes.shape[1] != k or np.shape(weight_scales) != (n, k // 32) or act_scales.shape[1] != k // 32:
        raise ValueError("Mismatched GEMV dimensions")
    w = fp4_values(split_nibbles(packed_weight)).astype(np.float64)
    dots = block_dots(act_codes, w)
    return scaled_group_sum(dots, act_scales, e8m0_values(weight_scales))


def mxfp4_gemv_spec(act_codes, act_scales, packed_weight, weight_scales) -> np.ndarray:
    """BF16 output bits of the E4M3 x MXFP4 block GEMV (formats.py:97-118), batched over tokens."""
    return bf16_bits(mxfp4_gemv_fp32(act_codes, act_scales, packed_weight, weight_scales))


def fp8_block32_gemv_fp32(act_codes, act_scales, weight_codes, weight_scales) -> np.ndarray:
    """E4M3 [T,K] x E4M3 [N,K] with one E8M0 scale per 32x32 weight block (shared_probe.cu:36-38).

    Same order as the MXFP4 spec; the weight scale index is (row/32, group).
    E4M3 x E4M3 products are multiples of 2^-18 below 2^18, so 32-term sums stay
    exact in float64.
    """
    act_codes = np.atleast_2d(np.asarray(act_codes, dtype=np.uint8))
    act_scales = np.atleast_2d(np.asarray(act_scales, dtype=np.uint8))
    weight_codes = np.asarray(weight_codes, dtype=np.uint8)
    n, k = weight_codes.shape
    if act_codes.shape[1] != k or np.shape(weight_scales) != (n // 32, k // 32):
        raise ValueError("Mismatched FP8 block-32 GEMV dimensions")
    w = e4m3_values(weight_codes).astype(np.float64)
    dots = block_dots(act_codes, w)
    row_scales = np.repeat(e8m0_values(weight_scales), 32, axis=0)  # [N, G]
    return scaled_group_sum(dots, act_scales, row_scales)
