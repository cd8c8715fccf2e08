// Scalar numerics shared by the gfx950 kernels and the host-side check build.
//
// Every function here is bit-exact by construction (integer arithmetic on FP32
// bit patterns, or a single IEEE-rounded FP32 operation). The same text is
// compiled by hipcc for the device and by g++ into libmxmoe_hostcheck.so, which
// the CPU tests compare exhaustively against the NumPy oracle.
//
// Reference behaviour restated (shell-term/vesper):
//   fp4 decode          src/vesper/kernels/format_probe.cu:7-11, formats.py:11-21
//   e8m0 decode         format_probe.cu:13-15, formats.py:24-29
//   e4m3 encode         formats.py:55-66 (RNE, saturate to 448, NaN -> 0x7F)
//   bf16 rounding       formats.py:69-73 (RNE, NaN quieted)
//   per-32 act quant    formats.py:80-94, format_probe.cu:37-52
#pragma once
#include <stdint.h>

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define MX_HD __host__ __device__ __forceinline__
#else
#include <math.h>
#include <string.h>
#define MX_HD static inline
#endif

namespace mx {

MX_HD uint32_t f2u(float f) { return __builtin_bit_cast(uint32_t, f); }
MX_HD float u2f(uint32_t u) { return __builtin_bit_cast(float, u); }

// FP32 nearest to 1/448 (the block quantizer's reciprocal of the E4M3 maximum).
constexpr uint32_t kInv448Bits = 0x3B124925u;
// FP32 nearest to 1e-4 (the per-block amax floor).
constexpr uint32_t kAmaxFloorBits = 0x38D1B717u;

// E2M1 code (4 bits) -> FP32; bit 3 is the sign, -0 preserved.
MX_HD float fp4_value(uint32_t code) {
  // magnitudes {0, .5, 1, 1.5, 2, 3, 4, 6} as FP32 bit patterns
  const uint32_t e = (code >> 1) & 3u, m = code & 1u;
  uint32_t bits = 0;
  if (e == 0) bits = m ? 0x3F000000u : 0u;                       // 0.5 or 0
  else bits = ((126u + e) << 23) | (m << 22);                     // (1 + m/2) * 2^(e-1)
  return u2f(bits | ((code & 8u) << 28));
}

// E8M0 scale byte -> FP32: 2^(c-127); c = 0 -> 2^-127 (subnormal); c = 255 -> NaN.
MX_HD float e8m0_value(uint32_t code) {
  return u2f(code == 0 ? 0x00400000u : code == 255 ? 0x7FC00000u : (code << 23));
}

// E4M3FN code -> FP32 (bias 7, subnormal m/512, 0x7F/0xFF NaN).
MX_HD float e4m3_value(uint32_t code) {
  const uint32_t e = (code >> 3) & 15u, m = code & 7u, s = (code & 0x80u) << 24;
  if (e == 15 && m == 7) return u2f(s | 0x7FC00000u);
  if (e == 0) {
    if (m == 0) return u2f(s);
    // m * 2^-9: normalise the 3-bit mantissa
    uint32_t shift = m >= 4 ? 0 : m >= 2 ? 1 : 2;               // leading one to bit 2
    uint32_t mm = (m << shift) & 3u;                             // bits below the leading one
    uint32_t exp = 127 - 9 + 2 - shift;                          // value = (4+mm)/4 * 2^(2-shift-9)
    return u2f(s | (exp << 23) | (mm << 21));
  }
  return u2f(s | ((e + 120u) << 23) | (m << 20));
}

// FP32 -> E4M3FN code: round-to-nearest-even, |v| >= 448 (incl. inf) saturates to
// +-448 (0x7E/0xFE), NaN -> 0x7F.
MX_HD uint32_t e4m3_encode(float v) {
  const uint32_t b = f2u(v);
  const uint32_t sign = (b >> 24) & 0x80u;
  const uint32_t mag = b & 0x7FFFFFFFu;
  if (mag > 0x7F800000u) return 0x7Fu;
  if (mag >= 0x43E00000u) return sign | 0x7Eu;                   // 448.0
  const uint32_t ef = mag >> 23;
  if (ef >= 121) {                                               // |v| >= 2^-6: E4M3 normal range
    const uint32_t lsb = (mag >> 20) & 1u;
    const uint32_t r = (mag + 0x7FFFFu + lsb) >> 20;             // RNE to 3 mantissa bits (carry ok)
    return sign | (r - (120u << 3));
  }
  if (ef == 0) return sign;                                      // FP32 subnormal: rounds to 0
  // E4M3 subnormal: code = rint(|v| * 2^9) with |v| = M * 2^(ef-150), M = 1.m * 2^23
  const uint32_t M = (mag & 0x7FFFFFu) | 0x800000u;
  const uint32_t s = 141u - ef;                                  // >= 21
  if (s >= 32) return sign;
  const uint32_t q = M >> s;
  const uint32_t rem = M & ((1u << s) - 1u);
  const uint32_t half = 1u << (s - 1);
  const uint32_t up = (rem > half) || (rem == half && (q & 1u));
  return sign | (q + up);
}

// FP32 -> BF16 bits, round-to-nearest-even, NaN quieted.
MX_HD uint32_t bf16_bits(float f) {
  const uint32_t b = f2u(f);
  if ((b & 0x7F800000u) == 0x7F800000u && (b & 0x7FFFFFu)) return (b >> 16) | 0x40u;
  return (b + 0x7FFFu + ((b >> 16) & 1u)) >> 16;
}

MX_HD float bf16_value(uint32_t bits) { return u2f(bits << 16); }
MX_HD float bf16_round(float f) { return bf16_value(bf16_bits(f)); }

// E8M0 code of one activation block from its (floored) amax:
// e = unbiased exponent of f32(amax * f32(1/448)), +1 when its mantissa is nonzero.
MX_HD uint32_t act_scale_code(float amax_floored) {
  const uint32_t bits = f2u(amax_floored * u2f(kInv448Bits));
  const int32_t e = (int32_t)((bits >> 23) & 255u) - 127 + ((bits & 0x7FFFFFu) != 0);
  return (uint32_t)(e + 127);
}

// One activation value -> E4M3 code given its block's E8M0 scale value s = 2^e:
// q = E4M3(clamp(x / s, -448, 448)) with IEEE division (exact except underflow).
MX_HD uint32_t act_quant_value(float x, float s) {
  float y = x / s;
  y = y > 448.f ? 448.f : (y < -448.f ? -448.f : y);
  return e4m3_encode(y);
}

// act_quant_value for a power-of-two scale s = 2^e (an E8M0 value), given inv_s = 1 / s = 2^-e: x * 2^-e
// and x / 2^e are the same exact value, correctly rounded by either operation (in the subnormal range
// too), so the codes are identical; a multiply replaces an IEEE division per value.
MX_HD uint32_t act_quant_pow2(float x, float inv_s) {
  float y = x * inv_s;
  y = y > 448.f ? 448.f : (y < -448.f ? -448.f : y);
  return e4m3_encode(y);
}

// FP32 scale of one per-token 128-wide activation block (the FP32-scale FP8 profile):
// s = f32(max(amax, 1e-4)) / 448 with one IEEE division; the codes are then act_quant_value(x, s).
MX_HD float act128_scale(float amax) {
  const float floor = u2f(kAmaxFloorBits);
  return (amax > floor ? amax : floor) / 448.0f;
}

// x / s correctly rounded, from inv = RN(1 / s) computed once per block: q0 = RN(x inv) is within an ulp
// of x / s, the remainder x - q0 s is exact in one fused multiply-add, and q0 + r inv rounded once is the
// correctly rounded quotient (Markstein's correction step); the sign is taken from x so that -0 / s stays
// -0. Three operations per value instead of an IEEE division. Over every BF16 x (NaN and infinities
// included) and every scale s = act128_scale(amax) with |x| <= amax (the only quotients the quantizers
// form) the result equals x / s bit for bit wherever |x / s| >= 2^-90, and below that both encode to a
// signed zero in E4M3, so the codes are the division's on every input -- checked exhaustively on the host
// (mxh_act128_quotient_check). An infinite s (infinite amax; s is never NaN) has inv = 0, where x * inv is
// already x / s (signed zero, or NaN for an infinite or NaN x); selected without a branch.
MX_HD float act128_quotient(float x, float s, float inv) {
  const float q0 = x * inv;
  const float r = fmaf(-q0, s, x);
  const float q = copysignf(fmaf(r, inv, q0), x);
  return s <= 3.4028234663852886e38f ? q : q0;
}

}  // namespace mx
