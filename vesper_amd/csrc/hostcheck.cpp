// Host build of the device numerics (mx_numerics.h) for exhaustive CPU comparison with the oracle.
// Nothing here runs on the GPU path; libmxmoe.so compiles the same header for gfx950.
#include <cmath>
#include <cstdint>

#include "mx_numerics.h"

extern "C" {

void mxh_e4m3_encode(const float* in, uint8_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = (uint8_t)mx::e4m3_encode(in[i]);
}

void mxh_e4m3_decode(const uint8_t* in, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = mx::e4m3_value(in[i]);
}

void mxh_fp4_decode(const uint8_t* codes, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = mx::fp4_value(codes[i] & 15u);
}

void mxh_e8m0_decode(const uint8_t* codes, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = mx::e8m0_value(codes[i]);
}

void mxh_bf16_bits(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = (uint16_t)mx::bf16_bits(in[i]);
}

// Same block algorithm as act_quant32_kernel: BF16-round, amax with floor, E8M0 code, E4M3 codes.
void mxh_act_quant32(const float* x, uint8_t* q, uint8_t* s, int64_t rows, int64_t width) {
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t b = 0; b < width / 32; ++b) {
      const float* v = x + r * width + b * 32;
      float amax = 0.f;
      for (int j = 0; j < 32; ++j) amax = std::fmax(amax, std::fabs(mx::bf16_round(v[j])));
      amax = std::fmax(amax, mx::u2f(mx::kAmaxFloorBits));
      const uint32_t code = mx::act_scale_code(amax);
      const float sc = mx::e8m0_value(code);
      for (int j = 0; j < 32; ++j) q[r * width + b * 32 + j] = (uint8_t)mx::act_quant_value(mx::bf16_round(v[j]), sc);
      s[r * (width / 32) + b] = (uint8_t)code;
    }
}

// Exhaustive check of mx::act128_quotient against IEEE division over the quantizer's whole domain: every
// positive BF16 amax up to infinity (amax below the floor shares the floor's scale, checked once), s =
// act128_scale(amax), and every BF16 x of either sign with |x| <= amax, plus a NaN x (a block's amax passes
// over NaN). Returns the number of (amax, x)
// pairs whose quotient bits differ; *code_mismatches the number whose E4M3 codes differ, *max_quotient the
// largest |x / s| among the differing quotients, *pairs the pairs checked.
int64_t mxh_act128_quotient_check(int64_t* code_mismatches, float* max_quotient, int64_t* pairs) {
  int64_t bad = 0, bad_code = 0, n = 0;
  float qmax = 0.f;
  const float floor = mx::u2f(mx::kAmaxFloorBits);
  for (uint32_t a = 0; a <= 0x7F80u; ++a) {
    const float amax = mx::u2f(a << 16);
    const bool at_floor = !(amax > floor);
    // below the floor every amax gives the floor's scale: check it once, with the largest such amax
    if (at_floor && !(mx::u2f((a + 1) << 16) > floor)) continue;
    const float s = mx::act128_scale(amax);
    const float inv = 1.0f / s;
    for (uint32_t v = 0; v <= a + 1; ++v)
      for (uint32_t sign = 0; sign < 2; ++sign) {
        // v = a + 1 stands for a NaN x
        const float x = v <= a ? mx::u2f((v << 16) | (sign << 31)) : mx::u2f(0x7FC00000u | (sign << 31));
        const float want = x / s, got = mx::act128_quotient(x, s, inv);
        ++n;
        if (want != want && got != got) continue;   // both NaN: E4M3 0x7F either way
        if (mx::f2u(want) != mx::f2u(got)) {
          ++bad;
          qmax = std::fmax(qmax, std::fabs(want));
          if (mx::e4m3_encode(want > 448.f ? 448.f : (want < -448.f ? -448.f : want)) !=
              mx::e4m3_encode(got > 448.f ? 448.f : (got < -448.f ? -448.f : got)))
            ++bad_code;
        }
      }
  }
  *code_mismatches = bad_code;
  *max_quotient = qmax;
  *pairs = n;
  return bad;
}

}  // extern "C"
