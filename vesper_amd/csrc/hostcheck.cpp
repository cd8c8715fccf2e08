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

}  // extern "C"
