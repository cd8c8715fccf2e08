// Device-side helpers shared by the kernel translation units (gfx950 only).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mx_numerics.h"

namespace mxd {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

// Loads through the global address space. Pointers that come from device tables or structs are
// otherwise treated as generic (flat) addresses.
__device__ __forceinline__ uint32_t ldg32(const uint8_t* p) {
  return *(const __attribute__((address_space(1))) uint32_t*)(p);
}

__device__ __forceinline__ uint4 ldg128(const uint8_t* p) {
  const u32x4_t v = *(const __attribute__((address_space(1))) u32x4_t*)(p);
  return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float ldgf(const float* p) {
  return *(const __attribute__((address_space(1))) float*)(p);
}

// V_MFMA_SCALE_F32_16X16X128_F8F6F4 operand layouts (measured on gfx950 with one-hot probes):
//   FP4 A (cbsz 4, 4 VGPRs): lane l = row l % 16, K = 32 (l / 16) + nibble j, low nibble first.
//   FP8 A (cbsz 0) and FP8 B (blgp 0), 8 VGPRs: lane l = row / column l % 16; bytes 0-15 hold
//     K = 16 (l / 16) + j and bytes 16-31 hold K = 64 + 16 (l / 16) + j.
//   scale_a / scale_b: lane l scales row / column l % 16 over the 32-wide K block l / 16.
//   D: lane l, register i = row 4 (l / 16) + i, column l % 16.
__device__ __forceinline__ v4f mfma_fp4_fp8(uint4 a, uint4 b0, uint4 b1, v4f c, int sa, int sb) {
  const v8i av = {(int)a.x, (int)a.y, (int)a.z, (int)a.w, 0, 0, 0, 0};
  const v8i bv = {(int)b0.x, (int)b0.y, (int)b0.z, (int)b0.w, (int)b1.x, (int)b1.y, (int)b1.z, (int)b1.w};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bv, c, 4, 0, 0, sa, 0, sb);
}

__device__ __forceinline__ v4f mfma_fp8_fp8(uint4 a0, uint4 a1, uint4 b0, uint4 b1, v4f c, int sa, int sb) {
  const v8i av = {(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w, (int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
  const v8i bv = {(int)b0.x, (int)b0.y, (int)b0.z, (int)b0.w, (int)b1.x, (int)b1.y, (int)b1.z, (int)b1.w};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bv, c, 0, 0, 0, sa, 0, sb);
}

// silu(g) = g / (1 + exp(-g)); exp is evaluated in float64 and rounded once to FP32.
__device__ __forceinline__ float silu_f32(float g) {
  const float e = (float)exp(-(double)g);
  return g / (1.0f + e);
}

// SwiGLU epilogue of one intermediate element (expert_probe.cu:10-25): W1/W3 outputs as BF16 bits ->
// clamp (limit > 0: gate <= limit, -limit <= up <= limit) -> silu(gate) * up -> times the route weight
// when weighted -> BF16. Returns the BF16-valued down input; `tr` (nullable) receives the FP32 trace
// {clamped gate, clamped up, silu, product, routed}.
__device__ __forceinline__ float swiglu_element(uint32_t b1, uint32_t b3, float limit, bool weighted, float rw,
                                                float* tr) {
  float gate = mx::bf16_value(b1), upf = mx::bf16_value(b3);
  if (limit > 0.f) {
    if (gate > limit) gate = limit;
    if (upf > limit) upf = limit;
    if (upf < -limit) upf = -limit;
  }
  const float silu = silu_f32(gate);
  const float product = silu * upf;
  const float routed = weighted ? rw * product : product;
  if (tr) {
    tr[0] = gate;
    tr[1] = upf;
    tr[2] = silu;
    tr[3] = product;
    tr[4] = routed;
  }
  return mx::bf16_round(routed);
}

// Byte offsets of the tiled expert blob for hidden H and intermediate I:
//   [0, I*H)            gate/up A operands: row group g (I/32 groups) x chunk c (H/128) x tile t x lane
//                       (16 B), tile t = W1 rows 32g + 8t + (0..7) as MFMA rows 0-7 and the same W3
//                       rows as MFMA rows 8-15; lane l = MFMA row l % 16, K block 4c + l / 16
//   [gu_s, +I*H/16)     gate/up scale words: g x c x lane (4 B, byte t = tile t)
//   [dn_w, +H*I/2)      down A operands: row group b (H/64) x chunk c (I/128) x tile t x lane, tile t =
//                       W2 rows 64b + 16t + (0..15)
//   [dn_s, +H*I/32)     down scale words: b x c x lane
struct TiledOffsets {
  size_t gu_s, dn_w, dn_s, total;
};

__host__ __device__ __forceinline__ TiledOffsets tiled_offsets(int H, int I) {
  const size_t ih = (size_t)I * H;
  TiledOffsets o;
  o.gu_s = ih;
  o.dn_w = ih + ih / 16;
  o.dn_s = o.dn_w + ih / 2;
  o.total = o.dn_s + ih / 32;
  return o;
}

}  // namespace mxd
