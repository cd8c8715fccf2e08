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

// Non-temporal (streaming) loads, the `nt` bit: for data read once per call, such as expert weights
// in decode. A plain blocked read of 2 GiB on MI355X runs at 6.9-7.0 TB/s with them, 6.0-6.2 TB/s without.
__device__ __forceinline__ uint32_t ldg32_nt(const uint8_t* p) {
  return __builtin_nontemporal_load((const __attribute__((address_space(1))) uint32_t*)(p));
}

__device__ __forceinline__ uint4 ldg128_nt(const uint8_t* p) {
  const u32x4_t v = __builtin_nontemporal_load((const __attribute__((address_space(1))) u32x4_t*)(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float ldgf(const float* p) {
  return *(const __attribute__((address_space(1))) float*)(p);
}

// Workgroup barrier ordering LDS only: the fences are restricted to the local address space, so the
// barrier waits for this wave's LDS operations (lgkmcnt) but leaves its global loads in flight. A plain
// __syncthreads() also waits for every outstanding global load (vmcnt(0)), which drains a kernel's
// register prefetch rings at every barrier.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// The s_waitcnt immediate that waits until at most n vector-memory operations of this wave are
// outstanding (lgkm and export counts left at their maxima: no wait on them).
constexpr int vm_wait_imm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// Asynchronous copies from global memory into LDS of 16 (4) bytes per lane: lane l's bytes land at
// lds + 16 l (4 l); lds is the wave-uniform LDS byte address. Counted by vmcnt like any other
// vector-memory load. Inline assembly rather than the compiler builtin: for the builtin the compiler
// treats every later wait on vmcnt as unordered (copies and register loads mixed) and widens it to
// vmcnt(0), which drains the copies in flight at each use of a register load; with the copies invisible
// to it, its waits for its own loads are exact (and cover a few more copies than needed, as the
// hardware counter also holds them). The caller orders its LDS reads after the copies with explicit
// waits. One wait state between the M0 write and the copy.
__device__ __forceinline__ void global_to_lds16(const void* src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(src), "s"(lds) : "m0");
}
__device__ __forceinline__ void global_to_lds4(const void* src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" : : "v"(src), "s"(lds) : "m0");
}

// Workgroup barrier for the global->LDS copy pipelines: the caller has already waited for its own copies
// and LDS reads (s_waitcnt) as far as the barrier must cover. Even the local-only fences of lds_barrier
// would wait for every copy in flight (the copies write LDS), so the barrier is issued bare; the empty
// assembly statements with a memory clobber keep the compiler from moving memory operations across it.
__device__ __forceinline__ void copy_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// Device-coherent 8-byte store and load: agent-scope relaxed atomics, which gfx950 issues with the sc1
// scope bit, so the store is written through to the device's coherence point and the load does not hit a
// stale line of this XCD's L2. Workgroups on different XCDs exchange data this way without the whole-L2
// write-back and invalidate that an agent-scope fence costs.
__device__ __forceinline__ void store_device(float* p, float a, float b) {
  const uint64_t v = (uint64_t)__float_as_uint(a) | ((uint64_t)__float_as_uint(b) << 32);
  __hip_atomic_store(reinterpret_cast<uint64_t*>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float2 load_device(const float* p) {
  const uint64_t v =
      __hip_atomic_load(reinterpret_cast<const uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return make_float2(__uint_as_float((uint32_t)v), __uint_as_float((uint32_t)(v >> 32)));
}

// Handoff buffers between workgroups (the split-K GEMV's partial sums) hold this FP32 pattern wherever no
// value is published: a signalling NaN, which FP32 arithmetic never produces (its NaN results are quiet).
constexpr uint32_t kHandoffEmpty = 0x7FA0DEADu;
constexpr int kHandoffPolls = 1 << 16;

// The pair `first` read from p, re-read until it is no longer the empty pattern (a pair is published by one
// 64-bit atomic, so its halves arrive together); at most kHandoffPolls reads, then NaN instead of a hang.
__device__ __forceinline__ float2 await_pair(float2 first, const float* p) {
  float2 v = first;
  for (int i = 0; __float_as_uint(v.x) == kHandoffEmpty; ++i) {
    if (i == kHandoffPolls) return make_float2(__builtin_nanf(""), __builtin_nanf(""));
    __builtin_amdgcn_s_sleep(1);
    v = load_device(p);
  }
  return v;
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

// As mfma_fp4_fp8, with the A scale taken from byte kByte of the word sa4 (the instruction's opsel
// selects it; checked against the extracted byte on gfx950).
template <int kByte>
__device__ __forceinline__ v4f mfma_fp4_fp8_sel(uint4 a, uint4 b0, uint4 b1, v4f c, uint32_t sa4, int sb) {
  const v8i av = {(int)a.x, (int)a.y, (int)a.z, (int)a.w, 0, 0, 0, 0};
  const v8i bv = {(int)b0.x, (int)b0.y, (int)b0.z, (int)b0.w, (int)b1.x, (int)b1.y, (int)b1.z, (int)b1.w};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bv, c, 4, 0, kByte, (int)sa4, 0, sb);
}

// Maximum over each aligned group of lanes, in every lane of the group, by DPP (VALU steps instead of
// LDS-routed swizzles; a maximum is exact in any order): 16-lane rows by rotations of 8, 4, 2 and 1, and
// quads by two quad permutations. Every lane of a group must be active.
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xF, 0xF, false)));   // row_ror:8
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x124, 0xF, 0xF, false)));   // row_ror:4
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x122, 0xF, 0xF, false)));   // row_ror:2
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x121, 0xF, 0xF, false)));   // row_ror:1
  return v;
}
__device__ __forceinline__ float quad_max(float v) {
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false)));   // [1,0,3,2]
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false)));   // [2,3,0,1]
  return v;
}

// E4M3 codes of four FP32 values clamped to [-448, 448] (NaN -> 0x7F), packed low value first: equal to
// mx::e4m3_encode(clamp(v)) for every FP32 input. The gfx950 pair conversion (round to nearest even,
// OCP E4M3) was checked against mx::e4m3_encode on every FP32 value with |v| <= 448; it encodes NaN as
// 0xFF, so NaN lanes are patched to the encoder's 0x7F.
__device__ __forceinline__ uint32_t e4m3x4(float a, float b, float c, float d) {
  auto clamp = [](float y) { return y > 448.f ? 448.f : (y < -448.f ? -448.f : y); };
  const uint32_t lo = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(clamp(a), clamp(b), 0, false);
  uint32_t w = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(clamp(c), clamp(d), (int)lo, true);
  w = a != a ? (w & 0xFFFFFF00u) | 0x7Fu : w;
  w = b != b ? (w & 0xFFFF00FFu) | 0x7F00u : w;
  w = c != c ? (w & 0xFF00FFFFu) | 0x7F0000u : w;
  w = d != d ? (w & 0x00FFFFFFu) | 0x7F000000u : w;
  return w;
}

// mx::bf16_round written with selects only (no divergent branch): round to nearest even, NaN quieted.
__device__ __forceinline__ float bf16_round_sel(float f) {
  const uint32_t b = mx::f2u(f);
  const uint32_t rne = (b + 0x7FFFu + ((b >> 16) & 1u)) & 0xFFFF0000u;
  const uint32_t qnan = (b & 0xFFFF0000u) | 0x400000u;
  return mx::u2f((b & 0x7FFFFFFFu) > 0x7F800000u ? qnan : rne);
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

// Entries of the SiLU table: silu_f32 of every BF16 gate value (index = BF16 bits), then of the clamp
// limit (index kSiluLimit, used when limit > 0 and the gate exceeds it).
constexpr uint32_t kSiluLimit = 65536, kSiluEntries = 65537;

// swiglu_element with silu_f32(gate) read from the SiLU table: the table holds the same function of the
// same inputs (the gate is a BF16 value or, clamped, the limit), so the result has the same bits.
__device__ __forceinline__ float swiglu_table(const float* silu_table, uint32_t b1, uint32_t b3, float limit,
                                              bool weighted, float rw) {
  const float gate = mx::bf16_value(b1);
  float upf = mx::bf16_value(b3);
  uint32_t idx = b1;
  if (limit > 0.f) {
    if (gate > limit) idx = kSiluLimit;
    if (upf > limit) upf = limit;
    if (upf < -limit) upf = -limit;
  }
  const float silu = ldgf(silu_table + idx);
  const float product = silu * upf;
  const float routed = weighted ? rw * product : product;
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

// One token's routing list made valid in place: an id outside [0, E) or equal to an earlier id of the token
// is replaced by the smallest expert the token does not name, with route weight 0, so every later step sees
// k distinct in-range experts and stays in bounds. Returns how many ids were replaced (the caller counts
// them in the layer's routing error word; the host refuses the call's output when it is nonzero).
__device__ __forceinline__ int repair_token_routes(int32_t* ids, float* w, int k, int E) {
  int replaced = 0;
  for (int i = 0; i < k; ++i) {
    bool bad = ids[i] < 0 || ids[i] >= E;
    for (int j = 0; j < i && !bad; ++j) bad = ids[j] == ids[i];
    if (!bad) continue;
    for (int e = 0; e < E; ++e) {
      bool used = false;
      for (int j = 0; j < k && !used; ++j) used = j != i && ids[j] == e;
      if (!used) {
        ids[i] = e;
        break;
      }
    }
    w[i] = 0.f;
    ++replaced;
  }
  return replaced;
}

}  // namespace mxd
