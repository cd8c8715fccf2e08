// The BF16-activation MXFP4 expert: y = W2 . (silu(W1 . x) * (W3 . x)) with BF16 activations, FP32
// accumulation, no activation quantization and no clamp (the benchmark's configuration 0), on the same tiled
// expert bytes the decode layer streams (mx_tile_expert).
//
// The reference's expert (ExpertExecutor.execute, src/vesper/expert.py:51-79) quantizes x and the down
// input to E4M3 per 32-block and feeds scaled MFMAs; this profile keeps the activations exact, so its
// products run on the VALU: every 16-byte MX block of a weight row (32 E2M1 values, one E8M0 scale) is
// converted to exact values with V_CVT_SCALEF32_PK_* at scale 1, dotted with the activations, and the block's
// partial sum is multiplied by its scale (a power of two: exact) and accumulated in FP32.
//
// Three launches on the caller's stream:
//   gate/up (I/32 row groups x KS K-splits, per group of up to 4 tokens): W1 and W3 rows against BF16 x staged in LDS,
//     V_DOT2C_F32_BF16 per pair (the products of two BF16 values are exact in FP32); partial sums per K-split
//     to scratch [KS][T][2I];
//   SwiGLU (T x I threads): g, u = the K-split partials summed in split order; h = silu(g) * u (* route
//     weight) in FP32 (optionally written out with g and u);
//   down (H/64 row blocks, per group of up to 4 tokens): W2 rows against FP32 h staged in LDS, V_FMA_F32 per element;
//     y rounded once to BF16.
// Every sum runs in a fixed order (lanes' blocks, then waves, then splits), so results do not depend on
// scheduling. At T = 1 the products cost ~1.3 VALU instructions per weight byte, below the HBM stream.
#include <algorithm>
#include <cmath>

#include "mx_device.h"
#include "mx_internal.h"
#include "mx_numerics.h"

namespace {

using mxd::ldg128_nt;
using mxd::ldg32_nt;
using mxd::tiled_offsets;
using mxd::TiledOffsets;

typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef float v2f __attribute__((ext_vector_type(2)));

constexpr int kTok = 4;          // tokens per workgroup pass (LDS holds their activations)
constexpr int kMaxTokens = 16;
constexpr int kMaxSplits = 8;
constexpr int kMaxHidden = 8192; // gate/up LDS: kTok x H BF16 = 64 KB
constexpr int kMaxInter = 4096;  // down LDS: kTok x I FP32 = 64 KB

struct GateUpArgs {
  const uint8_t* blob;
  const uint16_t* x;   // [T][H] BF16
  float* part;         // [KS][T][2I]: g partials in [0, I), u partials in [I, 2I)
  int H, I, T, splits;
};

struct SwigluArgs {
  const float* part;
  const float* route_w;   // [T] or null
  float* h;               // [T][I]
  float* gu;              // [T][2I] or null
  int I, T, splits;
};

struct DownArgs {
  const uint8_t* blob;
  const float* h;   // [T][I]
  uint16_t* y;      // [T][H]
  int H, I, T;
};

// 32 E2M1 values of one 16-byte MX block as 16 BF16 pairs (element 2j in .x, 2j + 1 in .y), exact.
__device__ __forceinline__ void fp4_block_bf16(const uint4 w, v2bf (&p)[16]) {
  const uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    p[4 * d + 0] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(words[d], 1.0f, 0);
    p[4 * d + 1] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(words[d], 1.0f, 1);
    p[4 * d + 2] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(words[d], 1.0f, 2);
    p[4 * d + 3] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(words[d], 1.0f, 3);
  }
}

// The same block as 16 FP32 pairs.
__device__ __forceinline__ void fp4_block_f32(const uint4 w, v2f (&p)[16]) {
  const uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    p[4 * d + 0] = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(words[d], 1.0f, 0);
    p[4 * d + 1] = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(words[d], 1.0f, 1);
    p[4 * d + 2] = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(words[d], 1.0f, 2);
    p[4 * d + 3] = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(words[d], 1.0f, 3);
  }
}

// grid (I/32, KS), 256 threads, dynamic LDS kTok * H * 2 bytes; one launch per group of up to 4 tokens (x and
// part point at the group's first token). Row group g holds W1 and W3 rows
// [32g, 32g + 32) in the tiled gate/up layout: per 128-wide K chunk, tile t's lane l = (m, q) carries row
// 32g + 8t + (m & 7) of W1 (m < 8) or W3 (m >= 8), K block 4c + q, and its E8M0 code in byte t of the lane's
// scale word. The workgroup's chunk range is split K-split ks of the H/128 chunks, quartered over the waves.
template <int NT>
__global__ __launch_bounds__(256) void bf16_gateup_kernel(GateUpArgs a) {
  extern __shared__ uint32_t s_x[];   // [kTok][H/2] BF16 pairs
  __shared__ float red[4][4][kTok][64];
  const int g = blockIdx.x, ks = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int H = a.H, I = a.I, hw = H / 2;
  for (int i = tid; i < NT * hw; i += 256) {
    const int k = i / hw, j = i - k * hw;
    s_x[k * hw + j] = reinterpret_cast<const uint32_t*>(a.x + (size_t)k * H)[j];
  }
  __syncthreads();
  const int chunks = H / 128;
  const int c_lo = chunks * ks / a.splits, c_hi = chunks * (ks + 1) / a.splits;
  const int n = c_hi - c_lo;
  const int c0 = c_lo + n * wave / 4, c1 = c_lo + n * (wave + 1) / 4;
  const int q = lane >> 4;
  const uint8_t* wp = a.blob + (size_t)g * chunks * 4096 + 16 * lane;
  const uint8_t* sp = a.blob + tiled_offsets(H, I).gu_s + (size_t)g * chunks * 256 + 4 * lane;
  float acc[4][NT];
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int k = 0; k < NT; ++k) acc[t][k] = 0.f;
  uint4 w[4];
  uint32_t sw = 0;
  if (c0 < c1) {
#pragma unroll
    for (int t = 0; t < 4; ++t) w[t] = ldg128_nt(wp + (size_t)c0 * 4096 + t * 1024);
    sw = ldg32_nt(sp + (size_t)c0 * 256);
  }
  for (int c = c0; c < c1; ++c) {
    uint4 cur[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) cur[t] = w[t];
    const uint32_t scur = sw;
    if (c + 1 < c1) {   // the next chunk's loads are in flight while this one is multiplied
#pragma unroll
      for (int t = 0; t < 4; ++t) w[t] = ldg128_nt(wp + (size_t)(c + 1) * 4096 + t * 1024);
      sw = ldg32_nt(sp + (size_t)(c + 1) * 256);
    }
    const int kb = 4 * c + q;   // this lane's 32-wide K block
    uint4 xv[NT][4];
#pragma unroll
    for (int k = 0; k < NT; ++k)
#pragma unroll
      for (int j = 0; j < 4; ++j) xv[k][j] = reinterpret_cast<const uint4*>(s_x + k * hw + 16 * kb)[j];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      v2bf p[16];
      fp4_block_bf16(cur[t], p);
      const float scale = mx::e8m0_value((scur >> (8 * t)) & 0xFF);
#pragma unroll
      for (int k = 0; k < NT; ++k) {
        const uint32_t xs[16] = {xv[k][0].x, xv[k][0].y, xv[k][0].z, xv[k][0].w, xv[k][1].x, xv[k][1].y,
                                 xv[k][1].z, xv[k][1].w, xv[k][2].x, xv[k][2].y, xv[k][2].z, xv[k][2].w,
                                 xv[k][3].x, xv[k][3].y, xv[k][3].z, xv[k][3].w};
        float part = 0.f;
#pragma unroll
        for (int j = 0; j < 16; ++j)
          part = __builtin_amdgcn_fdot2_f32_bf16(p[j], __builtin_bit_cast(v2bf, xs[j]), part, false);
        acc[t][k] = fmaf(part, scale, acc[t][k]);
      }
    }
  }
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int k = 0; k < NT; ++k) red[wave][t][k][lane] = acc[t][k];
  __syncthreads();
  // thread (t, m, k): the row's sum over the 4 K quarters of the chunk and the 4 waves, in that order
  const int t = tid >> 6, m = (tid >> 2) & 15, k = tid & 3;
  if (k < NT) {
    float s = 0.f;
#pragma unroll
    for (int wv = 0; wv < 4; ++wv)
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) s += red[wv][t][k][m + 16 * qq];
    const int row = 32 * g + 8 * t + (m & 7);
    a.part[((size_t)ks * a.T + k) * (2 * I) + (m < 8 ? row : I + row)] = s;
  }
}

// grid ceil(T * I / 256), 256 threads.
__global__ __launch_bounds__(256) void bf16_swiglu_kernel(SwigluArgs a) {
  const int idx = blockIdx.x * 256 + threadIdx.x;
  if (idx >= a.T * a.I) return;
  const int tok = idx / a.I, i = idx - tok * a.I;
  const size_t stride = (size_t)a.T * 2 * a.I;
  const float* p = a.part + (size_t)tok * 2 * a.I;
  float g = 0.f, u = 0.f;
  for (int ks = 0; ks < a.splits; ++ks) {
    g += p[ks * stride + i];
    u += p[ks * stride + a.I + i];
  }
  float h = g / (1.0f + expf(-g)) * u;
  if (a.route_w) h *= a.route_w[tok];
  a.h[idx] = h;
  if (a.gu) {
    a.gu[(size_t)tok * 2 * a.I + i] = g;
    a.gu[(size_t)tok * 2 * a.I + a.I + i] = u;
  }
}

// grid (H/64), 256 threads, dynamic LDS kTok * I * 4 bytes; one launch per group of up to 4 tokens (h and y
// point at the group's first token). Row block b holds W2 rows
// [64b, 64b + 64) in the tiled down layout: per 128-wide K chunk, tile t's lane (m, q) carries row
// 64b + 16t + m, K block 4c + q. The I/128 chunks are quartered over the waves.
template <int NT>
__global__ __launch_bounds__(256) void bf16_down_kernel(DownArgs a) {
  extern __shared__ float s_h[];   // [kTok][I]
  __shared__ float red[4][4][kTok][64];
  const int b = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int H = a.H, I = a.I;
  for (int i = tid; i < NT * I; i += 256) s_h[i] = a.h[i];
  __syncthreads();
  const int chunks = I / 128;
  const int c0 = chunks * wave / 4, c1 = chunks * (wave + 1) / 4;
  const int q = lane >> 4;
  const TiledOffsets off = tiled_offsets(H, I);
  const uint8_t* wp = a.blob + off.dn_w + (size_t)b * chunks * 4096 + 16 * lane;
  const uint8_t* sp = a.blob + off.dn_s + (size_t)b * chunks * 256 + 4 * lane;
  float acc[4][NT];
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int k = 0; k < NT; ++k) acc[t][k] = 0.f;
  uint4 w[4];
  uint32_t sw = 0;
  if (c0 < c1) {
#pragma unroll
    for (int t = 0; t < 4; ++t) w[t] = ldg128_nt(wp + (size_t)c0 * 4096 + t * 1024);
    sw = ldg32_nt(sp + (size_t)c0 * 256);
  }
  for (int c = c0; c < c1; ++c) {
    uint4 cur[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) cur[t] = w[t];
    const uint32_t scur = sw;
    if (c + 1 < c1) {
#pragma unroll
      for (int t = 0; t < 4; ++t) w[t] = ldg128_nt(wp + (size_t)(c + 1) * 4096 + t * 1024);
      sw = ldg32_nt(sp + (size_t)(c + 1) * 256);
    }
    const int kb = 4 * c + q;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      v2f p[16];
      fp4_block_f32(cur[t], p);
      const float scale = mx::e8m0_value((scur >> (8 * t)) & 0xFF);
#pragma unroll
      for (int k = 0; k < NT; ++k) {
        const float4* hv = reinterpret_cast<const float4*>(s_h + k * I + 32 * kb);
        float part = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float4 v = hv[j];
          part = fmaf(p[2 * j].x, v.x, part);
          part = fmaf(p[2 * j].y, v.y, part);
          part = fmaf(p[2 * j + 1].x, v.z, part);
          part = fmaf(p[2 * j + 1].y, v.w, part);
        }
        acc[t][k] = fmaf(part, scale, acc[t][k]);
      }
    }
  }
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int k = 0; k < NT; ++k) red[wave][t][k][lane] = acc[t][k];
  __syncthreads();
  const int t = tid >> 6, m = (tid >> 2) & 15, k = tid & 3;
  if (k < NT) {
    float s = 0.f;
#pragma unroll
    for (int wv = 0; wv < 4; ++wv)
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) s += red[wv][t][k][m + 16 * qq];
    a.y[(size_t)k * H + 64 * b + 16 * t + m] = (uint16_t)mx::bf16_bits(s);
  }
}

bool is_aligned(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

}  // namespace

using mxi::as_stream;
using mxi::use;

static uint64_t bf16_scratch_bytes(int32_t I, int32_t T) {
  return (uint64_t)kMaxSplits * T * 2 * I * sizeof(float) + (uint64_t)T * I * sizeof(float);
}

int mx_expert_forward_bf16(mx_ctx* ctx, const void* tiled, int32_t H, int32_t I, const uint16_t* x, int32_t T,
                           const float* route_w, float* h, float* gu, uint16_t* y, void* stream) {
  if (int s = use(ctx)) return s;
  MX_REQUIRE(tiled != nullptr && is_aligned(tiled, 256), "mx_expert_forward_bf16: 256-byte aligned tiled expert required");
  MX_REQUIRE(H > 0 && H % 128 == 0 && H <= kMaxHidden && I > 0 && I % 128 == 0 && I <= kMaxInter,
             "mx_expert_forward_bf16: H and I must be positive multiples of 128, H <= %d and I <= %d", kMaxHidden,
             kMaxInter);
  MX_REQUIRE(T >= 0 && T <= kMaxTokens, "token count %d outside [0, %d]", T, kMaxTokens);
  if (T == 0) return MX_OK;
  MX_REQUIRE(x && y && is_aligned(x, 16) && is_aligned(y, 4), "mx_expert_forward_bf16: x (16-byte) and y required");
  MX_REQUIRE(!h || is_aligned(h, 16), "mx_expert_forward_bf16: h must be 16-byte aligned");
  hipStream_t st = as_stream(stream);
  const int groups = I / 32;
  // enough K-splits to give the chip about 256 gate/up workgroups, at least 4 chunks per split
  const int splits = std::max(1, std::min({kMaxSplits, (256 + groups - 1) / groups, (H / 128) / 4}));
  void* base = nullptr;
  if (int s = mxi::scratch(ctx, bf16_scratch_bytes(I, T), &base)) return s;
  float* part = (float*)base;
  float* hbuf = h ? h : part + (size_t)kMaxSplits * T * 2 * I;
  GateUpArgs ga{(const uint8_t*)tiled, x, part, H, I, T, splits};
  for (int t0 = 0; t0 < T; t0 += kTok) {
    GateUpArgs a = ga;
    a.x = x + (size_t)t0 * H;
    a.part = part + (size_t)t0 * 2 * I;
    const int nt = std::min(kTok, T - t0);
    const dim3 grid(groups, splits, 1);
    const size_t lds = (size_t)kTok * H * 2;
    switch (nt) {
      case 1: hipLaunchKernelGGL(bf16_gateup_kernel<1>, grid, dim3(256), lds, st, a); break;
      case 2: hipLaunchKernelGGL(bf16_gateup_kernel<2>, grid, dim3(256), lds, st, a); break;
      case 3: hipLaunchKernelGGL(bf16_gateup_kernel<3>, grid, dim3(256), lds, st, a); break;
      default: hipLaunchKernelGGL(bf16_gateup_kernel<4>, grid, dim3(256), lds, st, a); break;
    }
    MX_LAUNCH_CHECK("bf16_gateup_kernel");
  }
  SwigluArgs sa{part, route_w, hbuf, gu, I, T, splits};
  hipLaunchKernelGGL(bf16_swiglu_kernel, dim3((T * I + 255) / 256), dim3(256), 0, st, sa);
  MX_LAUNCH_CHECK("bf16_swiglu_kernel");
  for (int t0 = 0; t0 < T; t0 += kTok) {
    DownArgs a{(const uint8_t*)tiled, hbuf + (size_t)t0 * I, y + (size_t)t0 * H, H, I, T};
    const int nt = std::min(kTok, T - t0);
    const dim3 grid(H / 64, 1, 1);
    const size_t lds = (size_t)kTok * I * 4;
    switch (nt) {
      case 1: hipLaunchKernelGGL(bf16_down_kernel<1>, grid, dim3(256), lds, st, a); break;
      case 2: hipLaunchKernelGGL(bf16_down_kernel<2>, grid, dim3(256), lds, st, a); break;
      case 3: hipLaunchKernelGGL(bf16_down_kernel<3>, grid, dim3(256), lds, st, a); break;
      default: hipLaunchKernelGGL(bf16_down_kernel<4>, grid, dim3(256), lds, st, a); break;
    }
    MX_LAUNCH_CHECK("bf16_down_kernel");
  }
  return MX_OK;
}
