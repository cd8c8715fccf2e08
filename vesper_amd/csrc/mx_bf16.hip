// The BF16-activation MXFP4 expert: y = W2 . (silu(W1 . x) * (W3 . x)) with BF16 activations, FP32
// accumulation, no activation quantization and no clamp (the benchmark's configuration 0), on the same tiled
// expert bytes the decode layer streams (mx_tile_expert).
//
// The reference's expert (ExpertExecutor.execute, src/vesper/expert.py:51-79) quantizes x and the down
// input to E4M3 per 32-block and feeds scaled MFMAs; this profile keeps the activations exact, so the
// products run on the BF16 MFMA (V_MFMA_F32_16X16X32_BF16, FP32 accumulation) with the weights converted
// exactly: each E2M1 value times its block's E8M0 scale has at most two significant bits, so
// V_CVT_SCALEF32_PK_BF16_FP4 gives it exactly in BF16 (the scale operand's exponent field is the E8M0 code;
// checked on gfx950 for every code and value, code 255 giving NaN as the format defines).
//
// MFMA mapping (measured on gfx950): A lane l = row l % 16, K 8 (l / 16) + 0..7; B lane l = column l % 16,
// same K; D lane l register i = row 4 (l / 16) + i, column l % 16. A is 16 weight rows, B is up to 16 tokens.
// In the tiled layout a lane (m, q) of tile t holds the 32 E2M1 values of row m, K block 4c + q as four
// 32-bit words; MFMA r of chunk c takes word r of every lane, i.e. K = 32 (4c + q) + 8r + 0..7 at lane group
// q, and the activations are read with the same map, so every product pairs the right operands.
//
// Three launches on the caller's stream:
//   gate/up (I/32 row groups x KS K-splits, 256 threads): the four waves split the workgroup's K range; all
//     tokens in one pass (MFMA columns); partial sums per K-split to scratch [KS][T][2I];
//   SwiGLU (T x I threads): g, u = the K-split partials summed in split order; h = silu(g) * u (* route
//     weight) in FP32 (optionally written out with g and u), and h as two BF16 terms hi + lo for the down
//     product (hi = bf16(h), lo = bf16(h - hi): their sum holds h to about 16 significant bits);
//   down (H/64 row blocks, 256 threads): W2 rows against hi and lo (two MFMAs per step), the four waves'
//     sums added in wave order and rounded once to BF16.
// Every sum runs in a fixed order (MFMA chains per wave, then waves, then splits), independent of T and of
// scheduling, so a token's result does not depend on the batch it runs in.
#include <algorithm>
#include <cmath>

#include "mx_device.h"
#include "mx_internal.h"
#include "mx_numerics.h"

namespace {

using mxd::ldg128;
using mxd::ldg128_nt;
using mxd::ldg32_nt;
using mxd::tiled_offsets;
using mxd::TiledOffsets;

constexpr int kMaxTokens = 16;
constexpr int kMaxSplits = 8;
constexpr int kMaxHidden = 8192;
constexpr int kMaxInter = 4096;
constexpr int kRing = 3;         // chunks of weights (and their activations) in flight per wave

typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
using mxd::v4f;

struct GateUpArgs {
  const uint8_t* blob;
  const uint16_t* x;   // [T][H] BF16
  float* part;         // [KS][T][2I]: g partials in [0, I), u partials in [I, 2I)
  int H, I, T, splits;
};

struct SwigluArgs {
  const float* part;
  const float* route_w;   // [T] or null
  float* h;               // [T][I] or null
  float* gu;              // [T][2I] or null
  uint16_t* hs;           // [2][T][I] BF16: hi, then lo
  int I, T, splits;
};

struct DownArgs {
  const uint8_t* blob;
  const uint16_t* hs;   // [2][T][I]
  uint16_t* y;          // [T][H]
  int H, I, T;
};

// Word r of a lane's 16-byte block (8 E2M1 values) times 2^(code - 127), as the 8 BF16 values of an MFMA
// operand (exact).
__device__ __forceinline__ v8bf fp4_word_bf16(uint32_t word, uint32_t code) {
  const float scale = __uint_as_float(code << 23);
  const v2bf p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, scale, 0);
  const v2bf p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, scale, 1);
  const v2bf p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, scale, 2);
  const v2bf p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, scale, 3);
  return v8bf{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
}

__device__ __forceinline__ uint32_t word_of(const uint4 v, int r) {
  return r == 0 ? v.x : r == 1 ? v.y : r == 2 ? v.z : v.w;
}

// One 128-wide K chunk of a 4-tile weight group against up to 16 tokens: 4 MFMAs per tile, one per word.
// w[t] = tile t's 16 bytes of this lane, sw = its scale word (byte t = tile t), xv[r] = the tokens' BF16
// operand for word r; acc[t] accumulates tile t.
template <int kTerms>
__device__ __forceinline__ void chunk_mfma(const uint4 (&w)[4], uint32_t sw, const uint4 (&xv)[kTerms][4],
                                           v4f (&acc)[4]) {
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const uint32_t code = (sw >> (8 * t)) & 0xFF;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const v8bf a = fp4_word_bf16(word_of(w[t], r), code);
#pragma unroll
      for (int term = 0; term < kTerms; ++term)
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, __builtin_bit_cast(v8bf, xv[term][r]), acc[t], 0, 0, 0);
    }
  }
}

// The wave's chunks [c0, c1) of a 4-tile group whose chunk c starts at wp + c * 4096 (tile t at + t * 1024,
// lane at + 16 lane) with scale words at sp + c * 256 (+ 4 lane); act(term, c, r) = the address of this
// lane's 16-byte activation operand. Loads run kRing chunks ahead in a statically indexed ring.
template <int kTerms, typename Act>
__device__ __forceinline__ void stream_group(const uint8_t* wp, const uint8_t* sp, int c0, int c1, Act act,
                                             v4f (&acc)[4]) {
  uint4 w[kRing][4];
  uint32_t sw[kRing];
  uint4 xv[kRing][kTerms][4];
  auto load = [&](int j, int c) {
#pragma unroll
    for (int t = 0; t < 4; ++t) w[j][t] = ldg128_nt(wp + (size_t)c * 4096 + t * 1024);
    sw[j] = ldg32_nt(sp + (size_t)c * 256);
#pragma unroll
    for (int term = 0; term < kTerms; ++term)
#pragma unroll
      for (int r = 0; r < 4; ++r) xv[j][term][r] = ldg128(act(term, c, r));
  };
#pragma unroll
  for (int j = 0; j < kRing; ++j)
    if (c0 + j < c1) load(j, c0 + j);
  for (int base = c0; base < c1; base += kRing) {
#pragma unroll
    for (int j = 0; j < kRing; ++j) {
      const int c = base + j;
      if (c < c1) {
        chunk_mfma<kTerms>(w[j], sw[j], xv[j], acc);
        if (c + kRing < c1) load(j, c + kRing);
      }
    }
  }
}

// grid (I/32, KS), 256 threads. Row group g holds W1 and W3 rows [32g, 32g + 32): tile t's MFMA rows 0-7 are
// W1 rows 32g + 8t + 0..7, rows 8-15 the same W3 rows. The workgroup's chunk range is split ks of the H/128
// chunks, quartered over the waves.
__global__ __launch_bounds__(256) void bf16_gateup_kernel(GateUpArgs a) {
  __shared__ float red[4][4][64][4];
  const int g = blockIdx.x, ks = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int H = a.H, I = a.I;
  const int chunks = H / 128;
  const int c_lo = chunks * ks / a.splits, c_hi = chunks * (ks + 1) / a.splits;
  const int n = c_hi - c_lo;
  const int c0 = c_lo + n * wave / 4, c1 = c_lo + n * (wave + 1) / 4;
  const int q = lane >> 4, tok = min(lane & 15, a.T - 1);
  const uint8_t* wp = a.blob + (size_t)g * chunks * 4096 + 16 * lane;
  const uint8_t* sp = a.blob + tiled_offsets(H, I).gu_s + (size_t)g * chunks * 256 + 4 * lane;
  const uint8_t* xrow = reinterpret_cast<const uint8_t*>(a.x + (size_t)tok * H) + 64 * q;
  auto act = [&](int, int c, int r) { return xrow + (size_t)c * 256 + 16 * r; };
  v4f acc[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) acc[t] = v4f{0.f, 0.f, 0.f, 0.f};
  stream_group<1>(wp, sp, c0, c1, act, acc);
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) red[wave][t][lane][i] = acc[t][i];
  __syncthreads();
  // thread (t, lane): tile t's rows 4 (lane / 16) + 0..3 for token lane % 16, the 4 waves summed in order
  const int t = tid >> 6, col = lane & 15;
  if (col < a.T) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float s = ((red[0][t][lane][i] + red[1][t][lane][i]) + red[2][t][lane][i]) + red[3][t][lane][i];
      const int m = 4 * q + i;
      const int row = 32 * g + 8 * t + (m & 7);
      a.part[((size_t)ks * a.T + col) * (2 * I) + (m < 8 ? row : I + row)] = s;
    }
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
  if (a.h) a.h[idx] = h;
  if (a.gu) {
    a.gu[(size_t)tok * 2 * a.I + i] = g;
    a.gu[(size_t)tok * 2 * a.I + a.I + i] = u;
  }
  const uint32_t hi = mx::bf16_bits(h);
  const float rest = h - __uint_as_float(hi << 16);
  a.hs[idx] = (uint16_t)hi;
  a.hs[(size_t)a.T * a.I + idx] = (uint16_t)mx::bf16_bits(rest);
}

// grid (H/64), 256 threads. Row block b holds W2 rows [64b, 64b + 64): tile t's MFMA rows are rows
// 64b + 16t + 0..15. The I/128 chunks are quartered over the waves.
__global__ __launch_bounds__(256) void bf16_down_kernel(DownArgs a) {
  __shared__ float red[4][4][64][4];
  const int b = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int H = a.H, I = a.I;
  const int chunks = I / 128;
  const int c0 = chunks * wave / 4, c1 = chunks * (wave + 1) / 4;
  const int q = lane >> 4, tok = min(lane & 15, a.T - 1);
  const TiledOffsets off = tiled_offsets(H, I);
  const uint8_t* wp = a.blob + off.dn_w + (size_t)b * chunks * 4096 + 16 * lane;
  const uint8_t* sp = a.blob + off.dn_s + (size_t)b * chunks * 256 + 4 * lane;
  const uint8_t* hrow = reinterpret_cast<const uint8_t*>(a.hs + (size_t)tok * I) + 64 * q;
  const size_t lo = (size_t)a.T * I * 2;   // bytes from the hi term to the lo term
  auto act = [&](int term, int c, int r) { return hrow + term * lo + (size_t)c * 256 + 16 * r; };
  v4f acc[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) acc[t] = v4f{0.f, 0.f, 0.f, 0.f};
  stream_group<2>(wp, sp, c0, c1, act, acc);
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) red[wave][t][lane][i] = acc[t][i];
  __syncthreads();
  const int t = tid >> 6, col = lane & 15;
  if (col < a.T) {
    uint32_t out[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      out[i] = mx::bf16_bits(((red[0][t][lane][i] + red[1][t][lane][i]) + red[2][t][lane][i]) + red[3][t][lane][i]);
    uint2 packed;
    packed.x = out[0] | (out[1] << 16);
    packed.y = out[2] | (out[3] << 16);
    *reinterpret_cast<uint2*>(a.y + (size_t)col * H + 64 * b + 16 * t + 4 * q) = packed;
  }
}

bool is_aligned(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

}  // namespace

using mxi::as_stream;
using mxi::use;

static uint64_t bf16_scratch_bytes(int32_t I, int32_t T) {
  return (uint64_t)kMaxSplits * T * 2 * I * sizeof(float) + (uint64_t)2 * T * I * sizeof(uint16_t);
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
  MX_REQUIRE(x && y && is_aligned(x, 16) && is_aligned(y, 8), "mx_expert_forward_bf16: x (16-byte) and y (8-byte) required");
  MX_REQUIRE(!h || is_aligned(h, 4), "mx_expert_forward_bf16: h must be 4-byte aligned");
  hipStream_t st = as_stream(stream);
  const int groups = I / 32;
  // enough K-splits to give the chip about 256 gate/up workgroups, at least 8 chunks per split
  const int splits = std::max(1, std::min({kMaxSplits, (256 + groups - 1) / groups, (H / 128) / 8}));
  void* base = nullptr;
  if (int s = mxi::scratch(ctx, bf16_scratch_bytes(I, T), &base)) return s;
  float* part = (float*)base;
  uint16_t* hs = reinterpret_cast<uint16_t*>(part + (size_t)kMaxSplits * T * 2 * I);
  GateUpArgs ga{(const uint8_t*)tiled, x, part, H, I, T, splits};
  hipLaunchKernelGGL(bf16_gateup_kernel, dim3(groups, splits, 1), dim3(256), 0, st, ga);
  MX_LAUNCH_CHECK("bf16_gateup_kernel");
  SwigluArgs sa{part, route_w, h, gu, hs, I, T, splits};
  hipLaunchKernelGGL(bf16_swiglu_kernel, dim3((T * I + 255) / 256), dim3(256), 0, st, sa);
  MX_LAUNCH_CHECK("bf16_swiglu_kernel");
  DownArgs da{(const uint8_t*)tiled, hs, y, H, I, T};
  hipLaunchKernelGGL(bf16_down_kernel, dim3(H / 64), dim3(256), 0, st, da);
  MX_LAUNCH_CHECK("bf16_down_kernel");
  return MX_OK;
}
