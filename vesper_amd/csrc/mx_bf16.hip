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
// Two launches on the caller's stream:
//   gate/up + SwiGLU (I/8 tiles, 8 waves each): workgroup j owns gate/up tile j (8 W1 rows and the same 8
//     W3 rows) over all of K, the waves taking contiguous eighths of the chunks, all tokens in one pass
//     (MFMA columns); the eight partial tiles are added through LDS in wave order, and the workgroup finishes
//     its 8 intermediate positions: h = silu(g) * u (* route weight) in FP32 (optionally written out with g
//     and u), and h as two BF16 terms hi + lo for the down product (hi = bf16(h), lo = bf16(h - hi): their
//     sum holds h to about 16 significant bits);
//   down (H/64 row blocks, 256 threads): W2 rows against hi and lo (two MFMAs per step), the four waves'
//     sums added in wave order and rounded once to BF16.
// Every sum runs in a fixed order (MFMA chains per wave, then waves), independent of T and of scheduling, so
// a token's result does not depend on the batch it runs in.
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
constexpr int kGuWaves = 8;      // gate/up: waves per tile, each a contiguous eighth of K
constexpr int kMaxHidden = 8192;
constexpr int kMaxInter = 4096;
constexpr int kRing = 3;         // chunks of weights (and their activations) in flight per wave

typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
using mxd::v4f;

struct GateUpArgs {
  const uint8_t* blob;
  const uint16_t* x;      // [T][H] BF16
  const float* route_w;   // [T] or null
  float* h;               // [T][I] or null
  float* gu;              // [T][2I] or null
  uint16_t* hs;           // [2][T][I] BF16: hi, then lo
  int H, I, T;
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

// One 128-wide K chunk of one gate/up tile against up to 16 tokens: 4 MFMAs, one per word. w = this lane's 16
// bytes of the tile, code = its E8M0 code, xv[r] = the tokens' BF16 operand for word r.
__device__ __forceinline__ void tile_chunk_mfma(const uint4& w, uint32_t code, const uint4 (&xv)[4], v4f& acc) {
#pragma unroll
  for (int r = 0; r < 4; ++r)
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fp4_word_bf16(word_of(w, r), code), __builtin_bit_cast(v8bf, xv[r]),
                                                  acc, 0, 0, 0);
}

// grid (I/8), 64 kGuWaves threads. Tile j = 4 g + t of row group g: MFMA rows 0-7 are W1 rows 8j + 0..7, rows
// 8-15 the same W3 rows; chunk c of the tile at (g C + c) 4096 + 1024 t, its codes byte t of the chunk's scale
// words. Wave w streams chunks [C w / 8, C (w + 1) / 8) through a register ring.
__global__ __launch_bounds__(64 * kGuWaves) void bf16_gateup_swiglu_kernel(GateUpArgs a) {
  __shared__ float4 red[kGuWaves][64];
  __shared__ float tile[16][kMaxTokens + 1];
  const int j = blockIdx.x, g = j >> 2, t = j & 3;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int H = a.H, I = a.I;
  const int chunks = H / 128;
  const int c0 = chunks * wave / kGuWaves, c1 = chunks * (wave + 1) / kGuWaves;
  const int q = lane >> 4, tok = min(lane & 15, a.T - 1);
  const uint8_t* wp = a.blob + (size_t)g * chunks * 4096 + t * 1024 + 16 * lane;
  const uint8_t* sp = a.blob + tiled_offsets(H, I).gu_s + (size_t)g * chunks * 256 + 4 * lane;
  const uint8_t* xrow = reinterpret_cast<const uint8_t*>(a.x + (size_t)tok * H) + 64 * q;
  uint4 w[kRing];
  uint32_t sw[kRing];
  uint4 xv[kRing][4];
  auto load = [&](int k, int c) {
    w[k] = ldg128_nt(wp + (size_t)c * 4096);
    sw[k] = ldg32_nt(sp + (size_t)c * 256);
#pragma unroll
    for (int r = 0; r < 4; ++r) xv[k][r] = ldg128(xrow + (size_t)c * 256 + 16 * r);
  };
  v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int k = 0; k < kRing; ++k)
    if (c0 + k < c1) load(k, c0 + k);
  for (int base = c0; base < c1; base += kRing) {
#pragma unroll
    for (int k = 0; k < kRing; ++k) {
      const int c = base + k;
      if (c < c1) {
        tile_chunk_mfma(w[k], (sw[k] >> (8 * t)) & 0xFF, xv[k], acc);
        if (c + kRing < c1) load(k, c + kRing);
      }
    }
  }
  red[wave][lane] = make_float4(acc[0], acc[1], acc[2], acc[3]);
  __syncthreads();
  if (wave == 0) {
    // lane l holds MFMA rows 4 (l / 16) + 0..3 of token column l % 16; the waves' tiles added in wave order
    float4 s = red[0][lane];
#pragma unroll
    for (int v = 1; v < kGuWaves; ++v) {
      const float4 r = red[v][lane];
      s.x = s.x + r.x;
      s.y = s.y + r.y;
      s.z = s.z + r.z;
      s.w = s.w + r.w;
    }
    const int col = lane & 15;
    tile[4 * q + 0][col] = s.x;
    tile[4 * q + 1][col] = s.y;
    tile[4 * q + 2][col] = s.z;
    tile[4 * q + 3][col] = s.w;
  }
  __syncthreads();
  // thread (token, i): intermediate position 8 j + i, gate row i and up row 8 + i of the tile
  if (tid >= 8 * a.T) return;
  const int n = tid >> 3, i = tid & 7, pos = 8 * j + i;
  const float gv = tile[i][n], uv = tile[8 + i][n];
  float h = gv / (1.0f + expf(-gv)) * uv;
  if (a.route_w) h *= a.route_w[n];
  const size_t idx = (size_t)n * I + pos;
  if (a.h) a.h[idx] = h;
  if (a.gu) {
    a.gu[(size_t)n * 2 * I + pos] = gv;
    a.gu[(size_t)n * 2 * I + I + pos] = uv;
  }
  const uint32_t hi = mx::bf16_bits(h);
  const float rest = h - __uint_as_float(hi << 16);
  a.hs[idx] = (uint16_t)hi;
  a.hs[(size_t)a.T * I + idx] = (uint16_t)mx::bf16_bits(rest);
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

static uint64_t bf16_scratch_bytes(int32_t I, int32_t T) { return (uint64_t)2 * T * I * sizeof(uint16_t); }

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
  void* base = nullptr;
  if (int s = mxi::scratch(ctx, bf16_scratch_bytes(I, T), &base)) return s;
  uint16_t* hs = (uint16_t*)base;
  GateUpArgs ga{(const uint8_t*)tiled, x, route_w, h, gu, hs, H, I, T};
  hipLaunchKernelGGL(bf16_gateup_swiglu_kernel, dim3(I / 8), dim3(64 * kGuWaves), 0, st, ga);
  MX_LAUNCH_CHECK("bf16_gateup_swiglu_kernel");
  DownArgs da{(const uint8_t*)tiled, hs, y, H, I, T};
  hipLaunchKernelGGL(bf16_down_kernel, dim3(H / 64), dim3(256), 0, st, da);
  MX_LAUNCH_CHECK("bf16_down_kernel");
  return MX_OK;
}
