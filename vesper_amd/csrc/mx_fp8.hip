// FP8 E4M3 block-scaled projections on gfx950 (NativeProjections.fp8, src/vesper/projections.py:135-154;
// projection_probe.cu:9-51).
//
// Two scale profiles, one kernel body:
//   block 32  (the reference's projection): weight E8M0 per 32 x 32 block [N/32][K/32], activations
//             per-32 E8M0 (the activation32 quantizer). Both scales are powers of two and are fed to the
//             scaled MFMA, which applies them exactly.
//   block 128 (DeepSeek-style FP32 scales): weight FP32 per 128 x 128 block
//             [ceil(N/128)][K/128], activations per-token per-128 FP32. Per 128-wide chunk the MFMA gives
//             the block dot d (unit scales) and the kernel accumulates acc += (d * sa) * sw in FP32,
//             the reference's order.
//
// Weights are held in a device-native tiled layout (mx_fp8_tile): for each group of 64 rows and each
// 128-wide K chunk, 4 tiles of 16 rows x 2 KB, each stored as two 1 KB halves of 16 bytes per lane in
// MFMA operand order, so every wave load reads 1 KB of contiguous HBM.
#include <algorithm>
#include <cmath>

#include "mx_device.h"
#include "mx_internal.h"
#include "mx_numerics.h"

namespace {

using mxd::ldg128;
using mxd::ldg32;
using mxd::ldgf;
using mxd::mfma_fp8_fp8;
using mxd::v4f;

constexpr int kTiles = 4;   // 16-row MFMA tiles per workgroup: 64 weight rows
constexpr int kTok = 16;    // token columns per MFMA

struct Fp8Blob {
  size_t scales;   // byte offset of the scale section
  size_t total;    // blob bytes (256-byte multiple)
};

__host__ __device__ inline Fp8Blob fp8_blob(int N, int K, int block) {
  const size_t w = (size_t)N * K;
  const size_t s = block == 32 ? w / 32 : (size_t)((N + 127) / 128) * (size_t)(K / 128) * 4;
  Fp8Blob b;
  b.scales = w;
  b.total = (w + s + 255) & ~(size_t)255;
  return b;
}

// Reference layout -> tiled blob. Weight piece i (16 bytes): lane l = i % 64, half h, tile t, chunk c,
// row group g; row 64g + 16t + l % 16, K 128c + 64h + 16 (l / 16). Block-32 scale word (g, c, l): byte t is
// the E8M0 code of (row block (64g + 16t) / 32, K block 4c + l / 16). Block-128 scales are copied as is.
__global__ void fp8_tile_kernel(const uint8_t* __restrict__ w, const void* __restrict__ sw, uint8_t* __restrict__ blob,
                                int N, int K, int block) {
  const int64_t C = K / 128;
  const int64_t pieces = (int64_t)N * K / 16;
  const int64_t words = block == 32 ? (int64_t)(N / 64) * C * 64 : 0;
  const int64_t fscales = block == 32 ? 0 : (int64_t)((N + 127) / 128) * C;
  const Fp8Blob off = fp8_blob(N, K, block);
  const int64_t total = pieces + words + fscales;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    if (i < pieces) {
      const int l = (int)(i & 63), h = (int)((i >> 6) & 1), t = (int)((i >> 7) & 3);
      const int64_t rest = i >> 9, c = rest % C, g = rest / C;
      const int64_t row = 64 * g + 16 * t + (l & 15);
      const int64_t k0 = 128 * c + 64 * h + 16 * (l >> 4);
      *reinterpret_cast<uint4*>(blob + i * 16) = *reinterpret_cast<const uint4*>(w + row * K + k0);
    } else if (i < pieces + words) {
      const int64_t j = i - pieces;
      const int l = (int)(j & 63);
      const int64_t rest = j >> 6, c = rest % C, g = rest / C;
      const uint8_t* s8 = (const uint8_t*)sw;
      uint32_t word = 0;
#pragma unroll
      for (int t = 0; t < 4; ++t) word |= (uint32_t)s8[((64 * g + 16 * t) / 32) * (K / 32) + 4 * c + (l >> 4)] << (8 * t);
      *reinterpret_cast<uint32_t*>(blob + off.scales + j * 4) = word;
    } else {
      const int64_t j = i - pieces - words;
      reinterpret_cast<float*>(blob + off.scales)[j] = ((const float*)sw)[j];
    }
  }
}

// Per-token per-128 FP32-scale quantizer: one wave per 128-wide block, 2 values per lane.
__global__ __launch_bounds__(256) void act_quant128_kernel(const uint16_t* __restrict__ x, uint8_t* __restrict__ q,
                                                           float* __restrict__ s, int64_t blocks) {
  const int64_t b = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (b >= blocks) return;
  const uint32_t pair = reinterpret_cast<const uint32_t*>(x + b * 128)[lane];
  const float v0 = mx::bf16_value(pair & 0xFFFFu), v1 = mx::bf16_value(pair >> 16);
  float amax = fmaxf(fabsf(v0), fabsf(v1));
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) amax = fmaxf(amax, __shfl_xor(amax, m, 64));
  const float sc = mx::act128_scale(amax);
  const uint32_t c0 = mx::act_quant_value(v0, sc), c1 = mx::act_quant_value(v1, sc);
  reinterpret_cast<uint16_t*>(q + b * 128)[lane] = (uint16_t)(c0 | (c1 << 8));
  if (lane == 0) s[b] = sc;
}

struct Fp8Args {
  const uint8_t* blob;
  int N, K, T;
  const uint8_t* xq;   // [T][K] E4M3
  const void* xs;      // block 32: uint8 [T][K/32]; block 128: float [T][K/128]
  uint16_t* y;         // [T][N] BF16
  float* trace;        // [T][N] FP32 sums, nullable
};

template <int kBlock>
struct Fp8Chunk {
  uint4 a[kTiles][2];
  uint4 b0, b1;
  uint32_t sw;   // block 32: scale word (byte t = tile t); block 128: FP32 bits of the weight block scale
  uint32_t sx;   // block 32: 4 activation E8M0 codes of the chunk; block 128: FP32 bits of the act scale
};

template <int kBlock>
__device__ __forceinline__ void fp8_load(Fp8Chunk<kBlock>& r, const Fp8Args& a, const uint8_t* wlane,
                                         const uint8_t* slane, const float* swrow, const uint8_t* xrow, int tok,
                                         int c, int q) {
#pragma unroll
  for (int t = 0; t < kTiles; ++t) {
    r.a[t][0] = ldg128(wlane + (size_t)c * 8192 + t * 2048);
    r.a[t][1] = ldg128(wlane + (size_t)c * 8192 + t * 2048 + 1024);
  }
  r.b0 = ldg128(xrow + (size_t)c * 128 + 16 * q);
  r.b1 = ldg128(xrow + (size_t)c * 128 + 64 + 16 * q);
  if constexpr (kBlock == 32) {
    r.sw = ldg32(slane + (size_t)c * 256);
    r.sx = ldg32((const uint8_t*)a.xs + (size_t)tok * (a.K / 32) + 4 * c);
  } else {
    r.sw = __float_as_uint(ldgf(swrow + c));
    r.sx = __float_as_uint(ldgf((const float*)a.xs + (size_t)tok * (a.K / 128) + c));
  }
}

template <int kBlock>
__device__ __forceinline__ void fp8_mma(const Fp8Chunk<kBlock>& r, v4f (&acc)[kTiles], int q, uint32_t keep) {
  const uint4 b0 = make_uint4(r.b0.x & keep, r.b0.y & keep, r.b0.z & keep, r.b0.w & keep);
  const uint4 b1 = make_uint4(r.b1.x & keep, r.b1.y & keep, r.b1.z & keep, r.b1.w & keep);
  if constexpr (kBlock == 32) {
    const int sx = (int)((r.sx >> (8 * q)) & 0xFF);
#pragma unroll
    for (int t = 0; t < kTiles; ++t)
      acc[t] = mfma_fp8_fp8(r.a[t][0], r.a[t][1], b0, b1, acc[t], (int)((r.sw >> (8 * t)) & 0xFF), sx);
  } else {
    const float sa = __uint_as_float(r.sx), sw = __uint_as_float(r.sw);
#pragma unroll
    for (int t = 0; t < kTiles; ++t) {
      const v4f d = mfma_fp8_fp8(r.a[t][0], r.a[t][1], b0, b1, v4f{0.f, 0.f, 0.f, 0.f}, 127, 127);
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[t][i] = acc[t][i] + (d[i] * sa) * sw;
    }
  }
}

// grid (N / 64, ceil(T / 16)), 256 threads: 64 weight rows x 16 tokens per workgroup. Wave w streams its
// quarter of the K chunks (P = 2 chunks of 8 KB in flight), the quarters are summed through LDS in wave
// order, then wave t writes tile t.
template <int kBlock>
__global__ __launch_bounds__(256) void fp8_gemv_kernel(Fp8Args a) {
  constexpr int P = 2;
  const int g = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q = lane >> 4, n = lane & 15;
  const int tok = blockIdx.y * kTok + n;
  const bool live = tok < a.T;
  const int rtok = live ? tok : a.T - 1;
  const int C = a.K / 128;
  const Fp8Blob off = fp8_blob(a.N, a.K, kBlock);
  const uint8_t* wlane = a.blob + (size_t)g * C * 8192 + 16 * lane;
  const uint8_t* slane = a.blob + off.scales + (size_t)g * C * 256 + 4 * lane;
  const float* swrow = reinterpret_cast<const float*>(a.blob + off.scales) + (size_t)((64 * g) / 128) * C;
  const uint8_t* xrow = a.xq + (size_t)rtok * a.K;
  v4f acc[kTiles];
#pragma unroll
  for (int t = 0; t < kTiles; ++t) acc[t] = v4f{0.f, 0.f, 0.f, 0.f};
  const int c0 = (C * wave) / 4;
  const int cn = (C * (wave + 1)) / 4 - c0;
  if (cn > 0) {
    const uint32_t keep = live ? 0xFFFFFFFFu : 0u;
    Fp8Chunk<kBlock> buf[P];
#pragma unroll
    for (int j = 0; j < P; ++j) fp8_load(buf[j], a, wlane, slane, swrow, xrow, rtok, c0 + min(j, cn - 1), q);
    int i = 0;
    for (; i + P < cn; i += P) {
#pragma unroll
      for (int j = 0; j < P; ++j) {
        fp8_mma(buf[j], acc, q, keep);
        fp8_load(buf[j], a, wlane, slane, swrow, xrow, rtok, c0 + min(i + j + P, cn - 1), q);
      }
    }
#pragma unroll
    for (int j = 0; j < P; ++j) fp8_mma(buf[j], acc, q, i + j < cn ? keep : 0u);
  }
  __shared__ float red[4][kTiles][64][4];
#pragma unroll
  for (int t = 0; t < kTiles; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) red[wave][t][lane][i] = acc[t][i];
  __syncthreads();
  float out[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    out[i] = ((red[0][wave][lane][i] + red[1][wave][lane][i]) + red[2][wave][lane][i]) + red[3][wave][lane][i];
  if (live) {
    const size_t o = (size_t)tok * a.N + 64 * g + 16 * wave + 4 * q;
    uint2 packed;
    packed.x = mx::bf16_bits(out[0]) | (mx::bf16_bits(out[1]) << 16);
    packed.y = mx::bf16_bits(out[2]) | (mx::bf16_bits(out[3]) << 16);
    *reinterpret_cast<uint2*>(a.y + o) = packed;
    if (a.trace) *reinterpret_cast<float4*>(a.trace + o) = make_float4(out[0], out[1], out[2], out[3]);
  }
}

int check_fp8_shape(int N, int K, int block, const char* who) {
  MX_REQUIRE(block == 32 || block == 128, "%s: block must be 32 or 128", who);
  MX_REQUIRE(N > 0 && N % 64 == 0 && K > 0 && K % 128 == 0, "%s: rows must be a multiple of 64 and width of 128",
             who);
  return MX_OK;
}

}  // namespace

using namespace mxi;

extern "C" {

uint64_t mx_fp8_tiled_bytes(int32_t N, int32_t K, int32_t block) {
  if ((block != 32 && block != 128) || N <= 0 || N % 64 || K <= 0 || K % 128) return 0;
  return fp8_blob(N, K, block).total;
}

int mx_fp8_tile(mx_ctx* ctx, const uint8_t* w, const void* sw, int32_t N, int32_t K, int32_t block, void* tiled,
                void* stream) {
  if (int s = use(ctx)) return s;
  if (int s = check_fp8_shape(N, K, block, "mx_fp8_tile")) return s;
  MX_REQUIRE(w && sw && tiled, "mx_fp8_tile: null pointer");
  MX_REQUIRE(((uintptr_t)w & 15) == 0 && ((uintptr_t)tiled & 255) == 0 && ((uintptr_t)sw & 3) == 0,
             "mx_fp8_tile: weights 16-byte, scales 4-byte and the tiled blob 256-byte aligned");
  hipLaunchKernelGGL(fp8_tile_kernel, dim3(2048), dim3(256), 0, as_stream(stream), w, sw, (uint8_t*)tiled, N, K,
                     block);
  MX_LAUNCH_CHECK("fp8_tile_kernel");
  return MX_OK;
}

int mx_act_quant128(mx_ctx* ctx, const uint16_t* x, uint8_t* q, float* s, int64_t rows, int64_t width, void* stream) {
  if (int s2 = use(ctx)) return s2;
  MX_REQUIRE(rows >= 0 && width > 0 && width % 128 == 0, "mx_act_quant128: width must be a positive multiple of 128");
  if (!rows) return MX_OK;
  MX_REQUIRE(x && q && s && ((uintptr_t)x & 3) == 0 && ((uintptr_t)q & 1) == 0,
             "mx_act_quant128: null or misaligned pointer");
  const int64_t blocks = rows * (width / 128);
  hipLaunchKernelGGL(act_quant128_kernel, dim3((unsigned)((blocks + 3) / 4)), dim3(256), 0, as_stream(stream), x, q, s,
                     blocks);
  MX_LAUNCH_CHECK("act_quant128_kernel");
  return MX_OK;
}

int mx_fp8_projection(mx_ctx* ctx, const void* tiled, int32_t N, int32_t K, int32_t block, const uint16_t* x,
                      int32_t T, uint16_t* y, float* trace, uint8_t* q_out, void* s_out, void* stream) {
  if (int s = use(ctx)) return s;
  if (int s = check_fp8_shape(N, K, block, "mx_fp8_projection")) return s;
  MX_REQUIRE(T >= 0, "mx_fp8_projection: negative token count");
  if (!T) return MX_OK;
  MX_REQUIRE(tiled && x && y, "mx_fp8_projection: null pointer");
  MX_REQUIRE(((uintptr_t)tiled & 255) == 0 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)y & 7) == 0 &&
                 ((uintptr_t)trace & 15) == 0,
             "mx_fp8_projection: tiled 256-byte, x 16-byte, y 8-byte and trace 16-byte alignment required");
  hipStream_t st = as_stream(stream);
  const uint64_t q_b = ((uint64_t)T * K + 255) & ~255ull;
  const uint64_t s_b = block == 32 ? (uint64_t)T * (K / 32) : (uint64_t)T * (K / 128) * 4;
  void* base = nullptr;
  if (!q_out || !s_out)
    if (int s = scratch(ctx, q_b + s_b + 256, &base)) return s;
  uint8_t* q = q_out ? q_out : (uint8_t*)base;
  void* sc = s_out ? s_out : (void*)((uint8_t*)base + q_b);
  MX_REQUIRE(((uintptr_t)q & 15) == 0 && ((uintptr_t)sc & 3) == 0, "mx_fp8_projection: q 16-byte, s 4-byte aligned");
  if (block == 32) {
    if (int s = mx_act_quant32(ctx, x, q, (uint8_t*)sc, T, K, stream)) return s;
  } else {
    if (int s = mx_act_quant128(ctx, x, q, (float*)sc, T, K, stream)) return s;
  }
  Fp8Args a{};
  a.blob = (const uint8_t*)tiled;
  a.N = N;
  a.K = K;
  a.T = T;
  a.xq = q;
  a.xs = sc;
  a.y = y;
  a.trace = trace;
  const dim3 grid(N / 64, (T + kTok - 1) / kTok);
  if (block == 32) hipLaunchKernelGGL(fp8_gemv_kernel<32>, grid, dim3(256), 0, st, a);
  else hipLaunchKernelGGL(fp8_gemv_kernel<128>, grid, dim3(256), 0, st, a);
  MX_LAUNCH_CHECK("fp8_gemv_kernel");
  return MX_OK;
}

}  // extern "C"
