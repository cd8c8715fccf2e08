// FP8 E4M3 block-scaled projections on gfx950 (NativeProjections.fp8, src/vesper/projections.py:135-154;
// projection_probe.cu:9-51).
//
// Two scale profiles, one kernel body:
//   block 32  (the reference's projection): weight E8M0 per 32 x 32 block [N/32][K/32], activations
//             per-32 E8M0 (the activation32 quantizer). Both scales are powers of two and are fed to the
//             scaled MFMA, which applies them exactly.
//   block 128 (DeepSeek-style FP32 scales): weight FP32 per 128 x 128 block
//             [ceil(N/128)][K/128], activations per-token per-128 FP32. Per 128-wide chunk the MFMA gives
//             the block dot d (unit scales) and the kernel accumulates acc = fma(d, f32(sa * sw), acc):
//             one rounding per output and chunk. (The reference's only FP8 projection has power-of-two
//             block-32 scales, where every order gives the same sums; this profile's order is this
//             build's own.)
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
using mxd::ldg128_nt;
using mxd::ldg32;
using mxd::ldgf;
using mxd::mfma_fp8_fp8;
using mxd::v4f;

constexpr int kTiles = 4;   // 16-row MFMA tiles per workgroup: 64 weight rows
constexpr int kTok = 16;    // token columns per MFMA
constexpr int kGemvMaxTokens = 32;   // above this the tiled GEMM reuses each weight tile for 128 tokens
// The GEMV's last workgroup per tile adds the split-K partial sums when they total at most this many
// bytes. Above it (the 7168- and 24576-row projections at 16 tokens, measured on MI355X) the
// device-coherent round trip through one workgroup per tile costs more than fp8_splitk_reduce_kernel.
constexpr uint64_t kTicketPartialBytes = MX_HANDOFF_BYTES;   // the context's handoff buffer

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

// E4M3 codes of 8 values over their block-128 scale sc: the quotients x / sc by mx::act128_quotient (one
// reciprocal per block, then a multiply and two fused multiply-adds per value instead of an IEEE division;
// the codes equal those of the division on every input), packed by mxd::e4m3x4 (equal to the encoder on
// every input).
__device__ __forceinline__ uint2 act128_codes8(const float (&v)[8], float sc) {
  const float inv = 1.0f / sc;
  uint2 c;
  c.x = mxd::e4m3x4(mx::act128_quotient(v[0], sc, inv), mx::act128_quotient(v[1], sc, inv),
                    mx::act128_quotient(v[2], sc, inv), mx::act128_quotient(v[3], sc, inv));
  c.y = mxd::e4m3x4(mx::act128_quotient(v[4], sc, inv), mx::act128_quotient(v[5], sc, inv),
                    mx::act128_quotient(v[6], sc, inv), mx::act128_quotient(v[7], sc, inv));
  return c;
}

// The same quantizer with 8 values per lane (16-byte loads, 8-byte stores), 16 lanes per block, blocks in
// a grid-stride loop; x 16-byte and q 8-byte aligned.
__global__ __launch_bounds__(256) void act_quant128_v8_kernel(const uint16_t* __restrict__ x, uint8_t* __restrict__ q,
                                                              float* __restrict__ s, int64_t blocks) {
  const int sub = threadIdx.x & 15;
  for (int64_t b = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 4; b < blocks;
       b += ((int64_t)gridDim.x * blockDim.x) >> 4) {
    const uint4 raw = *reinterpret_cast<const uint4*>(x + b * 128 + 8 * sub);
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
    float v[8];
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = mx::bf16_value(w[i] & 0xFFFFu);
      v[2 * i + 1] = mx::bf16_value(w[i] >> 16);
      amax = fmaxf(amax, fmaxf(fabsf(v[2 * i]), fabsf(v[2 * i + 1])));
    }
    amax = mxd::row16_max(amax);
    const float sc = mx::act128_scale(amax);
    *reinterpret_cast<uint2*>(q + b * 128 + 8 * sub) = act128_codes8(v, sc);
    if (sub == 0) s[b] = sc;
  }
}

struct Fp8Args {
  const uint8_t* blob;
  int N, K, T;
  const uint8_t* xq;   // [T][K] E4M3
  const void* xs;      // block 32: uint8 [T][K/32]; block 128: float [T][K/128]
  uint16_t* y;         // [T][N] BF16
  float* trace;        // [T][N] FP32 sums, nullable
  float* partial;      // split K: [splits][T][N] FP32 partial sums (the GEMV writes these instead of y)
  uint32_t* tickets;   // split-K GEMV: arrival counter per (row group, token tile), zero between launches;
                       // null = partial sums only, added by fp8_splitk_reduce_kernel
  float* handoff;      // with tickets: [splits][T][N] partial sums in this launch's half of the context's
                       // handoff buffer, which holds the empty pattern wherever this launch reads
  uint4* restore;      // with tickets: the other half, whose first restore_n 16-byte words the previous
  int64_t restore_n;   // launch wrote: every workgroup puts back the empty pattern over its share
  const uint16_t* x;   // fused tile GEMV (block 128, few tokens): the BF16 input [T][K], quantized in the kernel
  int64_t x_stride;    // activation elements per token: K, or groups x K when grouped
  int x_group_rows;    // grouped activations (block-32 GEMV): weight rows [g R, (g + 1) R) multiply
                       // activation group g, codes at xq + tok x_stride + g K; 0 = one group
};

// Block-128 calls of up to kFusedMaxTokens tokens run on fp8_tile_gemv_kernel, which can quantize its own
// activations into LDS rows of 128 codes + 16 bytes of padding; at 16 tokens the repeated quantization in
// every workgroup costs more than the quantizer launch (measured).
constexpr int kFusedMaxTokens = 4;
constexpr int kFusedRow = 144;

template <int kBlock>
struct Fp8Chunk {
  uint4 a[kTiles][2];
  uint4 b0, b1;
  uint32_t sw;   // block 32: scale word (byte t = tile t); block 128: FP32 bits of the weight block scale
  uint32_t sx;   // block 32: 4 activation E8M0 codes of the chunk; block 128: FP32 bits of the act scale
};

// xsrow: this lane's token's activation scales (block 32: E8M0 bytes, block 128: FP32), chunk 0 first.
template <int kBlock>
__device__ __forceinline__ void fp8_load(Fp8Chunk<kBlock>& r, const Fp8Args& a, const uint8_t* wlane,
                                         const uint8_t* slane, const float* swrow, const uint8_t* xrow,
                                         const uint8_t* xsrow, int c, int q) {
  // weights: non-temporal loads (each byte is read once per call); 48.8 against 53.0 us for the
  // configuration-3 projections at T = 1 with plain loads (MI355X)
#pragma unroll
  for (int t = 0; t < kTiles; ++t) {
    r.a[t][0] = ldg128_nt(wlane + (size_t)c * 8192 + t * 2048);
    r.a[t][1] = ldg128_nt(wlane + (size_t)c * 8192 + t * 2048 + 1024);
  }
  r.b0 = ldg128(xrow + (size_t)c * 128 + 16 * q);
  r.b1 = ldg128(xrow + (size_t)c * 128 + 64 + 16 * q);
  if constexpr (kBlock == 32) {
    r.sw = ldg32(slane + (size_t)c * 256);
    r.sx = ldg32(xsrow + 4 * c);
  } else {
    r.sw = __float_as_uint(ldgf(swrow + c));
    r.sx = __float_as_uint(ldgf(reinterpret_cast<const float*>(xsrow) + c));
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
    // the chunk's combined scale f32(sa * sw), then one fused multiply-add per output
    const float s = __uint_as_float(r.sx) * __uint_as_float(r.sw);
#pragma unroll
    for (int t = 0; t < kTiles; ++t) {
      const v4f d = mfma_fp8_fp8(r.a[t][0], r.a[t][1], b0, b1, v4f{0.f, 0.f, 0.f, 0.f}, 127, 127);
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[t][i] = fmaf(d[i], s, acc[t][i]);
    }
  }
}

// grid (N / 64, ceil(T / 16), splits), 256 threads: 64 weight rows x 16 tokens x one K range per
// workgroup. Wave w streams its quarter of the workgroup's K chunks (P = 2 chunks of 8 KB in flight), the
// quarters are summed through LDS in wave order, then wave t writes tile t: BF16 (and the FP32 trace)
// when K is not split, else its FP32 partial sums. With K split and a.tickets set, the last workgroup of
// the (row group, token tile) to arrive adds the partial sums in split order (fp8_splitk_reduce_kernel's
// arithmetic) and writes the outputs; without tickets fp8_splitk_reduce_kernel does it.
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
  // grouped activations: the row group's 64 rows lie in one activation group (x_group_rows % 64 == 0)
  const int xgroup = a.x_group_rows ? (64 * g) / a.x_group_rows : 0;
  const uint8_t* xrow = a.xq + (size_t)rtok * a.x_stride + (size_t)xgroup * a.K;
  const uint8_t* xsrow =
      kBlock == 32 ? (const uint8_t*)a.xs + (size_t)rtok * (a.x_stride / 32) + (size_t)xgroup * (a.K / 32)
                   : reinterpret_cast<const uint8_t*>((const float*)a.xs + (size_t)rtok * (a.K / 128));
  if (a.restore_n) {
    // this workgroup's share of the other handoff half (plain stores: the kernel boundary publishes them
    // to the launch that uses that half next)
    const int64_t wg = ((int64_t)blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x;
    const int64_t wgs = (int64_t)gridDim.x * gridDim.y * gridDim.z;
    const int64_t per = (a.restore_n + wgs - 1) / wgs;
    const uint4 empty = make_uint4(mxd::kHandoffEmpty, mxd::kHandoffEmpty, mxd::kHandoffEmpty, mxd::kHandoffEmpty);
    for (int64_t i = wg * per + tid; i < min((wg + 1) * per, a.restore_n); i += 256) a.restore[i] = empty;
  }
  v4f acc[kTiles];
#pragma unroll
  for (int t = 0; t < kTiles; ++t) acc[t] = v4f{0.f, 0.f, 0.f, 0.f};
  const int z = blockIdx.z, S = gridDim.z;
  const int cb = (C * z) / S, cw = (C * (z + 1)) / S - cb;   // this workgroup's chunk range
  const int c0 = cb + (cw * wave) / 4;
  const int cn = cb + (cw * (wave + 1)) / 4 - c0;
  const uint32_t keep = live ? 0xFFFFFFFFu : 0u;
  Fp8Chunk<kBlock> buf[P];
  if (cn > 0) {
#pragma unroll
    for (int j = 0; j < P; ++j) fp8_load<kBlock>(buf[j], a, wlane, slane, swrow, xrow, xsrow, c0 + min(j, cn - 1), q);
    int i = 0;
    for (; i + P < cn; i += P) {
#pragma unroll
      for (int j = 0; j < P; ++j) {
        fp8_mma<kBlock>(buf[j], acc, q, keep);
        fp8_load<kBlock>(buf[j], a, wlane, slane, swrow, xrow, xsrow, c0 + min(i + j + P, cn - 1), q);
      }
    }
#pragma unroll
    for (int j = 0; j < P; ++j) fp8_mma<kBlock>(buf[j], acc, q, i + j < cn ? keep : 0u);
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
  const size_t o = (size_t)tok * a.N + 64 * g + 16 * wave + 4 * q;
  if (S > 1) {
    float* part = a.partial + (size_t)z * a.T * a.N + o;
    if (!a.tickets) {
      if (live) *reinterpret_cast<float4*>(part) = make_float4(out[0], out[1], out[2], out[3]);
      return;
    }
    // The partial sums go to this launch's half of the context's handoff buffer (a.handoff, [S][T][N] FP32),
    // which holds the kHandoffEmpty pattern wherever this launch reads (the launch before restored it):
    // each pair of sums is published as one 64-bit agent-scope atomic, a relaxed atomic ticket per tile
    // elects the last of the S arrivals, and that workgroup reads every split's pairs, re-reading any
    // location that still holds the empty pattern until the published pair is visible, and adds them in
    // split order. In a launch a location only ever holds the empty pattern or this launch's pair, so
    // correctness rests on per-location coherence of the atomics (and the kernel boundaries between
    // launches) -- not on an order between different locations, which would need agent-scope fences: each
    // release fence writes back the XCD's whole L2, tens of microseconds over a launch. The stores have
    // completed before the ticket is taken (s_waitcnt 0, then the barrier), so the first read normally finds
    // them; the re-reads are bounded, and a pair still missing at the bound becomes NaN instead of a hang.
    const size_t stride = (size_t)a.T * a.N;
    float* hand = a.handoff + o;
    if (live) {
      mxd::store_device(hand + (size_t)z * stride, out[0], out[1]);
      mxd::store_device(hand + (size_t)z * stride + 2, out[2], out[3]);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __shared__ uint32_t arrived;
    __syncthreads();
    uint32_t* ticket = a.tickets + (size_t)blockIdx.y * gridDim.x + g;
    if (tid == 0) arrived = __hip_atomic_fetch_add(ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (arrived != (uint32_t)(S - 1)) return;
    if (tid == 0) __hip_atomic_store(ticket, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (!live) return;
    float2 p[16][2];
#pragma unroll
    for (int zz = 0; zz < 16; ++zz)
      if (zz < S) {
        p[zz][0] = mxd::load_device(hand + (size_t)zz * stride);
        p[zz][1] = mxd::load_device(hand + (size_t)zz * stride + 2);
      }
    // one check over every pair first; the re-reads are the rare path
    bool missing = false;
#pragma unroll
    for (int zz = 0; zz < 16; ++zz)
      if (zz < S)
        missing |= (int)(__float_as_uint(p[zz][0].x) == mxd::kHandoffEmpty) |
                    (int)(__float_as_uint(p[zz][1].x) == mxd::kHandoffEmpty);
    if (missing) {
#pragma unroll
      for (int zz = 0; zz < 16; ++zz)
        if (zz < S) {   // unrolled: p stays in registers
          p[zz][0] = mxd::await_pair(p[zz][0], hand + (size_t)zz * stride);
          p[zz][1] = mxd::await_pair(p[zz][1], hand + (size_t)zz * stride + 2);
        }
    }
    float4 t = make_float4(p[0][0].x, p[0][0].y, p[0][1].x, p[0][1].y);
#pragma unroll
    for (int zz = 1; zz < 16; ++zz)
      if (zz < S) {
        t.x = t.x + p[zz][0].x;
        t.y = t.y + p[zz][0].y;
        t.z = t.z + p[zz][1].x;
        t.w = t.w + p[zz][1].y;
      }
    out[0] = t.x;
    out[1] = t.y;
    out[2] = t.z;
    out[3] = t.w;
  }
  if (live) {
    uint2 packed;
    packed.x = mx::bf16_bits(out[0]) | (mx::bf16_bits(out[1]) << 16);
    packed.y = mx::bf16_bits(out[2]) | (mx::bf16_bits(out[3]) << 16);
    *reinterpret_cast<uint2*>(a.y + o) = packed;
    if (a.trace) *reinterpret_cast<float4*>(a.trace + o) = make_float4(out[0], out[1], out[2], out[3]);
  }
}

// Block-128 decode GEMV over 16-row tiles. A workgroup of W waves owns M consecutive 16-row MFMA tiles
// (one token tile) over all of K: wave w takes tile w % M and the (w / M)-th of W / M contiguous K parts,
// streams its chunks through a register ring of kTileRing chunks (2 KB of weights per chunk, non-temporal
// loads) into one FP32 16 x 16 partial tile, acc = fma(d, f32(sa sw), acc) in chunk order, and each tile's
// W / M partial tiles are added through LDS in K-part order. No K range is shared between workgroups, so no
// partial sums leave the workgroup (no handoff, no reduce launch); the host picks W and M so that the launch
// has a few thousand waves in a few hundred workgroups.
// Fused (few tokens): the M waves of a K part first quantize its chunks of the call's tokens (P passes of 4
// blocks of 128 each) into the part's LDS rows with act_quant128_v8_kernel's arithmetic, so the call needs no
// quantizer launch.
constexpr int kTileRing = 4;
constexpr int kTileQRows = 16;   // fused: at most 4 passes of 4 blocks per wave

struct TileChunk {
  uint4 a0, a1;   // weights: the tile's two 1 KB halves of the chunk, 16 bytes per lane
  uint4 b0, b1;   // activation codes (unfused)
  float sx;       // activation scale (unfused)
};

template <bool kFused>
__device__ __forceinline__ void tile_load(TileChunk& r, const uint8_t* wlane, const uint8_t* xrow,
                                          const float* xsrow, int c, int q) {
  r.a0 = ldg128_nt(wlane + (size_t)c * 8192);
  r.a1 = ldg128_nt(wlane + (size_t)c * 8192 + 1024);
  if constexpr (!kFused) {
    r.b0 = ldg128(xrow + (size_t)c * 128 + 16 * q);
    r.b1 = ldg128(xrow + (size_t)c * 128 + 64 + 16 * q);
    r.sx = ldgf(xsrow + c);
  }
}

// sw: the chunk's weight block scale; row / qs: fused, this lane's token's LDS row and scale for the chunk,
// unused otherwise
template <bool kFused>
__device__ __forceinline__ void tile_mma(const TileChunk& r, v4f& acc, int q, uint32_t keep, float sw,
                                         const uint8_t* row, const float* qs) {
  uint4 b0 = r.b0, b1 = r.b1;
  float sx = r.sx;
  if constexpr (kFused) {
    b0 = *reinterpret_cast<const uint4*>(row + 16 * q);
    b1 = *reinterpret_cast<const uint4*>(row + 64 + 16 * q);
    sx = *qs;
  }
  b0 = make_uint4(b0.x & keep, b0.y & keep, b0.z & keep, b0.w & keep);
  b1 = make_uint4(b1.x & keep, b1.y & keep, b1.z & keep, b1.w & keep);
  const float s = sx * sw;
  const v4f d = mfma_fp8_fp8(r.a0, r.a1, b0, b1, v4f{0.f, 0.f, 0.f, 0.f}, 127, 127);
#pragma unroll
  for (int i = 0; i < 4; ++i) acc[i] = fmaf(d[i], s, acc[i]);
}

__device__ __forceinline__ float chunk_scale(float swl, int i) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(swl), i));
}

// grid (N / 16 / M, ceil(T / 16)), 64 W threads.
template <bool kFused, int W, int M, int P>
__global__ __launch_bounds__(64 * W) void fp8_tile_gemv_kernel(Fp8Args a) {
  static_assert(W % M == 0 && 4 * P * M <= kTileQRows, "tile GEMV shape");
  constexpr int KP = W / M;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tile = blockIdx.x * M + w % M, kp = w / M;
  const int q = lane >> 4, nn = lane & 15;
  const int tok0 = blockIdx.y * kTok, tok = tok0 + nn;
  const int ntok = min(kTok, a.T - tok0);
  const bool live = nn < ntok;
  const int rtok = live ? tok : a.T - 1;
  const int C = a.K / 128;
  const Fp8Blob off = fp8_blob(a.N, a.K, 128);
  // tile t of row group g: chunk c's halves at (g C + c) 8192 + 2048 t + {0, 1024}
  const uint8_t* wlane = a.blob + (size_t)(tile >> 2) * C * 8192 + (tile & 3) * 2048 + 16 * lane;
  const float* swrow = reinterpret_cast<const float*>(a.blob + off.scales) + (size_t)(tile >> 3) * C;
  const uint8_t* xrow = a.xq + (size_t)rtok * a.K;
  const float* xsrow = reinterpret_cast<const float*>(a.xs) + (size_t)rtok * C;
  const int c0 = (C * kp) / KP, n = (C * (kp + 1)) / KP - c0;
  // fused: K part kp's rows, block b = i ntok + token (chunk c0 + i), 128 codes + 16 bytes of padding each,
  // quantized by the part's M waves together (wave w % M takes blocks 4 P (w % M) + 0 .. 4 P - 1), then one
  // spare row per wave that takes the stores of lanes past the part's blocks (no branch around the math:
  // branches would make the compiler wait for the weight loads before quantizing)
  constexpr int kPartRows = 4 * P * M;
  __shared__ __attribute__((aligned(16))) uint8_t qx[kFused ? (KP * kPartRows + W) * kFusedRow : 16];
  __shared__ float qsc[kFused ? KP * kPartRows + W : 1];
  const int sub = lane & 15, grp = lane >> 4;
  const int nb = n * ntok, nl = max(n - 1, 0), b0 = 4 * P * (w % M);
  uint4 xv[kFused ? P : 1];
  if constexpr (kFused) {
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int b = min(b0 + 4 * p + grp, max(nb - 1, 0));
      xv[p] = ldg128(reinterpret_cast<const uint8_t*>(a.x + (size_t)(tok0 + b % ntok) * a.K +
                                                      (size_t)(c0 + b / ntok) * 128 + 8 * sub));
    }
  }
  // the activation loads first, then the ring, then the quantization: loads return in order, so quantizing
  // waits for the activations alone (scheduling barriers keep the compiler from interleaving the three)
  __builtin_amdgcn_sched_barrier(0);
  // the wave's weight block scales, lane i holding chunk c0 + i's (at most 64 chunks a wave, checked on the
  // host); each chunk's is read out with v_readlane into a scalar register
  const float swl = ldgf(swrow + c0 + min(lane, nl));
  TileChunk buf[kTileRing];
#pragma unroll
  for (int j = 0; j < kTileRing; ++j) tile_load<kFused>(buf[j], wlane, xrow, xsrow, c0 + min(j, nl), q);
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (kFused) {
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int b = b0 + 4 * p + grp;
      const uint32_t wd[4] = {xv[p].x, xv[p].y, xv[p].z, xv[p].w};
      float v[8];
      float amax = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[2 * i] = mx::bf16_value(wd[i] & 0xFFFFu);
        v[2 * i + 1] = mx::bf16_value(wd[i] >> 16);
        amax = fmaxf(amax, fmaxf(fabsf(v[2 * i]), fabsf(v[2 * i + 1])));
      }
      amax = mxd::row16_max(amax);
      const float sc = mx::act128_scale(amax);
      const int row = b < nb ? kp * kPartRows + b : KP * kPartRows + w;
      *reinterpret_cast<uint2*>(qx + row * kFusedRow + 8 * sub) = act128_codes8(v, sc);
      if (sub == 0) qsc[row] = sc;
    }
    if constexpr (M == 1) {
      // the rows are this wave's own: its LDS writes complete before its reads (no workgroup barrier)
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    } else {
      mxd::lds_barrier();   // the part's rows come from M waves; LDS only, the weight loads stay in flight
    }
  }
  v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
  const uint32_t keep = live ? 0xFFFFFFFFu : 0u;
  const int qtok = kFused ? min(nn, ntok - 1) : 0;
  const uint8_t* qrow = qx + (kp * kPartRows + qtok) * kFusedRow;
  const float* qs = qsc + kp * kPartRows + qtok;
  int i = 0;
  for (; i + kTileRing < n; i += kTileRing) {
#pragma unroll
    for (int j = 0; j < kTileRing; ++j) {
      // a ring: chunk i + j is multiplied, then its slot is refilled with chunk i + j + kTileRing before the
      // next chunk is waited for (the barrier keeps the compiler from batching the loads after all four)
      tile_mma<kFused>(buf[j], acc, q, keep, chunk_scale(swl, i + j), qrow + (i + j) * ntok * kFusedRow,
                       qs + (i + j) * ntok);
      tile_load<kFused>(buf[j], wlane, xrow, xsrow, c0 + min(i + j + kTileRing, nl), q);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
#pragma unroll
  for (int j = 0; j < kTileRing; ++j) {
    const int ij = min(i + j, nl);
    tile_mma<kFused>(buf[j], acc, q, i + j < n ? keep : 0u, chunk_scale(swl, ij), qrow + ij * ntok * kFusedRow,
                     qs + ij * ntok);
  }
  __shared__ float4 red[W][64];
  red[w][lane] = make_float4(acc[0], acc[1], acc[2], acc[3]);
  __syncthreads();
  if (w >= M || !live) return;
  // wave w < M finishes tile w: K-part order, over the parts that own chunks (KP > C leaves some without)
  float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
  bool first = true;
#pragma unroll
  for (int v = 0; v < KP; ++v) {
    if ((C * (v + 1)) / KP == (C * v) / KP) continue;
    const float4 r = red[w + M * v][lane];
    if (first) {
      t = r;
      first = false;
    } else {
      t.x = t.x + r.x;
      t.y = t.y + r.y;
      t.z = t.z + r.z;
      t.w = t.w + r.w;
    }
  }
  const size_t o = (size_t)tok * a.N + 16 * tile + 4 * q;
  uint2 packed;
  packed.x = mx::bf16_bits(t.x) | (mx::bf16_bits(t.y) << 16);
  packed.y = mx::bf16_bits(t.z) | (mx::bf16_bits(t.w) << 16);
  *reinterpret_cast<uint2*>(a.y + o) = packed;
  if (a.trace) *reinterpret_cast<float4*>(a.trace + o) = t;
}

// Split-K epilogue: y = BF16(sum over splits in order), 4 outputs per thread.
__global__ void fp8_splitk_reduce_kernel(const float* __restrict__ partial, int splits, int64_t count,
                                         uint16_t* __restrict__ y, float* __restrict__ trace) {
  const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (i >= count) return;
  float4 s = *reinterpret_cast<const float4*>(partial + i);
  for (int z = 1; z < splits; ++z) {
    const float4 v = *reinterpret_cast<const float4*>(partial + (size_t)z * count + i);
    s.x = s.x + v.x;
    s.y = s.y + v.y;
    s.z = s.z + v.z;
    s.w = s.w + v.w;
  }
  uint2 packed;
  packed.x = mx::bf16_bits(s.x) | (mx::bf16_bits(s.y) << 16);
  packed.y = mx::bf16_bits(s.z) | (mx::bf16_bits(s.w) << 16);
  *reinterpret_cast<uint2*>(y + i) = packed;
  if (trace) *reinterpret_cast<float4*>(trace + i) = s;
}

// ---- GEMM for many tokens ------------------------------------------------------------------------
//
// grid (ceil(N / 256), ceil(T / 128), K splits), 768 threads = 12 waves. Waves 0-7 multiply: wave w owns
// the 64-row group 4 * blockIdx.x + (w % 4) and the token half w / 4 (64 tokens), 4 row tiles x 4 token
// tiles of 16 x 16. Waves 8-11 only copy operands global -> LDS (direct copies, no registers) into a
// 3-stage ring, two chunks ahead. Measured on MI355X: a CU moves at most 64 bytes per clock from L2 into
// LDS, and while a chunk is still on its way from HBM (the first workgroup of an XCD to ask for it, and
// every workgroup asking at the same time) a wave issuing copies stalls for most of their latency. When
// the multiplying waves issue the copies themselves, each 128-wide chunk takes about 2,700 clocks: the
// stalled copies hold up the MFMAs behind them. In waves of their own the stalls hold up no MFMA, since
// each SIMD issues from whichever of its waves is ready; the copy waves then set the pace (about 1,900
// clocks per chunk for the o projection at T = 2048, 1,000 when every chunk is already in L2) against
// about 1,450 for the multiplying waves. Stage layout: the 4 row groups' weight chunks
// (32 KB, piece 8 g + 2 t + h in the tiled blob's MFMA operand order), the 128 tokens' activation codes
// (16 KB, block 2 u + h holding at lane (q, n) bytes 64 h + 16 q .. of token 16 u + n: the B operand of
// token tile u), their scales (512 B) and the 4 row groups' weight-scale words (1 KB, 256 B each). Step
// c: the multiplying waves read chunk c from its stage and multiply; the copy waves issue chunk c + 2 into
// the stage chunk c - 1 left and wait for chunk c + 1; one barrier ends the step. The loops have no
// compiler-visible global loads (the copies are inline assembly), so the compiler adds no vmcnt waits.
constexpr int kGemmTok = 128;                 // tokens per workgroup
constexpr int kWaveTiles = 4;                 // token tiles per multiplying wave
constexpr int kGemmThreads = 768;
constexpr int kGemmA = 32768;
constexpr int kGemmB = 16384;
constexpr int kGemmSA = 512;
constexpr int kGemmSW = 1024;
constexpr int kGemmStage = kGemmA + kGemmB + kGemmSA + kGemmSW;
constexpr int kGemmStages = 3;
constexpr int kGemmCopies = 14;   // per copy wave and chunk: 8 weight, 4 activation, 1 + 1 scale
static_assert(kGemmStages * kGemmStage <= 160 * 1024, "GEMM LDS ring");

template <int kBlock>
__global__ __launch_bounds__(kGemmThreads) void fp8_gemm_kernel(Fp8Args a) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[kGemmStages * kGemmStage];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q = lane >> 4, n = lane & 15;
  const int chunks = a.K / 128, per = (chunks + gridDim.z - 1) / gridDim.z;
  const int c0 = blockIdx.z * per;
  const int C = min(per, chunks - c0);
  const int groups = a.N / 64;
  const int bx = blockIdx.x;
  const int m0 = blockIdx.y * kGemmTok;
  const Fp8Blob off = fp8_blob(a.N, a.K, kBlock);
  const uint32_t lds0 = mxd::lds_addr(lds);

  if (wave >= 8) {
    // copy wave p: row group p's 8 weight pieces and scale word(s), activation tiles 2p and 2p + 1 (both
    // blocks of each), the scales of tokens 32p .. 32p + 31. Rows past N and tokens past T repeat valid ones.
    const int p = wave - 8;
    const int gp = min(bx * 4 + p, groups - 1);
    const uint8_t* wsrc = a.blob + (size_t)gp * chunks * 8192 + 16 * lane;
    const uint8_t* bsrc0 = a.xq + (size_t)min(m0 + 32 * p + n, a.T - 1) * a.K + 16 * q;
    const uint8_t* bsrc1 = a.xq + (size_t)min(m0 + 32 * p + 16 + n, a.T - 1) * a.K + 16 * q;
    const int stok = min(m0 + 32 * p + (lane & 31), a.T - 1);
    const uint8_t* sasrc = kBlock == 32 ? (const uint8_t*)a.xs + (size_t)stok * (a.K / 32)
                                        : (const uint8_t*)a.xs + (size_t)stok * chunks * 4;
    const uint8_t* swsrc = kBlock == 32 ? a.blob + off.scales + (size_t)gp * chunks * 256 + 4 * lane
                                        : a.blob + off.scales + ((size_t)((64 * gp) / 128) * chunks) * 4;
    auto copy = [&](int cl) {
      const int c = c0 + cl;
      const uint32_t st = lds0 + (uint32_t)(cl % kGemmStages) * kGemmStage;
#pragma unroll
      for (int i = 0; i < 8; ++i)
        mxd::global_to_lds16(wsrc + (size_t)c * 8192 + i * 1024, __builtin_amdgcn_readfirstlane(st + (8 * p + i) * 1024));
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        mxd::global_to_lds16(bsrc0 + (size_t)c * 128 + 64 * h,
                             __builtin_amdgcn_readfirstlane(st + kGemmA + (4 * p + h) * 1024));
        mxd::global_to_lds16(bsrc1 + (size_t)c * 128 + 64 * h,
                             __builtin_amdgcn_readfirstlane(st + kGemmA + (4 * p + 2 + h) * 1024));
      }
      const uint32_t sa_lds = __builtin_amdgcn_readfirstlane(st + kGemmA + kGemmB + 128 * p);
      if (lane < 32) mxd::global_to_lds4(sasrc + (size_t)c * 4, sa_lds);
      const uint32_t sw_lds = __builtin_amdgcn_readfirstlane(st + kGemmA + kGemmB + kGemmSA + 256 * p);
      if (kBlock == 32 || lane == 0) mxd::global_to_lds4(swsrc + (size_t)c * (kBlock == 32 ? 256 : 4), sw_lds);
    };
    copy(0);
    if (C > 1) {
      copy(1);
      __builtin_amdgcn_s_waitcnt(mxd::vm_wait_imm(kGemmCopies));
    } else {
      __builtin_amdgcn_s_waitcnt(mxd::vm_wait_imm(0));
    }
    mxd::copy_barrier();
    for (int c = 0; c < C; ++c) {
      if (c + 2 < C) {
        copy(c + 2);
        __builtin_amdgcn_s_waitcnt(mxd::vm_wait_imm(kGemmCopies));   // chunk c + 1 has landed
      } else {
        __builtin_amdgcn_s_waitcnt(mxd::vm_wait_imm(0));
      }
      mxd::copy_barrier();
    }
    return;
  }

  const int g_raw = bx * 4 + (wave & 3);
  const bool has_rows = g_raw < groups;
  const int g = has_rows ? g_raw : groups - 1;
  const int u0 = (wave >> 2) * kWaveTiles;
  v4f acc[kTiles][kWaveTiles];
#pragma unroll
  for (int t = 0; t < kTiles; ++t)
#pragma unroll
    for (int u = 0; u < kWaveTiles; ++u) acc[t][u] = v4f{0.f, 0.f, 0.f, 0.f};
  mxd::copy_barrier();
  for (int c = 0; c < C; ++c) {
    const uint8_t* st = lds + (c % kGemmStages) * kGemmStage;
    uint4 am[kTiles][2], b[kWaveTiles][2];
    float sx[kWaveTiles];
#pragma unroll
    for (int t = 0; t < kTiles; ++t)
#pragma unroll
      for (int h = 0; h < 2; ++h)
        am[t][h] = *reinterpret_cast<const uint4*>(st + (8 * (wave & 3) + 2 * t + h) * 1024 + 16 * lane);
#pragma unroll
    for (int u = 0; u < kWaveTiles; ++u) {
      const int tile = u0 + u;
      b[u][0] = *reinterpret_cast<const uint4*>(st + kGemmA + (2 * tile) * 1024 + 16 * lane);
      b[u][1] = *reinterpret_cast<const uint4*>(st + kGemmA + (2 * tile + 1) * 1024 + 16 * lane);
      sx[u] = *reinterpret_cast<const float*>(st + kGemmA + kGemmB + 4 * (16 * tile + n));
    }
    const uint32_t swv = *reinterpret_cast<const uint32_t*>(st + kGemmA + kGemmB + kGemmSA + 256 * (wave & 3) +
                                                            (kBlock == 32 ? 4 * lane : 0));
    if constexpr (kBlock == 32) {
#pragma unroll
      for (int u = 0; u < kWaveTiles; ++u) {
        const int sxb = (int)((__float_as_uint(sx[u]) >> (8 * q)) & 0xFF);
#pragma unroll
        for (int t = 0; t < kTiles; ++t)
          acc[t][u] = mfma_fp8_fp8(am[t][0], am[t][1], b[u][0], b[u][1], acc[t][u], (int)((swv >> (8 * t)) & 0xFF),
                                   sxb);
      }
    } else {
      const float swf = __uint_as_float(swv);
      constexpr int kSteps = kTiles * kWaveTiles;
      v4f d[2];
      d[0] = mfma_fp8_fp8(am[0][0], am[0][1], b[0][0], b[0][1], v4f{0.f, 0.f, 0.f, 0.f}, 127, 127);
#pragma unroll
      for (int k = 0; k < kSteps; ++k) {
        const int t = k % kTiles, u = k / kTiles;
        if (k + 1 < kSteps) {
          const int t1 = (k + 1) % kTiles, u1 = (k + 1) / kTiles;
          d[(k + 1) & 1] = mfma_fp8_fp8(am[t1][0], am[t1][1], b[u1][0], b[u1][1], v4f{0.f, 0.f, 0.f, 0.f}, 127, 127);
        }
        __builtin_amdgcn_sched_barrier(0);
        const float sc = sx[u] * swf;
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[t][u][i] = fmaf(d[k & 1][i], sc, acc[t][u][i]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): this wave's reads of chunk c are done
    mxd::copy_barrier();
  }
  if (!has_rows) return;
#pragma unroll
  for (int u = 0; u < kWaveTiles; ++u) {
    const int tok = m0 + 16 * (u0 + u) + n;
    if (tok >= a.T) continue;
#pragma unroll
    for (int t = 0; t < kTiles; ++t) {
      const size_t o = (size_t)tok * a.N + 64 * g + 16 * t + 4 * q;
      const float4 v = make_float4(acc[t][u][0], acc[t][u][1], acc[t][u][2], acc[t][u][3]);
      if (gridDim.z > 1) {
        *reinterpret_cast<float4*>(a.partial + (size_t)blockIdx.z * a.T * a.N + o) = v;
        continue;
      }
      uint2 packed;
      packed.x = mx::bf16_bits(v.x) | (mx::bf16_bits(v.y) << 16);
      packed.y = mx::bf16_bits(v.z) | (mx::bf16_bits(v.w) << 16);
      *reinterpret_cast<uint2*>(a.y + o) = packed;
      if (a.trace) *reinterpret_cast<float4*>(a.trace + o) = v;
    }
  }
}

int check_fp8_shape(int N, int K, int block, const char* who) {
  MX_REQUIRE(block == 32 || block == 128, "%s: block must be 32 or 128", who);
  MX_REQUIRE(N > 0 && N % 64 == 0 && K > 0 && K % 128 == 0, "%s: rows must be a multiple of 64 and width of 128",
             who);
  return MX_OK;
}

// K splits. Decode GEMV: see below. GEMM: only when the rows and tokens alone give fewer workgroups than
// half the CUs (the partial sums cost a write and a read of splits x T x N floats and a reduce launch), then
// about 512, every split keeping 8 chunks. 2112 x 7168 at T = 2048 (144 workgroups) ran 97 us per call
// unsplit against 110 us with 4 splits (MI355X, quantizer included).
int fp8_splits(int N, int K, int T) {
  if (T > kGemvMaxTokens) {
    const int base_wgs = ((N / 64 + 3) / 4) * ((T + kGemmTok - 1) / kGemmTok);
    if (base_wgs >= 128) return 1;
    return std::max(1, std::min({8, (K / 128) / 8, (512 + base_wgs - 1) / base_wgs}));
  }
  // Split-K GEMV: up to kFusedMaxTokens tokens every workgroup takes up to 16 chunks of its row group, else
  // about 8; at most 16 splits. Fewer, longer workgroups measured faster than a fixed workgroup count on
  // MI355X (us per call, T = 1 / 16): 2112 x 7168 7 splits 11.3 / 13.1 against 14 splits (the former
  // ~512-workgroup rule) 12.5 / 16.9; 7168 x 16384 16 splits 28.9 / 33.8 against 5 splits 30.1 / 33.3. At T =
  // 1 with non-temporal weight loads: 24576 x 1536 unsplit 10.3 us against 12.5 us with 2 splits (no split-K
  // handoff); 2112 x 7168 4 splits 10.4 us, 7168 x 16384 8 splits 26.6 us, both as with 7 and 16. (Block-128
  // calls of up to 4 tokens now run on the tile GEMV, which splits K only within a workgroup.)
  const int chunks = K / 128;
  const int s = T <= kFusedMaxTokens ? (chunks + 15) / 16 : chunks / 8;
  return std::max(1, std::min(16, s));
}

// Shape of the block-128 decode GEMV (fp8_tile_gemv_kernel): W waves and M tiles per workgroup. Many tiles
// (q_b's 1536): 2 tiles of 4 K parts; few tiles (q_kv_a's 132): 8 K parts of one tile; otherwise (o's 448)
// 2 tiles of 8 K parts. Measured on MI355X at T = 1 (us per call, weights rotated): q_b 7.7-8.6 with 2 x 4
// against 9.6-10.2 with 4 tiles x 4 parts, 10.0 with 4 x 2 and 11.8-12.1 with 2 x 8; q_kv_a 6.6-6.7 with
// 1 x 8 against 6.9-7.0 with 1 x 16; o 21.1-21.4 with 2 x 8 against 22.0-22.5 with 1 x 8 and 22.8 with
// 1 x 16. A 6-chunk ring left o unchanged and slowed q_kv_a.
struct TileShape {
  int W, M;
};

TileShape fp8_tile_shape(int N, int T) {
  const int tiles = (N / 16) * ((T + kTok - 1) / kTok);
  if (tiles >= 1024) return {8, 2};
  if (tiles * 16 <= 4096) return {8, 1};
  return {16, 2};
}

// Whether fp8_tile_gemv_kernel takes the call: every wave's chunks within the 64 lanes that hold their weight
// scales (K up to 64 x 128 x the K parts).
bool fp8_tile_ok(int N, int K, int T) {
  const TileShape sh = fp8_tile_shape(N, T);
  const int kp = sh.W / sh.M;
  return (K / 128 + kp - 1) / kp <= 64;
}

// Fused quantization passes (4 blocks of 128 each per wave) for a K part's chunks x the tokens, shared by the
// part's M waves: 1, 2 or 4, or 0 when they exceed the part's LDS rows (the call then quantizes in its own
// launch).
int fp8_tile_passes(int N, int K, int T) {
  const TileShape sh = fp8_tile_shape(N, T);
  const int kp = sh.W / sh.M, blocks = ((K / 128 + kp - 1) / kp) * T;
  if (blocks > kTileQRows) return 0;
  const int per_wave = (blocks + sh.M - 1) / sh.M;
  return per_wave <= 4 ? 1 : per_wave <= 8 ? 2 : 4;
}

// Whether a block-128 call runs on fp8_tile_gemv_kernel: up to kFusedMaxTokens tokens (above that the split-K
// GEMV, whose 64-row workgroups load each activation chunk once for 4 tiles, measured faster).
bool fp8_tile_call(int N, int K, int T, int block) {
  return block == 128 && T <= kFusedMaxTokens && fp8_tile_ok(N, K, T);
}

// Whether the block-128 GEMV can quantize its own activations: a tile call whose every wave's blocks fit its
// LDS rows.
bool fp8_fused_ok(int N, int K, int T, int block) {
  return fp8_tile_call(N, K, T, block) && fp8_tile_passes(N, K, T) > 0;
}

// fp8_tile_gemv_kernel of shape (W, M): P fused quantization passes, or P = 0 when x comes quantized.
template <int W, int M>
void launch_tile_gemv(const Fp8Args& a, int P, dim3 grid, hipStream_t st) {
  const dim3 threads(64 * W);
  if (P == 1) hipLaunchKernelGGL((fp8_tile_gemv_kernel<true, W, M, 1>), grid, threads, 0, st, a);
  else if (P == 2) hipLaunchKernelGGL((fp8_tile_gemv_kernel<true, W, M, 2>), grid, threads, 0, st, a);
  else if (P == 4) {
    if constexpr (16 * M <= kTileQRows) hipLaunchKernelGGL((fp8_tile_gemv_kernel<true, W, M, 4>), grid, threads, 0, st, a);
  } else hipLaunchKernelGGL((fp8_tile_gemv_kernel<false, W, M, 1>), grid, threads, 0, st, a);
}

// The product on quantized activations: the tile GEMV (block 128, T <= kFusedMaxTokens: no K split across
// workgroups), the split-K GEMV (T <= 32) or the tiled GEMM, the latter two with K split over fp8_splits(N,
// K, T) workgroups whose FP32 partial sums are added in split order: by the GEMV's last workgroup per tile
// through the context's arrival counters and handoff buffer when they fit it (kTicketPartialBytes), else
// written to `partial` (fp8_splits * T * N floats) and added by fp8_splitk_reduce_kernel.
// x_fused: the BF16 input when the GEMV quantizes it itself (fp8_fused_ok), else null (q and sc given).
int launch_fp8_product(const uint8_t* blob, int N, int K, int block, const uint8_t* q, const void* sc, int T,
                       uint16_t* y, float* trace, float* partial, mx_ctx* ctx, hipStream_t st,
                       const uint16_t* x_fused = nullptr, int x_group_rows = 0) {
  Fp8Args a{};
  a.blob = blob;
  a.N = N;
  a.K = K;
  a.T = T;
  a.x_group_rows = x_group_rows;
  a.x_stride = x_group_rows ? (int64_t)K * (N / x_group_rows) : K;
  a.xq = q;
  a.xs = sc;
  a.y = y;
  a.trace = trace;
  a.partial = partial;
  a.x = x_fused;
  if (x_fused) a.xq = reinterpret_cast<const uint8_t*>(x_fused);   // not read: B comes from LDS
  if (fp8_tile_call(N, K, T, block)) {
    const TileShape sh = fp8_tile_shape(N, T);
    const dim3 grid(N / 16 / sh.M, (T + kTok - 1) / kTok);
    const int P = x_fused ? fp8_tile_passes(N, K, T) : 0;
    if (sh.W == 16) launch_tile_gemv<16, 2>(a, P, grid, st);
    else if (sh.M == 2) launch_tile_gemv<8, 2>(a, P, grid, st);
    else launch_tile_gemv<8, 1>(a, P, grid, st);
    MX_LAUNCH_CHECK("fp8_tile_gemv_kernel");
  } else if (T <= kGemvMaxTokens) {
    const int splits = fp8_splits(N, K, T);
    const dim3 grid(N / 64, (T + kTok - 1) / kTok, splits);
    if (splits > 1 && (size_t)grid.x * grid.y <= MX_TICKETS &&
        (uint64_t)splits * T * N * sizeof(float) <= kTicketPartialBytes) {
      // this launch's half, and the other half's extent the previous launch wrote (restored by this launch)
      const int h = ctx->handoff_half;
      a.tickets = ctx->tickets;
      a.handoff = ctx->handoff + (size_t)h * (MX_HANDOFF_BYTES / 4);
      a.restore = reinterpret_cast<uint4*>(ctx->handoff + (size_t)(1 - h) * (MX_HANDOFF_BYTES / 4));
      a.restore_n = (int64_t)(ctx->handoff_dirty[1 - h] / 16);
      ctx->handoff_dirty[1 - h] = 0;
      ctx->handoff_dirty[h] = ((uint64_t)splits * T * N * sizeof(float) + 15) / 16 * 16;
      ctx->handoff_half = 1 - h;
    }
    if (block == 32) hipLaunchKernelGGL(fp8_gemv_kernel<32>, grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL(fp8_gemv_kernel<128>, grid, dim3(256), 0, st, a);
    MX_LAUNCH_CHECK("fp8_gemv_kernel");
    if (splits > 1 && !a.tickets) {
      const int64_t count = (int64_t)T * N;
      hipLaunchKernelGGL(fp8_splitk_reduce_kernel, dim3((unsigned)((count / 4 + 255) / 256)), dim3(256), 0, st,
                         (const float*)partial, splits, count, y, trace);
      MX_LAUNCH_CHECK("fp8_splitk_reduce_kernel");
    }
  } else {
    const int splits = fp8_splits(N, K, T);
    const dim3 grid((N / 64 + 3) / 4, (T + kGemmTok - 1) / kGemmTok, splits);
    if (block == 32) hipLaunchKernelGGL(fp8_gemm_kernel<32>, grid, dim3(kGemmThreads), 0, st, a);
    else hipLaunchKernelGGL(fp8_gemm_kernel<128>, grid, dim3(kGemmThreads), 0, st, a);
    if (splits > 1) {
      const int64_t count = (int64_t)T * N;
      hipLaunchKernelGGL(fp8_splitk_reduce_kernel, dim3((unsigned)((count / 4 + 255) / 256)), dim3(256), 0, st,
                         (const float*)partial, splits, count, y, trace);
      MX_LAUNCH_CHECK("fp8_splitk_reduce_kernel");
    }
  }
  return MX_OK;
}

// SwiGLU of the FP8 expert, one element per thread (the gate/up kernel of the MXFP4 path applies the
// same mxd::swiglu_element in its epilogue).
__global__ void swiglu_kernel(const uint16_t* __restrict__ w1, const uint16_t* __restrict__ w3, int T, int I,
                              float limit, const float* __restrict__ route_w, uint16_t* __restrict__ din,
                              float* __restrict__ trace) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)T * I) return;
  const int t = (int)(i / I);
  const float v = mxd::swiglu_element(w1[i], w3[i], limit, route_w != nullptr, route_w ? route_w[t] : 1.f,
                                      trace ? trace + i * 5 : nullptr);
  din[i] = (uint16_t)mx::bf16_bits(v);
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
  if (((uintptr_t)x & 15) == 0 && ((uintptr_t)q & 7) == 0) {
    const int64_t want = (blocks + 15) / 16;   // 16 blocks per 256-thread workgroup and pass
    hipLaunchKernelGGL(act_quant128_v8_kernel, dim3((unsigned)(want < 8192 ? want : 8192)), dim3(256), 0,
                       as_stream(stream), x, q, s, blocks);
    MX_LAUNCH_CHECK("act_quant128_v8_kernel");
    return MX_OK;
  }
  MX_REQUIRE(blocks <= (int64_t)(1u << 31) * 4 - 4, "mx_act_quant128: too many blocks for one launch");
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
  const uint64_t s_b = ((block == 32 ? (uint64_t)T * (K / 32) : (uint64_t)T * (K / 128) * 4) + 255) & ~255ull;
  const uint64_t p_b = fp8_tile_call(N, K, T, block) ? 0 : (uint64_t)fp8_splits(N, K, T) * T * N * 4;
  void* base = nullptr;
  if (int s = scratch(ctx, q_b + s_b + p_b + 256, &base)) return s;
  uint8_t* q = q_out ? q_out : (uint8_t*)base;
  void* sc = s_out ? s_out : (void*)((uint8_t*)base + q_b);
  MX_REQUIRE(((uintptr_t)q & 15) == 0 && ((uintptr_t)sc & 3) == 0, "mx_fp8_projection: q 16-byte, s 4-byte aligned");
  float* partial = (float*)((uint8_t*)base + q_b + s_b);
  if (!q_out && !s_out && fp8_fused_ok(N, K, T, block))   // the GEMV quantizes x itself
    return launch_fp8_product((const uint8_t*)tiled, N, K, block, nullptr, nullptr, T, y, trace, partial, ctx, st,
                              x);
  if (block == 32) {
    if (int s = mx_act_quant32(ctx, x, q, (uint8_t*)sc, T, K, stream)) return s;
  } else {
    if (int s = mx_act_quant128(ctx, x, q, (float*)sc, T, K, stream)) return s;
  }
  return launch_fp8_product((const uint8_t*)tiled, N, K, block, q, sc, T, y, trace, partial, ctx, st);
}

int mx_fp8_grouped_projection(mx_ctx* ctx, const void* tiled, int32_t groups, int32_t rows, int32_t K,
                              const uint8_t* q, const uint8_t* s, int32_t T, uint16_t* y, float* trace, void* stream) {
  if (int st = use(ctx)) return st;
  MX_REQUIRE(groups >= 1 && groups <= 64 && rows > 0 && rows % 64 == 0 && rows <= (1 << 20),
             "mx_fp8_grouped_projection: 1 to 64 groups of a positive multiple of 64 rows required");
  const int N = groups * rows;
  if (int st = check_fp8_shape(N, K, 32, "mx_fp8_grouped_projection")) return st;
  MX_REQUIRE(T >= 0 && T <= kGemvMaxTokens, "mx_fp8_grouped_projection: token count %d outside [0, %d]", T,
             kGemvMaxTokens);
  if (!T) return MX_OK;
  MX_REQUIRE(tiled && q && s && y, "mx_fp8_grouped_projection: null pointer");
  MX_REQUIRE(((uintptr_t)tiled & 255) == 0 && ((uintptr_t)q & 15) == 0 && ((uintptr_t)s & 3) == 0 &&
                 ((uintptr_t)y & 7) == 0 && ((uintptr_t)trace & 15) == 0,
             "mx_fp8_grouped_projection: tiled 256-byte, q 16-byte, s 4-byte, y 8-byte, trace 16-byte alignment");
  void* base = nullptr;
  if (int st = scratch(ctx, (uint64_t)fp8_splits(N, K, T) * T * N * 4 + 256, &base)) return st;
  return launch_fp8_product((const uint8_t*)tiled, N, K, 32, q, s, T, y, trace, (float*)base, ctx,
                            as_stream(stream), nullptr, rows);
}

int mx_fp8_expert_forward(mx_ctx* ctx, const void* w1, const void* w3, const void* w2, int32_t H, int32_t I,
                          const uint16_t* x, int32_t T, float limit, const float* route_w, uint16_t* y,
                          const mx_expert_stages* stages, void* stream) {
  if (int s = use(ctx)) return s;
  MX_REQUIRE(w1 && w3 && w2, "mx_fp8_expert_forward: null tiled weight");
  MX_REQUIRE(((uintptr_t)w1 & 255) == 0 && ((uintptr_t)w3 & 255) == 0 && ((uintptr_t)w2 & 255) == 0,
             "mx_fp8_expert_forward: tiled weights must be 256-byte aligned");
  MX_REQUIRE(H > 0 && H % 128 == 0 && I > 0 && I % 128 == 0, "expert shapes must be positive multiples of 128");
  MX_REQUIRE(T >= 0 && T <= kTok, "token count %d outside [0, %d]", T, kTok);
  MX_REQUIRE(std::isfinite(limit) && limit >= 0.f, "Invalid SwiGLU limit");
  if (!T) return MX_OK;
  MX_REQUIRE(x && y && ((uintptr_t)x & 15) == 0 && ((uintptr_t)y & 15) == 0,
             "x and y must be 16-byte aligned device pointers");
  hipStream_t st = as_stream(stream);
  auto r256 = [](uint64_t b) { return (b + 255) & ~255ull; };
  const uint64_t sizes[7] = {r256((uint64_t)T * H),     r256((uint64_t)T * H / 32), r256((uint64_t)T * I * 2),
                             r256((uint64_t)T * I * 2), r256((uint64_t)T * I * 2),  r256((uint64_t)T * I),
                             r256((uint64_t)T * I / 32)};
  const uint64_t p_b = (uint64_t)std::max(fp8_splits(I, H, T) * I, fp8_splits(H, I, T) * H) * T * 4;
  uint64_t total = p_b;
  for (uint64_t b : sizes) total += b;
  void* base = nullptr;
  if (int s = scratch(ctx, total, &base)) return s;
  uint8_t* cur = (uint8_t*)base;
  uint8_t* buf[7];
  for (int i = 0; i < 7; ++i) {
    buf[i] = cur;
    cur += sizes[i];
  }
  float* partial = (float*)cur;
  uint8_t* q = (stages && stages->q) ? stages->q : buf[0];
  uint8_t* s = (stages && stages->s) ? stages->s : buf[1];
  uint16_t* b1 = (stages && stages->w1) ? stages->w1 : (uint16_t*)buf[2];
  uint16_t* b3 = (stages && stages->w3) ? stages->w3 : (uint16_t*)buf[3];
  uint16_t* din = (stages && stages->down_input) ? stages->down_input : (uint16_t*)buf[4];
  uint8_t* dq = (stages && stages->down_q) ? stages->down_q : buf[5];
  uint8_t* ds = (stages && stages->down_s) ? stages->down_s : buf[6];
  float* trace = stages ? stages->trace : nullptr;
  MX_REQUIRE(((uintptr_t)q & 15) == 0 && ((uintptr_t)dq & 15) == 0 && ((uintptr_t)b1 & 7) == 0 &&
                 ((uintptr_t)b3 & 7) == 0 && ((uintptr_t)din & 3) == 0 && ((uintptr_t)s & 3) == 0 &&
                 ((uintptr_t)ds & 3) == 0,
             "stage buffers: q/down_q 16-byte, w1/w3 8-byte, scales and down_input 4-byte aligned");
  if (int e = mx_act_quant32(ctx, x, q, s, T, H, stream)) return e;
  if (int e = launch_fp8_product((const uint8_t*)w1, I, H, 32, q, s, T, b1, nullptr, partial, ctx, st)) return e;
  if (int e = launch_fp8_product((const uint8_t*)w3, I, H, 32, q, s, T, b3, nullptr, partial, ctx, st)) return e;
  const int64_t n = (int64_t)T * I;
  hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, (const uint16_t*)b1,
                     (const uint16_t*)b3, T, I, limit, route_w, din, trace);
  MX_LAUNCH_CHECK("swiglu_kernel");
  if (int e = mx_act_quant32(ctx, din, dq, ds, T, I, stream)) return e;
  return launch_fp8_product((const uint8_t*)w2, H, I, 32, dq, ds, T, y, nullptr, partial, ctx, st);
}

}  // extern "C"
