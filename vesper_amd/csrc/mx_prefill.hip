// MoE prefill on gfx950: many tokens through a decode layer's experts as token-sorted grouped GEMMs on
// the scaled MXFP4 MFMA. Per token the arithmetic is the decode path's
// (ConnectedMoE.forward, src/vesper/connected.py:125-186: per-32 activation quantization, W1/W3,
// SwiGLU with the route weight before W2, down-input quantization, W2, ordered combine with the
// shared expert last); only the summation order inside the products differs.
//
//   plan      count pairs per expert, expert-major row offsets (shared expert last) and 128-row tiles;
//             a stable per-expert scatter gives each expert's rows in ascending token order
//             (participation, src/vesper/moe.py:18-30) and each (token, rank) pair its row
//   gate/up   grid (I/128, tiles), 8 waves: 4 groups of 32 intermediate rows (W1 + W3 interleaved per
//             MFMA tile, as in the tiled layout) x 2 halves of the tile's 128 tokens; the tokens' E4M3
//             rows are gathered into LDS per 128-wide K chunk; epilogue SwiGLU + route weight + the
//             per-token quantization of each 32-row block of the down input
//   down      grid (H/256, tiles), same shape over W2 with the tile's contiguous down-input rows
//   combine   per token: its expert rows in ascending expert ID, then the shared row; FP32 from +0,
//             one BF16 rounding (aggregation_probe.cu:4-25)
#include <algorithm>
#include <cmath>

#include "mx_device.h"
#include "mx_internal.h"
#include "mx_numerics.h"

namespace {

using mxd::ldg128;
using mxd::ldg32;
using mxd::mfma_fp4_fp8;
using mxd::tiled_offsets;
using mxd::TiledOffsets;
using mxd::v4f;

constexpr int kTileRows = 128;   // token rows per GEMM tile
constexpr int kThreads = 512;    // 8 waves
constexpr int kWaveTok = 4;      // token tiles of 16 per wave
constexpr int kLdsRow = 144;     // 128 bytes of a row's K chunk + 16 bytes of bank padding
constexpr int kDepth = 3;        // chunks of operands in flight per wave
constexpr int kMaxTopK = 32;

struct PrefillPlan {
  int32_t* counts;      // [E + 1] pairs per slot (slot E = shared expert)
  int32_t* row0;        // [E + 1] first row of each slot
  int32_t* tile_info;   // [max_tiles][4]: slot, first row, rows, unused
  int32_t* n_tiles;     // [1]
  int32_t* sorted_tok;  // [rows] token of each row
  float* sorted_w;      // [rows] route weight of each row
  int32_t* pair_row;    // [T * k] row of pair (t, rank)
};

__global__ void zero_i32_kernel(int32_t* p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

// Routing ids outside [0, E) (the C caller's responsibility) are skipped by every plan step and by the
// combine, so such input gives wrong rows for its token but never an access out of bounds.
// Per-workgroup LDS histogram, then one global atomic per nonzero bin (E <= 1024).
__global__ __launch_bounds__(256) void count_kernel(const int32_t* __restrict__ ids, int n, int E,
                                                    int32_t* __restrict__ counts) {
  __shared__ int32_t h[1024];
  for (int e = threadIdx.x; e < E; e += 256) h[e] = 0;
  __syncthreads();
  for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) {
    const int e = ids[i];
    if (e >= 0 && e < E) atomicAdd(&h[e], 1);
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += 256)
    if (h[e]) atomicAdd(&counts[e], h[e]);
}

// One wave: slot counts -> row offsets and the tile list (ascending slot, shared last).
__global__ __launch_bounds__(64) void offsets_kernel(PrefillPlan p, int E, int T, int has_shared) {
  const int lane = threadIdx.x;
  const int slots = E + 1;
  int row_carry = 0, tile_carry = 0;
  for (int base = 0; base < slots; base += 64) {
    const int s = base + lane;
    const int cnt = s < E ? p.counts[s] : (s == E && has_shared ? T : 0);
    const int tiles = (cnt + kTileRows - 1) / kTileRows;
    int rs = cnt, ts = tiles;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int r2 = __shfl_up(rs, d, 64), t2 = __shfl_up(ts, d, 64);
      if (lane >= d) {
        rs += r2;
        ts += t2;
      }
    }
    const int r0 = row_carry + rs - cnt, t0 = tile_carry + ts - tiles;
    if (s < slots) {
      p.row0[s] = r0;
      for (int j = 0; j < tiles; ++j) {
        int32_t* info = p.tile_info + (size_t)(t0 + j) * 4;
        info[0] = s;
        info[1] = r0 + j * kTileRows;
        info[2] = min(kTileRows, cnt - j * kTileRows);
        info[3] = 0;
      }
    }
    row_carry += __shfl(rs, 63, 64);
    tile_carry += __shfl(ts, 63, 64);
  }
  if (lane == 0) *p.n_tiles = tile_carry;
}

// grid (E + 1), 1024 threads. Workgroup s < E walks the (token, rank) pairs in order and appends those
// routed to expert s (each token names an expert at most once, so its rows come out in ascending token
// order); workgroup E lays out the shared expert's rows (every token, unweighted).
__global__ __launch_bounds__(1024) void scatter_kernel(PrefillPlan p, const int32_t* __restrict__ ids,
                                                       const float* __restrict__ w, int T, int k, int E,
                                                       int has_shared) {
  const int s = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int base_row = p.row0[s];
  if (s == E) {
    if (!has_shared) return;
    for (int t = tid; t < T; t += 1024) {
      p.sorted_tok[base_row + t] = t;
      p.sorted_w[base_row + t] = 1.0f;
    }
    return;
  }
  __shared__ int wave_cnt[16];
  int running = 0;
  const int n = T * k;
  for (int base = 0; base < n; base += 1024) {
    const int i = base + tid;
    const bool hit = i < n && ids[i] == s;
    const uint64_t mask = __ballot(hit);
    if (lane == 0) wave_cnt[wave] = __popcll(mask);
    __syncthreads();
    int before = running, total = 0;
    for (int v = 0; v < 16; ++v) {
      before += v < wave ? wave_cnt[v] : 0;
      total += wave_cnt[v];
    }
    if (hit) {
      const int pos = base_row + before + __popcll(mask & ((1ull << lane) - 1ull));
      p.sorted_tok[pos] = i / k;
      p.sorted_w[pos] = w[i];
      p.pair_row[i] = pos;
    }
    running += total;
    __syncthreads();
  }
}

struct GemmArgs {
  const uint8_t* const* tiles;   // [E + 1] tiled expert blobs
  PrefillPlan plan;
  int H, I, E;
  float limit;
  const uint8_t* xq;             // [T][H] E4M3 codes of the tokens
  const uint8_t* xs;             // [T][H / 32] E8M0
  uint8_t* dq;                   // [rows][I] down-input codes
  uint8_t* ds;                   // [rows][I / 32]
  uint16_t* out;                 // [rows][H] expert outputs (BF16)
};

// Down GEMM over one 128-row tile of one slot for H % 512 != 0: A = W2 tiles of 4 groups of 64 rows,
// B = the tile's rows of dq; 8 waves, each one group for 64 of the tile's token rows.
__global__ __launch_bounds__(kThreads) void down_tile_kernel(GemmArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t lds_b[2][kTileRows * kLdsRow];
  __shared__ uint32_t lds_s[2][kTileRows];
  const int ti = blockIdx.y;
  if (ti >= *a.plan.n_tiles) return;
  const int32_t* info = a.plan.tile_info + (size_t)ti * 4;
  const int slot = info[0], row0 = info[1], rows = info[2];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q = lane >> 4, n = lane & 15;
  const int C = a.I / 128;
  const int gg = blockIdx.x * 4 + (wave & 3);
  const int u0 = (wave >> 2) * kWaveTok;
  const uint8_t* blob = a.tiles[slot];
  const TiledOffsets off = tiled_offsets(a.H, a.I);
  const uint8_t* wlane = blob + off.dn_w + (size_t)gg * C * 4096 + 16 * lane;
  const uint8_t* slane = blob + off.dn_s + (size_t)gg * C * 256 + 4 * lane;

  // staging: pieces tid and tid + 512 of the tile's 128 rows x 8 x 16 bytes; rows past the tile repeat
  // its last row (results dropped)
  const uint8_t* xsrc[2];
  int ldst[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int pc = tid + kThreads * j, r = pc >> 3, part = pc & 7;
    xsrc[j] = a.dq + (size_t)(row0 + min(r, rows - 1)) * a.I + 16 * part;
    ldst[j] = r * kLdsRow + 16 * part;
  }
  const uint8_t* ssrc = a.ds + (size_t)(row0 + min(tid & (kTileRows - 1), rows - 1)) * (a.I / 32);

  // 16-token column tiles past the tile's rows hold padding: their MFMAs (and, for a wave with none left,
  // its weight loads) are skipped (a wave-uniform branch)
  const int live_tiles = min(kWaveTok, max(0, (rows - 16 * u0 + 15) / 16));
  auto load_b = [&](int c, uint4 (&bst)[2], uint32_t& sst) {
#pragma unroll
    for (int j = 0; j < 2; ++j) bst[j] = ldg128(xsrc[j] + (size_t)c * 128);
    sst = ldg32(ssrc + 4 * c);
  };
  auto store_b = [&](int stage, const uint4 (&bst)[2], uint32_t sst) {
#pragma unroll
    for (int j = 0; j < 2; ++j) *reinterpret_cast<uint4*>(&lds_b[stage][ldst[j]]) = bst[j];
    if (tid < kTileRows) lds_s[stage][tid] = sst;
  };
  auto load_a = [&](int c, uint4 (&am)[4], uint32_t& sw) {
    if (live_tiles == 0) return;
#pragma unroll
    for (int t = 0; t < 4; ++t) am[t] = ldg128(wlane + (size_t)c * 4096 + t * 1024);
    sw = ldg32(slane + (size_t)c * 256);
  };
  v4f acc[4][kWaveTok];
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int u = 0; u < kWaveTok; ++u) acc[t][u] = v4f{0.f, 0.f, 0.f, 0.f};
  auto compute = [&](int stage, const uint4 (&am)[4], uint32_t sw) {
#pragma unroll
    for (int u = 0; u < kWaveTok; ++u) {
      if (u >= live_tiles) break;
      const uint8_t* row = &lds_b[stage][(16 * (u0 + u) + n) * kLdsRow];
      const uint4 b0 = *reinterpret_cast<const uint4*>(row + 16 * q);
      const uint4 b1 = *reinterpret_cast<const uint4*>(row + 64 + 16 * q);
      const int sx = (int)((lds_s[stage][16 * (u0 + u) + n] >> (8 * q)) & 0xFF);
#pragma unroll
      for (int t = 0; t < 4; ++t) acc[t][u] = mfma_fp4_fp8(am[t], b0, b1, acc[t][u], (int)((sw >> (8 * t)) & 0xFF), sx);
    }
  };

  // Register ring of kDepth chunks: the loads of chunk c + kDepth are issued right after chunk c's MFMAs,
  // so about kDepth chunks of weights and gathered activations are in flight per wave while the
  // activations of chunk c + 1, loaded kDepth - 1 chunks earlier, move into the other LDS stage.
  uint4 a_ring[kDepth][4];
  uint32_t sw_ring[kDepth];
  uint4 b_ring[kDepth][2];
  uint32_t sx_ring[kDepth];
#pragma unroll
  for (int j = 0; j < kDepth; ++j) {
    const int c = min(j, C - 1);
    load_a(c, a_ring[j], sw_ring[j]);
    load_b(c, b_ring[j], sx_ring[j]);
  }
  store_b(0, b_ring[0], sx_ring[0]);
  __syncthreads();
  for (int base = 0; base < C; base += kDepth) {
#pragma unroll
    for (int j = 0; j < kDepth; ++j) {
      const int c = base + j;
      if (c < C) {
        compute(c & 1, a_ring[j], sw_ring[j]);
        const int jn = (j + 1) % kDepth;
        if (c + 1 < C) store_b((c + 1) & 1, b_ring[jn], sx_ring[jn]);
        if (c + kDepth < C) {
          load_a(c + kDepth, a_ring[j], sw_ring[j]);
          load_b(c + kDepth, b_ring[j], sx_ring[j]);
        }
        __syncthreads();
      }
    }
  }

#pragma unroll
  for (int u = 0; u < kWaveTok; ++u) {
    const int r = 16 * (u0 + u) + n;
    if (r >= rows) continue;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      uint2 packed;
      packed.x = mx::bf16_bits(acc[t][u][0]) | (mx::bf16_bits(acc[t][u][1]) << 16);
      packed.y = mx::bf16_bits(acc[t][u][2]) | (mx::bf16_bits(acc[t][u][3]) << 16);
      *reinterpret_cast<uint2*>(a.out + (size_t)(row0 + r) * a.H + 64 * gg + 16 * t + 4 * q) = packed;
    }
  }
}

// Grouped GEMM over one 128-row tile of one slot. kGateUp: A = W1/W3 tiles (a group = 32 intermediate rows
// of W1 and W3, 64 MFMA rows), B = the tile's gathered token rows of xq; else A = W2 tiles (a group = 64
// hidden rows), B = the tile's rows of dq. 256 threads = 4 waves, each owning kBigGroups groups for all 128
// token rows, so no weight byte is loaded twice within a workgroup; the accumulators live in the
// accumulation registers. Operand bytes per MFMA: 256 (one group per wave) or 192 (two), against 384 for
// down_tile_kernel. Grid x covers 2I / (256 kBigGroups) gate/up or H / (256 kBigGroups) down workgroups.
constexpr int kBigThreads = 256;
constexpr int kBigTok = 8;       // token tiles of 16 per wave
constexpr int kBigDepth = 2;     // chunks in flight

// kBigGroups = groups per wave: 2 where the grid divides (I % 256, H % 512), else 1 (gate/up) or
// down_tile_kernel (down).
template <bool kGateUp, int kBigGroups>
__global__ __launch_bounds__(kBigThreads) void grouped_kernel(GemmArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t lds_b[2][kTileRows * kLdsRow];
  __shared__ uint32_t lds_s[2][kTileRows];
  const int ti = blockIdx.y;
  if (ti >= *a.plan.n_tiles) return;
  const int32_t* info = a.plan.tile_info + (size_t)ti * 4;
  const int slot = info[0], row0 = info[1], rows = info[2];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q = lane >> 4, n = lane & 15;
  const int K = kGateUp ? a.H : a.I;
  const int C = K / 128;
  const int g0 = blockIdx.x * (4 * kBigGroups) + kBigGroups * wave;
  const uint8_t* blob = a.tiles[slot];
  const TiledOffsets off = tiled_offsets(a.H, a.I);
  const uint8_t* wbase = blob + (kGateUp ? 0 : off.dn_w) + 16 * lane;
  const uint8_t* sbase = blob + (kGateUp ? off.gu_s : off.dn_s) + 4 * lane;
  const int live_tiles = min(kBigTok, (rows + 15) / 16);

  // staging: pieces tid + 256 j (j < 4) of the tile's 128 rows x 8 x 16 bytes
  const uint8_t* xsrc[4];
  int ldst[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int pc = tid + kBigThreads * j, r = pc >> 3, part = pc & 7;
    const int row = row0 + min(r, rows - 1);
    const uint8_t* src = kGateUp ? a.xq + (size_t)a.plan.sorted_tok[row] * a.H : a.dq + (size_t)row * a.I;
    xsrc[j] = src + 16 * part;
    ldst[j] = r * kLdsRow + 16 * part;
  }
  const int srow = row0 + min(tid & (kTileRows - 1), rows - 1);
  const uint8_t* ssrc = kGateUp ? a.xs + (size_t)a.plan.sorted_tok[srow] * (a.H / 32)
                                : a.ds + (size_t)srow * (a.I / 32);
  auto load_b = [&](int c, uint4 (&bst)[4], uint32_t& sst) {
#pragma unroll
    for (int j = 0; j < 4; ++j) bst[j] = ldg128(xsrc[j] + (size_t)c * 128);
    sst = ldg32(ssrc + 4 * c);
  };
  auto store_b = [&](int stage, const uint4 (&bst)[4], uint32_t sst) {
#pragma unroll
    for (int j = 0; j < 4; ++j) *reinterpret_cast<uint4*>(&lds_b[stage][ldst[j]]) = bst[j];
    if (tid < kTileRows) lds_s[stage][tid] = sst;
  };
  auto load_a = [&](int c, uint4 (&am)[kBigGroups][4], uint32_t (&sw)[kBigGroups]) {
#pragma unroll
    for (int gi = 0; gi < kBigGroups; ++gi) {
      const size_t gb = (size_t)(g0 + gi) * C + c;
#pragma unroll
      for (int t = 0; t < 4; ++t) am[gi][t] = ldg128(wbase + gb * 4096 + t * 1024);
      sw[gi] = ldg32(sbase + gb * 256);
    }
  };
  v4f acc[kBigGroups][4][kBigTok];
#pragma unroll
  for (int gi = 0; gi < kBigGroups; ++gi)
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int u = 0; u < kBigTok; ++u) acc[gi][t][u] = v4f{0.f, 0.f, 0.f, 0.f};
  auto compute = [&](int stage, const uint4 (&am)[kBigGroups][4], const uint32_t (&sw)[kBigGroups]) {
#pragma unroll
    for (int u = 0; u < kBigTok; ++u) {
      if (u >= live_tiles) break;
      const uint8_t* row = &lds_b[stage][(16 * u + n) * kLdsRow];
      const uint4 b0 = *reinterpret_cast<const uint4*>(row + 16 * q);
      const uint4 b1 = *reinterpret_cast<const uint4*>(row + 64 + 16 * q);
      const int sx = (int)((lds_s[stage][16 * u + n] >> (8 * q)) & 0xFF);
#pragma unroll
      for (int gi = 0; gi < kBigGroups; ++gi)
#pragma unroll
        for (int t = 0; t < 4; ++t)
          acc[gi][t][u] = mfma_fp4_fp8(am[gi][t], b0, b1, acc[gi][t][u], (int)((sw[gi] >> (8 * t)) & 0xFF), sx);
    }
  };
  uint4 a_ring[kBigDepth][kBigGroups][4];
  uint32_t sw_ring[kBigDepth][kBigGroups];
  uint4 b_ring[kBigDepth][4];
  uint32_t sx_ring[kBigDepth];
#pragma unroll
  for (int j = 0; j < kBigDepth; ++j) {
    const int c = min(j, C - 1);
    load_a(c, a_ring[j], sw_ring[j]);
    load_b(c, b_ring[j], sx_ring[j]);
  }
  store_b(0, b_ring[0], sx_ring[0]);
  __syncthreads();
  for (int base = 0; base < C; base += kBigDepth) {
#pragma unroll
    for (int j = 0; j < kBigDepth; ++j) {
      const int c = base + j;
      if (c < C) {
        compute(c & 1, a_ring[j], sw_ring[j]);
        const int jn = (j + 1) % kBigDepth;
        if (c + 1 < C) store_b((c + 1) & 1, b_ring[jn], sx_ring[jn]);
        if (c + kBigDepth < C) {
          load_a(c + kBigDepth, a_ring[j], sw_ring[j]);
          load_b(c + kBigDepth, b_ring[j], sx_ring[j]);
        }
        __syncthreads();
      }
    }
  }

  if constexpr (kGateUp) {
    const bool weighted = slot < a.E;
    // The SwiGLU body is too large to unroll eight times, and a rolled loop may not index the accumulator
    // array by its counter (that would move the array to scratch memory): each pass copies token tile u
    // out of the array with constant indices and selects (uniform branch-free selects).
#pragma unroll 1
    for (int u = 0; u < live_tiles; ++u) {
      const int r = 16 * u + n;
      const bool live = r < rows;
      const int row = row0 + (live ? r : 0);
      const float rw = a.plan.sorted_w[row];
#pragma unroll
      for (int gi = 0; gi < kBigGroups; ++gi) {
        const int gg = g0 + gi;
        v4f cur[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          cur[t] = acc[gi][t][0];
#pragma unroll
          for (int uu = 1; uu < kBigTok; ++uu) cur[t] = uu == u ? acc[gi][t][uu] : cur[t];
        }
        float din[4][4];
        float amax = 0.f;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float up = __shfl_xor(cur[t][i], 32, 64);
            din[t][i] = mxd::swiglu_element(mx::bf16_bits(cur[t][i]), mx::bf16_bits(up), a.limit, weighted, rw,
                                            nullptr);
            amax = fmaxf(amax, fabsf(din[t][i]));
          }
        }
        amax = fmaxf(amax, __shfl_xor(amax, 16, 64));
        amax = fmaxf(amax, mx::u2f(mx::kAmaxFloorBits));
        const uint32_t code = mx::act_scale_code(amax);
        const float sc = mx::e8m0_value(code);
        if (q < 2 && live) {
          uint8_t* dst = a.dq + (size_t)row * a.I + 32 * gg + 4 * q;
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            uint32_t word = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) word |= mx::act_quant_value(din[t][i], sc) << (8 * i);
            *reinterpret_cast<uint32_t*>(dst + 8 * t) = word;
          }
          if (q == 0) a.ds[(size_t)row * (a.I / 32) + gg] = (uint8_t)code;
        }
      }
    }
  } else {
#pragma unroll
    for (int u = 0; u < kBigTok; ++u) {
      const int r = 16 * u + n;
      if (r >= rows) continue;
#pragma unroll
      for (int gi = 0; gi < kBigGroups; ++gi)
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          uint2 packed;
          packed.x = mx::bf16_bits(acc[gi][t][u][0]) | (mx::bf16_bits(acc[gi][t][u][1]) << 16);
          packed.y = mx::bf16_bits(acc[gi][t][u][2]) | (mx::bf16_bits(acc[gi][t][u][3]) << 16);
          *reinterpret_cast<uint2*>(a.out + (size_t)(row0 + r) * a.H + 64 * (g0 + gi) + 16 * t + 4 * q) = packed;
        }
    }
  }
}

// grid (T), 256 threads: one workgroup per token; thread 0 orders the token's rows by expert ID in LDS,
// then every thread sums 8 hidden positions per step over the rows (shared row last).
__global__ __launch_bounds__(256) void prefill_combine_kernel(PrefillPlan p, const int32_t* __restrict__ ids,
                                                              const uint16_t* __restrict__ rows, int T, int H, int k,
                                                              int E, int has_shared, uint16_t* __restrict__ y) {
  __shared__ int32_t order[kMaxTopK + 1];
  __shared__ int order_n;
  const int t = blockIdx.x;
  if (threadIdx.x == 0) {
    int32_t es[kMaxTopK], rs[kMaxTopK];
    int m = 0;
    for (int i = 0; i < k; ++i) {
      const int e = ids[t * k + i];
      if (e < 0 || e >= E) continue;
      const int r = p.pair_row[t * k + i];
      int j = m - 1;
      while (j >= 0 && es[j] > e) {
        es[j + 1] = es[j];
        rs[j + 1] = rs[j];
        --j;
      }
      es[j + 1] = e;
      rs[j + 1] = r;
      ++m;
    }
    for (int i = 0; i < m; ++i) order[i] = rs[i];
    if (has_shared) order[m++] = T * k + t;   // the shared expert's rows follow the routed ones
    order_n = m;
  }
  __syncthreads();
  const int n = order_n;
  for (int h = threadIdx.x * 8; h < H; h += 256 * 8) {
    float acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = 0.f;
    for (int i = 0; i < n; ++i) {
      const uint4 v = *reinterpret_cast<const uint4*>(rows + (size_t)order[i] * H + h);
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc[2 * j] = acc[2 * j] + mx::bf16_value(w[j] & 0xFFFFu);
        acc[2 * j + 1] = acc[2 * j + 1] + mx::bf16_value(w[j] >> 16);
      }
    }
    uint4 o;
    o.x = mx::bf16_bits(acc[0]) | (mx::bf16_bits(acc[1]) << 16);
    o.y = mx::bf16_bits(acc[2]) | (mx::bf16_bits(acc[3]) << 16);
    o.z = mx::bf16_bits(acc[4]) | (mx::bf16_bits(acc[5]) << 16);
    o.w = mx::bf16_bits(acc[6]) | (mx::bf16_bits(acc[7]) << 16);
    *reinterpret_cast<uint4*>(y + (size_t)t * H + h) = o;
  }
}

uint64_t r256(uint64_t b) { return (b + 255) & ~255ull; }

// Workspace layout (each piece 256-byte aligned).
struct Workspace {
  uint64_t logits, scores, selection, ids, w, xq, xs, counts, row0, tile_info, n_tiles, sorted_tok, sorted_w,
      pair_row, dq, ds, eout, total;
  int max_tiles, rows;
};

Workspace workspace_layout(const mx_moe_config& c, int T, int has_shared) {
  Workspace w{};
  const uint64_t E = c.experts, k = c.top_k, H = c.hidden, I = c.intermediate;
  const uint64_t pairs = (uint64_t)T * k;
  w.rows = (int)(pairs + (has_shared ? T : 0));
  w.max_tiles = (int)((pairs + kTileRows - 1) / kTileRows + E + (has_shared ? (T + kTileRows - 1) / kTileRows : 0));
  uint64_t o = 0;
  auto take = [&](uint64_t bytes) {
    const uint64_t at = o;
    o += r256(bytes);
    return at;
  };
  w.logits = take((uint64_t)T * E * 4);
  w.scores = take((uint64_t)T * E * 4);
  w.selection = take((uint64_t)T * E * 4);
  w.ids = take(pairs * 4);
  w.w = take(pairs * 4);
  w.xq = take((uint64_t)T * H);
  w.xs = take((uint64_t)T * H / 32);
  w.counts = take((E + 1) * 4);
  w.row0 = take((E + 1) * 4);
  w.tile_info = take((uint64_t)w.max_tiles * 16);
  w.n_tiles = take(4);
  w.sorted_tok = take((uint64_t)w.rows * 4);
  w.sorted_w = take((uint64_t)w.rows * 4);
  w.pair_row = take(pairs * 4);
  w.dq = take((uint64_t)w.rows * I);
  w.ds = take((uint64_t)w.rows * I / 32);
  w.eout = take((uint64_t)w.rows * H * 2);
  w.total = o;
  return w;
}

}  // namespace

using namespace mxi;

extern "C" {

uint64_t mx_prefill_workspace_bytes(mx_layer* layer, int32_t T) {
  const LayerView v = layer_view(layer);
  if (!v.ctx || T <= 0) return 0;
  return workspace_layout(v.cfg, T, v.has_shared).total;
}

int mx_moe_prefill(mx_layer* layer, const uint16_t* x, int32_t T, const int32_t* ids, const float* weights,
                   uint16_t* y, void* workspace, uint64_t workspace_bytes, void* stream) {
  const LayerView v = layer_view(layer);
  MX_REQUIRE(v.ctx != nullptr, "layer is closed");
  if (int s = use(v.ctx)) return s;
  const mx_moe_config& c = v.cfg;
  MX_REQUIRE(T >= 0 && T <= (1 << 20), "token count %d outside [0, 2^20]", T);
  if (!T) return MX_OK;
  MX_REQUIRE(x && y && ((uintptr_t)x & 15) == 0 && ((uintptr_t)y & 15) == 0,
             "x and y must be 16-byte aligned device pointers");
  MX_REQUIRE((ids == nullptr) == (weights == nullptr), "routing ids and weights are given together or not at all");
  MX_REQUIRE(c.intermediate % 128 == 0 && c.hidden % 256 == 0, "prefill needs I % 128 == 0 and H % 256 == 0");
  const Workspace ws = workspace_layout(c, T, v.has_shared);
  MX_REQUIRE(workspace && ((uintptr_t)workspace & 255) == 0 && workspace_bytes >= ws.total,
             "workspace must be 256-byte aligned and at least mx_prefill_workspace_bytes (%llu) bytes",
             (unsigned long long)ws.total);
  hipStream_t st = as_stream(stream);
  uint8_t* b = (uint8_t*)workspace;
  const int E = c.experts, k = c.top_k, H = c.hidden, I = c.intermediate;
  const int32_t* rid = ids;
  const float* rw = weights;
  if (!ids) {
    mx_router_out out{};
    out.logits = (float*)(b + ws.logits);
    out.scores = (float*)(b + ws.scores);
    out.selection = (float*)(b + ws.selection);
    out.indices = (int32_t*)(b + ws.ids);
    out.weights = (float*)(b + ws.w);
    if (int s = mx_router(v.ctx, v.router_weight, v.bias, x, T, H, E, k, c.score_func, c.route_scale, &out, stream))
      return s;
    rid = out.indices;
    rw = out.weights;
  }
  if (int s = mx_act_quant32(v.ctx, x, b + ws.xq, b + ws.xs, T, H, stream)) return s;
  PrefillPlan p{};
  p.counts = (int32_t*)(b + ws.counts);
  p.row0 = (int32_t*)(b + ws.row0);
  p.tile_info = (int32_t*)(b + ws.tile_info);
  p.n_tiles = (int32_t*)(b + ws.n_tiles);
  p.sorted_tok = (int32_t*)(b + ws.sorted_tok);
  p.sorted_w = (float*)(b + ws.sorted_w);
  p.pair_row = (int32_t*)(b + ws.pair_row);
  hipLaunchKernelGGL(zero_i32_kernel, dim3((E + 1 + 255) / 256), dim3(256), 0, st, p.counts, E + 1);
  MX_LAUNCH_CHECK("zero_i32_kernel");
  const int pairs = T * k;
  hipLaunchKernelGGL(count_kernel, dim3(std::min(64, (pairs + 255) / 256)), dim3(256), 0, st, rid, pairs, E, p.counts);
  MX_LAUNCH_CHECK("count_kernel");
  hipLaunchKernelGGL(offsets_kernel, dim3(1), dim3(64), 0, st, p, E, T, v.has_shared);
  MX_LAUNCH_CHECK("offsets_kernel");
  hipLaunchKernelGGL(scatter_kernel, dim3(E + 1), dim3(1024), 0, st, p, rid, rw, T, k, E, v.has_shared);
  MX_LAUNCH_CHECK("scatter_kernel");
  GemmArgs a{};
  a.tiles = v.tiles;
  a.plan = p;
  a.H = H;
  a.I = I;
  a.E = E;
  a.limit = c.swiglu_limit;
  a.xq = b + ws.xq;
  a.xs = b + ws.xs;
  a.dq = b + ws.dq;
  a.ds = b + ws.ds;
  a.out = (uint16_t*)(b + ws.eout);
  if (I % 256 == 0)
    hipLaunchKernelGGL((grouped_kernel<true, 2>), dim3(I / 256, ws.max_tiles), dim3(kBigThreads), 0, st, a);
  else
    hipLaunchKernelGGL((grouped_kernel<true, 1>), dim3(I / 128, ws.max_tiles), dim3(kBigThreads), 0, st, a);
  MX_LAUNCH_CHECK("grouped_kernel<gate/up>");
  if (H % 512 == 0)
    hipLaunchKernelGGL((grouped_kernel<false, 2>), dim3(H / 512, ws.max_tiles), dim3(kBigThreads), 0, st, a);
  else
    hipLaunchKernelGGL(down_tile_kernel, dim3(H / 256, ws.max_tiles), dim3(kThreads), 0, st, a);
  MX_LAUNCH_CHECK("grouped_kernel<down>");
  hipLaunchKernelGGL(prefill_combine_kernel, dim3(T), dim3(256), 0, st, p, rid,
                     (const uint16_t*)a.out, T, H, k, E, v.has_shared, y);
  MX_LAUNCH_CHECK("prefill_combine_kernel");
  return MX_OK;
}

}  // extern "C"
