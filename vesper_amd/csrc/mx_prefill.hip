// MoE prefill on gfx950: many tokens through a decode layer's experts as token-sorted grouped GEMMs on
// the scaled MXFP4 MFMA. Per token the arithmetic is the decode path's
// (ConnectedMoE.forward, src/vesper/connected.py:125-186: per-32 activation quantization, W1/W3,
// SwiGLU with the route weight before W2, down-input quantization, W2, ordered combine with the
// shared expert last); only the summation order inside the products differs.
//
//   plan      count pairs per expert, expert-major row offsets (shared expert last) and 128-row tiles;
//             a stable per-expert scatter gives each expert's rows in ascending token order
//             (participation, src/vesper/moe.py:18-30) and each (token, rank) pair its row
//   gate/up   grid (ceil(I/256), tiles), 8 waves: 8 groups of 32 intermediate rows (W1 + W3 interleaved
//             per MFMA tile, as in the tiled layout), each wave one group for all 128 tokens of the tile in
//             the block spec's exact order (one BF16 MFMA per 32-block, in-order FP32 additions), every wave
//             copying its share of each 128-wide K chunk -- weights and the tokens' exact BF16 activation
//             rows -- global -> LDS; epilogue SwiGLU + route weight + the per-token quantization of each
//             32-row block of the down input
//   down      grid (ceil(H/512), tiles), 8 multiplying waves over 64-row groups of W2 (scaled MXFP4 x E4M3
//             MFMA) with the tile's contiguous down-input rows, 4 copy waves bringing each chunk to LDS
//   combine   per token: its expert rows in ascending expert ID, then the shared row; FP32 from +0,
//             one BF16 rounding (aggregation_probe.cu:4-25). The down GEMM writes each row to the
//             token's contiguous [k + 1][H] block in that order, so the combine streams it.
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
constexpr int kMaxTopK = 32;

struct PrefillPlan {
  int32_t* counts;      // [E + 1] pairs per slot (slot E = shared expert)
  int32_t* row0;        // [E + 1] first row of each slot
  int32_t* tile_info;   // [max_tiles][4]: slot, first row, rows, unused
  int32_t* n_tiles;     // [1]
  int32_t* sorted_tok;  // [rows] token of each row
  float* sorted_w;      // [rows] route weight of each row
  int32_t* pair_row;    // [T * k] row of pair (t, rank)
  int32_t* row_dest;    // [rows] where the combine reads the row: t (k + 1) + j, j = the row's place in
                        // the token's ascending-expert order (the shared expert's row: j = k)
};

__global__ void zero_i32_kernel(int32_t* p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

// Given routing is first copied into the workspace with each token's list made valid (the decode path's
// rule, mxd::repair_token_routes) and the replacements counted in the layer's routing error word; the
// plan steps below additionally skip ids outside [0, E), so no input can take an access out of bounds.
__global__ __launch_bounds__(256) void repair_routes_kernel(const int32_t* __restrict__ ids, const float* __restrict__ w,
                                                            int T, int k, int E, int32_t* __restrict__ out_ids,
                                                            float* __restrict__ out_w, uint32_t* errors) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= T) return;
  int32_t row[kMaxTopK];
  float wr[kMaxTopK];
  for (int i = 0; i < k; ++i) {
    row[i] = ids[(size_t)t * k + i];
    wr[i] = w[(size_t)t * k + i];
  }
  const int replaced = mxd::repair_token_routes(row, wr, k, E);
  if (replaced) atomicAdd(errors, (uint32_t)replaced);
  for (int i = 0; i < k; ++i) {
    out_ids[(size_t)t * k + i] = row[i];
    out_w[(size_t)t * k + i] = wr[i];
  }
}

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
      p.row_dest[base_row + t] = t * (k + 1) + k;
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

// One thread per (token, rank) pair with a valid expert: the row's place in the combine's token-major
// layout, t (k + 1) + j with j = its position among the token's valid pairs ordered by (expert, rank).
__global__ __launch_bounds__(256) void dest_kernel(PrefillPlan p, const int32_t* __restrict__ ids, int T, int k,
                                                   int E) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= T * k) return;
  const int e = ids[i];
  if (e < 0 || e >= E) return;
  const int t = i / k, rank = i - t * k;
  const int32_t* tok_ids = ids + (size_t)t * k;
  int j = 0;
#pragma unroll 8
  for (int r = 0; r < k; ++r) {
    const int f = tok_ids[r];
    j += f >= 0 && f < E && (f < e || (f == e && r < rank));
  }
  p.row_dest[p.pair_row[i]] = t * (k + 1) + j;
}

struct GemmArgs {
  const uint8_t* const* tiles;   // [E + 1] tiled expert blobs
  PrefillPlan plan;
  int H, I, E;
  float limit;
  const float* silu;             // [mxd::kSiluEntries] the layer's SiLU table
  const uint8_t* xq;             // [T][H] E4M3 codes of the tokens
  const uint8_t* xs;             // [T][H / 32] E8M0
  const uint16_t* xd;            // [T][H] each code times its block scale, BF16 (exact)
  uint8_t* dq;                   // [rows][I] down-input codes
  uint8_t* ds;                   // [rows][I / 32]
  uint16_t* out;                 // [T][k + 1][H] expert outputs (BF16), token-major (plan.row_dest)
};

using mxd::copy_barrier;
using mxd::global_to_lds16;
using mxd::global_to_lds4;
using mxd::lds_addr;
using mxd::vm_wait_imm;

// One 16-token tile's MFMA B operand (two 16-byte reads 1 KB apart) and its scale byte (saddr: this lane's
// byte of the tile's scale words), read from LDS and waited for. Inline assembly: for compiler-visible LDS
// reads the compiler cannot tell which global->LDS copies they depend on and waits for all of them.
__device__ __forceinline__ void lds_read_b1(uint32_t addr, uint32_t saddr, uint4 (&b)[2], uint32_t& sw) {
  mxd::u32x4_t x0, x1;
  uint32_t s0;
  asm volatile(
      "ds_read_b128 %0, %3\n\t"
      "ds_read_b128 %1, %3 offset:1024\n\t"
      "ds_read_u8 %2, %4\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(x0), "=&v"(x1), "=&v"(s0)
      : "v"(addr), "v"(saddr));
  b[0] = uint4{x0.x, x0.y, x0.z, x0.w};
  b[1] = uint4{x1.x, x1.y, x1.z, x1.w};
  sw = s0;
}

constexpr int kGThreads = 768;   // 8 multiplying waves (two per SIMD, one 64-row group each) + 4 copy waves
constexpr int kStages = 3;       // operand chunks in LDS: chunk c + 2 is copied in while chunk c multiplies
constexpr int kCopies = 15;      // per copy wave and chunk: 8 weight pieces, 2 weight-scale, 4 activation,
                                 // 1 activation-scale copies
// a stage: the 8 groups' weight tiles (group w, tile t at 1 KB x (4 w + t)), their scale words (256 B per
// group), the 16 activation blocks of 1 KB, then the 128 rows' activation scale words
constexpr int kStageA = 0, kStageAS = 32768, kStageB = 34816, kStageBS = 51200, kStageBytes = 51712;
// epilogue tiles in the same LDS: gate and up [128][kEpiRowG] BF16, or the down output [128][kEpiRowD]
constexpr int kEpiRowG = 256 + 8, kEpiRowD = 512 + 8;
constexpr int kLdsBytes = kStages * kStageBytes;
static_assert(kLdsBytes <= 160 * 1024 && 2 * kTileRows * kEpiRowG * 2 <= kLdsBytes && kTileRows * kEpiRowD * 2 <= kLdsBytes,
              "LDS layout");

// The down GEMM over one 128-row tile of one slot: A = W2 tiles (a group = 64 hidden rows), B = the tile's
// rows of dq. Grid x covers the groups eight per workgroup (ceil(H / 512)), grid y the tiles.
//
// Waves 0-7 multiply: each keeps its 64 x 128 output block in 128 accumulator registers. Waves 8-11 only
// copy every operand of a 128-wide K chunk global -> LDS without registers (global_load_lds, 16 bytes a
// lane) into a 3-stage ring: the weight tiles as stored in the tiled layout (1 KB of MFMA operand per
// lane-ordered piece), their scale words, and the activations as 16 blocks of 1 KB, block 2u + h holding
// at lane (q, n) the bytes 64h + 16q.. of row 16u + n, which is exactly the MFMA B operand of lane (q, n)
// for token tile u, so every LDS read is one linear 1 KB wave access. A wave that issues copies stalls
// while its copies are on their way from HBM; in waves of their own those stalls hold up no MFMA, since
// each SIMD issues from whichever of its waves is ready. A step: the multiplying waves read chunk c from
// its stage and multiply; the copy waves issue chunk c + 2 into the stage chunk c - 1 left and wait for
// chunk c + 1; one barrier ends the step.
//
// Epilogue: the accumulators go to LDS as BF16 [token][column] and every thread then copies 16-byte row
// segments of the down output to the token-major output rows (plan.row_dest).
__global__ __launch_bounds__(kGThreads) void grouped_down_kernel(GemmArgs a) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[kLdsBytes];
  const int ti = blockIdx.y;
  if (ti >= *a.plan.n_tiles) return;
  const int32_t* info = a.plan.tile_info + (size_t)ti * 4;
  const int slot = info[0], row0 = info[1], rows = info[2];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q = lane >> 4, n = lane & 15;
  const int K = a.I;
  const int C = K / 128;
  // a multiplying wave past the last group (H / 64 groups) computes and stores nothing
  const int groups = a.H / 64;
  const int g = blockIdx.x * 8 + wave;
  const bool active = wave < 8 && g < groups;
  const uint8_t* blob = a.tiles[slot];
  const TiledOffsets off = tiled_offsets(a.H, a.I);
  const int live_tiles = min(8, (rows + 15) / 16);
  const uint32_t lds0 = lds_addr(lds);
  v4f acc[4][8];
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int u = 0; u < 8; ++u) acc[t][u] = v4f{0.f, 0.f, 0.f, 0.f};

  if (wave >= 8) {
    // copy wave p: groups 2p and 2p + 1 (weight tiles and scale words), activation tiles 2p and 2p + 1
    // (both blocks of each) and the scale words of rows 32p .. 32p + 31. Rows past the tile repeat its last
    // row; groups past the last repeat it. The activation offsets fit 32 bits (the host bounds the buffers).
    const int pw = wave - 8;
    const uint8_t* wsrc[2];
    const uint8_t* ssrc[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int gi = min((int)blockIdx.x * 8 + 2 * pw + i, groups - 1);
      wsrc[i] = blob + off.dn_w + (size_t)gi * C * 4096 + 16 * lane;
      ssrc[i] = blob + off.dn_s + (size_t)gi * C * 256 + 4 * lane;
    }
    const uint8_t* bbase = a.dq;
    const uint8_t* sbbase = a.ds;
    uint32_t boff[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int br = row0 + min(16 * (2 * pw + i) + n, rows - 1);
      boff[i] = (uint32_t)br * (uint32_t)a.I + 16 * q;
    }
    const int sr = row0 + min(32 * pw + (lane & 31), rows - 1);
    const uint32_t soff = (uint32_t)sr * (uint32_t)(a.I / 32);
    auto copy = [&](int c) {
      const uint32_t st = lds0 + (uint32_t)(c % kStages) * kStageBytes;
#pragma unroll
      for (int i = 0; i < 8; ++i)
        global_to_lds16(wsrc[i >> 2] + (size_t)c * 4096 + (i & 3) * 1024,
                        __builtin_amdgcn_readfirstlane(st + kStageA + (8 * pw + i) * 1024));
#pragma unroll
      for (int i = 0; i < 2; ++i)
        global_to_lds4(ssrc[i] + (size_t)c * 256, __builtin_amdgcn_readfirstlane(st + kStageAS + 256 * (2 * pw + i)));
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int h = 0; h < 2; ++h)
          global_to_lds16(bbase + (size_t)c * 128 + boff[i] + 64 * h,
                          __builtin_amdgcn_readfirstlane(st + kStageB + (4 * pw + 2 * i + h) * 1024));
      if (lane < 32) global_to_lds4(sbbase + (size_t)c * 4 + soff, __builtin_amdgcn_readfirstlane(st + kStageBS + 128 * pw));
    };
    copy(0);
    if (C > 1) {
      copy(1);
      __builtin_amdgcn_s_waitcnt(vm_wait_imm(kCopies));
    } else {
      __builtin_amdgcn_s_waitcnt(vm_wait_imm(0));
    }
    copy_barrier();
    for (int c = 0; c < C; ++c) {
      if (c + 2 < C) {
        copy(c + 2);
        __builtin_amdgcn_s_waitcnt(vm_wait_imm(kCopies));   // chunk c + 1 has landed
      } else {
        __builtin_amdgcn_s_waitcnt(vm_wait_imm(0));
      }
      copy_barrier();
    }
  } else {
    const uint32_t la = lds0 + kStageA + 1024 * 4 * wave + 16 * lane;
    const uint32_t las = lds0 + kStageAS + 256 * wave + 4 * lane;
    const uint32_t lb = lds0 + kStageB + 16 * lane;
    const uint32_t lsb = lds0 + kStageBS + 4 * n + q;   // byte q (K block q) of token n's scale word
    copy_barrier();
    for (int c = 0; c < C; ++c) {
      const uint32_t so = (c % kStages) * kStageBytes;
      if (active) {
        uint4 am[4];
#pragma unroll
        for (int t = 0; t < 4; ++t)
          am[t] = *reinterpret_cast<const uint4*>(lds + (la - lds0) + so + 1024 * t);
        const uint32_t sw = *reinterpret_cast<const uint32_t*>(lds + (las - lds0) + so);
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          if (u >= live_tiles) break;   // wave-uniform
          uint4 b[2];
          uint32_t sx;
          lds_read_b1(lb + so + 2 * u * 1024, lsb + so + 64 * u, b, sx);
          acc[0][u] = mxd::mfma_fp4_fp8_sel<0>(am[0], b[0], b[1], acc[0][u], sw, (int)sx);
          acc[1][u] = mxd::mfma_fp4_fp8_sel<1>(am[1], b[0], b[1], acc[1][u], sw, (int)sx);
          acc[2][u] = mxd::mfma_fp4_fp8_sel<2>(am[2], b[0], b[1], acc[2][u], sw, (int)sx);
          acc[3][u] = mxd::mfma_fp4_fp8_sel<3>(am[3], b[0], b[1], acc[3][u], sw, (int)sx);
          // pins this tile's MFMAs before the next tile's reads: the compiler would otherwise sink every MFMA
          // past the last read and keep all eight tiles' operands live at once
          asm volatile("" : "+v"(acc[0][u]), "+v"(acc[1][u]), "+v"(acc[2][u]), "+v"(acc[3][u]));
        }
      }
      __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): this wave's reads of chunk c are done
      copy_barrier();
    }
  }
  __syncthreads();

  // D[4q + i][n] of tile t: W2 rows 64g + 16t + 4q + i
  uint16_t* eo = reinterpret_cast<uint16_t*>(lds);
  if (active) {
    uint16_t* dst = eo + n * kEpiRowD + 64 * wave + 4 * q;
#pragma unroll
    for (int u = 0; u < 8; ++u)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        uint2 packed;
        packed.x = mx::bf16_bits(acc[t][u][0]) | (mx::bf16_bits(acc[t][u][1]) << 16);
        packed.y = mx::bf16_bits(acc[t][u][2]) | (mx::bf16_bits(acc[t][u][3]) << 16);
        *reinterpret_cast<uint2*>(dst + 16 * u * kEpiRowD + 16 * t) = packed;
      }
  }
  __syncthreads();
  // thread tid copies segment tid % 64 of rows tid / 64 + 8 i (i < 16); their destinations are loaded
  // together first
  const int cols = min(512, a.H - 512 * (int)blockIdx.x);
  const int seg = tid & 63, tok0 = tid >> 6;   // the multiplying waves' 512 threads
  int dest[kTileRows / 8];
#pragma unroll
  for (int i = 0; i < kTileRows / 8; ++i) dest[i] = a.plan.row_dest[row0 + min(tok0 + 8 * i, rows - 1)];
  if (tid < 512 && 8 * seg < cols) {
#pragma unroll
    for (int i = 0; i < kTileRows / 8; ++i) {
      const int tok = tok0 + 8 * i;
      if (tok < rows)
        *reinterpret_cast<uint4*>(a.out + (size_t)dest[i] * a.H + 512 * blockIdx.x + 8 * seg) =
            *reinterpret_cast<const uint4*>(eo + tok * kEpiRowD + 8 * seg);
    }
  }
}

// ---------------------------------------------------------------------------------------------------------
// Exact gate/up: W1 and W3 of the tile's tokens as the block spec defines them (E4M3 x MXFP4 per 32-block,
// src/vesper/formats.py:97-118 and src/vesper/kernels/format_probe.cu:90-118): every block dot is the exact
// 32-product sum of the scaled values rounded once to FP32, and the blocks are added to the FP32 result one
// at a time in ascending K order. The scaled FP4 x FP8 MFMA does not round its block sums exactly on gfx950
// (its adder drops low product bits), so each block runs on V_MFMA_F32_16X16X32_BF16 with a zero
// accumulator -- which returns the exact 32-product dot rounded once -- over operands converted exactly:
// weights by V_CVT_SCALEF32_PK_BF16_FP4 with the block's E8M0 scale as the scale operand (an E2M1 value
// times a power of two has at most two significant bits), activations as the quantizer's BF16 copy of each
// code times its block scale (four significant bits). The in-order chain acc = acc + d runs on the VALU:
// with a non-zero accumulator the MFMA does not round acc + dot as IEEE addition does.
//
// grid (ceil(I / 256), tiles), 512 threads: 8 waves, wave w one group of 32 intermediate rows (4 MFMA
// tiles, W1 rows 8t + 0..7 and the same W3 rows in tile t) for all 128 rows of the tile, 128 accumulator
// registers. Every wave copies its share of chunk c + 1's operands global -> LDS (global_load_lds, nine
// instructions: its group's four weight pieces and scale words, and token tile w's four BF16 activation
// blocks) into a 2-stage ring; a step waits for this wave's copies of chunk c, meets the barrier and
// multiplies chunk c, issuing chunk c + 1's copies a block at a time between its blocks. (Half-chunk steps
// through a 4-stage ring, which copy three steps ahead, and FP8 activations through a 3-stage ring,
// converted per wave, both measured slower: per-step costs -- the barrier, the first LDS reads, the last
// additions -- and the conversions outweigh the deeper prefetch.) Operands come from LDS with the bf16
// MFMA's lane map (A lane (m, q) = row m, K 8q..8q+7 of a block: word q of lane (m, b)'s 16 bytes in the
// tiled layout; B lane (n, q) = token n, the same K: the copy puts them at lane slot 16 q + n of the (token
// tile, block) KB). The reads are plain LDS loads: the copies are inline assembly, which the compiler does
// not see writing LDS, so it places no wait for them before a read -- the wave's own vmcnt wait and the
// barrier at the top of each step order them.
constexpr int kXThreads = 512;
constexpr int kXStages = 2;
// a stage: the 8 groups' weight tiles (group w, tile t at 1 KB x (4 w + t)), their scale words (256 B per
// group), then the activations: token tile u, block b at 1 KB x (4 u + b)
constexpr int kXStageA = 0, kXStageAS = 32768, kXStageB = 34816, kXStageBytes = 67584;
static_assert(kXStages * kXStageBytes <= 160 * 1024 && 2 * kTileRows * kEpiRowG * 2 <= kXStages * kXStageBytes,
              "exact gate/up LDS layout");

typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

// byte `kByte` of `word` shifted to an FP32 exponent field: the E8M0 code as the power of two it encodes
// (one SDWA instruction)
template <int kByte>
__device__ __forceinline__ float e8m0_scale(uint32_t word, uint32_t twenty_three) {
  uint32_t r;
  asm("v_lshlrev_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_%3"
      : "=v"(r) : "v"(twenty_three), "v"(word), "n"(kByte));
  return __uint_as_float(r);
}

// 8 E2M1 values (one 32-bit word) times the power of two `scale`, exact in BF16
__device__ __forceinline__ v8bf fp4_word_scaled(uint32_t word, float scale) {
  const v2bf p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, scale, 0);
  const v2bf p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, scale, 1);
  const v2bf p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, scale, 2);
  const v2bf p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, scale, 3);
  return v8bf{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
}

typedef __attribute__((address_space(3))) const uint32_t* lds_u32_ptr;
typedef __attribute__((address_space(3))) const mxd::u32x4_t* lds_u32x4_ptr;

// this lane's weight words of a chunk (word [t][b]: tile t, block b, at a_addr + 1 KB t + 256 B b) and its
// rows' scale words per block (at s_addr + 64 B b). Plain LDS loads: the compiler waits for each word just
// before its first use, so the conversions of block 0 start while the later words are still in flight
// (one wait for all twenty reads measured 0.8 % slower per prefill).
__device__ __forceinline__ void lds_read_weights(uint32_t a_addr, uint32_t s_addr, uint32_t (&w)[4][4],
                                                 uint32_t (&sw)[4]) {
  const lds_u32_ptr pa = (lds_u32_ptr)(size_t)a_addr;
  const lds_u32_ptr ps = (lds_u32_ptr)(size_t)s_addr;
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int b = 0; b < 4; ++b) w[t][b] = pa[256 * t + 64 * b];
#pragma unroll
  for (int b = 0; b < 4; ++b) sw[b] = ps[16 * b];
}

// four token tiles' activation operands of one block: 16 bytes at addr + 4 KB j, j < 4. Plain LDS loads, so
// that token tile j's MFMAs wait only for its own read (lgkmcnt(3 - j)) instead of all four (2.5 % slower
// per prefill with a single wait).
__device__ __forceinline__ void lds_read_acts4(uint32_t addr, mxd::u32x4_t (&x)[4]) {
  const lds_u32x4_ptr p = (lds_u32x4_ptr)(size_t)addr;
  x[0] = p[0];
  x[1] = p[256];
  x[2] = p[512];
  x[3] = p[768];
}

// One wave's copies and LDS operand addresses (see gateup_exact_kernel).
struct ExactStream {
  const uint8_t* wsrc;    // group's weight pieces, + 16 lane
  const uint8_t* ssrc;    // group's scale words, + 4 lane
  const uint8_t* xbase;   // the BF16 activations
  uint32_t boff;          // this lane's activation row and K offset
  uint32_t lds0, la, las, lb;
  int wave, C;
  bool active;
  // block b's share of the copies of chunk c: weight piece b and activation block b (and the scale words
  // with block 0)
  __device__ __forceinline__ void copy_block(int c, int b) const {
    const uint32_t st = lds0 + (uint32_t)(c % kXStages) * kXStageBytes;
    global_to_lds16(wsrc + (size_t)c * 4096 + b * 1024,
                    __builtin_amdgcn_readfirstlane(st + kXStageA + (4 * wave + b) * 1024));
    if (b == 0) global_to_lds4(ssrc + (size_t)c * 256, __builtin_amdgcn_readfirstlane(st + kXStageAS + 256 * wave));
    global_to_lds16(xbase + (size_t)c * 256 + boff + 64 * b,
                    __builtin_amdgcn_readfirstlane(st + kXStageB + (4 * wave + b) * 1024));
  }
  // all of chunk c's copies
  __device__ __forceinline__ void copy(int c) const {
#pragma unroll
    for (int b = 0; b < 4; ++b) copy_block(c, b);
  }
};

// The K loop for a tile with L live 16-row token tiles (L is a template argument so that the token-tile loop
// has no per-tile branches).
template <int L>
__device__ __forceinline__ void exact_stream(const ExactStream& s, v4f (&acc)[4][8]) {
  const uint32_t k23 = 23;
  s.copy(0);
  for (int c = 0; c < s.C; ++c) {
    __builtin_amdgcn_s_waitcnt(vm_wait_imm(0));   // this wave's copies of chunk c have landed
    copy_barrier();   // every wave's copies of chunk c are visible; chunk c - 1's stage is free
    // the next chunk's copies go out a block at a time between this chunk's blocks: issued together right
    // after the barrier, all eight waves' 72 copies queue at the CU's memory unit at once and each wave
    // stalled 750-1,060 clocks a chunk before its first conversion (per-wave clock stamps of a probe build)
    const bool more = c + 1 < s.C;
    if (!s.active) {
      if (more) s.copy(c + 1);
      continue;
    }
    const uint32_t so = (uint32_t)(c % kXStages) * kXStageBytes;
    uint32_t w[4][4], sw[4];
    lds_read_weights(s.la + so, s.las + so, w, sw);
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      if (more) s.copy_block(c + 1, b);
      const float ws[4] = {e8m0_scale<0>(sw[b], k23), e8m0_scale<1>(sw[b], k23), e8m0_scale<2>(sw[b], k23),
                           e8m0_scale<3>(sw[b], k23)};
      v8bf av[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) av[t] = fp4_word_scaled(w[t][b], ws[t]);
      // token tile u's four MFMAs are issued before tile u - 1's additions, so every addition reads a result
      // finished while other work issued; the empty statements fix that order (the compiler keeps them in
      // sequence) and keep at most two tiles' results live
      v4f d[2][4];   // results of token tiles u (d[u & 1]) and u - 1
      mxd::u32x4_t x[4];
#pragma unroll
      for (int u = 0; u <= L; ++u) {
        if (u < L) {
          if ((u & 3) == 0) lds_read_acts4(s.lb + so + (4 * u + b) * 1024, x);
          mxd::u32x4_t xw = x[u & 3];
          asm volatile("" : "+v"(xw));
          const v8bf xv = __builtin_bit_cast(v8bf, xw);
#pragma unroll
          for (int t = 0; t < 4; ++t)
            d[u & 1][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[t], xv, v4f{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
        }
        if (u >= 1) {
#pragma unroll
          for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[t][u - 1][i] = acc[t][u - 1][i] + d[(u - 1) & 1][t][i];
          asm volatile("" : "+v"(acc[0][u - 1]), "+v"(acc[1][u - 1]), "+v"(acc[2][u - 1]), "+v"(acc[3][u - 1]));
        }
      }
    }
  }
}

__global__ __launch_bounds__(kXThreads) void gateup_exact_kernel(GemmArgs a) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[kXStages * kXStageBytes];
  const int ti = blockIdx.y;
  if (ti >= *a.plan.n_tiles) return;
  const int32_t* info = a.plan.tile_info + (size_t)ti * 4;
  const int slot = info[0], row0 = info[1], rows = info[2];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q = lane >> 4, n = lane & 15, m = lane & 15;
  const int H = a.H;
  // a wave past the last group (I / 32 groups) copies the last group's weights and computes nothing
  const int groups = a.I / 32;
  const int g = blockIdx.x * 8 + wave;
  const bool active = g < groups;
  const uint8_t* blob = a.tiles[slot];
  const TiledOffsets off = tiled_offsets(H, a.I);
  const int live_tiles = __builtin_amdgcn_readfirstlane(min(8, (rows + 15) / 16));
  const uint32_t lds0 = lds_addr(lds);

  // this wave's copies: group gc's weight pieces and scale words, and token tile u = wave's four activation
  // blocks (rows past the tile repeat its last row); lane (n, q) of block b's copy takes 16 bytes at
  // K 32 b + 8 q of row 16 wave + n, so that it lands at lane slot 16 q + n. LDS operand addresses of this
  // lane (stage offset added per step): weight word q of lane (m, b) of tile t at kXStageA + (4 wave + t) KB
  // + 16 (16 b + m) + 4 q; its scale byte t of word 16 b + m; activation block b of token tile u at
  // kXStageB + (4 u + b) KB + 16 lane
  ExactStream s;
  const int gc = min(g, groups - 1);
  const int C = H / 128;
  s.C = C;
  s.wsrc = blob + (size_t)gc * C * 4096 + 16 * lane;
  s.ssrc = blob + off.gu_s + (size_t)gc * C * 256 + 4 * lane;
  s.xbase = reinterpret_cast<const uint8_t*>(a.xd);
  s.boff = (uint32_t)a.plan.sorted_tok[row0 + min(16 * wave + n, rows - 1)] * (uint32_t)(2 * H) + 16 * q;
  // the offset is loaded before the first copy is issued: a wait for it afterwards would also wait for the
  // copies (the vector memory counter retires in order)
  asm volatile("" : : "v"(s.boff));
  s.lds0 = lds0;
  s.la = lds0 + kXStageA + 4096 * wave + 16 * m + 4 * q;
  s.las = lds0 + kXStageAS + 256 * wave + 4 * m;
  s.lb = lds0 + kXStageB + 16 * lane;
  s.wave = wave;
  s.active = active;

  v4f acc[4][8];
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int u = 0; u < 8; ++u) acc[t][u] = v4f{0.f, 0.f, 0.f, 0.f};
  switch (live_tiles) {
    case 1: exact_stream<1>(s, acc); break;
    case 2: exact_stream<2>(s, acc); break;
    case 3: exact_stream<3>(s, acc); break;
    case 4: exact_stream<4>(s, acc); break;
    case 5: exact_stream<5>(s, acc); break;
    case 6: exact_stream<6>(s, acc); break;
    case 7: exact_stream<7>(s, acc); break;
    default: exact_stream<8>(s, acc); break;
  }
  __syncthreads();   // the last chunk's LDS reads are done before the epilogue reuses the LDS

  // D[4q + i][n] of tile t: lanes q < 2 hold W1 rows 32g + 8t + 4q + i, lanes q >= 2 the same W3 rows
  uint16_t* eg = reinterpret_cast<uint16_t*>(lds);
  if (active) {
    uint16_t* dst = eg + (q >> 1) * (kTileRows * kEpiRowG) + n * kEpiRowG + 32 * wave + 4 * (q & 1);
#pragma unroll
    for (int u = 0; u < 8; ++u)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        uint2 packed;
        packed.x = mx::bf16_bits(acc[t][u][0]) | (mx::bf16_bits(acc[t][u][1]) << 16);
        packed.y = mx::bf16_bits(acc[t][u][2]) | (mx::bf16_bits(acc[t][u][3]) << 16);
        *reinterpret_cast<uint2*>(dst + 16 * u * kEpiRowG + 8 * t) = packed;
      }
  }
  __syncthreads();
  const bool weighted = slot < a.E;
  // the clamp limit, or +inf when unclamped (no comparison then holds, as with no clamp)
  const float lim = a.limit > 0.f ? a.limit : __builtin_inff();
  for (int p = tid; p < kTileRows * 8; p += kXThreads) {
    const int tok = p >> 3, blk = p & 7, gg = blockIdx.x * 8 + blk;
    if (tok >= rows || gg >= groups) continue;
    const int row = row0 + tok;
    const float rw = a.plan.sorted_w[row];
    const uint4* gsrc = reinterpret_cast<const uint4*>(eg + tok * kEpiRowG + 32 * blk);
    const uint4* usrc = reinterpret_cast<const uint4*>(eg + kTileRows * kEpiRowG + tok * kEpiRowG + 32 * blk);
    // mxd::swiglu_table per element, written as three passes so that the 32 table loads are in flight
    // together: clamp and table index, loads, then the products
    uint32_t idx[32];
    float up[32];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint4 gv = gsrc[j], uv = usrc[j];
      const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w}, uw[4] = {uv.x, uv.y, uv.z, uv.w};
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const uint32_t gb = (gw[k >> 1] >> (16 * (k & 1))) & 0xFFFFu, ub = (uw[k >> 1] >> (16 * (k & 1))) & 0xFFFFu;
        float upf = mx::bf16_value(ub);
        upf = upf > lim ? lim : upf;
        upf = upf < -lim ? -lim : upf;
        idx[8 * j + k] = mx::bf16_value(gb) > lim ? mxd::kSiluLimit : gb;
        up[8 * j + k] = upf;
      }
    }
    float din[32];
#pragma unroll
    for (int k = 0; k < 32; ++k) din[k] = mxd::ldgf(a.silu + idx[k]);
    float amax = 0.f;
#pragma unroll
    for (int k = 0; k < 32; ++k) {
      const float product = din[k] * up[k];
      din[k] = mxd::bf16_round_sel(weighted ? rw * product : product);
      amax = fmaxf(amax, fabsf(din[k]));
    }
    amax = fmaxf(amax, mx::u2f(mx::kAmaxFloorBits));
    const uint32_t code = mx::act_scale_code(amax);
    // x / 2^e as x * 2^-e: both are exact or one rounding of the same exact value (code is in
    // [105, 246] for amax in [1e-4, FLT_MAX], so 2^-e is a normal float)
    const float inv = mx::u2f((254u - code) << 23);
    uint32_t words[8];
#pragma unroll
    for (int w = 0; w < 8; ++w)
      words[w] = mxd::e4m3x4(din[4 * w] * inv, din[4 * w + 1] * inv, din[4 * w + 2] * inv, din[4 * w + 3] * inv);
    uint4* dst = reinterpret_cast<uint4*>(a.dq + (size_t)row * a.I + 32 * gg);
    dst[0] = uint4{words[0], words[1], words[2], words[3]};
    dst[1] = uint4{words[4], words[5], words[6], words[7]};
    a.ds[(size_t)row * (a.I / 32) + gg] = (uint8_t)code;
  }
}

// Grid-stride over (token, 8 hidden positions) items, 256 threads a workgroup. The down GEMM stored each
// token's rows contiguously in ascending expert order (row_dest), the shared expert's at place k; an item
// sums its 8 positions over them in that order, loading up to 9 rows at once.
__global__ __launch_bounds__(256) void prefill_combine_kernel(const int32_t* __restrict__ ids,
                                                              const uint16_t* __restrict__ rows, int T, int H, int k,
                                                              int E, int has_shared, uint16_t* __restrict__ y) {
  const int per_tok = H / 8;
  const int64_t items = (int64_t)T * per_tok;
  constexpr int kBatch = 9;
  for (int64_t it = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; it < items; it += (int64_t)gridDim.x * blockDim.x) {
    const int t = (int)(it / per_tok), h = (int)(it - (int64_t)t * per_tok) * 8;
    int m = 0;   // the token's valid routed pairs
    for (int i = 0; i < k; ++i) {
      const int e = ids[t * k + i];
      m += e >= 0 && e < E;
    }
    const int n = m + (has_shared ? 1 : 0);
    const uint16_t* base = rows + (size_t)t * (k + 1) * H + h;
    float acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = 0.f;
    for (int i0 = 0; i0 < n; i0 += kBatch) {
      // all of a batch's loads first (places past n repeat the last one), then the sums in order
      uint4 v[kBatch];
#pragma unroll
      for (int b = 0; b < kBatch; ++b) {
        const int j = min(i0 + b, n - 1);
        v[b] = *reinterpret_cast<const uint4*>(base + (size_t)(j < m ? j : k) * H);
      }
      // no early exit: a fully unrolled loop keeps v[] in registers (a break would index it dynamically)
#pragma unroll
      for (int b = 0; b < kBatch; ++b) {
        if (i0 + b < n) {
          const uint32_t w[4] = {v[b].x, v[b].y, v[b].z, v[b].w};
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            acc[2 * j] = acc[2 * j] + mx::bf16_value(w[j] & 0xFFFFu);
            acc[2 * j + 1] = acc[2 * j + 1] + mx::bf16_value(w[j] >> 16);
          }
        }
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
  uint64_t logits, scores, selection, ids, w, xq, xs, xd, counts, row0, tile_info, n_tiles, sorted_tok, sorted_w,
      pair_row, row_dest, dq, ds, eout, total;
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
  w.xd = take((uint64_t)T * H * 2);
  w.counts = take((E + 1) * 4);
  w.row0 = take((E + 1) * 4);
  w.tile_info = take((uint64_t)w.max_tiles * 16);
  w.n_tiles = take(4);
  w.sorted_tok = take((uint64_t)w.rows * 4);
  w.sorted_w = take((uint64_t)w.rows * 4);
  w.pair_row = take(pairs * 4);
  w.row_dest = take((uint64_t)w.rows * 4);
  w.dq = take((uint64_t)w.rows * I);
  w.ds = take((uint64_t)w.rows * I / 32);
  w.eout = take((uint64_t)T * (k + 1) * H * 2);   // token-major: [T][k + 1][H]
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

int mx_prefill_stage_offsets(mx_layer* layer, int32_t T, uint64_t* offsets) {
  const LayerView v = layer_view(layer);
  MX_REQUIRE(v.ctx != nullptr, "layer is closed");
  MX_REQUIRE(T > 0 && T <= (1 << 20), "token count %d outside [1, 2^20]", T);
  MX_REQUIRE(offsets != nullptr, "mx_prefill_stage_offsets: null output");
  const Workspace ws = workspace_layout(v.cfg, T, v.has_shared);
  const uint64_t at[MX_PREFILL_STAGES] = {ws.dq, ws.ds, ws.pair_row, ws.row0, ws.eout};
  for (int i = 0; i < MX_PREFILL_STAGES; ++i) offsets[i] = at[i];
  return MX_OK;
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
  MX_REQUIRE((uint64_t)T * c.hidden <= 0xFFFFFFFFull && (uint64_t)ws.rows * c.intermediate <= 0xFFFFFFFFull,
             "prefill of %d tokens: the gathered activations (T * H and T * (top_k + shared) * I bytes) must stay "
             "below 4 GiB", T);
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
  } else {
    int32_t* fixed_ids = (int32_t*)(b + ws.ids);
    float* fixed_w = (float*)(b + ws.w);
    hipLaunchKernelGGL(repair_routes_kernel, dim3((T + 255) / 256), dim3(256), 0, st, ids, weights, T, k, E, fixed_ids,
                       fixed_w, v.route_errors);
    MX_LAUNCH_CHECK("repair_routes_kernel");
    rid = fixed_ids;
    rw = fixed_w;
  }
  if (int s = mxi::act_quant32_scaled(v.ctx, x, b + ws.xq, b + ws.xs, (uint16_t*)(b + ws.xd), T, H, st)) return s;
  PrefillPlan p{};
  p.counts = (int32_t*)(b + ws.counts);
  p.row0 = (int32_t*)(b + ws.row0);
  p.tile_info = (int32_t*)(b + ws.tile_info);
  p.n_tiles = (int32_t*)(b + ws.n_tiles);
  p.sorted_tok = (int32_t*)(b + ws.sorted_tok);
  p.sorted_w = (float*)(b + ws.sorted_w);
  p.pair_row = (int32_t*)(b + ws.pair_row);
  p.row_dest = (int32_t*)(b + ws.row_dest);
  hipLaunchKernelGGL(zero_i32_kernel, dim3((E + 1 + 255) / 256), dim3(256), 0, st, p.counts, E + 1);
  MX_LAUNCH_CHECK("zero_i32_kernel");
  const int pairs = T * k;
  hipLaunchKernelGGL(count_kernel, dim3(std::min(64, (pairs + 255) / 256)), dim3(256), 0, st, rid, pairs, E, p.counts);
  MX_LAUNCH_CHECK("count_kernel");
  hipLaunchKernelGGL(offsets_kernel, dim3(1), dim3(64), 0, st, p, E, T, v.has_shared);
  MX_LAUNCH_CHECK("offsets_kernel");
  hipLaunchKernelGGL(scatter_kernel, dim3(E + 1), dim3(1024), 0, st, p, rid, rw, T, k, E, v.has_shared);
  MX_LAUNCH_CHECK("scatter_kernel");
  hipLaunchKernelGGL(dest_kernel, dim3((pairs + 255) / 256), dim3(256), 0, st, p, rid, T, k, E);
  MX_LAUNCH_CHECK("dest_kernel");
  GemmArgs a{};
  a.tiles = v.tiles;
  a.plan = p;
  a.H = H;
  a.I = I;
  a.E = E;
  a.limit = c.swiglu_limit;
  a.silu = v.silu;
  a.xq = b + ws.xq;
  a.xs = b + ws.xs;
  a.xd = (const uint16_t*)(b + ws.xd);
  a.dq = b + ws.dq;
  a.ds = b + ws.ds;
  a.out = (uint16_t*)(b + ws.eout);
  hipLaunchKernelGGL(gateup_exact_kernel, dim3((I + 255) / 256, ws.max_tiles), dim3(kXThreads), 0, st, a);
  MX_LAUNCH_CHECK("gateup_exact_kernel");
  hipLaunchKernelGGL(grouped_down_kernel, dim3((H + 511) / 512, ws.max_tiles), dim3(kGThreads), 0, st, a);
  MX_LAUNCH_CHECK("grouped_down_kernel");
  const int64_t items = (int64_t)T * (H / 8);
  hipLaunchKernelGGL(prefill_combine_kernel, dim3((unsigned)std::min<int64_t>(2048, (items + 255) / 256)), dim3(256), 0,
                     st, rid, (const uint16_t*)a.out, T, H, k, E, v.has_shared, y);
  MX_LAUNCH_CHECK("prefill_combine_kernel");
  return MX_OK;
}

}  // extern "C"
