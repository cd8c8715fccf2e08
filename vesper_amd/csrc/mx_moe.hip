// Routed MoE decode on gfx950: router, top-k plan, fused MXFP4 expert GEMVs, ordered combine.
//
// Reference behaviour (shell-term/vesper) and where each piece lives here:
//   GateProjection.project (gate.py:133-147)        router_kernel: FP32 W_r . x, FMA per thread + fixed tree
//   router_scores / router_top6 (routing_probe.cu)  score_of + topk_token_wave (generalised E, k)
//   participation (moe.py:18-30)                    build_plan: ascending expert IDs, ascending tokens
//   ExpertExecutor.execute (expert.py:51-79)        gateup_kernel (W1/W3 + SwiGLU + down-input quant)
//                                                   + down_kernel (W2)
//   MoEAccumulator (moe.py:42-148)                  combine_kernel / acc_* kernels
//
// Expert GEMVs run on V_MFMA_SCALE_F32_16X16X128_F8F6F4: A = 16 weight rows of packed E2M1 (one
// 16-byte MX block per lane), B = up to 16 tokens of E4M3 activations, with the E8M0 block scales
// fed to the instruction. Decode streams each selected expert's weights from HBM exactly once and
// never materialises dequantized weights.
#include <algorithm>
#include <cmath>
#include <mutex>
#include <vector>

#include "mx_device.h"
#include "mx_internal.h"
#include "mx_numerics.h"

// Fixed device memory of the allocation-free tiled expert call (mx_expert_forward_tiled_noalloc): its plan,
// one-entry expert table and quantized activations, MX_NOALLOC_SCRATCH_BYTES on every GPU the library runs
// on, held until the process ends. Host code reaches it only through the device address that
// mxi::noalloc_scratch_init takes once per device. Every call on a GPU shares it: calls that overlap on one
// GPU race. Nothing in it needs to start at zero (each call writes what it reads).
static __device__ __align__(256) uint8_t scratch[MX_NOALLOC_SCRATCH_BYTES];

namespace {

using mxd::ldg128;
using mxd::ldg32;
using mxd::tiled_offsets;
using mxd::TiledOffsets;
using mxd::v4f;
using mxd::v8i;

constexpr int kMaxTokens = 16;   // MFMA N: tokens per expert per decode call
constexpr int kMaxTopK = 32;
constexpr int kMaxExperts = 1024;
constexpr int kMaxSlots = kMaxTokens * kMaxTopK + 1;
constexpr int kRouterKIter = 8;   // router GEMV: hidden size <= 8 * 1024 per thread-strided pass
constexpr int kRouteThreads = 1024;             // top-k + plan workgroup: one wave per token
constexpr int kRouteWaves = kRouteThreads / 64;

// Device-side execution plan of one decode call (written by the router's last workgroup).
struct Plan {
  int32_t n_slots;      // routed + shared
  int32_t n_routed;
  int32_t total_rows;   // rows of the compact per-(token, expert) buffers
  int32_t tokens;
  int32_t top_k;
  int32_t pad[3];
  int32_t slot_expert[kMaxSlots];   // expert ID per slot, ascending; E marks the shared expert
  int32_t slot_ntok[kMaxSlots];
  int32_t slot_row0[kMaxSlots];
  int32_t slot_weighted[kMaxSlots];
  int32_t slot_tok[kMaxSlots][kMaxTokens];
  float slot_w[kMaxSlots][kMaxTokens];
  int32_t tok_rows[kMaxTokens][kMaxTopK + 1];   // a token's rows in ascending expert order, shared last
};

// ----------------------------------------------------------------------------------------------
// small helpers

__device__ __forceinline__ uint32_t ordered_key(float v) {
  const uint32_t b = mx::f2u(v);
  return b ^ ((b & 0x80000000u) ? 0xFFFFFFFFu : 0x80000000u);
}

// ordered_key of +0, -0, +inf and -inf
constexpr uint32_t kKeyPosZero = 0x80000000u, kKeyNegZero = 0x7FFFFFFFu, kKeyPosInf = 0xFF800000u,
                   kKeyNegInf = 0x007FFFFFu;

// FP32 score of one logit: exp/log1p in float64 rounded once to FP32 (the oracle does the same).
__device__ __forceinline__ float score_of(float z, int score_func) {
  if (score_func == MX_SCORE_SIGMOID) {
    const float e = (float)exp(-(double)z);
    return 1.0f / (1.0f + e);
  }
  const float sp = z > 20.0f ? z : (float)log1p(exp((double)z));
  return sqrtf(sp);
}

// Wavefront reductions and scans on DPP (row_shr 1/2/4/8 inside 16-lane rows, then row_bcast 15/31
// across rows): VALU-latency steps instead of LDS-routed shuffles. `ident` fills lanes whose DPP
// source is out of range or whose row is masked off.
template <int kCtrl, int kRowMask>
__device__ __forceinline__ int dpp_i(int v, int ident) {
  return __builtin_amdgcn_update_dpp(ident, v, kCtrl, kRowMask, 0xF, false);
}

// inclusive prefix sum over the 64 lanes
__device__ __forceinline__ int wave_scan_i(int v, int /*lane*/) {
  v += dpp_i<0x111, 0xF>(v, 0);   // row_shr:1
  v += dpp_i<0x112, 0xF>(v, 0);   // row_shr:2
  v += dpp_i<0x114, 0xF>(v, 0);   // row_shr:4
  v += dpp_i<0x118, 0xF>(v, 0);   // row_shr:8
  v += dpp_i<0x142, 0xA>(v, 0);   // row_bcast:15 into rows 1 and 3
  v += dpp_i<0x143, 0xC>(v, 0);   // row_bcast:31 into rows 2 and 3
  return v;
}

// FP32 wavefront sum in the fixed DPP order (row scans, then across rows), result in every lane.
__device__ __forceinline__ float wave_sum_f(float v) {
  auto step = [](float x, int y) { return x + __int_as_float(y); };
  v = step(v, dpp_i<0x111, 0xF>(__float_as_int(v), 0));
  v = step(v, dpp_i<0x112, 0xF>(__float_as_int(v), 0));
  v = step(v, dpp_i<0x114, 0xF>(__float_as_int(v), 0));
  v = step(v, dpp_i<0x118, 0xF>(__float_as_int(v), 0));
  v = step(v, dpp_i<0x142, 0xA>(__float_as_int(v), 0));
  v = step(v, dpp_i<0x143, 0xC>(__float_as_int(v), 0));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

__device__ __forceinline__ uint32_t umax32(uint32_t a, uint32_t b) { return a > b ? a : b; }

__device__ __forceinline__ uint32_t wave_max_u(uint32_t v) {
  int x = (int)v;
  x = (int)umax32((uint32_t)x, (uint32_t)dpp_i<0x111, 0xF>(x, 0));
  x = (int)umax32((uint32_t)x, (uint32_t)dpp_i<0x112, 0xF>(x, 0));
  x = (int)umax32((uint32_t)x, (uint32_t)dpp_i<0x114, 0xF>(x, 0));
  x = (int)umax32((uint32_t)x, (uint32_t)dpp_i<0x118, 0xF>(x, 0));
  x = (int)umax32((uint32_t)x, (uint32_t)dpp_i<0x142, 0xA>(x, 0));
  x = (int)umax32((uint32_t)x, (uint32_t)dpp_i<0x143, 0xC>(x, 0));
  return (uint32_t)__builtin_amdgcn_readlane(x, 63);
}

// value of lane (lane ^ kXor) within each 32-lane half (ds_swizzle bit-mask mode: and 0x1F, xor kXor)
template <int kXor>
__device__ __forceinline__ int swizzle_xor(int v) {
  return __builtin_amdgcn_ds_swizzle(v, (kXor << 10) | 0x1F);
}

// ----------------------------------------------------------------------------------------------
// Top-k of one token by one wavefront (routing_probe.cu:17-86, router.py:23-61, generalised).
//
// 1. threshold = k-th largest order-preserving key, found by distinct-value rounds; a round whose
//    value occurs twice sets the tie flag (the reference's serial arg-max passes).
// 2. gather keys above the threshold by ascending ID, then keys equal to it by ascending ID, k total.
// 3. the 32-slot bitonic network (slot i pairs with i ^ stride; the pair's direction is bit `size`
//    of the lower slot for sizes 2..16, ascending-false for the final merge).
// 4. raw = score[id], denominator = halving-tree sum + 1e-20, weight = raw / den * route_scale.
// One compare-exchange stage of the 32-slot network on lanes (slot, slot ^ kStride).
template <int kSize, int kStride>
__device__ __forceinline__ void bitonic_stage(float& kv, int32_t& iv, int& vv, int slot) {
  const float pk = __int_as_float(swizzle_xor<kStride>(__float_as_int(kv)));
  const int32_t pi = swizzle_xor<kStride>(iv);
  const int pv = swizzle_xor<kStride>(vv);
  const bool lower = (slot & kStride) == 0;
  const int lo = lower ? slot : (slot ^ kStride);
  const float klo = lower ? kv : pk, khi = lower ? pk : kv;
  const int vlo = lower ? vv : pv, vhi = lower ? pv : vv;
  const bool promote = (klo > khi && vlo) || !vhi;
  const bool dir = kSize < 32 ? (lo & kSize) != 0 : false;
  if (promote == dir) { kv = pk; iv = pi; vv = pv; }
}

struct TopkOut {
  int32_t* indices;
  float* weights;
  float* raw;
  float* den;
  int32_t* tied;
};

template <int kPer>
__device__ void topk_token_wave_t(const float* __restrict__ selection, const float* __restrict__ scores, int E, int k,
                                  float route_scale, int t, const TopkOut& o) {
  const int lane = threadIdx.x & 63;
  const int per = kPer;
  uint32_t key[kPer];
  float sel[kPer], scr[kPer];
  // the raw scores are loaded with the selection values (no dependent load after the sort)
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int e = lane * per + j;
    const bool ok = e < E;
    sel[j] = ok ? selection[e] : 0.f;
    scr[j] = ok ? scores[e] : 0.f;
    key[j] = ok ? ordered_key(sel[j]) : 0u;
  }
  int taken = 0, tied = 0;
  uint32_t thr = 0;
  // While every round finds exactly one expert at a nonzero, non-NaN value, the rounds themselves are
  // the selection in descending order (float order equals key order there), which is what the sorting
  // network below produces for distinct values; lane r keeps round r's expert.
  bool distinct = true;
  int32_t round_id = 0;
  // 1a. Distinct rounds from sorted lanes: each lane orders its keys once (descending; invalid slots hold
  //     key 0), then a round is the wave maximum of the lanes' first keys, and the lane holding it shifts
  //     its keys down by one. A round whose value is held twice (by two lanes' first keys, or by the
  //     holder's next key) or is a signed zero or NaN ends this pass, and the threshold search below runs
  //     from the start; otherwise this pass is that search's rounds with a single candidate per lane
  //     (one wave maximum and two ballots a round instead of a scan of every key and kPer + 1 ballots).
  {
    uint32_t sk[kPer];
    int sj[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      sk[j] = lane * per + j < E ? key[j] : 0u;
      sj[j] = j;
    }
#pragma unroll
    for (int i = 1; i < kPer; ++i)
#pragma unroll
      for (int m = i; m >= 1; --m)
        if (sk[m] > sk[m - 1]) {
          const uint32_t tk = sk[m];
          sk[m] = sk[m - 1];
          sk[m - 1] = tk;
          const int tj = sj[m];
          sj[m] = sj[m - 1];
          sj[m - 1] = tj;
        }
    for (int round = 0; round < k; ++round) {
      const uint32_t best = wave_max_u(sk[0]);
      const bool mine = sk[0] == best;
      const uint64_t holders = __ballot(mine);
      const uint64_t twice = kPer > 1 ? __ballot(mine && sk[kPer > 1 ? 1 : 0] == best) : 0ull;
      if (__popcll(holders) != 1 || twice != 0ull || best == kKeyPosZero || best == kKeyNegZero ||
          best > kKeyPosInf || best < kKeyNegInf) {
        distinct = false;
        break;
      }
      const int hit = __builtin_ctzll(holders);
      const int32_t id = hit * per + __builtin_amdgcn_readlane(sj[0], hit);
      if (lane == round) round_id = id;
      if (mine) {
#pragma unroll
        for (int j = 0; j + 1 < kPer; ++j) {
          sk[j] = sk[j + 1];
          sj[j] = sj[j + 1];
        }
        sk[kPer - 1] = 0u;
      }
    }
  }
  // 1b. threshold search. Each round finds the next distinct key and how many experts hold it: lanes
  //    holding at least 1, 2, ... kPer of their keys at that value, counted by ballots.
  uint64_t bound = 1ull << 32;   // exclusive upper bound on keys still to rank
  const bool sorted_pass = distinct;
  distinct = true;
  for (int round = 0; !sorted_pass && round < k; ++round) {
    uint32_t m = 0;
    bool any = false;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int e = lane * per + j;
      if (e < E && (uint64_t)key[j] < bound && (!any || key[j] > m)) { m = key[j]; any = true; }
    }
    // lanes without a candidate contribute key 0; a real key 0 (-NaN pattern) is excluded upstream
    const uint32_t best = wave_max_u(any ? m : 0u);
    int cj = 0, jhit = 0;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int e = lane * per + j;
      if (e < E && key[j] == best) {
        ++cj;
        jhit = j;
      }
    }
    const uint64_t holders = __ballot(cj >= 1);
    int c = __popcll(holders);
#pragma unroll
    for (int mm = 2; mm <= kPer; ++mm) c += __popcll(__ballot(cj >= mm));
    tied |= c >= 2;
    taken += c;
    thr = best;
    const int hit = holders ? __builtin_ctzll(holders) : 0;
    const int32_t id = hit * per + __builtin_amdgcn_readlane(jhit, hit);
    distinct = distinct && c == 1 && best != kKeyPosZero && best != kKeyNegZero && best <= kKeyPosInf &&
               best >= kKeyNegInf;
    if (lane == round) round_id = id;
    if (taken >= k) break;
    bound = best;
  }
  const int slot = lane & 31;
  float kv;
  int32_t iv;
  int vv;
  if (distinct) {
    kv = 0.f;
    iv = round_id;
    vv = slot < k;
  } else {
    // 2. gather by ascending ID: lane-major then j (experts are laid out contiguously per lane)
    int n_gt = 0, n_eq = 0;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int e = lane * per + j;
      if (e < E) {
        n_gt += key[j] > thr;
        n_eq += key[j] == thr;
      }
    }
    const int inc_gt = wave_scan_i(n_gt, lane);
    const int inc_eq = wave_scan_i(n_eq, lane);
    const int total_gt = __builtin_amdgcn_readlane(inc_gt, 63);
    int pos_gt = inc_gt - n_gt, pos_eq = total_gt + inc_eq - n_eq;
    __shared__ float s_key[kRouteWaves][32];
    __shared__ int32_t s_id[kRouteWaves][32];
    const int wave = threadIdx.x >> 6;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int e = lane * per + j;
      if (e < E) {
        if (key[j] > thr) {
          if (pos_gt < k) { s_key[wave][pos_gt] = sel[j]; s_id[wave][pos_gt] = e; }
          ++pos_gt;
        } else if (key[j] == thr) {
          if (pos_eq < k) { s_key[wave][pos_eq] = sel[j]; s_id[wave][pos_eq] = e; }
          ++pos_eq;
        }
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    // 3. bitonic network on lanes 0..31 (lanes 32..63 mirror them and are ignored)
    kv = slot < k ? s_key[wave][slot] : 0.f;
    iv = slot < k ? s_id[wave][slot] : 0;
    vv = slot < k;
    bitonic_stage<2, 1>(kv, iv, vv, slot);
    bitonic_stage<4, 2>(kv, iv, vv, slot);
    bitonic_stage<4, 1>(kv, iv, vv, slot);
    bitonic_stage<8, 4>(kv, iv, vv, slot);
    bitonic_stage<8, 2>(kv, iv, vv, slot);
    bitonic_stage<8, 1>(kv, iv, vv, slot);
    bitonic_stage<16, 8>(kv, iv, vv, slot);
    bitonic_stage<16, 4>(kv, iv, vv, slot);
    bitonic_stage<16, 2>(kv, iv, vv, slot);
    bitonic_stage<16, 1>(kv, iv, vv, slot);
    bitonic_stage<32, 16>(kv, iv, vv, slot);
    bitonic_stage<32, 8>(kv, iv, vv, slot);
    bitonic_stage<32, 4>(kv, iv, vv, slot);
    bitonic_stage<32, 2>(kv, iv, vv, slot);
    bitonic_stage<32, 1>(kv, iv, vv, slot);
  }
  // 4. raw scores, tree denominator, weights
  // expert iv's raw score lives in lane iv / kPer, register iv % kPer
  float raw = 0.f;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const float v = __shfl(scr[j], iv / kPer, 64);
    raw = (iv % kPer == j) ? v : raw;
  }
  raw = slot < k ? raw : 0.f;
  float acc = raw;
  int width = 1;
  while (width < k) width <<= 1;
  int present = k;
  for (int stride = width >> 1; stride >= 1; stride >>= 1) {
    // lanes below `stride` read lane + stride, which is lane ^ stride for them
    const int bits = __float_as_int(acc);
    const int ob = stride == 16 ? swizzle_xor<16>(bits) : stride == 8 ? swizzle_xor<8>(bits)
                 : stride == 4 ? swizzle_xor<4>(bits) : stride == 2 ? swizzle_xor<2>(bits) : swizzle_xor<1>(bits);
    const float other = __int_as_float(ob);
    if (slot < stride && slot + stride < present) acc = acc + other;
    present = present < stride ? present : stride;
  }
  const float den = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), 0)) + 1e-20f;
  if (lane < k) {
    const float w = (raw / den) * route_scale;
    o.indices[t * k + lane] = iv;
    o.weights[t * k + lane] = w;
    if (o.raw) o.raw[t * k + lane] = raw;
  }
  if (lane == 0) {
    if (o.den) o.den[t] = den;
    if (o.tied) o.tied[t] = tied;
  }
}

// Experts are spread kPer per lane (E <= 64 * kPer); the smallest power-of-two kPer keeps the
// per-lane loops short for E = 256 (4 per lane).
__device__ __forceinline__ void topk_token_wave(const float* __restrict__ selection, const float* __restrict__ scores,
                                                int E, int k, float route_scale, int t, const TopkOut& o) {
  if (E <= 64) topk_token_wave_t<1>(selection, scores, E, k, route_scale, t, o);
  else if (E <= 128) topk_token_wave_t<2>(selection, scores, E, k, route_scale, t, o);
  else if (E <= 256) topk_token_wave_t<4>(selection, scores, E, k, route_scale, t, o);
  else if (E <= 512) topk_token_wave_t<8>(selection, scores, E, k, route_scale, t, o);
  else topk_token_wave_t<16>(selection, scores, E, k, route_scale, t, o);
}

// ----------------------------------------------------------------------------------------------
// Plan from the routed IDs (participation, moe.py:18-30): slots are the distinct experts in ascending
// ID order, each with its tokens ascending; rows are numbered expert-major; the shared expert is the
// last slot with every token.
//
// Two builders give the same plan; measured on MI355X (E = 256, k = 8), pair counting is faster for
// T * k < 32 pairs, the expert-indexed builder for more (T = 16: 2.7 us against 6.4 us).
//
// Expert-indexed (many pairs): each expert's tokens are collected as a bit mask (T <= 16) in LDS. One
// block-wide scan over the experts in ascending ID then gives every present expert its slot (present
// experts below it) and its first row (pairs below it). A pair's place within its expert is the number
// of earlier tokens in the expert's mask, and its place within its token the number of the token's
// experts with a smaller ID.
// `ids` and `w` are in LDS for both builders; every token's IDs are distinct and in [0, E).
__device__ void build_plan_experts(Plan* __restrict__ plan, const int32_t* ids, const float* w, int T, int k,
                                   int E, int has_shared) {
  __shared__ uint32_t s_mask[kMaxExperts];
  __shared__ int32_t s_slot[kMaxExperts];
  __shared__ int32_t s_row0[kMaxExperts];
  __shared__ int32_t s_wsum[2][kRouteWaves];
  const int tid = threadIdx.x, nth = blockDim.x, lane = tid & 63, wave = tid >> 6, waves = nth >> 6;
  const int n = T * k;
  for (int e = tid; e < E; e += nth) s_mask[e] = 0u;
  __syncthreads();
  for (int p = tid; p < n; p += nth) atomicOr(&s_mask[ids[p]], 1u << (p / k));
  __syncthreads();
  // thread tid owns the experts [run * tid, run * tid + run)
  const int run = (E + nth - 1) / nth;
  const int e0 = min(run * tid, E), e1 = min(e0 + run, E);
  int present = 0, pairs = 0;
  for (int e = e0; e < e1; ++e) {
    const int c = __popc(s_mask[e]);
    present += c > 0;
    pairs += c;
  }
  const int inc_p = wave_scan_i(present, lane), inc_r = wave_scan_i(pairs, lane);
  if (lane == 63) {
    s_wsum[0][wave] = inc_p;
    s_wsum[1][wave] = inc_r;
  }
  __syncthreads();
  int slot = inc_p - present, row = inc_r - pairs, routed = 0;
  for (int v = 0; v < waves; ++v) {
    if (v < wave) {
      slot += s_wsum[0][v];
      row += s_wsum[1][v];
    }
    routed += s_wsum[0][v];
  }
  for (int e = e0; e < e1; ++e) {
    const int c = __popc(s_mask[e]);
    s_slot[e] = slot;
    s_row0[e] = row;
    if (c) {
      plan->slot_expert[slot] = e;
      plan->slot_ntok[slot] = c;
      plan->slot_row0[slot] = row;
      plan->slot_weighted[slot] = 1;
      ++slot;
      row += c;
    }
  }
  __syncthreads();
  for (int p = tid; p < n; p += nth) {
    const int e = ids[p], t = p / k;
    const int before = __popc(s_mask[e] & ((1u << t) - 1u));
    int tok_before = 0;
    for (int j = 0; j < k; ++j) tok_before += ids[t * k + j] < e;
    plan->slot_tok[s_slot[e]][before] = t;
    plan->slot_w[s_slot[e]][before] = w[p];
    plan->tok_rows[t][tok_before] = s_row0[e] + before;
  }
  if (has_shared && tid < T) {
    plan->slot_tok[routed][tid] = tid;
    plan->slot_w[routed][tid] = 1.0f;
    plan->tok_rows[tid][k] = n + tid;
  }
  if (tid == 0) {
    plan->n_routed = routed;
    plan->n_slots = routed + has_shared;
    plan->total_rows = n + (has_shared ? T : 0);
    plan->tokens = T;
    plan->top_k = k;
    if (has_shared) {
      plan->slot_expert[routed] = E;
      plan->slot_ntok[routed] = T;
      plan->slot_row0[routed] = n;
      plan->slot_weighted[routed] = 0;
    }
  }
}

// Pair counting (few pairs): every routed pair (t, e) has the unique key e * 16 + t, and its row is the
// key's rank among all T * k keys: sorted by key, the pairs run expert-major with ascending tokens,
// which is exactly the row order. Ranks, slot numbers and positions are all counts over the staged keys, so the plan is
// two counting passes with one barrier between them. A group of S = 2^j lanes shares each pair's
// count and combines it with xor-shuffles. `ids` and `w` are in LDS.
__device__ void build_plan_pairs(Plan* __restrict__ plan, const int32_t* ids, const float* w, int T, int k, int E,
                                 int has_shared) {
  __shared__ int32_t s_start[kMaxTokens * kMaxTopK];   // 1 where the pair opens its expert's run
  const int tid = threadIdx.x, nth = blockDim.x;
  const int n = T * k;   // <= 32 * T <= nth / 2 (the launch has one wave per token)
  int S = 1;
  while (S < 64 && 2 * S * n <= nth) S <<= 1;
  const int p = tid / S, part = tid % S;
  const bool active = p < n;
  const int ep = active ? ids[p] : 0, tp = active ? p / k : 0;
  const int kp = ep * kMaxTokens + tp;
  int less = 0, same_before = 0, same = 0, tok_before = 0;
  if (active) {
    for (int u = part; u < n; u += S) {
      const int eu = ids[u], tu = u / k, ku = eu * kMaxTokens + tu;
      less += ku < kp;
      same_before += (eu == ep) & (tu < tp);
      same += eu == ep;
      tok_before += (tu == tp) & (eu < ep);
    }
  }
  for (int m = 1; m < S; m <<= 1) {
    less += __shfl_xor(less, m, 64);
    same_before += __shfl_xor(same_before, m, 64);
    same += __shfl_xor(same, m, 64);
    tok_before += __shfl_xor(tok_before, m, 64);
  }
  if (active && part == 0) s_start[p] = same_before == 0;
  __syncthreads();
  int slot = 0, routed = 0;
  if (active) {
    for (int u = part; u < n; u += S) {
      const int st = s_start[u];
      routed += st;
      slot += st & (ids[u] < ep);
    }
  }
  for (int m = 1; m < S; m <<= 1) {
    slot += __shfl_xor(slot, m, 64);
    routed += __shfl_xor(routed, m, 64);
  }
  if (active && part == 0) {
    if (same_before == 0) {
      plan->slot_expert[slot] = ep;
      plan->slot_ntok[slot] = same;
      plan->slot_row0[slot] = less;
      plan->slot_weighted[slot] = 1;
    }
    plan->slot_tok[slot][same_before] = tp;
    plan->slot_w[slot][same_before] = w[p];
    plan->tok_rows[tp][tok_before] = less;
    if (p == 0) {
      plan->n_routed = routed;
      plan->n_slots = routed + has_shared;
      plan->total_rows = n + (has_shared ? T : 0);
      plan->tokens = T;
      plan->top_k = k;
      if (has_shared) {
        plan->slot_expert[routed] = E;
        plan->slot_ntok[routed] = T;
        plan->slot_row0[routed] = n;
        plan->slot_weighted[routed] = 0;
        for (int t = 0; t < T; ++t) {
          plan->slot_tok[routed][t] = t;
          plan->slot_w[routed][t] = 1.0f;
          plan->tok_rows[t][k] = n + t;
        }
      }
    }
  }
}

__device__ __forceinline__ void build_plan(Plan* __restrict__ plan, const int32_t* ids, const float* w, int T, int k,
                                           int E, int has_shared) {
  if (T * k < 32) build_plan_pairs(plan, ids, w, T, k, E, has_shared);
  else build_plan_experts(plan, ids, w, T, k, E, has_shared);
}

// One slot holding all tokens of a single expert call (mx_expert_forward).
__global__ void single_plan_kernel(Plan* plan, int T, const float* __restrict__ route_w) {
  const int t = threadIdx.x;
  if (t < T) {
    plan->slot_tok[0][t] = t;
    plan->slot_w[0][t] = route_w ? route_w[t] : 1.0f;
    plan->tok_rows[t][0] = t;
  }
  if (t == 0) {
    plan->n_slots = 1;
    plan->n_routed = route_w ? 1 : 0;
    plan->total_rows = T;
    plan->tokens = T;
    plan->top_k = 1;
    plan->slot_expert[0] = 0;
    plan->slot_ntok[0] = T;
    plan->slot_row0[0] = 0;
    plan->slot_weighted[0] = route_w ? 1 : 0;
  }
}

// One workgroup ranks the tokens, one wave per token: wave t ranks token t, the results are staged in LDS and
// written out, then the same workgroup builds the plan from the staged IDs.
__global__ __launch_bounds__(kRouteThreads) void route_plan_kernel(const float* selection, const float* scores, int T,
                                                                   int E, int k, float route_scale, TopkOut o,
                                                                   Plan* plan, int has_shared) {
  __shared__ int32_t s_idx[kMaxTokens * kMaxTopK];
  __shared__ float s_w[kMaxTokens * kMaxTopK];
  const TopkOut staged{s_idx, s_w, o.raw, o.den, o.tied};
  const int t = threadIdx.x >> 6;
  if (t < T) topk_token_wave(selection + (size_t)t * E, scores + (size_t)t * E, E, k, route_scale, t, staged);
  __syncthreads();
  for (int i = threadIdx.x; i < T * k; i += blockDim.x) {
    o.indices[i] = s_idx[i];
    o.weights[i] = s_w[i];
  }
  build_plan(plan, s_idx, s_w, T, k, E, has_shared);
}

// Plan from given routing (decode with routing decided elsewhere): ids [T][k] and weights [T][k] are
// staged in LDS and each token's list is made valid first (mxd::repair_token_routes: an id outside [0, E)
// or repeated within the token becomes the smallest expert the token does not name, with weight 0), so any
// input keeps the plan's invariants (k distinct experts per token) and every access in bounds; the number
// of replaced ids is added to `errors`, which the host reads to refuse the call.
__global__ __launch_bounds__(kRouteThreads) void routed_plan_kernel(const int32_t* ids, const float* w, int T, int k,
                                                                    int E, int32_t* out_ids, float* out_w, Plan* plan,
                                                                    int has_shared, uint32_t* errors) {
  __shared__ int32_t s_idx[kMaxTokens * kMaxTopK];
  __shared__ float s_w[kMaxTokens * kMaxTopK];
  for (int i = threadIdx.x; i < T * k; i += blockDim.x) {
    s_idx[i] = ids[i];
    s_w[i] = w[i];
  }
  __syncthreads();
  if (threadIdx.x < T) {
    const int replaced = mxd::repair_token_routes(s_idx + threadIdx.x * k, s_w + threadIdx.x * k, k, E);
    if (replaced) atomicAdd(errors, (uint32_t)replaced);
  }
  __syncthreads();
  for (int i = threadIdx.x; i < T * k; i += blockDim.x) {
    out_ids[i] = s_idx[i];
    out_w[i] = s_w[i];
  }
  build_plan(plan, s_idx, s_w, T, k, E, has_shared);
}

__global__ void set_u32_kernel(uint32_t* p, uint32_t v) { *p = v; }

__global__ void set_experts_kernel(const uint8_t** table, int n, mx_expert_batch b) {
  const int i = threadIdx.x;
  if (i < n) table[b.expert[i]] = (const uint8_t*)b.tiled[i];
}

// Stand-alone top-k over supplied selection/scores: one wave per token.
__global__ __launch_bounds__(256) void topk_kernel(const float* selection, const float* scores, int T, int E, int k,
                                                   float route_scale, TopkOut o) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t < T) topk_token_wave(selection + (size_t)t * E, scores + (size_t)t * E, E, k, route_scale, t, o);
}

__global__ void scores_kernel(const float* logits, const float* bias, int T, int E, int score_func, float* scores,
                              float* selection) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= T * E) return;
  const float s = score_of(logits[i], score_func);
  scores[i] = s;
  selection[i] = bias ? s + bias[i % E] : s;
}

// ----------------------------------------------------------------------------------------------
// Expert GEMVs on scaled MFMA.

struct ExpertArgs {
  const uint8_t* const* tiles;   // tiled layout: device table [E+1] of expert blobs
  mx_expert_ptrs single;         // reference layout: the one expert of mx_expert_forward / mx_gemv_mxfp4
  const Plan* plan;
  int H, I;
  float limit;
  const uint8_t* xq;             // [T][H]
  const uint8_t* xs;             // [T][H/32]
  const uint16_t* xd;            // [T][H] BF16: each E4M3 code of xq times its block scale (exact)
  uint8_t* dq;                   // [rows][I]
  uint8_t* ds;                   // [rows][I/32]
  uint16_t* out;                 // [rows][H]
  int tokens;                    // the call's token count: bounds every slot's (sizes the gate/up LDS ring)
  // diagnostics (nullable)
  uint16_t* w1;
  uint16_t* w3;
  uint16_t* din;
  float* trace;
  // one-token decode with the routing folded into gate/up (gateup_kernel<true>): every workgroup selects the
  // token's experts from the router's outputs itself, and workgroup (0, 0) writes the routing and the plan
  // that the later launches read
  const float* selection;        // [E] selection values of the token
  const float* scores;           // [E] scores of the token
  TopkOut topk;                  // the routing outputs (indices, weights, raw scores, denominator, tie flag)
  Plan* plan_out;
  int E, k, has_shared;
  float route_scale;
};

// The gate/up workgroup's view of its slot: from the plan, or selected in the workgroup (gateup_kernel<true>).
struct SlotView {
  int n_slots, expert, ntok, row0, weighted;
  int32_t tok[kMaxTokens];
  float w[kMaxTokens];
};

// Operand layout of V_MFMA_SCALE_F32_16X16X128_F8F6F4 (measured on gfx950 with one-hot probe kernels):
//   A (FP4, 4 VGPRs): lane l holds row l%16, K = 32*(l/16) + j for nibble j (low nibble first),
//                     i.e. one whole 16-byte MX block of the reference layout.
//   B (FP8, 8 VGPRs): lane l holds column l%16; bytes 0-15 are K = 16*(l/16) + j and bytes 16-31
//                     are K = 64 + 16*(l/16) + j.
//   scale_a / scale_b: lane l scales row / column l%16 over the 32-wide K block l/16.
//   D: lane l, register i holds row 4*(l/16) + i, column l%16.
// So the FP8 side of a 128-wide K chunk is read as two 16-byte pieces at 16q and 64 + 16q.
__device__ __forceinline__ v4f mfma_fp4xfp8(uint4 a, uint4 b0, uint4 b1, v4f c, int sa, int sb) {
  v8i av = {(int)a.x, (int)a.y, (int)a.z, (int)a.w, 0, 0, 0, 0};
  v8i bv = {(int)b0.x, (int)b0.y, (int)b0.z, (int)b0.w, (int)b1.x, (int)b1.y, (int)b1.z, (int)b1.w};
  // cbsz = 4: A is FP4 E2M1; blgp = 0: B is FP8 E4M3; op_sel 0 selects scale byte 0.
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bv, c, 4, 0, 0, sa, 0, sb);
}

// ---- K-split streaming core shared by the gate/up and down kernels -------------------------------
//
// A workgroup of 4 waves owns a row group of 4 MFMA tiles x 16 weight rows. Wave w walks its own
// contiguous quarter of the 128-wide K chunks and multiplies every chunk into all 4 tiles, so one
// load of the activation operand serves 4 MFMAs. Loads run P chunks ahead of the MFMAs (a register
// ring unrolled so every index is static). The 4 partial accumulators per tile are then summed in a
// fixed wave order through LDS, so results do not depend on scheduling.
constexpr int kTiles = 4;

// Weight operand in the device-native tiled layout: for every (row group, K chunk) the 4 tiles'
// A operands are 4 consecutive KB (lane l's 16 bytes at 16 * l), so each load instruction of a
// wave reads 1 KB of contiguous memory, and one 4-byte word per lane (256 contiguous bytes per
// chunk) carries that lane's E8M0 code for each of the 4 tiles (byte t = tile t).
struct TiledW {
  const uint8_t* w;   // row group's weights + 16 * lane
  const uint8_t* s;   // row group's scale words + 4 * lane
  struct Regs {
    uint4 wa[kTiles];
    uint32_t sw;
  };
  __device__ __forceinline__ void load(Regs& r, int c, int /*q*/) const {
#pragma unroll
    for (int t = 0; t < kTiles; ++t) r.wa[t] = mxd::ldg128_nt(w + (size_t)c * 4096 + t * 1024);
    r.sw = mxd::ldg32_nt(s + (size_t)c * 256);
  }
  __device__ __forceinline__ static int scale(const Regs& r, int t, int /*q*/) { return (int)((r.sw >> (8 * t)) & 0xFF); }
};

// Weight operand in the reference row-major layout (w[row][K/2], s[row][K/32]): each load covers
// 16 rows x 64 bytes, and every tile needs its own scale load.
struct RowMajorW {
  const uint8_t* wrow[kTiles];   // this lane's weight row of each tile
  const uint8_t* srow[kTiles];   // and its E8M0 scale row
  struct Regs {
    uint4 wa[kTiles];
    uint32_t sw[kTiles];
  };
  __device__ __forceinline__ void load(Regs& r, int c, int q) const {
    const int kb = 4 * c + q;
#pragma unroll
    for (int t = 0; t < kTiles; ++t) {
      r.wa[t] = ldg128(wrow[t] + (size_t)kb * 16);
      r.sw[t] = ldg32(srow[t] + 4 * c);
    }
  }
  __device__ __forceinline__ static int scale(const Regs& r, int t, int q) { return (int)((r.sw[t] >> (8 * q)) & 0xFF); }
};

struct ActOperand {
  const uint8_t* xrow;    // this lane's token row of E4M3 activations
  const uint8_t* xsrow;   // and its E8M0 scales
  bool live;              // lane's token column is in use
  // chunk c's B operand (two 16-byte pieces) and the lane's scale word
  __device__ __forceinline__ void load(int c, int q, uint4& b0, uint4& b1, uint32_t& sx) const {
    const uint8_t* chunk = xrow + (size_t)c * 128;
    b0 = ldg128(chunk + 16 * q);
    b1 = ldg128(chunk + 64 + 16 * q);
    sx = ldg32(xsrow + 4 * c);
  }
};

template <class W>
struct ChunkRegs {
  typename W::Regs w;
  uint4 b0, b1;
  uint32_t sx;
};

template <class W, class X>
__device__ __forceinline__ void load_chunk(ChunkRegs<W>& r, const W& ws, const X& x, int c, int q) {
  ws.load(r.w, c, q);
  // Idle token columns read a valid row too (no divergent branch around the loads, which would
  // force the operands through scratch); mma_chunk zeroes them, and their outputs are dropped.
  x.load(c, q, r.b0, r.b1, r.sx);
}

template <class W>
__device__ __forceinline__ void mma_chunk(const ChunkRegs<W>& r, v4f (&acc)[kTiles], int q, uint32_t keep) {
  const int sx = (int)((r.sx >> (8 * q)) & 0xFF);
  const uint4 b0 = make_uint4(r.b0.x & keep, r.b0.y & keep, r.b0.z & keep, r.b0.w & keep);
  const uint4 b1 = make_uint4(r.b1.x & keep, r.b1.y & keep, r.b1.z & keep, r.b1.w & keep);
#pragma unroll
  for (int t = 0; t < kTiles; ++t) acc[t] = mfma_fp4xfp8(r.w.wa[t], b0, b1, acc[t], W::scale(r.w, t, q), sx);
}

// The K chunks [c0, c0 + n) of one wave, accumulated in place from zero, one MFMA per chunk in order. Loads
// run P chunks ahead; ring slots past the end repeat the last chunk (a cache hit) and are masked to zero.
template <int P, class W, class X>
__device__ __forceinline__ void stream_range(const W& ws, const X& x, int c0, int n, int q, v4f (&acc)[kTiles]) {
#pragma unroll
  for (int t = 0; t < kTiles; ++t) acc[t] = v4f{0.f, 0.f, 0.f, 0.f};
  if (n == 0) return;
  const uint32_t live = x.live ? 0xFFFFFFFFu : 0u;
  ChunkRegs<W> buf[P];
#pragma unroll
  for (int j = 0; j < P; ++j) load_chunk(buf[j], ws, x, c0 + min(j, n - 1), q);
  int i = 0;
  for (; i + P < n; i += P) {
#pragma unroll
    for (int j = 0; j < P; ++j) {
      mma_chunk(buf[j], acc, q, live);
      load_chunk(buf[j], ws, x, c0 + min(i + j + P, n - 1), q);
    }
  }
#pragma unroll
  for (int j = 0; j < P; ++j) mma_chunk(buf[j], acc, q, i + j < n ? live : 0u);
}

// Wave `wave` of 4 streams its contiguous quarter of the K chunks.
template <int P, class W, class X>
__device__ __forceinline__ void stream_ksplit(const W& ws, const X& x, int chunks, int wave, int q,
                                              v4f (&acc)[kTiles]) {
  const int c0 = (chunks * wave) / 4, c1 = (chunks * (wave + 1)) / 4;
  stream_range<P>(ws, x, c0, c1 - c0, q, acc);
}

// ---- Exact in-order core of the gate/up GEMVs ---------------------------------------------------
//
// fp4_gemv_spec (formats.py:97-118) rounds each 32-wide block dot to FP32 once, scales it by both E8M0
// codes, and adds the blocks to an FP32 sum in ascending block order. Here one wave owns one 16-row tile
// over the whole K range, so each (row, token) sum is a single chain in one lane, and every block is one
// V_MFMA_F32_16X16X32_BF16 whose operands carry the scales: the E2M1 weights times 2^(code - 127) (at most
// two significant bits: exact in BF16, converted by V_CVT_SCALEF32_PK_BF16_FP4) and the E4M3 activations
// times their block scale (four significant bits: exact in BF16, written by the quantizer). Measured on
// MI355X against the exact dot on 1.5 M random blocks (realistic, all-codes and sparse operands): with a zero
// accumulator the instruction returns the exact sum of its 32 products rounded once to FP32 in every case,
// so D = RN(dot) * sa * sw, the spec's block term; its accumulator input is not rounded that way, so the chain
// adds D in VALU: acc = acc + D, blocks 4c, 4c + 1, 4c + 2, 4c + 3 of chunk c in order.
//
// Operand map (gfx950): A lane l = row l % 16, K 8 (l / 16) + 0..7; B lane l = token column l % 16, same K;
// D lane l register i = row 4 (l / 16) + i, column l % 16. A lane (m, q) of the tiled layout holds the whole
// 32-value block 4c + q of row m as four words; two permlane32 and two permlane16 swaps transpose the
// 4 x 4 (lane group, word) matrix so that lane group g holds word g of every block, and MFMA b of the chunk
// takes register b: K = 32 (4c + b) + 8 g + 0..7 at lane group g.

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));

// The core's loop runs its own memory pipeline. Each wave streams its tile's weights into a register ring;
// the operands all four waves share -- the chunk's 256 bytes of scale words and the slot's activations -- are
// copied once per workgroup into an LDS ring (direct global -> LDS copies) and read from there. Loads, copies
// and LDS reads are issued from inline assembly with counted waits: with compiler-issued loads, register
// allocation around the ring made the compiler's in-order vmcnt waits cover loads issued a chunk earlier (a
// memory round trip per chunk), and nine loads per wave and chunk (codes and activations read by every
// wave) filled the address unit's queues. The compiler does not track these loads: every register
// destination passes through a tied wait before it is read, and the loop drains them before its registers
// are released.
using mxd::u32x4_t;
typedef int v4i __attribute__((ext_vector_type(4)));

// Loads and copies address memory as a wave-uniform base (SGPRs, advanced per chunk by scalar arithmetic) plus
// a constant per-lane 32-bit offset, so the per-chunk address arithmetic runs on the scalar unit.
__device__ __forceinline__ u32x4_t asm_ldg128_nt(const uint8_t* base, uint32_t off) {
  u32x4_t v;
  asm volatile("global_load_dwordx4 %0, %1, %2 nt" : "=v"(v) : "v"(off), "s"(base));
  return v;
}
__device__ __forceinline__ u32x4_t asm_ldg128(const uint8_t* base, uint32_t off) {
  u32x4_t v;
  asm volatile("global_load_dwordx4 %0, %1, %2" : "=v"(v) : "v"(off), "s"(base));
  return v;
}
// Direct global -> LDS copy of 16 bytes per lane at base + off: lane l's bytes land at lds + 16 l.
__device__ __forceinline__ void asm_copy16(const uint8_t* base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" : : "v"(off), "s"(base), "s"(lds) : "m0");
}

// Readable memory for the core's loads past the last chunk (each lane reads 16 bytes at 16 x lane): small
// enough to stay cached, read with plain loads.
__device__ __align__(256) uint8_t exact_dummy_page[1024];

// Exact-core LDS ring: kXStages stages of kStageChunks chunks each: the chunks' scale words (256 B each, 1 KB)
// and, per token of the slot, the chunks' scaled activations (256 B each, 1 KB per token); xstage_bytes(T)
// with the call's token count T bounding every slot's. The ring lives in the launch's dynamic LDS.
constexpr int kStageChunks = 4;
constexpr int kXStages = 2;
constexpr int kXStageScale = 0, kXStageAct = 1024;
__host__ __device__ constexpr int xstage_bytes(int T) { return 1024 + 1024 * T; }

// Stage g's shared operands (chunks 4g .. 4g + 3) into ring slot st, one 1 KB copy instruction each: the scale
// words, and one per token (token j by wave j % 4, the scale words by wave ntok % 4). In a last stage holding
// fewer than 4 chunks the lanes past the row's end copy its first bytes instead (those LDS bytes are never
// read), and past the last stage the copies read the dummy page, so a wave issues the same number of copies for
// every stage.
struct SharedCopies {
  const uint8_t* scale;   // row group's scale words (chunk c at + 256 c)
  const uint8_t* act;     // the scaled activations (token t's row at + 2 H t)
  const uint8_t* dummy;   // exact_dummy_page
  uint32_t act_row[kMaxTokens / 4];   // byte offsets of this wave's tokens' rows
  int act_tok[kMaxTokens / 4];        // and their token indices within the slot
  int n_act;                          // how many tokens this wave copies
  int n;                              // chunks of the row
  uint32_t lane;
  uint32_t lds;           // the ring's LDS byte address
  int stage_bytes;
  bool copies_scale;
  __device__ __forceinline__ int copies() const { return n_act + (copies_scale ? 1 : 0); }
  __device__ __forceinline__ void issue(int g, int st) const {
    const uint32_t base = lds + st * stage_bytes;
    if (kStageChunks * g < n) {
      const uint32_t k = (int)lane < 16 * (n - kStageChunks * g) ? (uint32_t)g * 1024 + 16 * lane : 0;
      if (copies_scale) asm_copy16(scale, k, base + kXStageScale);
#pragma unroll
      for (int i = 0; i < kMaxTokens / 4; ++i)
        if (i < n_act) asm_copy16(act, act_row[i] + k, base + kXStageAct + 1024 * act_tok[i]);
    } else {
      if (copies_scale) asm_copy16(dummy, 16 * lane, base + kXStageScale);
#pragma unroll
      for (int i = 0; i < kMaxTokens / 4; ++i)
        if (i < n_act) asm_copy16(dummy, 16 * lane, base + kXStageAct + 1024 * act_tok[i]);
    }
  }
};

__device__ __forceinline__ uint32_t fp4_scale_float_bits(uint32_t code) { return code << 23; }

// 8 E2M1 values (one word, low nibble first) times the scale whose FP32 bits are `scale_bits`, as 8 BF16 MFMA
// operand values (exact).
__device__ __forceinline__ v8bf fp4_word_bits(uint32_t word, uint32_t scale_bits) {
  const float scale = __uint_as_float(scale_bits);
  const v2bf p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, scale, 0);
  const v2bf p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, scale, 1);
  const v2bf p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, scale, 2);
  const v2bf p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, scale, 3);
  return v8bf{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
}

// 4 x 4 transpose across lane groups: afterwards lane group g register r holds what lane group r register g held
// (two permlane32 swaps exchange the upper half of v0 / v1 with the lower half of v2 / v3, two permlane16 swaps
// the odd 16-lane rows of v0 / v2 with the even rows of v1 / v3).
__device__ __forceinline__ void transpose_groups(uint32_t (&v)[4]) {
  auto a = __builtin_amdgcn_permlane32_swap(v[0], v[2], false, false);
  auto b = __builtin_amdgcn_permlane32_swap(v[1], v[3], false, false);
  auto c = __builtin_amdgcn_permlane16_swap(a[0], b[0], false, false);
  auto d = __builtin_amdgcn_permlane16_swap(a[1], b[1], false, false);
  v[0] = c[0];
  v[1] = c[1];
  v[2] = d[0];
  v[3] = d[1];
}

// Stage st's operands of this lane, read and waited for: the activations of blocks 0..3 at K 8 g (token column
// n, or the slot's first token for idle columns) and the E8M0 codes of row m, blocks 0..3 (byte t of scale
// word m + 16 b).
__device__ __forceinline__ void lds_read_stage(uint32_t xaddr, uint32_t caddr, u32x4_t (&xb)[4], uint32_t (&code)[4]) {
  asm volatile(
      "ds_read_b128 %0, %8\n\t"
      "ds_read_b128 %1, %8 offset:64\n\t"
      "ds_read_b128 %2, %8 offset:128\n\t"
      "ds_read_b128 %3, %8 offset:192\n\t"
      "ds_read_u8 %4, %9\n\t"
      "ds_read_u8 %5, %9 offset:64\n\t"
      "ds_read_u8 %6, %9 offset:128\n\t"
      "ds_read_u8 %7, %9 offset:192\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(xb[0]), "=&v"(xb[1]), "=&v"(xb[2]), "=&v"(xb[3]), "=&v"(code[0]), "=&v"(code[1]), "=&v"(code[2]),
        "=&v"(code[3])
      : "v"(xaddr), "v"(caddr));
}

// Multiply chunk c (this lane's 16 weight bytes wa, LDS stage operands) into the chains.
__device__ __forceinline__ void exact_chunk(const u32x4_t& wa, const u32x4_t (&xb)[4], const uint32_t (&code)[4],
                                            v4f& acc) {
  uint32_t wv[4] = {wa.x, wa.y, wa.z, wa.w};
  transpose_groups(wv);   // lane group g now holds word g of every block: K 32 (4c + b) + 8 g + 0..7 in wv[b]
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const v8bf av = fp4_word_bits(wv[b], fp4_scale_float_bits(code[b]));
    const v4f d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, __builtin_bit_cast(v8bf, xb[b]),
                                                          v4f{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = acc[i] + d[i];
  }
}

// The whole K range (n chunks) of tile `wave` of a row group, stage by stage. At the
// start of stage g a wave waits until its own copies of stage g have landed, a barrier makes every wave's copies
// visible, and the wave issues its copies of stage g + kXStages - 1 (into the ring slot of stage g - 1, which
// every wave finished reading before this barrier); then for each chunk c of the stage it reads the chunk's
// operands from LDS, multiplies chunk c and issues its weights for chunk c + kW. kW = kXStages x kStageChunks,
// so the weights of a stage's chunks are issued before that stage's copies, and past the end weights load from
// the dummy page and copies read it: every stage issues the same loads per wave, and when a wave waits for its
// copies of stage g, the loads issued after them -- the weights of stage g - kXStages + 1's chunks and, per
// later stage, copies + kStageChunks weights -- may still be in flight.
constexpr int kWRing = kXStages * kStageChunks;

template <int kAfter>
__device__ __forceinline__ void vm_wait() {
  static_assert(kAfter <= 63, "vmcnt holds at most 63 outstanding loads");
  __builtin_amdgcn_s_waitcnt(mxd::vm_wait_imm(kAfter));
}

// wait for this wave's copies of a stage, with `copies` copy instructions per stage (0 .. 5)
template <int kCopies>
__device__ __forceinline__ void wait_stage() {
  vm_wait<kStageChunks + (kXStages - 2) * (kCopies + kStageChunks)>();
}

__device__ __forceinline__ void stream_exact(const uint8_t* wbase, uint32_t woff, const SharedCopies& sc,
                                             uint32_t xaddr, uint32_t caddr, int n, v4f& acc) {
  constexpr int kW = kWRing, kX = kXStages, kC = kStageChunks;
  const int sb = sc.stage_bytes, n_stages = (n + kC - 1) / kC, copies = sc.copies();
  acc = v4f{0.f, 0.f, 0.f, 0.f};
  u32x4_t wr[kW];
  auto load_w = [&](u32x4_t& r, int c) {
    if (c < n) r = asm_ldg128_nt(wbase + (size_t)c * 4096, woff);
    else r = asm_ldg128(sc.dummy, 16 * sc.lane);
  };
  // the loads of stages -kX .. -1 in the steady state's order: stage g issues C(g + kX - 1) (when that stage
  // index is not negative), then the weights of chunks kC g + kW .. kC g + kW + kC - 1
#pragma unroll
  for (int vg = -kX; vg < 0; ++vg) {
    if (vg + kX - 1 >= 0) sc.issue(vg + kX - 1, (vg + kX - 1) % kX);
#pragma unroll
    for (int u = 0; u < kC; ++u) load_w(wr[kC * (vg + kX) + u], kC * vg + kW + u);
  }
  for (int g0 = 0; g0 < n_stages; g0 += kX) {
#pragma unroll
    for (int gs = 0; gs < kX; ++gs) {
      const int g = g0 + gs;
      // the waits and ties run for every slot, past the end too: a slot's registers are only released (and
      // reusable by the compiler) once the load that writes them has landed
      switch (copies) {
        case 0: wait_stage<0>(); break;
        case 1: wait_stage<1>(); break;
        case 2: wait_stage<2>(); break;
        case 3: wait_stage<3>(); break;
        case 4: wait_stage<4>(); break;
        default: wait_stage<5>(); break;
      }
#pragma unroll
      for (int u = 0; u < kC; ++u) asm volatile("" : "+v"(wr[kC * gs + u]));   // landed with the wait above
      // every wave's copies of stage g have landed, and every wave has finished reading stage g - 1, whose slot
      // this stage's copies overwrite (past the last stage only that one is still read)
      if (g <= n_stages) mxd::copy_barrier();
      sc.issue(g + kX - 1, (gs + kX - 1) % kX);
#pragma unroll
      for (int u = 0; u < kC; ++u) {
        const int c = kC * g + u;
        if (c < n) {
          u32x4_t xb[4];
          uint32_t code[4];
          lds_read_stage(xaddr + gs * sb + 256 * u, caddr + gs * sb + 256 * u, xb, code);
          exact_chunk(wr[kC * gs + u], xb, code, acc);
        }
        load_w(wr[kC * gs + u], c + kW);
      }
    }
  }
  // drain: no load may still be writing a ring register, and no copy the LDS, once the loop is left
  vm_wait<0>();
#pragma unroll
  for (int j = 0; j < kW; ++j) asm volatile("" : "+v"(wr[j]));
  mxd::copy_barrier();
}

// ----------------------------------------------------------------------------------------------
// Router: grid (E, ceil(T / kMaxTokens)); workgroup e computes logits/scores/selection of expert e
// for up to 16 tokens; workgroups also share the per-32 quantization of x. Top-k and the plan run in
// route_plan_kernel, the next launch on the same stream, so no workgroup waits on another.
struct RouterArgs {
  const float* W;
  const float* bias;
  const uint16_t* x;
  int T, H, E, k, score_func;
  float route_scale;
  float* logits;
  float* scores;
  float* selection;
  uint8_t* xq;
  uint8_t* xs;
  uint16_t* xd;   // each code times its block scale, BF16 (the exact gate/up GEMVs' activation operand)
};

__global__ __launch_bounds__(256) void router_kernel(RouterArgs a) {
  const int e = blockIdx.x;
  const int t0 = blockIdx.y * kMaxTokens;
  const int nt = min(kMaxTokens, a.T - t0);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float acc[kMaxTokens];
#pragma unroll
  for (int t = 0; t < kMaxTokens; ++t) acc[t] = 0.f;
  const float* wrow = a.W + (size_t)e * a.H;
  // All of this thread's W_r loads are issued before any FMA (kRouterKIter * 1024 >= H, checked on
  // the host); x rows are then read four tokens at a time with their loads hoisted likewise.
  float4 w[kRouterKIter];
#pragma unroll
  for (int i = 0; i < kRouterKIter; ++i) {
    const int k0 = tid * 4 + i * 1024;
    w[i] = k0 < a.H ? *reinterpret_cast<const float4*>(wrow + k0) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
#pragma unroll
  for (int t4 = 0; t4 < kMaxTokens; t4 += 4) {
    if (t4 < nt) {
      uint2 xb[4][kRouterKIter];
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int i = 0; i < kRouterKIter; ++i) {
          const int k0 = tid * 4 + i * 1024;
          xb[u][i] = (t4 + u < nt && k0 < a.H) ? *reinterpret_cast<const uint2*>(a.x + (size_t)(t0 + t4 + u) * a.H + k0)
                                               : make_uint2(0u, 0u);
        }
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int i = 0; i < kRouterKIter; ++i) {
          float v = acc[t4 + u];
          v = fmaf(w[i].x, mx::bf16_value(xb[u][i].x & 0xFFFFu), v);
          v = fmaf(w[i].y, mx::bf16_value(xb[u][i].x >> 16), v);
          v = fmaf(w[i].z, mx::bf16_value(xb[u][i].y & 0xFFFFu), v);
          v = fmaf(w[i].w, mx::bf16_value(xb[u][i].y >> 16), v);
          acc[t4 + u] = v;
        }
    }
  }
  __shared__ float part[4][kMaxTokens];
#pragma unroll
  for (int t = 0; t < kMaxTokens; ++t) {
    if (t < nt) {
      const float v = wave_sum_f(acc[t]);
      if (lane == 0) part[wave][t] = v;
    }
  }
  // share the per-32 quantization of x (blocks of 32 handled by 32-lane halves)
  if (a.xq && blockIdx.y == 0) {
    const int nblocks = a.T * (a.H / 32);
    const int half = tid >> 5, l32 = tid & 31;
    for (int b = blockIdx.x * 8 + half; b < nblocks; b += a.E * 8) {   // the E routing workgroups share it
      const float v = mx::bf16_value(a.x[(size_t)b * 32 + l32]);
      float amax = fabsf(v);
#pragma unroll
      for (int m = 16; m >= 1; m >>= 1) amax = fmaxf(amax, __shfl_xor(amax, m, 32));
      amax = fmaxf(amax, mx::u2f(mx::kAmaxFloorBits));
      const uint32_t code = mx::act_scale_code(amax);
      const uint32_t qc = mx::act_quant_pow2(v, 1.0f / mx::e8m0_value(code));
      a.xq[(size_t)b * 32 + l32] = (uint8_t)qc;
      a.xd[(size_t)b * 32 + l32] = (uint16_t)mx::bf16_bits(mx::e4m3_value(qc) * mx::e8m0_value(code));
      if (l32 == 0) a.xs[b] = (uint8_t)code;
    }
  }
  __syncthreads();
  if (tid < nt) {
    const float z = ((part[0][tid] + part[1][tid]) + part[2][tid]) + part[3][tid];
    const size_t o = (size_t)(t0 + tid) * a.E + e;
    a.logits[o] = z;
    const float s = score_of(z, a.score_func);
    if (a.scores) a.scores[o] = s;
    if (a.selection) a.selection[o] = a.bias ? s + a.bias[e] : s;
  }
}

// Sum the 4 waves' partial tiles in wave order; wave w returns tile w's accumulator.
__device__ __forceinline__ v4f reduce_tiles(const v4f (&acc)[kTiles], int wave, int lane, float (*red)[kTiles][64][4]) {
#pragma unroll
  for (int t = 0; t < kTiles; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) red[wave][t][lane][i] = acc[t][i];
  __syncthreads();
  v4f out;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    out[i] = ((red[0][wave][lane][i] + red[1][wave][lane][i]) + red[2][wave][lane][i]) + red[3][wave][lane][i];
  return out;
}

// SwiGLU epilogue of gate/up tile t of row group g: in `mine` (the in-order chains), lane (n, q) holds token
// column n; lanes with q < 2 hold W1 rows 4q + i of the tile (D[4q + i][n]) and lane + 32 the matching W3
// rows. Writes the down input of token n to s_din[n][8t + 4q + i] (and the diagnostic copies when requested).
__device__ __forceinline__ void gateup_tile_epilogue(const ExpertArgs& a, const SlotView& sv, int g, int t,
                                                     const v4f& mine, int lane, int ntok, float (*s_din)[32]) {
  float upv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) upv[i] = __shfl_xor(mine[i], 32, 64);
  const int q = lane >> 4, n = lane & 15;
  if (q < 2 && n < ntok) {
    const int row0 = sv.row0;
    const bool weighted = sv.weighted != 0;
    const float rw = sv.w[n];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int li = t * 8 + 4 * q + i;           // row within the 32-row block
      const int gi = g * 32 + li;                 // intermediate index
      const uint32_t b1 = mx::bf16_bits(mine[i]);
      const uint32_t b3 = mx::bf16_bits(upv[i]);
      const size_t o2 = (size_t)(row0 + n) * a.I + gi;
      const float din = mxd::swiglu_element(b1, b3, a.limit, weighted, rw, a.trace ? a.trace + o2 * 5 : nullptr);
      s_din[n][li] = din;
      if (a.w1) a.w1[o2] = (uint16_t)b1;
      if (a.w3) a.w3[o2] = (uint16_t)b3;
      if (a.din) a.din[o2] = (uint16_t)mx::bf16_bits(din);
    }
  }
}

// Per-token quantization of row group g's 32-row block of the down input (one E8M0 block per token):
// 16 consecutive threads j2 = 0..15 take token tn, 2 values each.
__device__ __forceinline__ void gateup_quantize_block(const ExpertArgs& a, const SlotView& sv, int g, int tn, int j2,
                                                      int ntok, const float (*s_din)[32]) {
  if (tn >= ntok) return;
  const int I = a.I;
  const float v0 = s_din[tn][2 * j2], v1 = s_din[tn][2 * j2 + 1];
  float amax = mxd::row16_max(fmaxf(fabsf(v0), fabsf(v1)));   // the token's 16 lanes are one row
  amax = fmaxf(amax, mx::u2f(mx::kAmaxFloorBits));
  const uint32_t code = mx::act_scale_code(amax);
  const float sc = mx::e8m0_value(code);
  const float inv = 1.0f / sc;   // exact: sc is a power of two
  const uint32_t q0 = mx::act_quant_pow2(v0, inv), q1 = mx::act_quant_pow2(v1, inv);
  const size_t r = (size_t)(sv.row0 + tn);
  *reinterpret_cast<uint16_t*>(a.dq + r * I + g * 32 + 2 * j2) = (uint16_t)(q0 | (q1 << 8));
  if (j2 == 0) a.ds[r * (I / 32) + g] = (uint8_t)code;
}

// One-token decode, routing folded into gate/up: wave 0 selects the token's k experts from the router's
// selection values and scores (topk_token_wave, the same selection and weights as route_plan_kernel), and
// slot s is the selected expert with s smaller selected IDs (row s, the token's route weight), or the shared
// expert for s = k (row k) -- route_plan_kernel's plan for one token, where pairs run expert-major. Workgroup
// (0, 0) also writes the routing outputs and the plan itself (build_plan) for the down and combine launches
// that follow on the stream; every workgroup computes the same selection from the same inputs.
__device__ void select_slot_one_token(const ExpertArgs& a, int s, SlotView& sv) {
  __shared__ int32_t s_idx[kMaxTopK];
  __shared__ float s_w[kMaxTopK];
  const bool first = blockIdx.x == 0 && blockIdx.y == 0;
  // the shared expert's slot (s = k) needs no selection, so its workgroups -- the last dispatched -- start
  // streaming without waiting for it; workgroup (0, 0), which publishes the routing and the plan, is a routed slot
  if (s < a.k && threadIdx.x < 64) {
    const TopkOut staged{s_idx, s_w, first ? a.topk.raw : nullptr, first ? a.topk.den : nullptr,
                         first ? a.topk.tied : nullptr};
    topk_token_wave(a.selection, a.scores, a.E, a.k, a.route_scale, 0, staged);
  }
  __syncthreads();
  if (first) {
    for (int i = threadIdx.x; i < a.k; i += blockDim.x) {
      a.topk.indices[i] = s_idx[i];
      a.topk.weights[i] = s_w[i];
    }
    build_plan_pairs(a.plan_out, s_idx, s_w, 1, a.k, a.E, a.has_shared);   // one token: k < 32 pairs
  }
  if (threadIdx.x == 0) {
    sv.n_slots = a.k + a.has_shared;
    sv.ntok = 1;
    sv.tok[0] = 0;
    if (s < a.k) {
      int e = 0;
      float w = 0.f;
      for (int j = 0; j < a.k; ++j) {
        int below = 0;
        for (int i = 0; i < a.k; ++i) below += s_idx[i] < s_idx[j];
        if (below == s) {
          e = s_idx[j];
          w = s_w[j];
        }
      }
      sv.expert = e;
      sv.row0 = s;
      sv.weighted = 1;
      sv.w[0] = w;
    } else {
      sv.expert = a.E;
      sv.row0 = a.k;
      sv.weighted = 0;
      sv.w[0] = 1.0f;
    }
  }
  __syncthreads();
}

// grid (I/32, slots), 256 threads, tiled experts. The workgroup computes intermediate rows [32g, 32g + 32) of
// W1 and W3 for the slot's tokens: tile t holds W1 rows 32g + 8t + (0..7) as MFMA rows 0-7 and the same W3
// rows as MFMA rows 8-15. Wave t streams tile t over all of K (the exact in-order core), applies the SwiGLU
// epilogue, and the workgroup quantizes its 32-row block of the down input per token (one E8M0 block).
// kPlanInGateup: the one-token form that selects its experts itself (a separate instantiation: the
// selection's LDS and registers stay out of the many-token kernel, whose occupancy they would lower).
template <bool kPlanInGateup>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void gateup_kernel(ExpertArgs a) {
  const int s = blockIdx.y, g = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63;
  __shared__ SlotView sv;
  if constexpr (kPlanInGateup) {
    select_slot_one_token(a, s, sv);
  } else {
    const Plan* __restrict__ plan = a.plan;
    if (tid == 0) {
      sv.n_slots = plan->n_slots;
      if (s < sv.n_slots) {
        sv.expert = plan->slot_expert[s];
        sv.ntok = plan->slot_ntok[s];
        sv.row0 = plan->slot_row0[s];
        sv.weighted = plan->slot_weighted[s];
      }
    }
    if (tid < kMaxTokens && s < plan->n_slots) {
      sv.tok[tid] = plan->slot_tok[s][tid];
      sv.w[tid] = plan->slot_w[s][tid];
    }
    __syncthreads();
  }
  if (s >= sv.n_slots) return;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q = lane >> 4, m = lane & 15, n = lane & 15;
  const int ntok = sv.ntok;
  const int H = a.H, I = a.I;
  const size_t chunks = H / 128;
  const uint8_t* blob = a.tiles[sv.expert];
  extern __shared__ __attribute__((aligned(16))) uint8_t ring[];   // kXStages x xstage_bytes(a.tokens)
  const uint32_t ring0 = mxd::lds_addr(ring);
  SharedCopies sc;
  sc.scale = blob + tiled_offsets(H, I).gu_s + (size_t)g * chunks * 256;
  sc.act = reinterpret_cast<const uint8_t*>(a.xd);
  sc.n_act = 0;
#pragma unroll
  for (int i = 0; i < kMaxTokens / 4; ++i) {   // tokens wave, wave + 4, ... of the slot
    const int j = wave + 4 * i;
    sc.act_tok[i] = j;
    sc.act_row[i] = (uint32_t)sv.tok[j < ntok ? j : 0] * (uint32_t)(2 * H);
    if (j < ntok) sc.n_act = i + 1;
  }
  sc.dummy = exact_dummy_page;
  sc.n = (int)chunks;
  sc.lane = lane;
  sc.lds = ring0;
  sc.stage_bytes = xstage_bytes(a.tokens);
  sc.copies_scale = wave == (ntok & 3);
  // this lane's LDS operands: token column n's row (the slot's first token for idle columns) at K 8 q, and the
  // scale byte of tile `wave` for row m (word m + 16 b holds block b)
  const uint32_t xaddr = ring0 + kXStageAct + 1024 * (n < ntok ? n : 0) + 16 * q;
  const uint32_t caddr = ring0 + kXStageScale + 4 * m + wave;
  const uint8_t* wbase = blob + (size_t)g * chunks * 4096 + (size_t)wave * 1024;
  v4f acc;
  stream_exact(wbase, 16 * lane, sc, xaddr, caddr, (int)chunks, acc);
  __shared__ float s_din[kMaxTokens][32];
  gateup_tile_epilogue(a, sv, g, wave, acc, lane, ntok, s_din);
  __syncthreads();
  gateup_quantize_block(a, sv, g, tid >> 4, tid & 15, ntok, s_din);
}

// Output rows [64b, 64b + 64) of slot s's W2 as 4 tiles of 16 rows; after the cross-wave sum wave t writes
// tile t as BF16 (the reference's w2 stage).
template <bool kTiled>
__device__ void down_rows(const ExpertArgs& a, int s, int b, float (*red)[kTiles][64][4]) {
  const Plan* __restrict__ plan = a.plan;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int m = lane & 15, q = lane >> 4, n = lane & 15;
  const int ntok = plan->slot_ntok[s];
  const int row0 = plan->slot_row0[s];
  const int H = a.H, I = a.I;
  const int hb = b * 64;
  ActOperand x;
  x.live = n < ntok;
  x.xrow = a.dq + (size_t)(row0 + (x.live ? n : 0)) * I;
  x.xsrow = a.ds + (size_t)(row0 + (x.live ? n : 0)) * (I / 32);
  v4f acc[kTiles];
  if constexpr (kTiled) {
    const uint8_t* blob = a.tiles[plan->slot_expert[s]];
    const TiledOffsets off = tiled_offsets(H, I);
    const size_t chunks = I / 128;
    TiledW ws;
    ws.w = blob + off.dn_w + (size_t)b * chunks * 4096 + 16 * lane;
    ws.s = blob + off.dn_s + (size_t)b * chunks * 256 + 4 * lane;
    stream_ksplit<4>(ws, x, I / 128, wave, q, acc);
  } else {
    RowMajorW ws;
#pragma unroll
    for (int t = 0; t < kTiles; ++t) {
      ws.wrow[t] = (const uint8_t*)a.single.w2_weight + (size_t)(hb + 16 * t + m) * (I / 2);
      ws.srow[t] = (const uint8_t*)a.single.w2_scale + (size_t)(hb + 16 * t + m) * (I / 32);
    }
    stream_ksplit<4>(ws, x, I / 128, wave, q, acc);
  }
  const v4f mine = reduce_tiles(acc, wave, lane, red);
  if (n < ntok) {
    uint2 packed;
    packed.x = mx::bf16_bits(mine[0]) | (mx::bf16_bits(mine[1]) << 16);
    packed.y = mx::bf16_bits(mine[2]) | (mx::bf16_bits(mine[3]) << 16);
    *reinterpret_cast<uint2*>(a.out + (size_t)(row0 + n) * H + hb + 16 * wave + 4 * q) = packed;
  }
}

// grid (H/64, slots), 256 threads.
template <bool kTiled>
__global__ __launch_bounds__(256) void down_kernel(ExpertArgs a) {
  const Plan* __restrict__ plan = a.plan;
  const int s = blockIdx.y;
  if (s >= plan->n_slots) return;
  __shared__ float red[4][kTiles][64][4];
  down_rows<kTiled>(a, s, blockIdx.x, red);
}

// Reference layout <-> tiled layout of one expert (both directions bit-for-bit; every byte of
// either layout has exactly one counterpart). One thread per 16-byte A operand piece, then one per
// 4-byte scale word; gate/up and down sections in one grid-stride pass.
__global__ void tile_expert_kernel(mx_expert_ptrs ref, uint8_t* blob, int H, int I, int to_tiled) {
  const TiledOffsets off = tiled_offsets(H, I);
  const int64_t cg = H / 128, cd = I / 128;
  const int64_t gu_pieces = (int64_t)I * H / 16, gu_words = (int64_t)I * H / 64;
  const int64_t dn_pieces = (int64_t)H * I / 32, dn_words = (int64_t)H * I / 128;
  const int64_t total = gu_pieces + gu_words + dn_pieces + dn_words;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    int64_t i = idx;
    if (i < gu_pieces) {
      const int l = (int)(i & 63), t = (int)((i >> 6) & 3), m = l & 15, q = l >> 4;
      const int64_t rest = i >> 8, c = rest % cg, g = rest / cg;
      const int64_t row = 32 * g + 8 * t + (m & 7);
      uint8_t* r = (uint8_t*)(m < 8 ? ref.w1_weight : ref.w3_weight) + row * (H / 2) + (4 * c + q) * 16;
      uint4* d = reinterpret_cast<uint4*>(blob + i * 16);
      if (to_tiled) *d = *reinterpret_cast<const uint4*>(r);
      else *reinterpret_cast<uint4*>(r) = *d;
      continue;
    }
    i -= gu_pieces;
    if (i < gu_words) {
      const int l = (int)(i & 63), m = l & 15, q = l >> 4;
      const int64_t rest = i >> 6, c = rest % cg, g = rest / cg;
      uint8_t* sref = (uint8_t*)(m < 8 ? ref.w1_scale : ref.w3_scale);
      uint32_t* d = reinterpret_cast<uint32_t*>(blob + off.gu_s + i * 4);
      uint32_t word = to_tiled ? 0u : *d;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        uint8_t* r = sref + (32 * g + 8 * t + (m & 7)) * (H / 32) + 4 * c + q;
        if (to_tiled) word |= (uint32_t)*r << (8 * t);
        else *r = (uint8_t)(word >> (8 * t));
      }
      if (to_tiled) *d = word;
      continue;
    }
    i -= gu_words;
    if (i < dn_pieces) {
      const int l = (int)(i & 63), t = (int)((i >> 6) & 3), m = l & 15, q = l >> 4;
      const int64_t rest = i >> 8, c = rest % cd, b = rest / cd;
      uint8_t* r = (uint8_t*)ref.w2_weight + (64 * b + 16 * t + m) * (I / 2) + (4 * c + q) * 16;
      uint4* d = reinterpret_cast<uint4*>(blob + off.dn_w + i * 16);
      if (to_tiled) *d = *reinterpret_cast<const uint4*>(r);
      else *reinterpret_cast<uint4*>(r) = *d;
      continue;
    }
    i -= dn_pieces;
    {
      const int l = (int)(i & 63), m = l & 15, q = l >> 4;
      const int64_t rest = i >> 6, c = rest % cd, b = rest / cd;
      uint32_t* d = reinterpret_cast<uint32_t*>(blob + off.dn_s + i * 4);
      uint32_t word = to_tiled ? 0u : *d;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        uint8_t* r = (uint8_t*)ref.w2_scale + (64 * b + 16 * t + m) * (I / 32) + 4 * c + q;
        if (to_tiled) word |= (uint32_t)*r << (8 * t);
        else *r = (uint8_t)(word >> (8 * t));
      }
      if (to_tiled) *d = word;
    }
  }
}

// Ordered combine (aggregation_probe.cu:4-25): per token, FP32 sum from +0 of its expert rows in
// ascending expert ID, the shared row last, one BF16 rounding. grid (H / 512, T) of 64 threads, 8
// hidden positions per thread; every row's load is issued before the first add (one memory round trip).
constexpr int kCombineThreads = 64;

__global__ __launch_bounds__(kCombineThreads) void combine_kernel(const Plan* __restrict__ plan,
                                                                  const uint16_t* __restrict__ rows, int H, int k,
                                                                  int has_shared, uint16_t* __restrict__ y) {
  const int t = blockIdx.y;
  const int h = (blockIdx.x * kCombineThreads + threadIdx.x) * 8;
  if (t >= plan->tokens || h >= H) return;
  const int n = k + has_shared;
  uint4 v[kMaxTopK + 1];
#pragma unroll
  for (int i = 0; i < kMaxTopK + 1; ++i)
    if (i < n) v[i] = *reinterpret_cast<const uint4*>(rows + (size_t)plan->tok_rows[t][i] * H + h);
  float acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = 0.f;
#pragma unroll
  for (int i = 0; i < kMaxTopK + 1; ++i) {
    if (i < n) {
      const uint32_t w[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc[2 * j] = acc[2 * j] + mx::bf16_value(w[j] & 0xFFFFu);
        acc[2 * j + 1] = acc[2 * j + 1] + mx::bf16_value(w[j] >> 16);
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

// MoEAccumulator kernels (aggregation_probe.cu:4-25), one element per thread.
__global__ void acc_zero_kernel(float* sum, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) sum[i] = 0.f;
}
__global__ void acc_add_rows_kernel(float* sum, const uint16_t* vals, const int32_t* rows, int nrows, int width) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)nrows * width) return;
  const int64_t target = (int64_t)rows[i / width] * width + i % width;
  sum[target] = sum[target] + mx::bf16_value(vals[i]);
}
__global__ void acc_add_kernel(float* sum, const uint16_t* vals, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) sum[i] = sum[i] + mx::bf16_value(vals[i]);
}
__global__ void acc_finish_kernel(const float* sum, uint16_t* out, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = (uint16_t)mx::bf16_bits(sum[i]);
}

__global__ void set_expert_kernel(const uint8_t** slot, const uint8_t* value) { *slot = value; }

unsigned blocks_for(int64_t n, int threads) { return (unsigned)((n + threads - 1) / threads); }

bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

int check_expert_ptrs(const mx_expert_ptrs& w, const char* who) {
  const void* ws[3] = {w.w1_weight, w.w3_weight, w.w2_weight};
  const void* ss[3] = {w.w1_scale, w.w3_scale, w.w2_scale};
  for (int i = 0; i < 3; ++i) {
    MX_REQUIRE(ws[i] && ss[i], "%s: expert tensor pointer is null", who);
    MX_REQUIRE(aligned(ws[i], 16), "%s: packed weights must be 16-byte aligned", who);
    MX_REQUIRE(aligned(ss[i], 4), "%s: scales must be 4-byte aligned", who);
  }
  return MX_OK;
}

}  // namespace

// ------------------------------------------------------------------------------------------------
// Layer object

// SiLU table of a layer: silu_f32 of every BF16 value, then of the clamp limit (0 when unclamped).
__global__ void silu_table_kernel(float* table, float limit) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < mxd::kSiluLimit) table[i] = mxd::silu_f32(mx::bf16_value(i));
  else if (i == mxd::kSiluLimit) table[i] = limit > 0.f ? mxd::silu_f32(limit) : 0.f;
}

struct mx_layer {
  mx_ctx* ctx = nullptr;
  mx_moe_config cfg{};
  const float* router_weight = nullptr;
  const float* bias = nullptr;
  int has_shared = 0;
  const uint8_t** tiles = nullptr;  // device [E + 1]: tiled expert blobs, shared last
  // per-call buffers
  float *logits = nullptr, *scores = nullptr, *selection = nullptr, *weights = nullptr, *raw = nullptr,
        *den = nullptr, *trace = nullptr;
  int32_t *indices = nullptr, *tied = nullptr;
  uint8_t *xq = nullptr, *xs = nullptr, *dq = nullptr, *ds = nullptr;
  uint16_t* xd = nullptr;             // [T][H] BF16: x's codes times their block scales
  uint16_t *w1 = nullptr, *w3 = nullptr, *din = nullptr, *eout = nullptr;
  Plan* plan = nullptr;
  float* silu = nullptr;   // [mxd::kSiluEntries] SiLU table (prefill epilogue)
  uint32_t* route_errors = nullptr;   // routing ids replaced by routed decode / prefill since the last clear
  int max_rows = 0;
  // the most recent decode call (mx_layer_time_stage repeats its stages)
  const uint16_t* last_x = nullptr;
  uint16_t* last_y = nullptr;
  int last_T = 0;
  bool last_diag = false;
  bool last_plan_in_gateup = false;   // the last decode call folded its routing into gate/up (one token)
  std::vector<std::pair<void*, uint64_t>> allocs;
  // profiling: events bracket each kernel of a call; a ring of kProfRing calls is recorded without
  // host synchronisation and folded into the totals when full or when the profile is read.
  static constexpr int kProfRing = 64;
  bool profile = false;
  std::vector<hipEvent_t> ev;   // kProfRing * 5
  int pending = 0;
  double stage_ms[4] = {0, 0, 0, 0};
  int profiled_calls = 0;
};

namespace {

int layer_alloc(mx_layer* L, uint64_t bytes, void** out) {
  void* p = nullptr;
  MX_HIP(hipMalloc(&p, bytes));
  L->allocs.emplace_back(p, bytes);
  *out = p;
  return MX_OK;
}

template <typename T>
int layer_alloc_t(mx_layer* L, uint64_t count, T** out) {
  void* p = nullptr;
  if (int s = layer_alloc(L, count * sizeof(T), &p)) return s;
  *out = (T*)p;
  return MX_OK;
}

void layer_release(mx_layer* L) {
  for (auto& a : L->allocs) (void)hipFree(a.first);
  L->allocs.clear();
  for (auto& e : L->ev)
    if (e) (void)hipEventDestroy(e);
  L->ev.clear();
}

int profile_flush(mx_layer* L) {
  if (!L->pending) return MX_OK;
  MX_HIP(hipEventSynchronize(L->ev[(L->pending - 1) * 5 + 4]));
  for (int c = 0; c < L->pending; ++c)
    for (int i = 0; i < 4; ++i) {
      float ms = 0.f;
      MX_HIP(hipEventElapsedTime(&ms, L->ev[c * 5 + i], L->ev[c * 5 + i + 1]));
      L->stage_ms[i] += ms;
    }
  L->profiled_calls += L->pending;
  L->pending = 0;
  return MX_OK;
}

int validate_config(const mx_moe_config* c) {
  MX_REQUIRE(c != nullptr, "mx_layer_create: null config");
  MX_REQUIRE(c->hidden > 0 && c->hidden % 128 == 0 && c->hidden <= kRouterKIter * 1024,
             "hidden size must be a positive multiple of 128, at most %d", kRouterKIter * 1024);
  MX_REQUIRE(c->intermediate > 0 && c->intermediate % 128 == 0,
             "intermediate size must be a positive multiple of 128");
  MX_REQUIRE(c->experts >= 1 && c->experts <= kMaxExperts, "experts must be in [1, %d]", kMaxExperts);
  MX_REQUIRE(c->top_k >= 1 && c->top_k <= kMaxTopK && c->top_k <= c->experts, "top_k must be in [1, min(32, E)]");
  MX_REQUIRE(c->score_func == MX_SCORE_SIGMOID || c->score_func == MX_SCORE_SQRTSOFTPLUS, "unknown score function");
  MX_REQUIRE(std::isfinite(c->route_scale), "route scale must be finite");
  MX_REQUIRE(std::isfinite(c->swiglu_limit) && c->swiglu_limit >= 0.f, "Invalid SwiGLU limit");
  MX_REQUIRE(c->shared_format == -1 || c->shared_format == MX_FMT_MXFP4,
             "shared expert format must be none or MXFP4 in the decode layer");
  MX_REQUIRE(c->max_tokens >= 1 && c->max_tokens <= kMaxTokens, "max_tokens must be in [1, %d]", kMaxTokens);
  return MX_OK;
}

}  // namespace

namespace mxi {

LayerView layer_view(mx_layer* L) {
  LayerView v{};
  if (!L) return v;
  v.ctx = L->ctx;
  v.cfg = L->cfg;
  v.router_weight = L->router_weight;
  v.bias = L->bias;
  v.tiles = L->tiles;
  v.has_shared = L->has_shared;
  v.silu = L->silu;
  v.route_errors = L->route_errors;
  return v;
}

namespace {
constexpr int kNoallocDevices = 64;
std::mutex g_noalloc_lock;
uint8_t* g_noalloc_ptr[kNoallocDevices] = {};   // scratch's device address on each GPU (null until set up)
}  // namespace

int noalloc_scratch_init(int device) {
  MX_REQUIRE(device >= 0 && device < kNoallocDevices, "device %d outside the %d the library supports", device,
             kNoallocDevices);
  std::lock_guard<std::mutex> guard(g_noalloc_lock);
  if (g_noalloc_ptr[device]) return MX_OK;
  // with `device` current: each GPU holds its own copy of the array at its own address; the host-side name is
  // only a stand-in, so every later use goes through this pointer
  void* p = nullptr;
  MX_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(::scratch)));   // the array, not mxi::scratch
  MX_REQUIRE(p != nullptr && ((uintptr_t)p & 255) == 0, "device scratch is not 256-byte aligned");
  g_noalloc_ptr[device] = (uint8_t*)p;
  return MX_OK;
}

int noalloc_scratch(int device, uint8_t** out) {
  MX_REQUIRE(device >= 0 && device < kNoallocDevices, "device %d outside the %d the library supports", device,
             kNoallocDevices);
  std::lock_guard<std::mutex> guard(g_noalloc_lock);
  if (!g_noalloc_ptr[device]) return fail(MX_ERR_STATE, "device scratch of device %d was not set up", device);
  *out = g_noalloc_ptr[device];
  return MX_OK;
}

}  // namespace mxi

namespace {

// One stage of a decode call on the arguments recorded in L->last_*.
int launch_stage(mx_layer* L, int stage, hipStream_t st) {
  const mx_moe_config& c = L->cfg;
  const int T = L->last_T;
  if (stage == MX_STAGE_ROUTER) {
    RouterArgs r{};
    r.W = L->router_weight;
    r.bias = L->bias;
    r.x = L->last_x;
    r.T = T;
    r.H = c.hidden;
    r.E = c.experts;
    r.k = c.top_k;
    r.score_func = c.score_func;
    r.route_scale = c.route_scale;
    r.logits = L->logits;
    r.scores = L->scores;
    r.selection = L->selection;
    r.xq = L->xq;
    r.xs = L->xs;
    r.xd = L->xd;
    hipLaunchKernelGGL(router_kernel, dim3(c.experts, 1), dim3(256), 0, st, r);
    MX_LAUNCH_CHECK("router_kernel");
    return MX_OK;
  }
  if (stage == MX_STAGE_ROUTE_PLAN) {
    if (L->last_plan_in_gateup) return MX_OK;   // selected inside the gate/up launch
    hipLaunchKernelGGL(route_plan_kernel, dim3(1), dim3(64 * T), 0, st, (const float*)L->selection,
                       (const float*)L->scores, T, c.experts, c.top_k, c.route_scale,
                       TopkOut{L->indices, L->weights, L->raw, L->den, L->tied}, L->plan, L->has_shared);
    MX_LAUNCH_CHECK("route_plan_kernel");
    return MX_OK;
  }
  if (stage == MX_STAGE_COMBINE) {
    hipLaunchKernelGGL(combine_kernel, dim3((c.hidden / 8 + kCombineThreads - 1) / kCombineThreads, T),
                       dim3(kCombineThreads), 0, st, (const Plan*)L->plan, (const uint16_t*)L->eout, c.hidden,
                       c.top_k, L->has_shared, L->last_y);
    MX_LAUNCH_CHECK("combine_kernel");
    return MX_OK;
  }
  ExpertArgs a{};
  a.tiles = L->tiles;
  a.plan = L->plan;
  a.H = c.hidden;
  a.I = c.intermediate;
  a.limit = c.swiglu_limit;
  a.xq = L->xq;
  a.xs = L->xs;
  a.xd = L->xd;
  a.dq = L->dq;
  a.ds = L->ds;
  a.out = L->eout;
  if (L->last_diag) {
    a.w1 = L->w1;
    a.w3 = L->w3;
    a.din = L->din;
    a.trace = L->trace;
  }
  // grid rows beyond the plan's slot count exit at once
  const int routed = std::min(c.experts, T * c.top_k);
  const int slots = routed + L->has_shared;
  if (stage == MX_STAGE_GATEUP) {
    a.tokens = T;
    if (L->last_plan_in_gateup) {
      a.selection = (const float*)L->selection;
      a.scores = (const float*)L->scores;
      a.topk = TopkOut{L->indices, L->weights, L->raw, L->den, L->tied};
      a.plan_out = L->plan;
      a.E = c.experts;
      a.k = c.top_k;
      a.has_shared = L->has_shared;
      a.route_scale = c.route_scale;
      hipLaunchKernelGGL(gateup_kernel<true>, dim3(c.intermediate / 32, slots), dim3(256), kXStages * xstage_bytes(T),
                         st, a);
    } else {
      hipLaunchKernelGGL(gateup_kernel<false>, dim3(c.intermediate / 32, slots), dim3(256), kXStages * xstage_bytes(T),
                         st, a);
    }
    MX_LAUNCH_CHECK("gateup_kernel");
  } else {
    hipLaunchKernelGGL(down_kernel<true>, dim3(c.hidden / 64, slots), dim3(256), 0, st, a);
    MX_LAUNCH_CHECK("down_kernel");
  }
  return MX_OK;
}

}  // namespace

using namespace mxi;

extern "C" {

int mx_layer_create(mx_ctx* ctx, const mx_moe_config* cfg, const float* router_weight, const float* bias,
                    const void* const* experts, const void* shared, mx_layer** out) {
  if (int s = use(ctx)) return s;
  if (int s = validate_config(cfg)) return s;
  MX_REQUIRE(out != nullptr, "mx_layer_create: null output");
  MX_REQUIRE(router_weight != nullptr && aligned(router_weight, 16), "router weight must be a 16-byte aligned pointer");
  MX_REQUIRE(experts != nullptr, "expert pointer table is null");
  for (int e = 0; e < cfg->experts; ++e)
    MX_REQUIRE(experts[e] && aligned(experts[e], 256), "expert %d: tiled expert must be a 256-byte aligned pointer", e);
  MX_REQUIRE((cfg->shared_format == -1) == (shared == nullptr), "shared expert pointer and format disagree");
  MX_REQUIRE(!shared || aligned(shared, 256), "shared expert: tiled expert must be 256-byte aligned");
  mx_layer* L = new mx_layer();
  L->ctx = ctx;
  L->cfg = *cfg;
  L->router_weight = router_weight;
  L->bias = bias;
  L->has_shared = shared != nullptr;
  const int T = cfg->max_tokens, E = cfg->experts, k = cfg->top_k, H = cfg->hidden, I = cfg->intermediate;
  L->max_rows = T * k + T;
  int s = MX_OK;
  auto fail_out = [&](int st) {
    layer_release(L);
    delete L;
    return st;
  };
  if ((s = layer_alloc_t(L, (uint64_t)E + 1, &L->tiles))) return fail_out(s);
  if ((s = layer_alloc_t(L, (uint64_t)T * E, &L->logits))) return fail_out(s);
  if ((s = layer_alloc_t(L, (uint64_t)T * E, &L->scores))) return fail_out(s);
  if ((s = layer_alloc_t(L, (uint64_t)T * E, &L->selection))) return fail_out(s);
  if ((s = layer_alloc_t(L, (uint64_t)T * k, &L->indices))) return fail_out(s);
  if ((s = layer_alloc_t(L, (uint64_t)T * k, &L->weights))) return fail_out(s);
  if ((s = layer_alloc_t(L, (uint64_t)T * k, &L->raw))) return fail_out(s);
  if ((s = layer_alloc_t(L, (uint64_t)T, &L->den))) return fail_out(s);
  if ((s = layer_alloc_t(L, (uint64_t)T, &L->tied))) return fail_out(s);
  if ((s = layer_alloc_t(L, (uint64_t)T * H, &L->xq))) return fail_out(s);
  if ((s = layer_alloc_t(L, (uint64_t)T * H / 32 + 16, &L->xs))) return fail_out(s);
  if ((s = layer_alloc_t(L, (uint64_t)T * H, &L->xd))) return fail_out(s);
  if ((s = layer_alloc_t(L, 1, &L->plan))) return fail_out(s);
  const uint64_t R = (uint64_t)L->max_rows;
  if ((s = layer_alloc_t(L, R * I, &L->w1))) return fail_out(s);
  if ((s = layer_alloc_t(L, R * I, &L->w3))) return fail_out(s);
  if ((s = layer_alloc_t(L, R * I, &L->din))) return fail_out(s);
  if ((s = layer_alloc_t(L, R * I * 5, &L->trace))) return fail_out(s);
  if ((s = layer_alloc_t(L, R * I, &L->dq))) return fail_out(s);
  if ((s = layer_alloc_t(L, R * I / 32 + 16, &L->ds))) return fail_out(s);
  if ((s = layer_alloc_t(L, R * H, &L->eout))) return fail_out(s);
  if ((s = layer_alloc_t(L, (uint64_t)mxd::kSiluEntries, &L->silu))) return fail_out(s);
  if ((s = layer_alloc_t(L, 64, &L->route_errors))) return fail_out(s);
  hipLaunchKernelGGL(silu_table_kernel, dim3((mxd::kSiluEntries + 255) / 256), dim3(256), 0, nullptr, L->silu,
                     cfg->swiglu_limit);
  if (hipError_t e = hipGetLastError(); e != hipSuccess) return fail_out(hip_fail(e, "mx_layer_create: SiLU table"));
  std::vector<const void*> host(E + 1);
  for (int e = 0; e < E; ++e) host[e] = experts[e];
  host[E] = shared ? shared : experts[0];
  hipError_t err = hipMemcpy(L->tiles, host.data(), sizeof(void*) * (E + 1), hipMemcpyHostToDevice);
  if (err == hipSuccess) err = hipMemset(L->plan, 0, sizeof(Plan));
  if (err == hipSuccess) err = hipMemset(L->route_errors, 0, 64 * sizeof(uint32_t));
  if (err == hipSuccess) err = hipDeviceSynchronize();
  if (err != hipSuccess) return fail_out(hip_fail(err, "mx_layer_create: table upload"));
  *out = L;
  return MX_OK;
}

int mx_layer_destroy(mx_layer* L) {
  if (!L) return MX_OK;
  if (int s = use(L->ctx)) return s;
  (void)hipDeviceSynchronize();
  layer_release(L);
  delete L;
  return MX_OK;
}

int mx_layer_set_expert(mx_layer* L, int32_t expert, const void* tiled, void* stream) {
  MX_REQUIRE(L != nullptr, "layer is closed");
  if (int s = use(L->ctx)) return s;
  MX_REQUIRE(expert >= 0 && expert < L->cfg.experts, "expert %d outside the layer", expert);
  MX_REQUIRE(tiled != nullptr && aligned(tiled, 256), "tiled expert must be a 256-byte aligned pointer");
  // A kernel on the caller's stream writes the table entry, ordered after a slot fill on that stream.
  hipLaunchKernelGGL(set_expert_kernel, dim3(1), dim3(1), 0, as_stream(stream), L->tiles + expert,
                     (const uint8_t*)tiled);
  MX_LAUNCH_CHECK("set_expert");
  return MX_OK;
}

int mx_layer_buffer(mx_layer* L, int32_t which, void** dptr, uint64_t* bytes) {
  MX_REQUIRE(L != nullptr && dptr != nullptr, "mx_layer_buffer: bad arguments");
  const uint64_t T = L->cfg.max_tokens, E = L->cfg.experts, k = L->cfg.top_k, H = L->cfg.hidden,
                 I = L->cfg.intermediate, R = L->max_rows;
  void* p = nullptr;
  uint64_t b = 0;
  switch (which) {
    case MX_BUF_LOGITS: p = L->logits; b = T * E * 4; break;
    case MX_BUF_SCORES: p = L->scores; b = T * E * 4; break;
    case MX_BUF_SELECTION: p = L->selection; b = T * E * 4; break;
    case MX_BUF_INDICES: p = L->indices; b = T * k * 4; break;
    case MX_BUF_WEIGHTS: p = L->weights; b = T * k * 4; break;
    case MX_BUF_XQ: p = L->xq; b = T * H; break;
    case MX_BUF_XS: p = L->xs; b = T * H / 32; break;
    case MX_BUF_PLAN: p = L->plan; b = sizeof(Plan); break;
    case MX_BUF_W1: p = L->w1; b = R * I * 2; break;
    case MX_BUF_W3: p = L->w3; b = R * I * 2; break;
    case MX_BUF_DOWN_INPUT: p = L->din; b = R * I * 2; break;
    case MX_BUF_DOWN_Q: p = L->dq; b = R * I; break;
    case MX_BUF_DOWN_S: p = L->ds; b = R * I / 32; break;
    case MX_BUF_EXPERT_OUT: p = L->eout; b = R * H * 2; break;
    case MX_BUF_TRACE: p = L->trace; b = R * I * 5 * 4; break;
    case MX_BUF_RAW: p = L->raw; b = T * k * 4; break;
    case MX_BUF_DENOMINATOR: p = L->den; b = T * 4; break;
    case MX_BUF_TIED: p = L->tied; b = T * 4; break;
    default: return fail(MX_ERR_INVALID, "mx_layer_buffer: unknown buffer %d", which);
  }
  *dptr = p;
  if (bytes) *bytes = b;
  return MX_OK;
}

int mx_layer_profile(mx_layer* L, int32_t enable, float* stage_ms, int32_t* calls) {
  MX_REQUIRE(L != nullptr, "layer is closed");
  if (int s = use(L->ctx)) return s;
  if (int s = profile_flush(L)) return s;
  if (stage_ms)
    for (int i = 0; i < 4; ++i) stage_ms[i] = L->profiled_calls ? (float)(L->stage_ms[i] / L->profiled_calls) : 0.f;
  if (calls) *calls = L->profiled_calls;
  if (enable && L->ev.empty()) {
    L->ev.assign(mx_layer::kProfRing * 5, nullptr);
    for (auto& e : L->ev) MX_HIP(hipEventCreate(&e));
  }
  if (enable) {
    for (auto& v : L->stage_ms) v = 0;
    L->profiled_calls = 0;
  }
  L->profile = enable != 0;
  return MX_OK;
}

int mx_moe_decode(mx_layer* L, const uint16_t* x, int32_t T, uint16_t* y, int32_t diagnostics, void* stream) {
  MX_REQUIRE(L != nullptr, "layer is closed");
  if (int s = use(L->ctx)) return s;
  const mx_moe_config& c = L->cfg;
  MX_REQUIRE(T >= 0 && T <= c.max_tokens, "token count %d outside [0, %d]", T, c.max_tokens);
  if (T == 0) return MX_OK;
  MX_REQUIRE(x && y && aligned(x, 16) && aligned(y, 16), "x and y must be 16-byte aligned device pointers");
  hipStream_t st = as_stream(stream);
  const bool prof = L->profile;
  hipEvent_t* ev = nullptr;
  if (prof) {
    if (L->pending == mx_layer::kProfRing)
      if (int s2 = profile_flush(L)) return s2;
    ev = &L->ev[L->pending * 5];
    MX_HIP(hipEventRecord(ev[0], st));
  }
  L->last_x = x;
  L->last_y = y;
  L->last_T = T;
  L->last_diag = diagnostics != 0;
  // one token: the gate/up launch selects the experts itself (no route_plan launch)
  L->last_plan_in_gateup = T == 1;
  // event i + 1 closes profiled stage i: router (GEMV + top-k/plan), gate/up, down, combine
  static const int kEventAfter[5] = {-1, 1, 2, 3, 4};
  for (int stage = 0; stage < 5; ++stage) {
    if (int s2 = launch_stage(L, stage, st)) return s2;
    if (prof && kEventAfter[stage] > 0) MX_HIP(hipEventRecord(ev[kEventAfter[stage]], st));
  }
  if (prof) ++L->pending;
  return MX_OK;
}

int mx_moe_decode_routed(mx_layer* L, const uint16_t* x, int32_t T, const int32_t* ids, const float* weights,
                         uint16_t* y, void* stream) {
  MX_REQUIRE(L != nullptr, "layer is closed");
  if (int s = use(L->ctx)) return s;
  const mx_moe_config& c = L->cfg;
  MX_REQUIRE(T >= 0 && T <= c.max_tokens, "token count %d outside [0, %d]", T, c.max_tokens);
  if (T == 0) return MX_OK;
  MX_REQUIRE(x && y && ids && weights && aligned(x, 16) && aligned(y, 16),
             "x, y (16-byte aligned), ids and weights must be device pointers");
  hipStream_t st = as_stream(stream);
  if (int s = act_quant32_scaled(L->ctx, x, L->xq, L->xs, L->xd, T, c.hidden, st)) return s;
  hipLaunchKernelGGL(routed_plan_kernel, dim3(1), dim3(64 * T), 0, st, ids, weights, T, c.top_k, c.experts, L->indices,
                     L->weights, L->plan, L->has_shared, L->route_errors);
  MX_LAUNCH_CHECK("routed_plan_kernel");
  L->last_x = x;
  L->last_y = y;
  L->last_T = T;
  L->last_diag = false;
  L->last_plan_in_gateup = false;
  for (int stage = MX_STAGE_GATEUP; stage <= MX_STAGE_COMBINE; ++stage)
    if (int s = launch_stage(L, stage, st)) return s;
  return MX_OK;
}

int mx_layer_route_errors(mx_layer* L, uint32_t* count, int32_t clear, void* stream) {
  MX_REQUIRE(L != nullptr, "layer is closed");
  if (int s = use(L->ctx)) return s;
  MX_REQUIRE(count != nullptr, "mx_layer_route_errors: null output");
  hipStream_t st = as_stream(stream);
  MX_HIP(hipMemcpyAsync(count, L->route_errors, sizeof(uint32_t), hipMemcpyDeviceToHost, st));
  MX_HIP(hipStreamSynchronize(st));
  if (clear) {
    hipLaunchKernelGGL(set_u32_kernel, dim3(1), dim3(1), 0, st, L->route_errors, 0u);
    MX_LAUNCH_CHECK("set_u32_kernel");
  }
  return MX_OK;
}

int mx_layer_set_experts(mx_layer* L, int32_t n, const int32_t* experts, const void* const* tiled, void* stream) {
  MX_REQUIRE(L != nullptr, "layer is closed");
  if (int s = use(L->ctx)) return s;
  MX_REQUIRE(n >= 0 && (n == 0 || (experts && tiled)), "mx_layer_set_experts: bad arguments");
  for (int i = 0; i < n; ++i) {
    MX_REQUIRE(experts[i] >= 0 && experts[i] < L->cfg.experts, "expert %d outside the layer", experts[i]);
    MX_REQUIRE(tiled[i] != nullptr && aligned(tiled[i], 256), "tiled expert must be a 256-byte aligned pointer");
  }
  for (int base = 0; base < n; base += MX_EXPERT_BATCH) {
    mx_expert_batch b{};
    const int m = std::min(MX_EXPERT_BATCH, n - base);
    for (int i = 0; i < m; ++i) {
      b.expert[i] = experts[base + i];
      b.tiled[i] = tiled[base + i];
    }
    hipLaunchKernelGGL(set_experts_kernel, dim3(1), dim3(64), 0, as_stream(stream), L->tiles, m, b);
    MX_LAUNCH_CHECK("set_experts_kernel");
  }
  return MX_OK;
}

int mx_layer_time_stage(mx_layer* L, int32_t stage, int32_t iters, float* us_per_launch, void* stream) {
  MX_REQUIRE(L != nullptr, "layer is closed");
  if (int s = use(L->ctx)) return s;
  MX_REQUIRE(L->last_T > 0, "mx_layer_time_stage: no decode call to repeat yet");
  MX_REQUIRE(stage >= MX_STAGE_ROUTER && stage <= MX_STAGE_COMBINE, "unknown stage %d", stage);
  MX_REQUIRE(iters >= 1 && us_per_launch != nullptr, "mx_layer_time_stage: need iters >= 1 and an output");
  hipStream_t st = as_stream(stream);
  hipEvent_t a = nullptr, b = nullptr;
  MX_HIP(hipEventCreate(&a));
  hipError_t err = hipEventCreate(&b);
  int status = MX_OK;
  if (err == hipSuccess) err = hipEventRecord(a, st);
  for (int i = 0; err == hipSuccess && status == MX_OK && i < iters; ++i) status = launch_stage(L, stage, st);
  if (err == hipSuccess && status == MX_OK) err = hipEventRecord(b, st);
  if (err == hipSuccess && status == MX_OK) err = hipEventSynchronize(b);
  float ms = 0.f;
  if (err == hipSuccess && status == MX_OK) err = hipEventElapsedTime(&ms, a, b);
  (void)hipEventDestroy(a);
  if (b) (void)hipEventDestroy(b);
  if (status != MX_OK) return status;
  if (err != hipSuccess) return hip_fail(err, "mx_layer_time_stage");
  *us_per_launch = ms * 1000.f / (float)iters;
  return MX_OK;
}

// ------------------------------------------------------------------------------------------------
// Single expert, T tokens (ExpertExecutor.execute / ResidentSharedExpert.forward)

// Bytes of device scratch one tiled expert call needs: plan | one-entry expert table | xq | xs | dq | ds | xd.
static uint64_t tiled_call_scratch_bytes(int32_t H, int32_t I, int32_t T) {
  const uint64_t plan_b = (sizeof(Plan) + 255) & ~255ull, table_b = 256;
  const uint64_t xq_b = ((uint64_t)T * H + 255) & ~255ull, xs_b = ((uint64_t)T * H / 32 + 255) & ~255ull;
  const uint64_t dq_b = ((uint64_t)T * I + 255) & ~255ull, ds_b = ((uint64_t)T * I / 32 + 255) & ~255ull;
  return plan_b + table_b + xq_b + xs_b + dq_b + ds_b + 2 * xq_b;
}

static int check_tiled_call(const char* what, const void* tiled, int32_t H, int32_t I, const uint16_t* x, int32_t T,
                            float limit, uint16_t* y) {
  MX_REQUIRE(tiled != nullptr && aligned(tiled, 256), "%s: 256-byte aligned tiled expert required", what);
  MX_REQUIRE(H > 0 && H % 128 == 0 && I > 0 && I % 128 == 0, "expert shapes must be positive multiples of 128");
  MX_REQUIRE(T >= 0 && T <= kMaxTokens, "token count %d outside [0, %d]", T, kMaxTokens);
  MX_REQUIRE(std::isfinite(limit) && limit >= 0.f, "Invalid SwiGLU limit");
  MX_REQUIRE(T == 0 || (x && y && aligned(x, 16) && aligned(y, 16)), "x and y must be 16-byte aligned device pointers");
  return MX_OK;
}

// The tiled expert call on a given scratch region of tiled_call_scratch_bytes(H, I, T) bytes, 256-byte
// aligned (the context's scratch, or the allocation-free entry point's fixed array).
static int tiled_call_on(mx_ctx* ctx, uint8_t* b8, const void* tiled, int32_t H, int32_t I, const uint16_t* x,
                         int32_t T, float limit, const float* route_w, uint16_t* y, const mx_expert_stages* stages,
                         void* stream) {
  hipStream_t st = as_stream(stream);
  const uint64_t plan_b = (sizeof(Plan) + 255) & ~255ull, table_b = 256;
  const uint64_t xq_b = ((uint64_t)T * H + 255) & ~255ull, xs_b = ((uint64_t)T * H / 32 + 255) & ~255ull;
  const uint64_t dq_b = ((uint64_t)T * I + 255) & ~255ull, ds_b = ((uint64_t)T * I / 32 + 255) & ~255ull;
  Plan* plan = (Plan*)b8;
  const uint8_t** table = (const uint8_t**)(b8 + plan_b);
  uint8_t* cur = b8 + plan_b + table_b;
  uint16_t* xd = (uint16_t*)(cur + xq_b + xs_b + dq_b + ds_b);
  uint8_t* xq = (stages && stages->q) ? stages->q : cur;
  uint8_t* xs = (stages && stages->s) ? stages->s : cur + xq_b;
  uint8_t* dq = (stages && stages->down_q) ? stages->down_q : cur + xq_b + xs_b;
  uint8_t* ds = (stages && stages->down_s) ? stages->down_s : cur + xq_b + xs_b + dq_b;
  MX_REQUIRE(aligned(xq, 16) && aligned(dq, 16) && aligned(xs, 4) && aligned(ds, 4),
             "stage buffers q/down_q must be 16-byte and s/down_s 4-byte aligned");
  hipLaunchKernelGGL(set_expert_kernel, dim3(1), dim3(1), 0, st, table, (const uint8_t*)tiled);
  MX_LAUNCH_CHECK("set_expert_kernel");
  hipLaunchKernelGGL(single_plan_kernel, dim3(1), dim3(64), 0, st, plan, T, route_w);
  MX_LAUNCH_CHECK("single_plan_kernel");
  if (int s = act_quant32_scaled(ctx, x, xq, xs, xd, T, H, st)) return s;
  ExpertArgs a{};
  a.tiles = table;
  a.xd = xd;
  a.plan = plan;
  a.H = H;
  a.I = I;
  a.limit = limit;
  a.xq = xq;
  a.xs = xs;
  a.dq = dq;
  a.ds = ds;
  a.out = y;
  if (stages) {
    a.w1 = stages->w1;
    a.w3 = stages->w3;
    a.din = stages->down_input;
    a.trace = stages->trace;
  }
  a.tokens = T;
  hipLaunchKernelGGL(gateup_kernel<false>, dim3(I / 32, 1), dim3(256), kXStages * xstage_bytes(T), st, a);
  MX_LAUNCH_CHECK("gateup_kernel");
  hipLaunchKernelGGL(down_kernel<true>, dim3(H / 64, 1), dim3(256), 0, st, a);
  MX_LAUNCH_CHECK("down_kernel");
  return MX_OK;
}

int mx_expert_forward(mx_ctx* ctx, const mx_expert_ptrs* w, int32_t format, int32_t H, int32_t I,
                      const uint16_t* x, int32_t T, float limit, const float* route_w, uint16_t* y,
                      const mx_expert_stages* stages, void* stream) {
  if (int s = use(ctx)) return s;
  MX_REQUIRE(w != nullptr, "mx_expert_forward: null expert pointers");
  MX_REQUIRE(format == MX_FMT_MXFP4, "mx_expert_forward: only the MXFP4 format runs on this path");
  MX_REQUIRE(H > 0 && H % 128 == 0 && I > 0 && I % 128 == 0, "expert shapes must be positive multiples of 128");
  MX_REQUIRE(T >= 0 && T <= kMaxTokens, "token count %d outside [0, %d]", T, kMaxTokens);
  MX_REQUIRE(std::isfinite(limit) && limit >= 0.f, "Invalid SwiGLU limit");
  if (int s = check_expert_ptrs(*w, "mx_expert_forward")) return s;
  if (T == 0) return MX_OK;
  MX_REQUIRE(x && y && aligned(x, 16) && aligned(y, 16), "x and y must be 16-byte aligned device pointers");
  // the reference layout is tiled into scratch (one pass over the expert's bytes) and the tiled call runs on it
  const uint64_t blob_b = (tiled_offsets(H, I).total + 255) & ~255ull;
  void* base = nullptr;
  if (int s = mxi::scratch(ctx, blob_b + tiled_call_scratch_bytes(H, I, T), &base)) return s;
  uint8_t* b8 = (uint8_t*)base;
  hipLaunchKernelGGL(tile_expert_kernel, dim3(2048), dim3(256), 0, as_stream(stream), *w, b8, H, I, 1);
  MX_LAUNCH_CHECK("tile_expert_kernel");
  return tiled_call_on(ctx, b8 + blob_b, b8, H, I, x, T, limit, route_w, y, stages, stream);
}

int mx_expert_forward_tiled(mx_ctx* ctx, const void* tiled, int32_t H, int32_t I, const uint16_t* x, int32_t T,
                            float limit, const float* route_w, uint16_t* y, const mx_expert_stages* stages,
                            void* stream) {
  if (int s = use(ctx)) return s;
  if (int s = check_tiled_call("mx_expert_forward_tiled", tiled, H, I, x, T, limit, y)) return s;
  if (T == 0) return MX_OK;
  void* base = nullptr;
  if (int s = mxi::scratch(ctx, tiled_call_scratch_bytes(H, I, T), &base)) return s;
  return tiled_call_on(ctx, (uint8_t*)base, tiled, H, I, x, T, limit, route_w, y, stages, stream);
}

int mx_expert_forward_tiled_noalloc(mx_ctx* ctx, const void* tiled, int32_t H, int32_t I, const uint16_t* x,
                                    int32_t T, float limit, const float* route_w, uint16_t* y,
                                    const mx_expert_stages* stages, void* stream) {
  if (int s = use(ctx)) return s;
  if (int s = check_tiled_call("mx_expert_forward_tiled_noalloc", tiled, H, I, x, T, limit, y)) return s;
  const uint64_t need = tiled_call_scratch_bytes(H, I, T);
  MX_REQUIRE(need <= MX_NOALLOC_SCRATCH_BYTES,
             "mx_expert_forward_tiled_noalloc: %d tokens of a %d x %d expert need %llu bytes of scratch, more than "
             "the fixed %llu (use mx_expert_forward_tiled)",
             T, H, I, (unsigned long long)need, (unsigned long long)MX_NOALLOC_SCRATCH_BYTES);
  if (T == 0) return MX_OK;
  uint8_t* base = nullptr;
  if (int s = noalloc_scratch(ctx->device, &base)) return s;
  return tiled_call_on(ctx, base, tiled, H, I, x, T, limit, route_w, y, stages, stream);
}

int mx_gemv_mxfp4(mx_ctx* ctx, const uint8_t* q, const uint8_t* sa, const uint8_t* w, const uint8_t* sw,
                  uint16_t* y, int32_t T, int32_t N, int32_t K, void* stream) {
  if (int s = use(ctx)) return s;
  MX_REQUIRE(T >= 0 && T <= kMaxTokens, "token count %d outside [0, %d]", T, kMaxTokens);
  MX_REQUIRE(N > 0 && N % 64 == 0 && K > 0 && K % 128 == 0, "mx_gemv_mxfp4 needs N %% 64 == 0 and K %% 128 == 0");
  if (!T) return MX_OK;
  MX_REQUIRE(q && sa && w && sw && y, "mx_gemv_mxfp4: null pointer");
  MX_REQUIRE(aligned(q, 16) && aligned(w, 16) && aligned(sa, 4) && aligned(sw, 4) && aligned(y, 8),
             "mx_gemv_mxfp4: q/w 16-byte, scales 4-byte and y 8-byte alignment required");
  hipStream_t st = as_stream(stream);
  void* base = nullptr;
  if (int s = mxi::scratch(ctx, sizeof(Plan), &base)) return s;
  Plan* plan = (Plan*)base;
  hipLaunchKernelGGL(single_plan_kernel, dim3(1), dim3(64), 0, st, plan, T, (const float*)nullptr);
  MX_LAUNCH_CHECK("single_plan_kernel");
  ExpertArgs a{};
  a.single.w2_weight = w;
  a.single.w2_scale = sw;
  a.plan = plan;
  a.H = N;
  a.I = K;
  a.dq = const_cast<uint8_t*>(q);
  a.ds = const_cast<uint8_t*>(sa);
  a.out = y;
  hipLaunchKernelGGL(down_kernel<false>, dim3(N / 64, 1), dim3(256), 0, st, a);
  MX_LAUNCH_CHECK("down_kernel");
  return MX_OK;
}

// ------------------------------------------------------------------------------------------------
// Tiled expert layout

uint64_t mx_tiled_expert_bytes(int32_t H, int32_t I) {
  if (H <= 0 || I <= 0 || H % 128 || I % 128) return 0;
  return tiled_offsets(H, I).total;
}

static int tile_common(mx_ctx* ctx, const mx_expert_ptrs* ref, const void* blob, int32_t H, int32_t I,
                       const char* who) {
  if (int s = use(ctx)) return s;
  MX_REQUIRE(ref != nullptr && blob != nullptr, "%s: null pointer", who);
  MX_REQUIRE(H > 0 && H % 128 == 0 && I > 0 && I % 128 == 0, "%s: shapes must be positive multiples of 128", who);
  MX_REQUIRE(aligned(blob, 256), "%s: the tiled expert must be 256-byte aligned", who);
  return check_expert_ptrs(*ref, who);
}

int mx_tile_expert(mx_ctx* ctx, const mx_expert_ptrs* ref, int32_t H, int32_t I, void* tiled, void* stream) {
  if (int s = tile_common(ctx, ref, tiled, H, I, "mx_tile_expert")) return s;
  hipLaunchKernelGGL(tile_expert_kernel, dim3(2048), dim3(256), 0, as_stream(stream), *ref, (uint8_t*)tiled, H, I, 1);
  MX_LAUNCH_CHECK("tile_expert_kernel");
  return MX_OK;
}

int mx_untile_expert(mx_ctx* ctx, const void* tiled, int32_t H, int32_t I, const mx_expert_ptrs* ref, void* stream) {
  if (int s = tile_common(ctx, ref, tiled, H, I, "mx_untile_expert")) return s;
  hipLaunchKernelGGL(tile_expert_kernel, dim3(2048), dim3(256), 0, as_stream(stream), *ref,
                     (uint8_t*)const_cast<void*>(tiled), H, I, 0);
  MX_LAUNCH_CHECK("tile_expert_kernel");
  return MX_OK;
}

// ------------------------------------------------------------------------------------------------
// Router entry points

static int router_common(mx_ctx* ctx, int T, int E, int k, int score_func, float route_scale,
                         const mx_router_out* out) {
  if (int s = use(ctx)) return s;
  MX_REQUIRE(out && out->indices && out->weights, "router outputs indices and weights are required");
  MX_REQUIRE(T >= 0, "negative token count");
  MX_REQUIRE(E >= 1 && E <= kMaxExperts, "experts must be in [1, %d]", kMaxExperts);
  MX_REQUIRE(k >= 1 && k <= kMaxTopK && k <= E, "top_k must be in [1, min(32, E)]");
  MX_REQUIRE(score_func == MX_SCORE_SIGMOID || score_func == MX_SCORE_SQRTSOFTPLUS, "unknown score function");
  MX_REQUIRE(std::isfinite(route_scale), "route scale must be finite");
  return MX_OK;
}

int mx_router(mx_ctx* ctx, const float* W, const float* bias, const uint16_t* x, int32_t T, int32_t H, int32_t E,
              int32_t k, int32_t score_func, float route_scale, const mx_router_out* out, void* stream) {
  if (int s = router_common(ctx, T, E, k, score_func, route_scale, out)) return s;
  MX_REQUIRE(H > 0 && H % 4 == 0 && H <= kRouterKIter * 1024, "hidden size must be a positive multiple of 4, at most %d",
             kRouterKIter * 1024);
  MX_REQUIRE(out->logits != nullptr, "router logits output is required");
  MX_REQUIRE(W && x && aligned(W, 16) && aligned(x, 8), "W must be 16-byte and x 8-byte aligned");
  if (!T) return MX_OK;
  hipStream_t st = as_stream(stream);
  // scores/selection scratch when the caller does not keep them
  float *scores = out->scores, *selection = out->selection;
  if (!scores || !selection) {
    void* base = nullptr;
    if (int s = mxi::scratch(ctx, (uint64_t)T * E * 8, &base)) return s;
    if (!scores) scores = (float*)base;
    if (!selection) selection = (float*)base + (uint64_t)T * E;
  }
  RouterArgs r{};
  r.W = W;
  r.bias = bias;
  r.x = x;
  r.T = T;
  r.H = H;
  r.E = E;
  r.k = k;
  r.score_func = score_func;
  r.route_scale = route_scale;
  r.logits = out->logits;
  r.scores = scores;
  r.selection = selection;
  hipLaunchKernelGGL(router_kernel, dim3(E, (T + kMaxTokens - 1) / kMaxTokens), dim3(256), 0, st, r);
  MX_LAUNCH_CHECK("router_kernel");
  TopkOut o{out->indices, out->weights, out->raw, out->denominator, out->tied};
  hipLaunchKernelGGL(topk_kernel, dim3((T + 3) / 4), dim3(256), 0, st, (const float*)selection, (const float*)scores,
                     T, E, k, route_scale, o);
  MX_LAUNCH_CHECK("topk_kernel");
  return MX_OK;
}

int mx_gate_project(mx_ctx* ctx, const float* W, const uint16_t* x, int32_t T, int32_t H, int32_t E, float* logits,
                    void* stream) {
  if (int s = use(ctx)) return s;
  MX_REQUIRE(T >= 0 && H > 0 && H % 4 == 0 && H <= kRouterKIter * 1024,
             "hidden size must be a positive multiple of 4, at most %d", kRouterKIter * 1024);
  MX_REQUIRE(E >= 1, "experts must be positive");
  if (!T) return MX_OK;
  MX_REQUIRE(W && x && logits && aligned(W, 16) && aligned(x, 8), "W must be 16-byte and x 8-byte aligned");
  RouterArgs r{};
  r.W = W;
  r.x = x;
  r.T = T;
  r.H = H;
  r.E = E;
  r.logits = logits;
  hipLaunchKernelGGL(router_kernel, dim3(E, (T + kMaxTokens - 1) / kMaxTokens), dim3(256), 0, as_stream(stream), r);
  MX_LAUNCH_CHECK("router_kernel");
  return MX_OK;
}

int mx_router_postprocess(mx_ctx* ctx, const float* logits, const float* bias, int32_t T, int32_t E, int32_t k,
                          int32_t score_func, float route_scale, const mx_router_out* out, void* stream) {
  if (int s = router_common(ctx, T, E, k, score_func, route_scale, out)) return s;
  MX_REQUIRE(logits != nullptr, "logits are required");
  if (!T) return MX_OK;
  hipStream_t st = as_stream(stream);
  float *scores = out->scores, *selection = out->selection;
  if (!scores || !selection) {
    void* base = nullptr;
    if (int s = mxi::scratch(ctx, (uint64_t)T * E * 8, &base)) return s;
    if (!scores) scores = (float*)base;
    if (!selection) selection = (float*)base + (uint64_t)T * E;
  }
  hipLaunchKernelGGL(scores_kernel, dim3(blocks_for((int64_t)T * E, 256)), dim3(256), 0, st, logits, bias, T, E,
                     score_func, scores, selection);
  MX_LAUNCH_CHECK("scores_kernel");
  TopkOut o{out->indices, out->weights, out->raw, out->denominator, out->tied};
  hipLaunchKernelGGL(topk_kernel, dim3((T + 3) / 4), dim3(256), 0, st, (const float*)selection, (const float*)scores,
                     T, E, k, route_scale, o);
  MX_LAUNCH_CHECK("topk_kernel");
  return MX_OK;
}

int mx_router_select(mx_ctx* ctx, const float* scores, const float* selection, int32_t T, int32_t E, int32_t k,
                     float route_scale, const mx_router_out* out, void* stream) {
  if (int s = router_common(ctx, T, E, k, MX_SCORE_SIGMOID, route_scale, out)) return s;
  MX_REQUIRE(scores && selection, "scores and selection are required");
  if (!T) return MX_OK;
  TopkOut o{out->indices, out->weights, out->raw, out->denominator, out->tied};
  hipLaunchKernelGGL(topk_kernel, dim3((T + 3) / 4), dim3(256), 0, as_stream(stream), selection, scores, T, E, k,
                     route_scale, o);
  MX_LAUNCH_CHECK("topk_kernel");
  return MX_OK;
}

// ------------------------------------------------------------------------------------------------
// MoEAccumulator kernels

int mx_acc_zero(mx_ctx* ctx, float* sum, int64_t n, void* stream) {
  if (int s = use(ctx)) return s;
  MX_REQUIRE(n >= 0 && (n == 0 || sum), "mx_acc_zero: bad arguments");
  if (!n) return MX_OK;
  hipLaunchKernelGGL(acc_zero_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, as_stream(stream), sum, n);
  MX_LAUNCH_CHECK("acc_zero_kernel");
  return MX_OK;
}

int mx_acc_add_rows(mx_ctx* ctx, float* sum, const uint16_t* vals, const int32_t* rows, int32_t nrows, int32_t width,
                    void* stream) {
  if (int s = use(ctx)) return s;
  MX_REQUIRE(nrows >= 0 && width > 0, "mx_acc_add_rows: bad shape");
  if (!nrows) return MX_OK;
  MX_REQUIRE(sum && vals && rows, "mx_acc_add_rows: null pointer");
  hipLaunchKernelGGL(acc_add_rows_kernel, dim3(blocks_for((int64_t)nrows * width, 256)), dim3(256), 0,
                     as_stream(stream), sum, vals, rows, nrows, width);
  MX_LAUNCH_CHECK("acc_add_rows_kernel");
  return MX_OK;
}

int mx_acc_add(mx_ctx* ctx, float* sum, const uint16_t* vals, int64_t n, void* stream) {
  if (int s = use(ctx)) return s;
  MX_REQUIRE(n >= 0, "mx_acc_add: bad count");
  if (!n) return MX_OK;
  MX_REQUIRE(sum && vals, "mx_acc_add: null pointer");
  hipLaunchKernelGGL(acc_add_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, as_stream(stream), sum, vals, n);
  MX_LAUNCH_CHECK("acc_add_kernel");
  return MX_OK;
}

int mx_acc_finish(mx_ctx* ctx, const float* sum, uint16_t* out, int64_t n, void* stream) {
  if (int s = use(ctx)) return s;
  MX_REQUIRE(n >= 0, "mx_acc_finish: bad count");
  if (!n) return MX_OK;
  MX_REQUIRE(sum && out, "mx_acc_finish: null pointer");
  hipLaunchKernelGGL(acc_finish_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, as_stream(stream), sum, out, n);
  MX_LAUNCH_CHECK("acc_finish_kernel");
  return MX_OK;
}

}  // extern "C"
