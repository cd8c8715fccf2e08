// Format hooks: MXFP4 dequantization, E4M3 encoding and the per-32 activation quantizer.
//
// Bit-exact counterparts of the reference's conformance kernels decode_fp4,
// encode_fp8 and activation32 (src/vesper/kernels/format_probe.cu:23-52). The
// production path never materialises dequantized weights; these exist so the
// formats can be checked on the device against the oracle.
#include <vector>

#include "mx_device.h"
#include "mx_internal.h"
#include "mx_numerics.h"

namespace {

// One thread per packed byte (two outputs); 8 bytes per thread would not help: this is a test hook.
__global__ void dequant_mxfp4_kernel(const uint8_t* __restrict__ packed, const uint8_t* __restrict__ scales,
                                     float* __restrict__ out, int64_t rows, int64_t k) {
  const int64_t half = k / 2;
  const int64_t total = rows * half;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / half, c = i % half;
    const uint32_t byte = packed[i];
    const float s = mx::e8m0_value(scales[r * (k / 32) + (2 * c) / 32]);
    float2 v;
    v.x = mx::fp4_value(byte & 15u) * s;
    v.y = mx::fp4_value(byte >> 4) * s;
    reinterpret_cast<float2*>(out + r * k)[c] = v;
  }
}

__global__ void encode_e4m3_kernel(const float* __restrict__ in, uint8_t* __restrict__ out, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    out[i] = (uint8_t)mx::e4m3_encode(in[i]);
}

// One 32-lane half-wave per 32-element block: lane j holds element j, the amax is a
// butterfly max over the 32 lanes, and each lane encodes its own element.
template <typename In>
__global__ void act_quant32_kernel(const In* __restrict__ x, uint8_t* __restrict__ q, uint8_t* __restrict__ s,
                                   int64_t blocks) {
  const int lane = threadIdx.x & 31;
  const int64_t block = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 5;
  const bool live = block < blocks;
  float v = 0.f;
  if (live) {
    if constexpr (sizeof(In) == 2) v = mx::bf16_value(x[block * 32 + lane]);
    else v = mx::bf16_round(x[block * 32 + lane]);
  }
  float amax = fabsf(v);
#pragma unroll
  for (int m = 16; m >= 1; m >>= 1) amax = fmaxf(amax, __shfl_xor(amax, m, 32));
  amax = fmaxf(amax, mx::u2f(mx::kAmaxFloorBits));
  const uint32_t code = mx::act_scale_code(amax);
  if (live) {
    q[block * 32 + lane] = (uint8_t)mx::act_quant_pow2(v, 1.0f / mx::e8m0_value(code));
    if (lane == 0) s[block] = (uint8_t)code;
  }
}

// BF16 input, 8 values per thread (one 16-byte load), 4 threads per 32-block: the block amax is two
// xor-shuffles inside the quad, the 8 codes are one 8-byte store. Grid-stride over the groups of 8.
// rounded (nullable): the quantize-dequantize round trip BF16(E4M3(code) x scale), one 16-byte store.
__global__ __launch_bounds__(256) void act_quant32_v8_kernel(const uint16_t* __restrict__ x, uint8_t* __restrict__ q,
                                                             uint8_t* __restrict__ s, int64_t groups,
                                                             uint16_t* __restrict__ rounded) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t base = (int64_t)blockIdx.x * blockDim.x; base < groups; base += stride) {
    const int64_t i = base + threadIdx.x;   // quads never straddle the bound: groups is a multiple of 4
    const bool live = i < groups;
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (live) v = reinterpret_cast<const uint4*>(x)[i];
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    float f[8];
    float amax = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      f[2 * j] = mx::bf16_value(w[j] & 0xFFFFu);
      f[2 * j + 1] = mx::bf16_value(w[j] >> 16);
      amax = fmaxf(amax, fmaxf(fabsf(f[2 * j]), fabsf(f[2 * j + 1])));
    }
    amax = mxd::quad_max(amax);   // the block's 4 lanes are one quad
    amax = fmaxf(amax, mx::u2f(mx::kAmaxFloorBits));
    const uint32_t code = mx::act_scale_code(amax);
    const float sc = mx::e8m0_value(code);
    if (live) {
      uint2 out;
      // act_quant_pow2 of the 8 values: x * (1 / sc) is exact scaling (sc a power of two), and the
      // hardware pair conversion equals mx::e4m3_encode of the clamped value for every FP32 input
      const float r = 1.0f / sc;
      out.x = mxd::e4m3x4(f[0] * r, f[1] * r, f[2] * r, f[3] * r);
      out.y = mxd::e4m3x4(f[4] * r, f[5] * r, f[6] * r, f[7] * r);
      reinterpret_cast<uint2*>(q)[i] = out;
      if ((i & 3) == 0) s[i >> 2] = (uint8_t)code;
      if (rounded) {
        // E4M3 value x power of two is exact in FP32 and has at most 4 significant bits: the BF16
        // rounding keeps it exactly
        uint32_t r[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t lo = mx::bf16_bits(mx::e4m3_value((j < 2 ? out.x : out.y) >> (16 * (j & 1)) & 0xFFu) * sc);
          const uint32_t hi = mx::bf16_bits(mx::e4m3_value((j < 2 ? out.x : out.y) >> (16 * (j & 1) + 8) & 0xFFu) * sc);
          r[j] = lo | (hi << 16);
        }
        reinterpret_cast<uint4*>(rounded)[i] = make_uint4(r[0], r[1], r[2], r[3]);
      }
    }
  }
}

unsigned grid_for(int64_t items, int threads) {
  const int64_t g = (items + threads - 1) / threads;
  return (unsigned)(g < 1 ? 1 : g > 1048576 ? 1048576 : g);
}

}  // namespace

using namespace mxi;

// Exhaustive comparison of the hardware E4M3 packing (mxd::e4m3x4) with the software encoder on every
// FP32 bit pattern, clamped to [-448, 448] as the activation quantizers clamp: per-thread mismatch counts.
__global__ __launch_bounds__(256) void e4m3_pack_check_kernel(uint32_t* counts) {
  const uint32_t tid = blockIdx.x * blockDim.x + threadIdx.x, threads = gridDim.x * blockDim.x;
  auto clamp = [](float y) { return y > 448.f ? 448.f : (y < -448.f ? -448.f : y); };
  uint32_t bad = 0;
  for (uint64_t m = (uint64_t)tid * 4; m < (1ull << 32); m += (uint64_t)threads * 4) {
    float v[4];
    uint32_t want = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[i] = mx::u2f((uint32_t)(m + i));
      want |= mx::e4m3_encode(clamp(v[i])) << (8 * i);
    }
    bad += mxd::e4m3x4(v[0], v[1], v[2], v[3]) != want;
  }
  counts[tid] = bad;
}

namespace mxi {

int act_quant32_scaled(mx_ctx* ctx, const uint16_t* x, uint8_t* q, uint8_t* scales, uint16_t* scaled, int64_t rows,
                       int64_t width, hipStream_t stream) {
  if (int st = use(ctx)) return st;
  MX_REQUIRE(rows >= 0 && width > 0 && width % 32 == 0, "act_quant32_scaled: width must be a positive multiple of 32");
  if (!rows) return MX_OK;
  MX_REQUIRE(x && q && scales && scaled && ((uintptr_t)x & 15) == 0 && ((uintptr_t)q & 7) == 0 &&
                 ((uintptr_t)scaled & 15) == 0,
             "act_quant32_scaled: x and scaled 16-byte, q 8-byte aligned pointers required");
  const int64_t groups = rows * (width / 32) * 4;
  const int64_t want = (groups + 255) / 256;
  hipLaunchKernelGGL(act_quant32_v8_kernel, dim3((unsigned)(want < 65536 ? want : 65536)), dim3(256), 0, stream, x, q,
                     scales, groups, scaled);
  MX_LAUNCH_CHECK("act_quant32_v8_kernel");
  return MX_OK;
}

}  // namespace mxi

extern "C" {

int mx_check_e4m3_pack(mx_ctx* ctx, uint64_t* mismatches) {
  if (int st = use(ctx)) return st;
  MX_REQUIRE(mismatches != nullptr, "mx_check_e4m3_pack: null output");
  constexpr int kBlocks = 4096, kThreads = 256;
  uint32_t* d = nullptr;
  MX_HIP(hipMalloc(&d, sizeof(uint32_t) * kBlocks * kThreads));
  std::vector<uint32_t> h(kBlocks * kThreads);
  hipLaunchKernelGGL(e4m3_pack_check_kernel, dim3(kBlocks), dim3(kThreads), 0, nullptr, d);
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) e = hipMemcpy(h.data(), d, sizeof(uint32_t) * h.size(), hipMemcpyDeviceToHost);
  (void)hipFree(d);
  if (e != hipSuccess) return hip_fail(e, "mx_check_e4m3_pack");
  uint64_t total = 0;
  for (uint32_t c : h) total += c;
  *mismatches = total;
  return MX_OK;
}

int mx_dequant_mxfp4(mx_ctx* ctx, const uint8_t* packed, const uint8_t* scales, float* out, int64_t rows,
                     int64_t k, void* stream) {
  if (int st = use(ctx)) return st;
  MX_REQUIRE(rows >= 0 && k >= 0 && k % 32 == 0, "mx_dequant_mxfp4: k must be a multiple of 32");
  if (!rows || !k) return MX_OK;
  MX_REQUIRE(packed && scales && out, "mx_dequant_mxfp4: null pointer");
  hipLaunchKernelGGL(dequant_mxfp4_kernel, dim3(grid_for(rows * k / 2, 256)), dim3(256), 0, as_stream(stream),
                     packed, scales, out, rows, k);
  MX_LAUNCH_CHECK("dequant_mxfp4_kernel");
  return MX_OK;
}

int mx_encode_e4m3(mx_ctx* ctx, const float* in, uint8_t* out, int64_t n, void* stream) {
  if (int st = use(ctx)) return st;
  MX_REQUIRE(n >= 0, "mx_encode_e4m3: negative count");
  if (!n) return MX_OK;
  MX_REQUIRE(in && out, "mx_encode_e4m3: null pointer");
  hipLaunchKernelGGL(encode_e4m3_kernel, dim3(grid_for(n, 256)), dim3(256), 0, as_stream(stream), in, out, n);
  MX_LAUNCH_CHECK("encode_e4m3_kernel");
  return MX_OK;
}

int mx_act_quant32(mx_ctx* ctx, const uint16_t* x, uint8_t* q, uint8_t* scales, int64_t rows, int64_t width,
                   void* stream) {
  if (int st = use(ctx)) return st;
  MX_REQUIRE(rows >= 0 && width > 0 && width % 32 == 0, "mx_act_quant32: width must be a positive multiple of 32");
  if (!rows) return MX_OK;
  MX_REQUIRE(x && q && scales, "mx_act_quant32: null pointer");
  const int64_t blocks = rows * (width / 32);
  if (((uintptr_t)x & 15) == 0 && ((uintptr_t)q & 7) == 0) {
    const int64_t groups = blocks * 4;
    const int64_t want = (groups + 255) / 256;
    hipLaunchKernelGGL(act_quant32_v8_kernel, dim3((unsigned)(want < 65536 ? want : 65536)), dim3(256), 0,
                       as_stream(stream), x, q, scales, groups, (uint16_t*)nullptr);
    MX_LAUNCH_CHECK("act_quant32_v8_kernel");
    return MX_OK;
  }
  MX_REQUIRE(blocks * 32 <= (int64_t)1048576 * 256, "mx_act_quant32: unaligned input limited to 2^28 values");
  hipLaunchKernelGGL(act_quant32_kernel<uint16_t>, dim3(grid_for(blocks * 32, 256)), dim3(256), 0,
                     as_stream(stream), x, q, scales, blocks);
  MX_LAUNCH_CHECK("act_quant32_kernel");
  return MX_OK;
}

int mx_kv_round32(mx_ctx* ctx, const uint16_t* x, int64_t count, uint16_t* rounded, uint8_t* codes, uint8_t* scales,
                  void* stream) {
  if (int st = use(ctx)) return st;
  MX_REQUIRE(count >= 0 && count % 32 == 0, "mx_kv_round32: the value count must be a multiple of 32");
  if (!count) return MX_OK;
  MX_REQUIRE(x && rounded && codes && scales, "mx_kv_round32: null pointer");
  MX_REQUIRE(((uintptr_t)x & 15) == 0 && ((uintptr_t)rounded & 15) == 0 && ((uintptr_t)codes & 7) == 0,
             "mx_kv_round32: x and rounded 16-byte, codes 8-byte alignment required");
  const int64_t groups = count / 8;
  const int64_t want = (groups + 255) / 256;
  hipLaunchKernelGGL(act_quant32_v8_kernel, dim3((unsigned)(want < 65536 ? want : 65536)), dim3(256), 0,
                     as_stream(stream), x, codes, scales, groups, rounded);
  MX_LAUNCH_CHECK("act_quant32_v8_kernel");
  return MX_OK;
}

int mx_act_quant32_f32(mx_ctx* ctx, const float* x, uint8_t* q, uint8_t* scales, int64_t rows, int64_t width,
                       void* stream) {
  if (int st = use(ctx)) return st;
  MX_REQUIRE(rows >= 0 && width > 0 && width % 32 == 0, "mx_act_quant32_f32: width must be a positive multiple of 32");
  if (!rows) return MX_OK;
  MX_REQUIRE(x && q && scales, "mx_act_quant32_f32: null pointer");
  const int64_t blocks = rows * (width / 32);
  MX_REQUIRE(blocks * 32 <= (int64_t)1048576 * 256, "mx_act_quant32_f32: limited to 2^28 values per call");
  hipLaunchKernelGGL(act_quant32_kernel<float>, dim3(grid_for(blocks * 32, 256)), dim3(256), 0, as_stream(stream),
                     x, q, scales, blocks);
  MX_LAUNCH_CHECK("act_quant32_kernel");
  return MX_OK;
}

}  // extern "C"
