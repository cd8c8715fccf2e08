// Context, memory, stream and event entry points of the C ABI.
//
// Replaces the reference's ctypes Driver/Device layer (src/vesper/cuda.py:28-222):
// an explicit-allocation map with a byte cap, pinned host buffers, copies, and
// device-wide errors surfaced as status codes plus a thread-local message.
#include "mx_device.h"
#include "mx_internal.h"

namespace mxi {

static thread_local std::string g_error = "no error";

int fail(int status, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_error = buf;
  return status;
}

int hip_fail(hipError_t err, const char* what) {
  (void)hipGetLastError();  // clear the sticky launch error so the next call starts clean
  if (err == hipErrorOutOfMemory) return fail(MX_ERR_MEMORY, "%s: %s", what, hipGetErrorString(err));
  return fail(MX_ERR_HIP, "%s: %s (%s)", what, hipGetErrorName(err), hipGetErrorString(err));
}

void clear_error() { g_error = "no error"; }

int use(mx_ctx* ctx) {
  if (!ctx) return fail(MX_ERR_STATE, "context is closed");
  MX_HIP(hipSetDevice(ctx->device));
  return MX_OK;
}

int scratch(mx_ctx* ctx, uint64_t bytes, void** out) {
  if (ctx->scratch_bytes < bytes) {
    if (ctx->scratch) MX_HIP(hipFree(ctx->scratch));
    ctx->scratch = nullptr;
    ctx->scratch_bytes = 0;
    MX_HIP(hipMalloc(&ctx->scratch, bytes));
    ctx->scratch_bytes = bytes;
  }
  *out = ctx->scratch;
  return MX_OK;
}

}  // namespace mxi

namespace {

__global__ void fill_u32_kernel(uint32_t* p, int64_t n, uint32_t v) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

}  // namespace

using namespace mxi;

extern "C" {

const char* mx_last_error(void) { return g_error.c_str(); }

int mx_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  return n;
}

int mx_create(int device, uint64_t cap_bytes, mx_ctx** out) {
  MX_REQUIRE(out != nullptr, "mx_create: null output");
  int n = mx_device_count();
  MX_REQUIRE(device >= 0 && device < n, "mx_create: device %d not present (%d visible)", device, n);
  MX_HIP(hipSetDevice(device));
  MX_HIP(hipFree(nullptr));  // initialise the device's primary context now
  if (int s = noalloc_scratch_init(device)) return s;
  uint32_t* tickets = nullptr;
  float* handoff = nullptr;
  MX_HIP(hipMalloc(&tickets, MX_TICKETS * sizeof(uint32_t)));
  hipError_t err = hipMalloc(&handoff, 2 * (size_t)MX_HANDOFF_BYTES);
  if (err == hipSuccess) err = hipMemset(tickets, 0, MX_TICKETS * sizeof(uint32_t));
  if (err == hipSuccess) {
    hipLaunchKernelGGL(fill_u32_kernel, dim3(2 * MX_HANDOFF_BYTES / 4 / 256), dim3(256), 0, nullptr,
                       (uint32_t*)handoff, (int64_t)(2 * MX_HANDOFF_BYTES / 4), mxd::kHandoffEmpty);
    err = hipGetLastError();
  }
  if (err == hipSuccess) err = hipDeviceSynchronize();
  if (err != hipSuccess) {
    (void)hipFree(tickets);
    if (handoff) (void)hipFree(handoff);
    return hip_fail(err, "mx_create: set up the arrival counters and handoff buffer");
  }
  mx_ctx* ctx = new mx_ctx();
  ctx->device = device;
  ctx->cap = cap_bytes;
  ctx->tickets = tickets;
  ctx->handoff = handoff;
  *out = ctx;
  return MX_OK;
}

int mx_destroy(mx_ctx* ctx) {
  if (!ctx) return MX_OK;
  int status = MX_OK;
  if (hipSetDevice(ctx->device) == hipSuccess) {
    if (hipDeviceSynchronize() != hipSuccess) status = hip_fail(hipGetLastError(), "mx_destroy: synchronize");
    for (auto& kv : ctx->owned) (void)hipFree(kv.first);
    for (auto& kv : ctx->pinned) (void)hipHostFree(kv.first);
    if (ctx->scratch) (void)hipFree(ctx->scratch);
    if (ctx->tickets) (void)hipFree(ctx->tickets);
    if (ctx->handoff) (void)hipFree(ctx->handoff);
  }
  delete ctx;
  return status;
}

int mx_device_name(mx_ctx* ctx, char* name, size_t name_bytes, char* arch, size_t arch_bytes) {
  if (int s = use(ctx)) return s;
  hipDeviceProp_t prop;
  MX_HIP(hipGetDeviceProperties(&prop, ctx->device));
  if (name && name_bytes) snprintf(name, name_bytes, "%s", prop.name);
  if (arch && arch_bytes) snprintf(arch, arch_bytes, "%s", prop.gcnArchName);
  return MX_OK;
}

int mx_device_memory(mx_ctx* ctx, uint64_t* free_bytes, uint64_t* total_bytes) {
  if (int s = use(ctx)) return s;
  MX_REQUIRE(free_bytes != nullptr && total_bytes != nullptr, "mx_device_memory: null output");
  size_t f = 0, t = 0;
  MX_HIP(hipMemGetInfo(&f, &t));
  *free_bytes = f;
  *total_bytes = t;
  return MX_OK;
}

int mx_malloc(mx_ctx* ctx, uint64_t bytes, void** dptr) {
  if (int s = use(ctx)) return s;
  MX_REQUIRE(dptr != nullptr, "mx_malloc: null output");
  MX_REQUIRE(bytes > 0, "mx_malloc: zero-byte allocation");
  std::lock_guard<std::mutex> g(ctx->lock);
  if (ctx->cap && ctx->live + bytes > ctx->cap)
    return fail(MX_ERR_MEMORY, "mx_malloc: %llu bytes would exceed the context cap (%llu live of %llu)",
                (unsigned long long)bytes, (unsigned long long)ctx->live, (unsigned long long)ctx->cap);
  void* p = nullptr;
  MX_HIP(hipMalloc(&p, bytes));
  ctx->owned[p] = bytes;
  ctx->live += bytes;
  if (ctx->live > ctx->peak) ctx->peak = ctx->live;
  *dptr = p;
  return MX_OK;
}

int mx_free(mx_ctx* ctx, void* dptr) {
  if (int s = use(ctx)) return s;
  if (!dptr) return MX_OK;
  std::lock_guard<std::mutex> g(ctx->lock);
  auto it = ctx->owned.find(dptr);
  MX_REQUIRE(it != ctx->owned.end(), "mx_free: pointer not owned by this context");
  MX_HIP(hipFree(dptr));
  ctx->live -= it->second;
  ctx->owned.erase(it);
  return MX_OK;
}

int mx_owned_size(mx_ctx* ctx, const void* dptr, uint64_t* bytes) {
  MX_REQUIRE(ctx != nullptr, "mx_owned_size: context is closed");
  MX_REQUIRE(bytes != nullptr, "mx_owned_size: null output");
  std::lock_guard<std::mutex> g(ctx->lock);
  auto it = ctx->owned.find(const_cast<void*>(dptr));
  *bytes = it == ctx->owned.end() ? 0 : it->second;
  return MX_OK;
}

int mx_owned_bytes(mx_ctx* ctx, uint64_t* live, uint64_t* peak) {
  MX_REQUIRE(ctx != nullptr, "mx_owned_bytes: context is closed");
  std::lock_guard<std::mutex> g(ctx->lock);
  if (live) *live = ctx->live;
  if (peak) *peak = ctx->peak;
  return MX_OK;
}

int mx_host_alloc_pinned(mx_ctx* ctx, uint64_t bytes, void** hptr) {
  if (int s = use(ctx)) return s;
  MX_REQUIRE(hptr != nullptr && bytes > 0, "mx_host_alloc_pinned: bad arguments");
  void* p = nullptr;
  MX_HIP(hipHostMalloc(&p, bytes, hipHostMallocDefault));
  std::lock_guard<std::mutex> g(ctx->lock);
  ctx->pinned[p] = bytes;
  *hptr = p;
  return MX_OK;
}

int mx_host_free_pinned(mx_ctx* ctx, void* hptr) {
  if (int s = use(ctx)) return s;
  if (!hptr) return MX_OK;
  std::lock_guard<std::mutex> g(ctx->lock);
  auto it = ctx->pinned.find(hptr);
  MX_REQUIRE(it != ctx->pinned.end(), "mx_host_free_pinned: pointer not owned by this context");
  MX_HIP(hipHostFree(hptr));
  ctx->pinned.erase(it);
  return MX_OK;
}

static int copy(mx_ctx* ctx, void* dst, const void* src, uint64_t bytes, void* stream, hipMemcpyKind kind,
                const char* what) {
  if (int s = use(ctx)) return s;
  if (!bytes) return MX_OK;
  MX_REQUIRE(dst && src, "%s: null pointer", what);
  MX_HIP(hipMemcpyAsync(dst, src, bytes, kind, as_stream(stream)));
  if (kind == hipMemcpyDeviceToHost) MX_HIP(hipStreamSynchronize(as_stream(stream)));
  return MX_OK;
}

int mx_memcpy_h2d(mx_ctx* ctx, void* dst, const void* src, uint64_t bytes, void* stream) {
  return copy(ctx, dst, src, bytes, stream, hipMemcpyHostToDevice, "mx_memcpy_h2d");
}
int mx_memcpy_d2h(mx_ctx* ctx, void* dst, const void* src, uint64_t bytes, void* stream) {
  return copy(ctx, dst, src, bytes, stream, hipMemcpyDeviceToHost, "mx_memcpy_d2h");
}
int mx_memcpy_d2d(mx_ctx* ctx, void* dst, const void* src, uint64_t bytes, void* stream) {
  return copy(ctx, dst, src, bytes, stream, hipMemcpyDeviceToDevice, "mx_memcpy_d2d");
}

int mx_stream_create(mx_ctx* ctx, void** stream) {
  if (int s = use(ctx)) return s;
  MX_REQUIRE(stream != nullptr, "mx_stream_create: null output");
  hipStream_t st;
  MX_HIP(hipStreamCreate(&st));  // default flags and priority: ordered with the null stream
  *stream = st;
  return MX_OK;
}
int mx_stream_destroy(mx_ctx* ctx, void* stream) {
  if (int s = use(ctx)) return s;
  if (stream) MX_HIP(hipStreamDestroy(as_stream(stream)));
  return MX_OK;
}
int mx_stream_sync(mx_ctx* ctx, void* stream) {
  if (int s = use(ctx)) return s;
  MX_HIP(hipStreamSynchronize(as_stream(stream)));
  return MX_OK;
}
int mx_device_sync(mx_ctx* ctx) {
  if (int s = use(ctx)) return s;
  MX_HIP(hipDeviceSynchronize());
  return MX_OK;
}
int mx_event_create(mx_ctx* ctx, void** event) {
  if (int s = use(ctx)) return s;
  MX_REQUIRE(event != nullptr, "mx_event_create: null output");
  hipEvent_t ev;
  MX_HIP(hipEventCreate(&ev));
  *event = ev;
  return MX_OK;
}
int mx_event_destroy(mx_ctx* ctx, void* event) {
  if (int s = use(ctx)) return s;
  if (event) MX_HIP(hipEventDestroy(reinterpret_cast<hipEvent_t>(event)));
  return MX_OK;
}
int mx_event_record(mx_ctx* ctx, void* event, void* stream) {
  if (int s = use(ctx)) return s;
  MX_HIP(hipEventRecord(reinterpret_cast<hipEvent_t>(event), as_stream(stream)));
  return MX_OK;
}
int mx_event_sync(mx_ctx* ctx, void* event) {
  if (int s = use(ctx)) return s;
  MX_HIP(hipEventSynchronize(reinterpret_cast<hipEvent_t>(event)));
  return MX_OK;
}
int mx_event_elapsed_ms(mx_ctx* ctx, void* start, void* stop, float* ms) {
  if (int s = use(ctx)) return s;
  MX_HIP(hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(start), reinterpret_cast<hipEvent_t>(stop)));
  return MX_OK;
}
int mx_stream_wait_event(mx_ctx* ctx, void* stream, void* event) {
  if (int s = use(ctx)) return s;
  MX_HIP(hipStreamWaitEvent(as_stream(stream), reinterpret_cast<hipEvent_t>(event), 0));
  return MX_OK;
}

}  // extern "C"

// ---------------------------------------------------------------------------------------------
// Deterministic synthetic fill (SplitMix64 finaliser over (seed, index)); used to create the
// 6 GB expert bank of the benchmark directly in HBM instead of pushing it over PCIe.

__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__global__ void fill_uniform_u8_kernel(uint8_t* dst, uint64_t bytes, uint64_t seed, uint32_t lo, uint32_t span) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t w = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; w * 8 < bytes; w += stride) {
    const uint64_t base = seed * 0x632BE59BD9B4E019ull + 2 * w;
    const uint64_t h[2] = {splitmix64(base), splitmix64(base + 1)};
    uint64_t out = 0;
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const uint32_t r16 = (uint32_t)((h[b >> 2] >> (16 * (b & 3))) & 0xFFFF);
      out |= (uint64_t)(lo + ((r16 * span) >> 16)) << (8 * b);
    }
    if (w * 8 + 8 <= bytes) {
      reinterpret_cast<uint64_t*>(dst)[w] = out;
    } else {
      for (uint64_t b = 0; w * 8 + b < bytes; ++b) dst[w * 8 + b] = (uint8_t)(out >> (8 * b));
    }
  }
}

extern "C" int mx_fill_uniform_u8(mx_ctx* ctx, void* dst, uint64_t bytes, uint64_t seed, uint32_t lo, uint32_t hi,
                                  void* stream) {
  if (int s = use(ctx)) return s;
  MX_REQUIRE(dst != nullptr, "mx_fill_uniform_u8: null destination");
  MX_REQUIRE(lo <= hi && hi <= 255, "mx_fill_uniform_u8: need lo <= hi <= 255");
  MX_REQUIRE(((uintptr_t)dst & 7) == 0, "mx_fill_uniform_u8: destination must be 8-byte aligned");
  if (!bytes) return MX_OK;
  const uint32_t span = hi - lo + 1;  // (r16 * span) >> 16 maps 16 hash bits onto [0, span)
  const uint64_t words = (bytes + 7) / 8;
  const uint64_t want = (words + 255) / 256;
  const unsigned blocks = (unsigned)(want < 65536 ? want : 65536);
  hipLaunchKernelGGL(fill_uniform_u8_kernel, dim3(blocks), dim3(256), 0, as_stream(stream), (uint8_t*)dst, bytes,
                     seed, lo, span);
  MX_LAUNCH_CHECK("fill_uniform_u8_kernel");
  return MX_OK;
}

// Plain streaming copy, 16 bytes per thread per step: the known-size workload against which the
// profiler's HBM byte counters (FETCH_SIZE, WRITE_SIZE) are calibrated.
__global__ void copy_u8x16_kernel(uint4* __restrict__ dst, const uint4* __restrict__ src, uint64_t n16) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) dst[i] = src[i];
}

// Streaming read at the best rate measured for a plain kernel on MI355X: workgroup g owns the bytes
// [g * per, (g + 1) * per); wave w of 4 reads 4 KB steps w, w + 4, ... (four 1 KB loads, 16 bytes per
// lane), three steps in flight, with non-temporal loads. Each wave writes the XOR of the 32-bit words
// it read, so the launch cannot be elided and its coverage can be checked.
constexpr int kReadWorkgroups = 4096;
constexpr int kReadDepth = 3;

__global__ __launch_bounds__(256) void read_ceiling_kernel(const uint8_t* __restrict__ src, uint64_t per,
                                                           uint32_t* __restrict__ out) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint8_t* base = src + (uint64_t)blockIdx.x * per + 16 * lane;
  const uint64_t steps = per / 4096;
  uint32_t acc = 0;
  uint64_t s0 = wave;
  for (; s0 + 4 * (kReadDepth - 1) < steps; s0 += 4 * kReadDepth) {
    uint4 v[kReadDepth][4];
#pragma unroll
    for (int s = 0; s < kReadDepth; ++s)
#pragma unroll
      for (int t = 0; t < 4; ++t) v[s][t] = mxd::ldg128_nt(base + (s0 + 4 * s) * 4096 + t * 1024);
#pragma unroll
    for (int s = 0; s < kReadDepth; ++s)
#pragma unroll
      for (int t = 0; t < 4; ++t) acc ^= v[s][t].x ^ v[s][t].y ^ v[s][t].z ^ v[s][t].w;
  }
  for (; s0 < steps; s0 += 4)
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const uint4 v = mxd::ldg128_nt(base + s0 * 4096 + t * 1024);
      acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) acc ^= (uint32_t)__shfl_xor((int)acc, m, 64);
  if (lane == 0) out[blockIdx.x * 4 + wave] = acc;
}

extern "C" int mx_read_kernel(mx_ctx* ctx, const void* src, uint64_t bytes, uint32_t* out, void* stream) {
  if (int s = use(ctx)) return s;
  MX_REQUIRE(src != nullptr && out != nullptr, "mx_read_kernel: null pointer");
  const uint64_t unit = (uint64_t)kReadWorkgroups * 4096;
  MX_REQUIRE(((uintptr_t)src & 15) == 0 && bytes > 0 && bytes % unit == 0,
             "mx_read_kernel: 16-byte aligned source and a positive multiple of %llu bytes required",
             (unsigned long long)unit);
  hipLaunchKernelGGL(read_ceiling_kernel, dim3(kReadWorkgroups), dim3(256), 0, as_stream(stream),
                     (const uint8_t*)src, bytes / kReadWorkgroups, out);
  MX_LAUNCH_CHECK("read_ceiling_kernel");
  return MX_OK;
}

extern "C" int mx_copy_kernel(mx_ctx* ctx, void* dst, const void* src, uint64_t bytes, void* stream) {
  if (int s = use(ctx)) return s;
  MX_REQUIRE(dst != nullptr && src != nullptr, "mx_copy_kernel: null pointer");
  MX_REQUIRE(((uintptr_t)dst & 15) == 0 && ((uintptr_t)src & 15) == 0 && bytes % 16 == 0,
             "mx_copy_kernel: 16-byte aligned pointers and a multiple of 16 bytes required");
  if (!bytes) return MX_OK;
  const uint64_t n16 = bytes / 16;
  const uint64_t want = (n16 + 255) / 256;
  const unsigned blocks = (unsigned)(want < 8192 ? want : 8192);
  hipLaunchKernelGGL(copy_u8x16_kernel, dim3(blocks), dim3(256), 0, as_stream(stream), (uint4*)dst,
                     (const uint4*)src, n16);
  MX_LAUNCH_CHECK("copy_u8x16_kernel");
  return MX_OK;
}
