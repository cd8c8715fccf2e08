// SHA-256 admission audit of device bytes: one digest per consecutive 4 KiB chunk
// (integrity.py:9-27 digest layout, kernels/integrity_probe.cu sha256_chunks), written from
// FIPS 180-4 (sections 4.1.2 functions, 4.2.2 constants, 5.1.1 padding, 5.3.3 initial value,
// 6.2.2 computation).
//
// Chunks are independent and each chunk's 65 compressions are a dependent chain, so one lane owns
// one chunk: a wave hashes 64 chunks side by side. Per 64-byte block a lane runs about 1,500 integer
// VALU instructions against 64 bytes of loads, so the kernel is bound by the VALU issue rate (about
// 1.4-1.5 TB/s of hashed bytes over the whole chip), not by HBM; a lane's next block is loaded while
// the current one is compressed, and the padding block of a full chunk is built from constants.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <thread>
#include <vector>

// OpenSSL 3 marks the one-shot SHA256() deprecated in favour of EVP; it remains the plain FIPS 180-4 digest
#define OPENSSL_SUPPRESS_DEPRECATED
#include <openssl/sha.h>

#include "mx_internal.h"

namespace {

constexpr uint32_t kChunkBytes = 4096;
constexpr uint64_t kMaxPayload = 1ull << 30;   // integrity.py:15-17

// FIPS 180-4 section 4.2.2: first 32 bits of the fractional parts of the cube roots of the first 64 primes.
constexpr uint32_t kRound[64] = {
    0x428a2f98u, 0x71374491u, 0xb5c0fbcfu, 0xe9b5dba5u, 0x3956c25bu, 0x59f111f1u, 0x923f82a4u, 0xab1c5ed5u,
    0xd807aa98u, 0x12835b01u, 0x243185beu, 0x550c7dc3u, 0x72be5d74u, 0x80deb1feu, 0x9bdc06a7u, 0xc19bf174u,
    0xe49b69c1u, 0xefbe4786u, 0x0fc19dc6u, 0x240ca1ccu, 0x2de92c6fu, 0x4a7484aau, 0x5cb0a9dcu, 0x76f988dau,
    0x983e5152u, 0xa831c66du, 0xb00327c8u, 0xbf597fc7u, 0xc6e00bf3u, 0xd5a79147u, 0x06ca6351u, 0x14292967u,
    0x27b70a85u, 0x2e1b2138u, 0x4d2c6dfcu, 0x53380d13u, 0x650a7354u, 0x766a0abbu, 0x81c2c92eu, 0x92722c85u,
    0xa2bfe8a1u, 0xa81a664bu, 0xc24b8b70u, 0xc76c51a3u, 0xd192e819u, 0xd6990624u, 0xf40e3585u, 0x106aa070u,
    0x19a4c116u, 0x1e376c08u, 0x2748774cu, 0x34b0bcb5u, 0x391c0cb3u, 0x4ed8aa4au, 0x5b9cca4fu, 0x682e6ff3u,
    0x748f82eeu, 0x78a5636fu, 0x84c87814u, 0x8cc70208u, 0x90befffau, 0xa4506cebu, 0xbef9a3f7u, 0xc67178f2u};

// Section 5.3.3: first 32 bits of the fractional parts of the square roots of the first 8 primes.
constexpr uint32_t kInitial[8] = {0x6a09e667u, 0xbb67ae85u, 0x3c6ef372u, 0xa54ff53au,
                                  0x510e527fu, 0x9b05688cu, 0x1f83d9abu, 0x5be0cd19u};

// rotate right by n (0 < n < 32): one v_alignbit_b32
__device__ __forceinline__ uint32_t rotr(uint32_t x, int n) { return __builtin_amdgcn_alignbit(x, x, n); }

// Three-input bitwise functions as one v_bitop3_b32 each; both truth tables are symmetric in their
// inputs (odd parity 0x96, at least two set 0xE8), so the operand order of the encoding does not matter.
__device__ __forceinline__ uint32_t xor3(uint32_t x, uint32_t y, uint32_t z) {
  return __builtin_amdgcn_bitop3_b32(x, y, z, 0x96);
}
__device__ __forceinline__ uint32_t majority3(uint32_t x, uint32_t y, uint32_t z) {
  return __builtin_amdgcn_bitop3_b32(x, y, z, 0xE8);
}

// One compression (section 6.2.2) of the block in w (big-endian words); w is consumed as the rolling
// 16-word message schedule. Fully unrolled so every index and round constant is static.
__device__ __forceinline__ void compress(uint32_t (&h)[8], uint32_t (&w)[16]) {
  uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], k = h[7];
#pragma unroll
  for (int i = 0; i < 64; ++i) {
    if (i >= 16) {
      const uint32_t x = w[(i - 15) & 15], y = w[(i - 2) & 15];
      const uint32_t sigma0 = xor3(rotr(x, 7), rotr(x, 18), x >> 3);
      const uint32_t sigma1 = xor3(rotr(y, 17), rotr(y, 19), y >> 10);
      w[i & 15] = w[i & 15] + sigma0 + w[(i - 7) & 15] + sigma1;
    }
    const uint32_t big1 = xor3(rotr(e, 6), rotr(e, 11), rotr(e, 25));
    const uint32_t choose = (e & f) | (~e & g);
    const uint32_t t1 = k + big1 + choose + kRound[i] + w[i & 15];
    const uint32_t big0 = xor3(rotr(a, 2), rotr(a, 13), rotr(a, 22));
    const uint32_t majority = majority3(a, b, c);
    const uint32_t t2 = big0 + majority;
    k = g;
    g = f;
    f = e;
    e = d + t1;
    d = c;
    c = b;
    b = a;
    a = t1 + t2;
  }
  h[0] += a;
  h[1] += b;
  h[2] += c;
  h[3] += d;
  h[4] += e;
  h[5] += f;
  h[6] += g;
  h[7] += k;
}

// 64 message bytes at p (16-byte aligned, inside the payload) as four 16-byte loads
__device__ __forceinline__ void load_block(uint4 (&v)[4], const uint8_t* p) {
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = *reinterpret_cast<const uint4*>(p + 16 * i);
}

// little-endian loads -> the block's big-endian message words
__device__ __forceinline__ void to_words(uint32_t (&w)[16], const uint4 (&v)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    w[4 * i + 0] = __builtin_bswap32(v[i].x);
    w[4 * i + 1] = __builtin_bswap32(v[i].y);
    w[4 * i + 2] = __builtin_bswap32(v[i].z);
    w[4 * i + 3] = __builtin_bswap32(v[i].w);
  }
}

// SHA-256 of the len (1..4096) bytes at src into h (the eight state words).
__device__ __forceinline__ void hash_chunk(const uint8_t* src, uint32_t len, uint32_t (&h)[8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) h[i] = kInitial[i];
  // Blocks wholly inside the chunk's bytes come from memory (block b + 1 is in flight while block b is
  // compressed). Padding (section 5.1.1) follows: the rem = len % 64 remaining bytes, the 0x80 marker,
  // zeros, and the 64-bit message length in bits in the last two words, with one more block when
  // rem >= 56. For a whole 4 KiB chunk rem = 0 and the padding block is constant. One loop over all
  // blocks keeps a single copy of the unrolled compression in the kernel.
  const uint32_t whole = len / 64;
  const uint32_t rem = len - 64 * whole;
  const uint32_t total = whole + (rem < 56 ? 1 : 2);
  const uint8_t* tail = src + 64 * whole;
  const uint32_t bits = len * 8;   // len <= 4096: the high word of the length is zero
  uint4 cur[4], next[4];
  if (whole > 0) load_block(cur, src);
  for (uint32_t b = 0; b < total; ++b) {
    uint32_t w[16];
    if (b < whole) {
      if (b + 1 < whole) load_block(next, src + 64 * (b + 1));
      to_words(w, cur);
#pragma unroll
      for (int i = 0; i < 4; ++i) cur[i] = next[i];
    } else if (b == whole) {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        uint32_t word = 0;
        if (4 * j <= rem) {   // data bytes or the marker: assemble the word byte by byte
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const uint32_t p = 4 * j + t;
            const uint32_t byte = p < rem ? tail[p] : (p == rem ? 0x80u : 0u);
            word |= byte << (24 - 8 * t);
          }
        }
        w[j] = word;
      }
      if (rem < 56) w[15] = bits;
    } else {
#pragma unroll
      for (int j = 0; j < 15; ++j) w[j] = 0;
      w[15] = bits;
    }
    compress(h, w);
  }
}

// the digest bytes (state words big-endian) as two 16-byte vectors
__device__ __forceinline__ void digest_words(const uint32_t (&h)[8], uint4& d0, uint4& d1) {
  d0 = make_uint4(__builtin_bswap32(h[0]), __builtin_bswap32(h[1]), __builtin_bswap32(h[2]), __builtin_bswap32(h[3]));
  d1 = make_uint4(__builtin_bswap32(h[4]), __builtin_bswap32(h[5]), __builtin_bswap32(h[6]), __builtin_bswap32(h[7]));
}

// grid ceil(chunks / 256) x 256 threads: lane c hashes bytes [4096 c, min(4096 (c + 1), bytes)) and
// writes its 32-byte digest to digests + 32 c.
__global__ __launch_bounds__(256) void sha256_chunks_kernel(const uint8_t* __restrict__ data,
                                                            uint8_t* __restrict__ digests, uint64_t bytes,
                                                            uint32_t chunks) {
  const uint32_t chunk = blockIdx.x * 256u + threadIdx.x;
  if (chunk >= chunks) return;
  const uint64_t start = (uint64_t)chunk * kChunkBytes;
  const uint32_t len = (uint32_t)(bytes - start < kChunkBytes ? bytes - start : kChunkBytes);
  uint32_t h[8];
  hash_chunk(data + start, len, h);
  uint4* out = reinterpret_cast<uint4*>(digests + (size_t)chunk * 32);
  digest_words(h, out[0], out[1]);
}

// Admission audit of up to kVerifyBatch slots in one launch: the slots' device bytes and their expected
// digest tables (device memory, chunk c's 32 bytes at 32 c).
constexpr int kVerifyBatch = 64;
struct VerifyBatch {
  const uint8_t* slot[kVerifyBatch];
  const uint8_t* expected[kVerifyBatch];
  int32_t counter[kVerifyBatch];   // the mismatch counter each slot adds to
};

// grid ceil(n x chunks / 256) x 256 threads: lane i hashes chunk i % chunks of slot i / chunks, compares
// the digest with the expected one and counts a difference in mismatches[counter[slot]] (a vector atomic).
__global__ __launch_bounds__(256) void sha256_verify_kernel(VerifyBatch batch, int n, uint64_t bytes, uint32_t chunks,
                                                            uint32_t* __restrict__ mismatches) {
  const uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x;
  const uint32_t s = (uint32_t)(i / chunks), chunk = (uint32_t)(i % chunks);
  if (s >= (uint32_t)n) return;
  const uint64_t start = (uint64_t)chunk * kChunkBytes;
  const uint32_t len = (uint32_t)(bytes - start < kChunkBytes ? bytes - start : kChunkBytes);
  uint32_t h[8];
  hash_chunk(batch.slot[s] + start, len, h);
  uint4 d0, d1;
  digest_words(h, d0, d1);
  const uint4* want = reinterpret_cast<const uint4*>(batch.expected[s] + (size_t)chunk * 32);
  const uint4 w0 = want[0], w1 = want[1];
  const bool same = d0.x == w0.x && d0.y == w0.y && d0.z == w0.z && d0.w == w0.w && d1.x == w1.x && d1.y == w1.y &&
                    d1.z == w1.z && d1.w == w1.w;
  if (!same) atomicAdd(mismatches + batch.counter[s], 1u);
}

// Audit gate: the counters of up to kGateBatch audited experts; when any is nonzero, every workgroup of the
// grid overwrites its share of y with BF16 NaN, so nothing computed from a slot that failed its audit can
// pass as a number.
constexpr int kGateBatch = 512;
struct GateBatch {
  int32_t index[kGateBatch];
};

__global__ __launch_bounds__(256) void audit_gate_kernel(const uint32_t* __restrict__ counters, GateBatch g, int n,
                                                         uint16_t* __restrict__ y, uint64_t count) {
  int flagged = 0;
  for (int i = threadIdx.x; i < n; i += 256) flagged |= counters[g.index[i]] != 0u;
  if (!__syncthreads_or(flagged)) return;
  for (uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x; i < count; i += (uint64_t)gridDim.x * 256u)
    y[i] = 0x7FC0u;
}

}  // namespace

using namespace mxi;

extern "C" int mx_audit_gate(mx_ctx* ctx, const uint32_t* counters, int32_t n_counters, const int32_t* index,
                             int32_t n, uint16_t* y, uint64_t count, void* stream) {
  if (int s = use(ctx)) return s;
  MX_REQUIRE(n >= 0 && n <= kGateBatch, "mx_audit_gate: 0 to %d counters per call", kGateBatch);
  if (n == 0 || count == 0) return MX_OK;
  MX_REQUIRE(counters && index && y, "mx_audit_gate: null pointer");
  GateBatch g{};
  for (int i = 0; i < n; ++i) {
    MX_REQUIRE(index[i] >= 0 && index[i] < n_counters, "mx_audit_gate: counter index %d outside [0, %d)", index[i],
               n_counters);
    g.index[i] = index[i];
  }
  const uint64_t blocks = (count + 255) / 256;
  hipLaunchKernelGGL(audit_gate_kernel, dim3((unsigned)(blocks < 256 ? blocks : 256)), dim3(256), 0, as_stream(stream),
                     counters, g, n, y, count);
  MX_LAUNCH_CHECK("audit_gate_kernel");
  return MX_OK;
}

// Host digest tables (the store's verified reads in GPU-integrity mode): OpenSSL's SHA-256 per chunk, the
// chunk range split over `threads` host threads. The interpreter lock is released around the whole call, so
// several experts of a batch promotion hash side by side without per-chunk Python work.
extern "C" int mx_host_sha256_chunks(const void* data, uint64_t bytes, void* digests, int32_t threads) {
  MX_REQUIRE(data != nullptr && digests != nullptr, "mx_host_sha256_chunks: null pointer");
  MX_REQUIRE(bytes > 0 && bytes <= kMaxPayload, "Invalid bounded integrity payload size");
  MX_REQUIRE(threads >= 1 && threads <= 64, "mx_host_sha256_chunks: threads must be in [1, 64]");
  const uint64_t chunks = (bytes + kChunkBytes - 1) / kChunkBytes;
  const uint8_t* d = (const uint8_t*)data;
  uint8_t* o = (uint8_t*)digests;
  MX_REQUIRE(o + chunks * 32 <= d || d + bytes <= o, "Digest destination must not overwrite source bytes");
  auto range = [&](uint64_t first, uint64_t last) {
    for (uint64_t c = first; c < last; ++c)
      SHA256(d + c * kChunkBytes, std::min<uint64_t>(kChunkBytes, bytes - c * kChunkBytes), o + 32 * c);
  };
  const uint64_t parts = std::min<uint64_t>((uint64_t)threads, chunks);
  std::vector<std::thread> pool;
  for (uint64_t i = 1; i < parts; ++i) pool.emplace_back(range, chunks * i / parts, chunks * (i + 1) / parts);
  range(0, chunks / parts);
  for (std::thread& t : pool) t.join();
  return MX_OK;
}

extern "C" int mx_sha256_chunks(mx_ctx* ctx, const void* data, uint64_t bytes, void* digests, void* stream) {
  if (int s = use(ctx)) return s;
  MX_REQUIRE(data != nullptr && digests != nullptr, "mx_sha256_chunks: null pointer");
  MX_REQUIRE(bytes > 0 && bytes <= kMaxPayload, "Invalid bounded integrity payload size");
  MX_REQUIRE(((uintptr_t)data & 15) == 0 && ((uintptr_t)digests & 15) == 0,
             "mx_sha256_chunks: data and digests must be 16-byte aligned");
  const uint64_t chunks = (bytes + kChunkBytes - 1) / kChunkBytes;
  const uint8_t* d = (const uint8_t*)data;
  uint8_t* o = (uint8_t*)digests;
  MX_REQUIRE(o + chunks * 32 <= d || d + bytes <= o, "Digest destination must not overwrite source bytes");
  hipLaunchKernelGGL(sha256_chunks_kernel, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0,
                     as_stream(stream), d, o, bytes, (uint32_t)chunks);
  MX_LAUNCH_CHECK("sha256_chunks_kernel");
  return MX_OK;
}

extern "C" int mx_sha256_verify(mx_ctx* ctx, const void* const* slots, const void* const* expected,
                                const int32_t* counters, int32_t n, uint64_t bytes, uint32_t* mismatches,
                                void* stream) {
  if (int s = use(ctx)) return s;
  MX_REQUIRE(n >= 0, "mx_sha256_verify: negative slot count");
  if (n == 0) return MX_OK;
  MX_REQUIRE(slots && expected && mismatches, "mx_sha256_verify: null pointer");
  MX_REQUIRE(bytes > 0 && bytes <= kMaxPayload, "Invalid bounded integrity payload size");
  for (int i = 0; i < n; ++i) {
    MX_REQUIRE(slots[i] && expected[i] && ((uintptr_t)slots[i] & 15) == 0 && ((uintptr_t)expected[i] & 15) == 0,
               "mx_sha256_verify: slot %d: 16-byte aligned device pointers required", i);
    MX_REQUIRE(!counters || counters[i] >= 0, "mx_sha256_verify: slot %d: negative counter index", i);
  }
  const uint64_t chunks = (bytes + kChunkBytes - 1) / kChunkBytes;
  hipStream_t st = as_stream(stream);
  for (int base = 0; base < n; base += kVerifyBatch) {
    VerifyBatch b{};
    const int m = n - base < kVerifyBatch ? n - base : kVerifyBatch;
    for (int i = 0; i < m; ++i) {
      b.slot[i] = (const uint8_t*)slots[base + i];
      b.expected[i] = (const uint8_t*)expected[base + i];
      b.counter[i] = counters ? counters[base + i] : base + i;
    }
    const uint64_t lanes = (uint64_t)m * chunks;
    hipLaunchKernelGGL(sha256_verify_kernel, dim3((unsigned)((lanes + 255) / 256)), dim3(256), 0, st, b, m, bytes,
                       (uint32_t)chunks, mismatches);
    MX_LAUNCH_CHECK("sha256_verify_kernel");
  }
  return MX_OK;
}
