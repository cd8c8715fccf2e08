// Internal declarations shared by the library's translation units.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>
#include <unordered_map>

#include "../../include/mxmoe.h"

struct mx_ctx {
  int device = 0;
  uint64_t cap = 0;      // 0 = unlimited explicit allocations
  uint64_t live = 0;
  uint64_t peak = 0;
  std::mutex lock;
  std::unordered_map<void*, uint64_t> owned;        // device allocations
  std::unordered_map<void*, uint64_t> pinned;       // host pinned allocations
  void* scratch = nullptr;                          // small reusable device scratch
  uint64_t scratch_bytes = 0;
  uint32_t* tickets = nullptr;                      // [MX_TICKETS] arrival counters, zero between launches
  float* handoff = nullptr;                         // 2 halves of MX_HANDOFF_BYTES, used on alternate launches
  int handoff_half = 0;                             // the half the next single-launch split-K GEMV uses
  uint64_t handoff_dirty[2] = {0, 0};               // bytes of each half a launch wrote and nobody restored yet
};

// Arrival counters of split-K kernels: the last workgroup of an output tile to arrive finishes the tile
// and puts its counter back to zero, so the array is zero again whenever the launch has ended.
#define MX_TICKETS 16384
// The split-K GEMV's partial sums on its single-launch path, per half. A launch writes its partial sums into
// one half, which holds the empty pattern (mxd::kHandoffEmpty) everywhere it reads, and restores the pattern
// over what the previous launch wrote into the other half; the next launch then uses that half.
#define MX_HANDOFF_BYTES (2u << 20)

// By-value kernel argument of mx_layer_set_experts: up to 64 table entries per launch.
#define MX_EXPERT_BATCH 64
struct mx_expert_batch {
  int32_t expert[MX_EXPERT_BATCH];
  const void* tiled[MX_EXPERT_BATCH];
};

namespace mxi {

// Thread-local error text; every failing entry point sets it.
int fail(int status, const char* fmt, ...);
int hip_fail(hipError_t err, const char* what);
void clear_error();

// Make the context's device current for this thread.
int use(mx_ctx* ctx);

// Context-owned scratch of at least `bytes` (grows; never shrinks until destroy).
int scratch(mx_ctx* ctx, uint64_t bytes, void** out);

// The allocation-free tiled expert call's fixed device array (mx_moe.hip): its device address is taken once
// per device, with the device current (mx_create), and looked up by later calls on that device.
int noalloc_scratch_init(int device);
int noalloc_scratch(int device, uint8_t** out);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// mx_act_quant32 that also writes each code times its block scale as BF16 (exact: at most 4 significant bits)
// into `scaled` [rows][width], the activation operand of the exact gate/up GEMVs. x 16-byte and q 8-byte
// aligned (mx_formats.hip).
int act_quant32_scaled(mx_ctx* ctx, const uint16_t* x, uint8_t* q, uint8_t* scales, uint16_t* scaled, int64_t rows,
                       int64_t width, hipStream_t stream);

// What other translation units need of a decode layer (defined with the layer in mx_moe.hip).
struct LayerView {
  mx_ctx* ctx;
  mx_moe_config cfg;
  const float* router_weight;
  const float* bias;
  const uint8_t** tiles;   // device [E + 1] tiled expert blobs, shared last
  int has_shared;
  const float* silu;       // device [65537]: mxd::silu_f32 of every BF16 gate value, then of the limit
  uint32_t* route_errors;  // device word: routing ids replaced by routed decode / prefill since the last clear
};
LayerView layer_view(mx_layer* layer);

}  // namespace mxi

#define MX_HIP(call)                                           \
  do {                                                         \
    hipError_t _e = (call);                                    \
    if (_e != hipSuccess) return mxi::hip_fail(_e, #call);     \
  } while (0)

#define MX_REQUIRE(cond, ...)                                  \
  do {                                                         \
    if (!(cond)) return mxi::fail(MX_ERR_INVALID, __VA_ARGS__); \
  } while (0)

#define MX_LAUNCH_CHECK(what)                                  \
  do {                                                         \
    hipError_t _e = hipGetLastError();                         \
    if (_e != hipSuccess) return mxi::hip_fail(_e, what);      \
  } while (0)
