/* mxmoe: MI355X (gfx950) quantized MoE expert arithmetic behind a C ABI.
 *
 * Plain pointers and sizes only. Device pointers are HIP device addresses;
 * `stream` is a hipStream_t (NULL = the device's default stream). Every entry
 * point returns MX_OK (0) or a negative status; mx_last_error() describes the
 * most recent failure on the calling thread. Shapes are validated on the host
 * before any device work, mirroring the reference's ValueError-before-device
 * rule (tests/test_expert_boundaries.py:31-40 of shell-term/vesper).
 *
 * The reference binds CUDA probe kernels through ctypes (src/vesper/cuda.py);
 * each declaration below names the reference interface it replaces.
 *
 * A context keeps small reusable device buffers (scratch, and the arrival
 * counters of split-K kernels, which are zero between launches), and a layer
 * keeps its per-call buffers: calls on one context, or on one layer, must not
 * run concurrently on different streams. Use one context per stream that runs
 * alongside others, as the reference serialises calls per Device
 * (src/vesper/connected.py:131-133).
 */
#ifndef MXMOE_H
#define MXMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes; the Python adapter maps them to the reference's exception
 * classes (src/vesper/cuda.py:18-19,62-67 and the ValueError/MemoryError/
 * RuntimeError conventions of src/vesper/expert.py and src/vesper/moe.py). */
#define MX_OK 0
#define MX_ERR_INVALID (-1) /* ValueError: bad shape, range or argument      */
#define MX_ERR_MEMORY (-2)  /* MemoryError: allocation cap or device memory */
#define MX_ERR_STATE (-3)   /* RuntimeError: lifecycle misuse               */
#define MX_ERR_HIP (-4)     /* CudaError analogue: HIP runtime failure      */

typedef struct mx_ctx mx_ctx;
typedef struct mx_layer mx_layer;

/* ---- context, memory, streams (replaces Driver/Device, src/vesper/cuda.py:28-191) ---- */

/* Description of the most recent failure on this thread (never NULL). */
const char* mx_last_error(void);
/* Number of visible HIP devices (0 when none; never fails). */
int mx_device_count(void);
/* Open device `device` with an explicit-allocation cap in bytes (0 = no cap);
 * replaces Device(driver, ordinal, cap) (src/vesper/cuda.py:93-138). */
int mx_create(int device, uint64_t cap_bytes, mx_ctx** out);
/* Frees every allocation the context still owns (src/vesper/cuda.py:180-191). */
int mx_destroy(mx_ctx* ctx);
/* Name and gfx architecture of the context's device, e.g. "gfx950". */
int mx_device_name(mx_ctx* ctx, char* name, size_t name_bytes, char* arch, size_t arch_bytes);
/* Free and total bytes of the context's device (Device.memory, src/vesper/cuda.py:115-119). */
int mx_device_memory(mx_ctx* ctx, uint64_t* free_bytes, uint64_t* total_bytes);
int mx_malloc(mx_ctx* ctx, uint64_t bytes, void** dptr);       /* Device.allocate (cuda.py:121-138) */
int mx_free(mx_ctx* ctx, void* dptr);                           /* Device.free                        */
int mx_owned_bytes(mx_ctx* ctx, uint64_t* live, uint64_t* peak);/* Device.peak / allocations          */
/* Size of the allocation this context owns at base pointer `dptr` (0 when it owns none): the
 * allocation lookup of Device.allocations, src/vesper/cuda.py:121-138, that DeviceIntegrity.digests
 * uses to refuse unowned sources (src/vesper/integrity.py:53-54). */
int mx_owned_size(mx_ctx* ctx, const void* dptr, uint64_t* bytes);
int mx_host_alloc_pinned(mx_ctx* ctx, uint64_t bytes, void** hptr); /* Pinned (cuda.py:200-222)       */
int mx_host_free_pinned(mx_ctx* ctx, void* hptr);
int mx_memcpy_h2d(mx_ctx* ctx, void* dst, const void* src, uint64_t bytes, void* stream); /* Device.upload   */
int mx_memcpy_d2h(mx_ctx* ctx, void* dst, const void* src, uint64_t bytes, void* stream); /* Device.download */
int mx_memcpy_d2d(mx_ctx* ctx, void* dst, const void* src, uint64_t bytes, void* stream);
int mx_stream_create(mx_ctx* ctx, void** stream);
int mx_stream_destroy(mx_ctx* ctx, void* stream);
int mx_stream_sync(mx_ctx* ctx, void* stream);
int mx_device_sync(mx_ctx* ctx);
int mx_event_create(mx_ctx* ctx, void** event);
int mx_event_destroy(mx_ctx* ctx, void* event);
int mx_event_record(mx_ctx* ctx, void* event, void* stream);
int mx_event_sync(mx_ctx* ctx, void* event);
int mx_event_elapsed_ms(mx_ctx* ctx, void* start, void* stop, float* ms);
/* Make `stream` wait for `event` (cross-stream ordering for slot reuse). */
int mx_stream_wait_event(mx_ctx* ctx, void* stream, void* event);
/* Deterministic synthetic bytes on the device: dst[i] = lo + hash(seed, i) % (hi - lo + 1). */
int mx_fill_uniform_u8(mx_ctx* ctx, void* dst, uint64_t bytes, uint64_t seed, uint32_t lo, uint32_t hi, void* stream);

/* Device-side copy by a plain streaming kernel (16 B per thread): the known-size workload used to
 * calibrate the profiler's HBM byte counters. Pointers 16-byte aligned, bytes a multiple of 16. */
int mx_copy_kernel(mx_ctx* ctx, void* dst, const void* src, uint64_t bytes, void* stream);

/* SHA-256 of every consecutive 4 KiB chunk of `bytes` device bytes (0 < bytes <= 2^30): digests
 * receives ceil(bytes / 4096) x 32 bytes, chunk c's digest at 32 c; the last chunk may be short.
 * Replaces the sha256_chunks kernel (src/vesper/kernels/integrity_probe.cu) launched by
 * DeviceIntegrity.digests (src/vesper/integrity.py:44-66) for the cache's admission audit
 * (src/vesper/tiered.py:78-95). data and digests 16-byte aligned and not overlapping. */
int mx_sha256_chunks(mx_ctx* ctx, const void* data, uint64_t bytes, void* digests, void* stream);

/* The same digest table of `bytes` HOST bytes (0 < bytes <= 2^30), computed on the host with `threads`
 * threads (1..64); no context or device. Replaces hash_chunks (src/vesper/integrity.py:21-34), the host
 * table of a verified store read that the GPU audit compares a slot with. */
int mx_host_sha256_chunks(const void* data, uint64_t bytes, void* digests, int32_t threads);

/* Batched admission audit: for each of the n slots (device pointers, `bytes` each) hash every 4 KiB chunk
 * as mx_sha256_chunks does, compare with expected[i] (device digest table, ceil(bytes / 4096) x 32 bytes)
 * and add slot i's count of differing chunks to mismatches[counters[i]] (device; counters NULL = i). The
 * counters are not cleared, so several admissions in flight can accumulate into per-expert counters that
 * the host reads and clears after synchronising. One launch per 64 slots on `stream` (e.g. the cache's
 * copy stream right after the copies it audits). The batched, asynchronous form of DeviceIntegrity.verify
 * (src/vesper/integrity.py:67-94); each slot must hold `bytes`. */
int mx_sha256_verify(mx_ctx* ctx, const void* const* slots, const void* const* expected, const int32_t* counters,
                     int32_t n, uint64_t bytes, uint32_t* mismatches, void* stream);

/* Audit gate for outputs computed from audited slots: if any of counters[index[i]] (device mismatch counters
 * as mx_sha256_verify fills them, n_counters of them; index a host array, n <= 512) is nonzero, the `count`
 * BF16 values at y are overwritten with NaN, ordered on `stream` after the work that wrote y. Placed after
 * each layer that read audited slots, it keeps an output computed from bytes that failed their audit from
 * passing as a number until the host has read the counters and dropped the slots -- the asynchronous
 * counterpart of the reference's refusal before a failing slot is used (src/vesper/cache.py:131-146). */
int mx_audit_gate(mx_ctx* ctx, const uint32_t* counters, int32_t n_counters, const int32_t* index, int32_t n,
                  uint16_t* y, uint64_t count, void* stream);

/* Streaming read of `bytes` (a multiple of 16 MiB, 16-byte aligned source) by the fastest plain read
 * kernel measured on MI355X (4096 workgroups of contiguous ranges, non-temporal 16-byte loads, three
 * 4 KB steps in flight per wave): the HBM read rate the weight-streaming kernels are compared with.
 * out[4 * 4096] receives the XOR of the 32-bit words each wave read. No reference counterpart: a
 * measurement workload. */
int mx_read_kernel(mx_ctx* ctx, const void* src, uint64_t bytes, uint32_t* out, void* stream);

/* ---- format hooks (replaces format_probe.cu decode_fp4/encode_fp8/activation32, lines 23-52) ---- */

/* Self-check with no counterpart in the reference: compares the gfx950 hardware E4M3 packing used by the
 * prefill epilogue with the bit-exact software encoder on every FP32 bit pattern (clamped to +-448 as the
 * activation quantizers clamp); *mismatches receives the count, 0 when they agree. Synchronous. */
int mx_check_e4m3_pack(mx_ctx* ctx, uint64_t* mismatches);

/* out[r][k] = E2M1(packed[r][k/2] nibble, low first) * E8M0(scales[r][k/32]); bit-exact. */
int mx_dequant_mxfp4(mx_ctx* ctx, const uint8_t* packed, const uint8_t* scales, float* out,
                     int64_t rows, int64_t k, void* stream);
/* out[i] = E4M3(in[i]) (RNE, saturating, NaN -> 0x7F); bit-exact with formats.py:55-66. */
int mx_encode_e4m3(mx_ctx* ctx, const float* in, uint8_t* out, int64_t n, void* stream);
/* Per-32 activation quantizer over BF16 input [rows][width] (formats.py:80-94). */
int mx_act_quant32(mx_ctx* ctx, const uint16_t* x_bf16, uint8_t* q, uint8_t* scales,
                   int64_t rows, int64_t width, void* stream);
/* Same quantizer over FP32 input (BF16-rounded first), the activation32 signature. */
int mx_act_quant32_f32(mx_ctx* ctx, const float* x, uint8_t* q, uint8_t* scales,
                       int64_t rows, int64_t width, void* stream);
/* Per-32 quantize-dequantize of `count` BF16 values (a multiple of 32): E4M3 codes, E8M0 scales (the
 * mx_act_quant32 arithmetic) and the round trip rounded = BF16(E4M3(code) x 2^(scale - 127)). Replaces
 * kv_round32 (src/vesper/kernels/kv_probe.cu:4-25). x and rounded 16-byte, codes 8-byte aligned. */
int mx_kv_round32(mx_ctx* ctx, const uint16_t* x, int64_t count, uint16_t* rounded, uint8_t* codes, uint8_t* scales,
                  void* stream);

/* ---- expert arithmetic ---- */

/* E4M3 x MXFP4 block GEMV (gemv_fp4 / gemv_fp4_mma, format_probe.cu:54-129; formats.py:97-118):
 * y[t][n] = BF16(sum_g dot(q[t][g], W[n][g]) * sa[t][g] * sw[n][g]) for T <= 16 tokens;
 * q [T][K] E4M3, sa [T][K/32] E8M0, W [N][K/2] packed E2M1, sw [N][K/32] E8M0. N % 64 == 0, K % 128 == 0. */
int mx_gemv_mxfp4(mx_ctx* ctx, const uint8_t* q, const uint8_t* sa, const uint8_t* w, const uint8_t* sw,
                  uint16_t* y_bf16, int32_t tokens, int32_t n, int32_t k, void* stream);

/* One expert's six tensors in the reference layout (src/vesper/checkpoint.py:139-149):
 * MXFP4: w*_weight [rows][width/2] bytes, w*_scale [rows][width/32] E8M0.
 * FP8 block-32 (shared expert, src/vesper/shared.py:20-24): w*_weight [rows][width] E4M3,
 * w*_scale [rows/32][width/32] E8M0. */
typedef struct mx_expert_ptrs {
  const void* w1_weight;
  const void* w1_scale;
  const void* w3_weight;
  const void* w3_scale;
  const void* w2_weight;
  const void* w2_scale;
} mx_expert_ptrs;

#define MX_FMT_MXFP4 0
#define MX_FMT_FP8_BLOCK32 1

/* Per-stage device buffers of one expert call (all optional; NULL skips the stage copy).
 * Row r of every buffer is token r. Mirrors the stage dict of ExpertExecutor.execute
 * (src/vesper/expert.py:71-79): q, s, w1, w3, down_input (BF16 bits here), trace, down_q,
 * down_s, w2. */
typedef struct mx_expert_stages {
  uint8_t* q;            /* [T][H]     */
  uint8_t* s;            /* [T][H/32]  */
  uint16_t* w1;          /* [T][I]     */
  uint16_t* w3;          /* [T][I]     */
  uint16_t* down_input;  /* [T][I]     */
  float* trace;          /* [T][I][5]: clamped gate, clamped up, silu, product, routed */
  uint8_t* down_q;       /* [T][I]     */
  uint8_t* down_s;       /* [T][I/32]  */
} mx_expert_stages;

/* y[T][H] (BF16 bits) = expert(x[T][H] BF16) for 1 <= T <= 16 tokens; route_w[T] (device FP32)
 * multiplies the SwiGLU product before W2, NULL = unweighted (shared expert).
 * Replaces ExpertExecutor.execute (src/vesper/expert.py:51-79) and ResidentSharedExpert.forward
 * (src/vesper/shared.py:169-170). */
int mx_expert_forward(mx_ctx* ctx, const mx_expert_ptrs* w, int32_t format, int32_t hidden, int32_t intermediate,
                      const uint16_t* x_bf16, int32_t tokens, float swiglu_limit, const float* route_w,
                      uint16_t* y_bf16, const mx_expert_stages* stages, void* stream);

/* ---- device-native expert layout ----
 *
 * The decode layer reads experts in a tiled layout chosen for the gfx950 scaled MFMA: per 128-wide
 * K chunk, a group of 64 MFMA rows stores its four 16-row A operands as 4 consecutive KB (lane l's
 * 16-byte MX block at 16*l), so every wave load is 1 KB of contiguous HBM, and one 4-byte word per
 * lane carries that lane's E8M0 code for all four tiles. Gate/up groups interleave 32 W1 rows and
 * the same 32 W3 rows (8 + 8 per tile) so the SwiGLU pair lands in one accumulator. Same byte count
 * as the reference layout (1.59375 * H * I); conversion is bit-for-bit in both directions.
 * The reference stores experts row-major (src/vesper/checkpoint.py:139-149, storage.py:33-41);
 * these calls are the boundary between that store layout and the resident one. */

/* Bytes of one tiled expert (0 if H or I is not a positive multiple of 128). */
uint64_t mx_tiled_expert_bytes(int32_t hidden, int32_t intermediate);
/* Reference layout (six device tensors) -> tiled blob (256-byte aligned device memory). */
int mx_tile_expert(mx_ctx* ctx, const mx_expert_ptrs* ref, int32_t hidden, int32_t intermediate, void* tiled,
                   void* stream);
/* Tiled blob -> reference layout; writes through the six pointers of `ref`. */
int mx_untile_expert(mx_ctx* ctx, const void* tiled, int32_t hidden, int32_t intermediate, const mx_expert_ptrs* ref,
                     void* stream);

/* mx_expert_forward on a tiled expert (a cache slot or bank entry): same stages and arithmetic as the
 * decode layer's expert kernels. Used by the tiered runtime (TieredExpertRuntime.forward,
 * src/vesper/tiered.py:199-211). */
int mx_expert_forward_tiled(mx_ctx* ctx, const void* tiled, int32_t hidden, int32_t intermediate,
                            const uint16_t* x_bf16, int32_t tokens, float swiglu_limit, const float* route_w,
                            uint16_t* y_bf16, const mx_expert_stages* stages, void* stream);

/* The benchmark's configuration-0 expert on a tiled expert: BF16 activations, FP32 accumulation, no
 * activation quantization and no clamp. y[T][H] (BF16, rounded once, 8-byte aligned) = W2 . h with
 * h[T][I] = silu(W1 . x) * (W3 . x) [* route_w[t]] in FP32, x BF16 [T][H] (16-byte aligned). `h` (FP32 [T][I])
 * and `gu` (FP32 [T][2I]: W1 . x then W3 . x) receive the intermediates when non-null; the down product
 * takes h as two BF16 terms (hi + lo, about 16 significant bits). tokens <= 16, hidden <= 8192,
 * intermediate <= 4096; uses the context scratch. The reference's expert
 * (ExpertExecutor.execute, src/vesper/expert.py:51-79) quantizes both activations to E4M3 instead; this is
 * the same weights under configuration 0's formula (expert_reference_fp32 of the oracle). */
int mx_expert_forward_bf16(mx_ctx* ctx, const void* tiled, int32_t hidden, int32_t intermediate,
                           const uint16_t* x_bf16, int32_t tokens, const float* route_w, float* h, float* gu,
                           uint16_t* y_bf16, void* stream);

/* mx_expert_forward_tiled without any device allocation: no counterpart in the reference. For callers that
 * cannot allocate -- code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc.
 * Same arguments, kernels and results; the call's plan, expert table and quantized activations live in a
 * fixed device array of MX_NOALLOC_SCRATCH_BYTES per GPU (taken by mx_create, held until the process ends)
 * instead of the context's growable scratch. A call whose plan + tokens x (H + I) x 33/32 bytes exceed it is
 * refused with MX_ERR_INVALID (16 tokens of a 7168 x 2048 expert need about 0.23 MiB). Every call on one GPU
 * shares the array, so calls that overlap on one GPU race: serialise them (one stream, or events). */
#define MX_NOALLOC_SCRATCH_BYTES (1u << 20)
int mx_expert_forward_tiled_noalloc(mx_ctx* ctx, const void* tiled, int32_t hidden, int32_t intermediate,
                                    const uint16_t* x_bf16, int32_t tokens, float swiglu_limit, const float* route_w,
                                    uint16_t* y_bf16, const mx_expert_stages* stages, void* stream);

/* ---- router (replaces GateProjection.project + RouterProbe, src/vesper/gate.py:133-147,
 *      src/vesper/router.py:227-264, routing_probe.cu:5-86) ---- */

#define MX_SCORE_SIGMOID 0
#define MX_SCORE_SQRTSOFTPLUS 1

typedef struct mx_router_out {
  float* logits;       /* [T][E]  (required)   */
  float* scores;       /* [T][E]  (optional)   */
  float* selection;    /* [T][E]  (optional)   */
  int32_t* indices;    /* [T][k]  (required)   */
  float* weights;      /* [T][k]  (required)   */
  float* raw;          /* [T][k]  (optional)   */
  float* denominator;  /* [T]     (optional)   */
  int32_t* tied;       /* [T]     (optional)   */
} mx_router_out;

/* logits[T][E] = W_r[E][H] (FP32) . x[T][H] (BF16 -> FP32) only: GateProjection.project
 * (src/vesper/gate.py:133-147) with cublasSgemm(T, N, E, T, H) (src/vesper/blas.py:70-73). */
int mx_gate_project(mx_ctx* ctx, const float* router_weight, const uint16_t* x_bf16, int32_t tokens,
                    int32_t hidden, int32_t experts, float* logits, void* stream);

/* logits = W_r[E][H] (FP32) . x[T][H] (BF16 -> FP32), then scores, selection = score + bias,
 * top-k (reference tie order), route weights. E <= 1024, k <= 32. */
int mx_router(mx_ctx* ctx, const float* router_weight, const float* bias, const uint16_t* x_bf16,
              int32_t tokens, int32_t hidden, int32_t experts, int32_t top_k, int32_t score_func,
              float route_scale, const mx_router_out* out, void* stream);
/* Selection postprocessing on supplied logits (RouterProbe.inspect, router.py:227-241):
 * scores/selection/indices/weights from logits[T][E]. */
int mx_router_postprocess(mx_ctx* ctx, const float* logits, const float* bias, int32_t tokens, int32_t experts,
                          int32_t top_k, int32_t score_func, float route_scale, const mx_router_out* out,
                          void* stream);
/* Selection on supplied scores and selection values (RouterProbe.inspect_selection, router.py:243-258). */
int mx_router_select(mx_ctx* ctx, const float* scores, const float* selection, int32_t tokens, int32_t experts,
                     int32_t top_k, float route_scale, const mx_router_out* out, void* stream);

/* ---- FP8 E4M3 block-scaled projections (replaces NativeProjections.fp8, src/vesper/projections.py:135-154,
 *      and projection_fp8, src/vesper/kernels/projection_probe.cu:9-51) ----
 *
 * block 32:  weight E8M0 scales [N/32][K/32] (the reference's layout), activations per-32 E8M0
 *            (mx_act_quant32); the scales are applied inside the scaled MFMA (exact powers of two).
 * block 128: weight FP32 scales [ceil(N/128)][K/128], activations per-token per-128 FP32
 *            (mx_act_quant128); per 128-wide chunk acc += (dot * sa) * sw in FP32.
 * Weights are tiled once (mx_fp8_tile) into 64-row groups of MFMA-ordered 1 KB pieces plus scales.
 * N % 64 == 0, K % 128 == 0. */

#define MX_FP8_BLOCK32 32
#define MX_FP8_BLOCK128 128
/* Bytes of a tiled FP8 weight (0 for unsupported shapes or block). */
uint64_t mx_fp8_tiled_bytes(int32_t n, int32_t k, int32_t block);
/* Reference layout (E4M3 codes [N][K] + scales) -> tiled blob (256-byte aligned device memory). */
int mx_fp8_tile(mx_ctx* ctx, const uint8_t* weight, const void* scales, int32_t n, int32_t k, int32_t block,
                void* tiled, void* stream);
/* Per-token per-128 quantizer of BF16 x [rows][width]: q E4M3 codes, s FP32 = max(amax, 1e-4) / 448. */
int mx_act_quant128(mx_ctx* ctx, const uint16_t* x_bf16, uint8_t* q, float* s, int64_t rows, int64_t width,
                    void* stream);
/* y[T][N] (BF16) = projection of x[T][H=K] (BF16): quantize with the block's activation quantizer, then the
 * block-scaled product. Optional outputs: trace [T][N] FP32 sums, q_out [T][K] codes, s_out scales
 * ([T][K/32] E8M0 or [T][K/128] FP32) -- the stage dict of projections.py:146-154. */
int mx_fp8_projection(mx_ctx* ctx, const void* tiled, int32_t n, int32_t k, int32_t block, const uint16_t* x_bf16,
                      int32_t tokens, uint16_t* y_bf16, float* trace, uint8_t* q_out, void* s_out, void* stream);

/* Grouped block-32 FP8 projection (the attention output projection wo_a): weight rows [g rows, (g + 1)
 * rows) of `tiled` (mx_fp8_tile, block 32, groups x rows by K) multiply activation group g, so
 * y[t][g rows + r] = sum_k W[g rows + r][k] x[t][g][k] with x given as per-32 E4M3 codes q[T][groups][K]
 * and E8M0 scales s[T][groups][K/32] (mx_kv_round32). Replaces the dequantize-to-BF16 + batched BF16
 * GEMM of NativeProjections.grouped (src/vesper/projections.py:60-67,156-171): the weights stay E4M3 and
 * the scaled MFMA applies both block scales. 1 <= T <= 32 tokens, rows a multiple of 64. */
int mx_fp8_grouped_projection(mx_ctx* ctx, const void* tiled, int32_t groups, int32_t rows, int32_t K,
                              const uint8_t* q, const uint8_t* s, int32_t T, uint16_t* y, float* trace, void* stream);

/* FP8 block-32 expert (the shared expert's format, src/vesper/shared.py:20-24,141-170 with
 * gemv_fp8_shared, shared_probe.cu:4-49): the MXFP4 expert's stage sequence with E4M3 weights and E8M0
 * scales per 32 x 32 block. w1/w3/w2 are tiled blobs (mx_fp8_tile, block 32) of W1 [I][H], W3 [I][H] and
 * W2 [H][I]; route_w NULL = unweighted. Same stage buffers and semantics as mx_expert_forward. */
int mx_fp8_expert_forward(mx_ctx* ctx, const void* w1_tiled, const void* w3_tiled, const void* w2_tiled,
                          int32_t hidden, int32_t intermediate, const uint16_t* x_bf16, int32_t tokens,
                          float swiglu_limit, const float* route_w, uint16_t* y_bf16,
                          const mx_expert_stages* stages, void* stream);

/* ---- ordered combine (replaces MoEAccumulator, src/vesper/moe.py:42-148, aggregation_probe.cu:4-25) ---- */

int mx_acc_zero(mx_ctx* ctx, float* sum, int64_t count, void* stream);                     /* moe_zero       */
int mx_acc_add_rows(mx_ctx* ctx, float* sum, const uint16_t* rows_bf16, const int32_t* token_rows,
                    int32_t nrows, int32_t width, void* stream);                           /* moe_add_expert */
int mx_acc_add(mx_ctx* ctx, float* sum, const uint16_t* values_bf16, int64_t count, void* stream); /* moe_add_shared */
int mx_acc_finish(mx_ctx* ctx, const float* sum, uint16_t* out_bf16, int64_t count, void* stream); /* moe_finish     */

/* ---- routed MoE layer (replaces ConnectedMoE.forward, src/vesper/connected.py:125-186) ---- */

typedef struct mx_moe_config {
  int32_t hidden;         /* H, multiple of 128          */
  int32_t intermediate;   /* I, multiple of 128          */
  int32_t experts;        /* E <= 1024                   */
  int32_t top_k;          /* k <= 32                     */
  int32_t score_func;     /* MX_SCORE_*                  */
  float route_scale;      /* 2.5 (BASELINE), 1.5 (ref)   */
  float swiglu_limit;     /* 0 disables the clamp        */
  int32_t shared_format;  /* -1 none, MX_FMT_*           */
  int32_t max_tokens;     /* decode batch capacity, <= 16 */
} mx_moe_config;

/* Register a layer: FP32 router weight [E][H], optional FP32 selection bias [E], E tiled expert
 * blobs (host array of device pointers, copied to a device table) and the optional shared expert. */
int mx_layer_create(mx_ctx* ctx, const mx_moe_config* cfg, const float* router_weight, const float* bias,
                    const void* const* experts_tiled, const void* shared_tiled, mx_layer** out);
int mx_layer_destroy(mx_layer* layer);
/* Re-point expert `expert` to another tiled blob (e.g. after a cache slot fill); ordered on `stream`. */
int mx_layer_set_expert(mx_layer* layer, int32_t expert, const void* tiled, void* stream);

/* y[T][H] = MoE(x[T][H]) for 1 <= T <= max_tokens, inputs resident in HBM: router -> top-k + plan ->
 * fused gate/up + SwiGLU + down-input quantization -> down -> ordered combine (shared last). At one token
 * the top-k and plan run inside the gate/up launch (four launches).
 * `diagnostics` != 0 also writes the per-stage buffers that mx_layer_buffer exposes. */
int mx_moe_decode(mx_layer* layer, const uint16_t* x_bf16, int32_t tokens, uint16_t* y_bf16,
                  int32_t diagnostics, void* stream);

/* Decode with routing decided elsewhere (a seeded trace, an expert-parallel dispatcher): ids [T][k] and
 * weights [T][k] on the device replace the router. An id outside [0, E) or repeated within a token is
 * replaced (smallest expert the token does not name, weight 0) so the call stays in bounds, and counted in
 * the layer's routing error word (mx_layer_route_errors): the reference refuses such routing before any
 * device work (participation, src/vesper/moe.py:18-30), so a caller that cannot validate ids on the host
 * must read the word after the call and discard the output when it is nonzero. */
int mx_moe_decode_routed(mx_layer* layer, const uint16_t* x_bf16, int32_t tokens, const int32_t* ids,
                         const float* weights, uint16_t* y_bf16, void* stream);
/* Routing ids that mx_moe_decode_routed and mx_moe_prefill replaced since the last clear (see above).
 * Synchronises `stream` and reads the count into *count; clear != 0 then resets it, ordered on `stream`.
 * The device-side form of participation's refusals (src/vesper/moe.py:18-30). */
int mx_layer_route_errors(mx_layer* layer, uint32_t* count, int32_t clear, void* stream);
/* Re-point n experts at once (one launch per 64), ordered on `stream`: experts[i] -> tiled[i]. */
int mx_layer_set_experts(mx_layer* layer, int32_t n, const int32_t* experts, const void* const* tiled, void* stream);

/* ---- expert streaming: device slot cache over host-pinned experts (replaces TieredCache /
 *      CudaCacheBackend / TieredExpertRuntime, src/vesper/cache.py:19-287, src/vesper/tiered.py:50-216) ----
 *
 * `slots` device slots of `slot_bytes` (an expert's tiled bytes); keys are caller-chosen 64-bit ids
 * (e.g. layer << 32 | expert), each registered with its host-pinned source. mx_cache_ensure maps a batch
 * of keys to slot pointers: hits refresh the LRU order, misses evict the least recently used slot that
 * the batch does not need and copy the source with hipMemcpyAsync on the cache's copy stream, after the
 * evicted slot's release event. The caller makes its compute stream wait for mx_cache_ready_event (after
 * each ensure) and records mx_cache_release on the compute stream after the work that reads the slots.
 * No host synchronisation; copies overlap compute. */
typedef struct mx_cache mx_cache;
int mx_cache_create(mx_ctx* ctx, uint64_t slot_bytes, int32_t slots, mx_cache** out);
int mx_cache_destroy(mx_cache* cache);
/* host_src must be pinned (mx_host_alloc_pinned) and hold slot_bytes bytes. */
int mx_cache_register(mx_cache* cache, int64_t key, const void* host_src);
/* dev_ptrs[i] <- slot of keys[i] (n <= slots, distinct registered keys); hit[i] (nullable) = 1 if resident. */
int mx_cache_ensure(mx_cache* cache, const int64_t* keys, int32_t n, void** dev_ptrs, int32_t* hit);
/* Drop `key`'s slot so it is never served (a slot whose admission audit failed): the key becomes a miss
 * again and the slot free. The reference publishes a slot only after its audit (src/vesper/cache.py:
 * 131-146). No-op when the key is not resident. */
int mx_cache_forget(mx_cache* c, int64_t key);
int mx_cache_ready_event(mx_cache* cache, void** event);
int mx_cache_release(mx_cache* cache, const int64_t* keys, int32_t n, void* stream);
int mx_cache_copy_stream(mx_cache* cache, void** stream);
/* Counters since the last mx_cache_set_timing; copy_ms sums per-copy event pairs (timing enabled). */
int mx_cache_stats(mx_cache* cache, uint64_t* hits, uint64_t* misses, uint64_t* bytes_copied, double* copy_ms,
                   int32_t* resident);
int mx_cache_set_timing(mx_cache* cache, int32_t enable);

/* Prefill: T tokens through the layer (routed experts + shared) as token-sorted grouped GEMMs on the
 * scaled MXFP4 MFMA; same per-token arithmetic as mx_moe_decode.
 * ids [T][k] (device int32, distinct per token) and weights [T][k] (device FP32) give the routing, or both
 * NULL to run the layer's router on x. Invalid given ids are replaced and counted as in
 * mx_moe_decode_routed. The caller provides a device workspace of at least
 * mx_prefill_workspace_bytes(layer, T) bytes, 256-byte aligned (no allocation inside the call).
 * H % 256 == 0. Replaces the reference's per-token ConnectedMoE.forward loop (connected.py:125-186). */
uint64_t mx_prefill_workspace_bytes(mx_layer* layer, int32_t tokens);
/* Byte offsets, inside a prefill workspace of `tokens` rows, of the intermediate stages a finished
 * mx_moe_prefill call leaves there: offsets[0] the down-input E4M3 codes [rows][I] (uint8), [1] their
 * E8M0 scales [rows][I/32], [2] the row of each routed pair (token t, rank j) [T][k] (int32), [3] the
 * first row of each expert [E + 1] (int32; the shared expert's rows, one per token in order, start at
 * entry E), [4] the expert outputs [T][k + 1][H] (BF16; token t's j-th routed expert in ascending ID at
 * place j, the shared expert at place k). The reference returns these stages from its per-token call
 * (ConnectedMoE.forward's expert dicts, connected.py:154-160); here they are read from the batched call's
 * workspace. */
#define MX_PREFILL_STAGES 5
int mx_prefill_stage_offsets(mx_layer* layer, int32_t tokens, uint64_t* offsets);
int mx_moe_prefill(mx_layer* layer, const uint16_t* x_bf16, int32_t tokens, const int32_t* ids, const float* weights,
                   uint16_t* y_bf16, void* workspace, uint64_t workspace_bytes, void* stream);

/* Internal per-call buffers of a layer (device pointers, valid after mx_moe_decode on the same stream). */
#define MX_BUF_LOGITS 0      /* float [T][E]          */
#define MX_BUF_SCORES 1      /* float [T][E]          */
#define MX_BUF_SELECTION 2   /* float [T][E]          */
#define MX_BUF_INDICES 3     /* int32 [T][k]          */
#define MX_BUF_WEIGHTS 4     /* float [T][k]          */
#define MX_BUF_XQ 5          /* uint8 [T][H]          */
#define MX_BUF_XS 6          /* uint8 [T][H/32]       */
#define MX_BUF_PLAN 7        /* int32 plan: struct Plan of csrc/mx_moe.hip (slot experts, rows, tokens) */
#define MX_BUF_W1 8          /* uint16 [rows][I]      */
#define MX_BUF_W3 9          /* uint16 [rows][I]      */
#define MX_BUF_DOWN_INPUT 10 /* uint16 [rows][I]      */
#define MX_BUF_DOWN_Q 11     /* uint8 [rows][I]       */
#define MX_BUF_DOWN_S 12     /* uint8 [rows][I/32]    */
#define MX_BUF_EXPERT_OUT 13 /* uint16 [rows][H]      */
#define MX_BUF_TRACE 14      /* float [rows][I][5]    */
#define MX_BUF_RAW 15        /* float [T][k]          */
#define MX_BUF_DENOMINATOR 16 /* float [T]            */
#define MX_BUF_TIED 17       /* int32 [T]             */
int mx_layer_buffer(mx_layer* layer, int32_t which, void** dptr, uint64_t* bytes);

/* Per-kernel HIP event timing of mx_moe_decode: while enabled, each call records events around its
 * four kernels on its stream (no host synchronisation; a ring of 64 calls is folded into the totals
 * when full). Reading (any call) reports stage_ms[0..3] = router, gate/up, down, combine averaged
 * over the calls recorded since profiling was last enabled. */
int mx_layer_profile(mx_layer* layer, int32_t enable, float* stage_ms, int32_t* calls);

/* Measurement hook: re-launch one stage of the layer's most recent mx_moe_decode call `iters` times
 * back to back on `stream` (each stage is idempotent given its inputs) and report the average
 * duration per launch from HIP events around the loop. Stages: MX_STAGE_*. After a one-token call the
 * route-plan stage is part of the gate/up launch and launches nothing. No reference counterpart (the
 * reference times whole Python calls); used by the benchmark's roofline figure. */
#define MX_STAGE_ROUTER 0
#define MX_STAGE_ROUTE_PLAN 1
#define MX_STAGE_GATEUP 2
#define MX_STAGE_DOWN 3
#define MX_STAGE_COMBINE 4
int mx_layer_time_stage(mx_layer* layer, int32_t stage, int32_t iters, float* us_per_launch, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* MXMOE_H */
