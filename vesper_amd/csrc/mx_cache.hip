// Device expert-slot cache over host-pinned expert bytes (TieredCache + CudaCacheBackend,
// src/vesper/cache.py:19-287 and src/vesper/tiered.py:50-127, made asynchronous).
//
// The reference promotes an expert with blocking copies and a host sync per request. Here a fixed pool
// of HBM slots is indexed by an LRU map from 64-bit keys (e.g. layer << 32 | expert) to slots; a miss
// takes the least recently used slot that the same batch does not need (preferring one that no queued work
// still reads), and its bytes are copied from
// the key's registered host-pinned source with hipMemcpyAsync on the cache's own copy stream. Ordering is
// carried by events, never by host waits:
//   * each slot has a release event, recorded by the caller on the compute stream after the work that
//     reads the slot; a copy into the slot first makes the copy stream wait for it;
//   * each ensure() records a ready event on the copy stream after its copies, which the caller makes
//     the compute stream wait for (mx_cache_ready_event + mx_stream_wait_event).
// So copies for the next layer run while the current layer computes. Per-copy event pairs (optional)
// measure the time the copy engine spent on each transfer.
#include <algorithm>
#include <cstring>
#include <list>
#include <unordered_map>
#include <vector>

#include "mx_internal.h"

struct mx_cache {
  mx_ctx* ctx = nullptr;
  uint64_t slot_bytes = 0;
  int slots = 0;
  uint8_t* pool = nullptr;                       // slots * slot_bytes device bytes
  hipStream_t copy = nullptr;                    // default-priority side stream
  std::vector<hipEvent_t> released;              // per slot: last compute use (caller-recorded)
  std::vector<bool> release_pending;
  hipEvent_t ready = nullptr;                    // after the most recent ensure's copies
  std::unordered_map<int64_t, const void*> source;   // key -> host pinned bytes
  std::list<int64_t> lru;                        // front = least recently used key
  std::unordered_map<int64_t, std::pair<int, std::list<int64_t>::iterator>> where;   // key -> slot
  std::vector<int> free_slots;
  std::vector<int64_t> owner;                    // slot -> key (or -1)
  // statistics and optional per-copy timing
  uint64_t hits = 0, misses = 0, bytes_copied = 0;
  bool timing = false;
  std::vector<hipEvent_t> copy_events;           // pairs, reused
  int copy_events_used = 0;
  double copy_ms = 0.0;
};

using namespace mxi;

namespace {

int flush_copy_timing(mx_cache* c) {
  if (!c->copy_events_used) return MX_OK;
  MX_HIP(hipEventSynchronize(c->copy_events[c->copy_events_used - 1]));
  for (int i = 0; i + 1 < c->copy_events_used; i += 2) {
    float ms = 0.f;
    MX_HIP(hipEventElapsedTime(&ms, c->copy_events[i], c->copy_events[i + 1]));
    c->copy_ms += ms;
  }
  c->copy_events_used = 0;
  return MX_OK;
}

void release_all(mx_cache* c) {
  if (c->copy) (void)hipStreamSynchronize(c->copy);
  for (auto& e : c->released)
    if (e) (void)hipEventDestroy(e);
  for (auto& e : c->copy_events)
    if (e) (void)hipEventDestroy(e);
  if (c->ready) (void)hipEventDestroy(c->ready);
  if (c->copy) (void)hipStreamDestroy(c->copy);
  if (c->pool) (void)hipFree(c->pool);
}

}  // namespace

extern "C" {

int mx_cache_create(mx_ctx* ctx, uint64_t slot_bytes, int32_t slots, mx_cache** out) {
  if (int s = use(ctx)) return s;
  MX_REQUIRE(out != nullptr, "mx_cache_create: null output");
  MX_REQUIRE(slots >= 1 && slot_bytes > 0 && slot_bytes % 256 == 0,
             "mx_cache_create: need at least one slot and a slot size that is a positive multiple of 256");
  mx_cache* c = new mx_cache();
  c->ctx = ctx;
  c->slot_bytes = slot_bytes;
  c->slots = slots;
  hipError_t err = hipMalloc((void**)&c->pool, slot_bytes * (uint64_t)slots);
  if (err == hipSuccess) err = hipStreamCreateWithFlags(&c->copy, hipStreamNonBlocking);
  if (err == hipSuccess) err = hipEventCreateWithFlags(&c->ready, hipEventDisableTiming);
  c->released.assign(slots, nullptr);
  c->release_pending.assign(slots, false);
  for (int i = 0; err == hipSuccess && i < slots; ++i) err = hipEventCreateWithFlags(&c->released[i], hipEventDisableTiming);
  if (err != hipSuccess) {
    const int st = err == hipErrorOutOfMemory ? fail(MX_ERR_MEMORY, "mx_cache_create: %llu device bytes unavailable",
                                                     (unsigned long long)(slot_bytes * (uint64_t)slots))
                                              : hip_fail(err, "mx_cache_create");
    release_all(c);
    delete c;
    return st;
  }
  c->owner.assign(slots, -1);
  for (int i = slots - 1; i >= 0; --i) c->free_slots.push_back(i);
  *out = c;
  return MX_OK;
}

int mx_cache_destroy(mx_cache* c) {
  if (!c) return MX_OK;
  if (int s = use(c->ctx)) return s;
  release_all(c);
  delete c;
  return MX_OK;
}

int mx_cache_register(mx_cache* c, int64_t key, const void* host_src) {
  MX_REQUIRE(c != nullptr, "cache is closed");
  MX_REQUIRE(key >= 0 && host_src != nullptr, "mx_cache_register: need a non-negative key and a host source");
  hipPointerAttribute_t attr{};
  const hipError_t err = hipPointerGetAttributes(&attr, host_src);
  MX_REQUIRE(err == hipSuccess && attr.type == hipMemoryTypeHost,
             "mx_cache_register: the source must be pinned host memory (mx_host_alloc_pinned)");
  c->source[key] = host_src;
  return MX_OK;
}

int mx_cache_ensure(mx_cache* c, const int64_t* keys, int32_t n, void** dev_ptrs, int32_t* hit) {
  MX_REQUIRE(c != nullptr, "cache is closed");
  if (int s = use(c->ctx)) return s;
  MX_REQUIRE(n >= 0 && (n == 0 || (keys && dev_ptrs)), "mx_cache_ensure: bad arguments");
  MX_REQUIRE(n <= c->slots, "mx_cache_ensure: %d keys exceed the %d slots", n, c->slots);
  for (int i = 0; i < n; ++i) {
    MX_REQUIRE(c->source.count(keys[i]), "Requested expert %lld is absent from the pinned store", (long long)keys[i]);
    for (int j = 0; j < i; ++j) MX_REQUIRE(keys[j] != keys[i], "mx_cache_ensure: repeated key %lld", (long long)keys[i]);
  }
  // pass 1: hits move to the most-recent end, so the batch's own keys are never chosen as victims
  std::vector<int> slot_of(n, -1);
  for (int i = 0; i < n; ++i) {
    auto it = c->where.find(keys[i]);
    if (it == c->where.end()) continue;
    c->lru.splice(c->lru.end(), c->lru, it->second.second);
    slot_of[i] = it->second.first;
  }
  // the batch's keys present in the LRU list: its hits now, plus each miss once inserted (all at the back)
  int batch_in_lru = 0;
  for (int i = 0; i < n; ++i) batch_in_lru += slot_of[i] >= 0;
  bool copied = false;
  for (int i = 0; i < n; ++i) {
    if (hit) hit[i] = slot_of[i] >= 0;
    if (slot_of[i] >= 0) {
      ++c->hits;
      continue;
    }
    ++c->misses;
    int s;
    if (!c->free_slots.empty()) {
      s = c->free_slots.back();
      c->free_slots.pop_back();
    } else {
      // Least recently used first, but skip a slot whose last release is still in flight on the GPU (the
      // host may run ahead of the device): copying into it would make the copy stream wait for that work.
      // Batch keys sit at the back and are never reached; with none idle, take the front and wait.
      auto pick = c->lru.begin();
      const int candidates = std::min<int>(64, (int)c->lru.size() - batch_in_lru);
      int scanned = 0;
      for (auto it = c->lru.begin(); scanned < candidates; ++it, ++scanned) {
        const int cand = c->where[*it].first;
        if (!c->release_pending[cand] || hipEventQuery(c->released[cand]) == hipSuccess) {
          pick = it;
          break;
        }
      }
      auto vit = c->where.find(*pick);
      s = vit->second.first;
      c->lru.erase(pick);
      c->where.erase(vit);
    }
    if (c->release_pending[s]) MX_HIP(hipStreamWaitEvent(c->copy, c->released[s], 0));
    c->release_pending[s] = false;
    uint8_t* dst = c->pool + (uint64_t)s * c->slot_bytes;
    if (c->timing) {
      if (c->copy_events_used + 2 > (int)c->copy_events.size()) {
        if (c->copy_events.size() >= 4096)
          if (int st = flush_copy_timing(c)) return st;
        while (c->copy_events_used + 2 > (int)c->copy_events.size()) {
          hipEvent_t e;
          MX_HIP(hipEventCreate(&e));
          c->copy_events.push_back(e);
        }
      }
      MX_HIP(hipEventRecord(c->copy_events[c->copy_events_used++], c->copy));
    }
    MX_HIP(hipMemcpyAsync(dst, c->source[keys[i]], c->slot_bytes, hipMemcpyHostToDevice, c->copy));
    if (c->timing) MX_HIP(hipEventRecord(c->copy_events[c->copy_events_used++], c->copy));
    c->bytes_copied += c->slot_bytes;
    c->owner[s] = keys[i];
    ++batch_in_lru;
    c->lru.push_back(keys[i]);
    c->where[keys[i]] = {s, std::prev(c->lru.end())};
    slot_of[i] = s;
    copied = true;
  }
  for (int i = 0; i < n; ++i) dev_ptrs[i] = c->pool + (uint64_t)slot_of[i] * c->slot_bytes;
  // the ready event always marks this batch (recorded even without copies: it then completes at once)
  MX_HIP(hipEventRecord(c->ready, c->copy));
  (void)copied;
  return MX_OK;
}

int mx_cache_forget(mx_cache* c, int64_t key) {
  MX_REQUIRE(c != nullptr, "cache is closed");
  auto it = c->where.find(key);
  if (it == c->where.end()) return MX_OK;
  const int s = it->second.first;
  c->lru.erase(it->second.second);
  c->where.erase(it);
  c->owner[s] = -1;
  c->free_slots.push_back(s);   // its release event, if pending, still orders the next copy into it
  return MX_OK;
}

int mx_cache_ready_event(mx_cache* c, void** event) {
  MX_REQUIRE(c != nullptr && event != nullptr, "mx_cache_ready_event: bad arguments");
  *event = c->ready;
  return MX_OK;
}

int mx_cache_release(mx_cache* c, const int64_t* keys, int32_t n, void* stream) {
  MX_REQUIRE(c != nullptr, "cache is closed");
  if (int s = use(c->ctx)) return s;
  MX_REQUIRE(n >= 0 && (n == 0 || keys), "mx_cache_release: bad arguments");
  for (int i = 0; i < n; ++i) {
    auto it = c->where.find(keys[i]);
    MX_REQUIRE(it != c->where.end(), "mx_cache_release: key %lld is not resident", (long long)keys[i]);
    const int s = it->second.first;
    MX_HIP(hipEventRecord(c->released[s], as_stream(stream)));
    c->release_pending[s] = true;
  }
  return MX_OK;
}

int mx_cache_stats(mx_cache* c, uint64_t* hits, uint64_t* misses, uint64_t* bytes_copied, double* copy_ms,
                   int32_t* resident) {
  MX_REQUIRE(c != nullptr, "cache is closed");
  if (int s = use(c->ctx)) return s;
  if (c->timing)
    if (int s = flush_copy_timing(c)) return s;
  if (hits) *hits = c->hits;
  if (misses) *misses = c->misses;
  if (bytes_copied) *bytes_copied = c->bytes_copied;
  if (copy_ms) *copy_ms = c->copy_ms;
  if (resident) *resident = (int32_t)c->where.size();
  return MX_OK;
}

int mx_cache_set_timing(mx_cache* c, int32_t enable) {
  MX_REQUIRE(c != nullptr, "cache is closed");
  if (int s = use(c->ctx)) return s;
  if (int s = flush_copy_timing(c)) return s;
  c->timing = enable != 0;
  c->hits = c->misses = c->bytes_copied = 0;
  c->copy_ms = 0.0;
  return MX_OK;
}

int mx_cache_copy_stream(mx_cache* c, void** stream) {
  MX_REQUIRE(c != nullptr && stream != nullptr, "mx_cache_copy_stream: bad arguments");
  *stream = c->copy;
  return MX_OK;
}

}  // extern "C"
