// Runtime half of the C ABI: device/stream setup, caching device allocator, copies, events.
//
// One process drives one GPU through one HIP stream.  Every kernel and copy the library issues is
// ordered on that stream, so a block returned to the allocator's free lists can be handed to the
// next request at once: any later use is enqueued after every earlier use of the same memory.
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <unordered_map>

#include "common.h"

namespace kh {

namespace {

thread_local char g_err[1024] = {0};

struct State {
  bool init = false;
  int device = -1;
  hipStream_t stream = nullptr;
};
State g_state;

// Size classes: requests up to 1 MiB round to 512 B, larger ones to 2 MiB.
constexpr size_t kSmallLimit = size_t(1) << 20;
constexpr size_t kSmallRound = 512;
constexpr size_t kLargeRound = size_t(2) << 20;

size_t round_size(size_t bytes) {
  if (bytes == 0) bytes = 1;
  if (bytes <= kSmallLimit) return (bytes + kSmallRound - 1) / kSmallRound * kSmallRound;
  return (bytes + kLargeRound - 1) / kLargeRound * kLargeRound;
}

struct Allocator {
  std::mutex mu;
  std::multimap<size_t, void*> free_blocks;   // size -> block
  std::unordered_map<void*, size_t> live;     // block -> size
  kh_alloc_stats stats{};

  int alloc(void** out, size_t bytes) {
    std::lock_guard<std::mutex> lock(mu);
    const size_t sz = round_size(bytes);
    // Reuse the smallest cached block that fits and wastes at most half of itself.
    auto it = free_blocks.lower_bound(sz);
    if (it != free_blocks.end() && it->first <= 2 * sz) {
      void* p = it->second;
      const size_t bsz = it->first;
      free_blocks.erase(it);
      stats.cached_bytes -= bsz;
      live[p] = bsz;
      stats.live_bytes += bsz;
      if (stats.live_bytes > stats.peak_bytes) stats.peak_bytes = stats.live_bytes;
      stats.n_cache_hits++;
      *out = p;
      return KH_OK;
    }
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, sz);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      release_cached_locked();
      e = hipMalloc(&p, sz);
      if (e != hipSuccess) {
        (void)hipGetLastError();
        set_error("kh_alloc: out of device memory for %zu bytes (%s)", sz, hipGetErrorString(e));
        return KH_ERR_OOM;
      }
    }
    live[p] = sz;
    stats.live_bytes += sz;
    if (stats.live_bytes > stats.peak_bytes) stats.peak_bytes = stats.live_bytes;
    stats.n_device_allocs++;
    *out = p;
    return KH_OK;
  }

  int free(void* p) {
    if (p == nullptr) return KH_OK;
    std::lock_guard<std::mutex> lock(mu);
    auto it = live.find(p);
    if (it == live.end()) {
      set_error("kh_free: %p was not allocated by kh_alloc (or was freed twice)", p);
      return KH_ERR_INVALID;
    }
    const size_t sz = it->second;
    live.erase(it);
    stats.live_bytes -= sz;
    free_blocks.emplace(sz, p);
    stats.cached_bytes += sz;
    return KH_OK;
  }

  // Caller holds `mu`.  Waits for the stream so no queued kernel still uses a released block.
  void release_cached_locked() {
    if (g_state.stream) (void)hipStreamSynchronize(g_state.stream);
    for (auto& kv : free_blocks) (void)hipFree(kv.second);
    free_blocks.clear();
    stats.cached_bytes = 0;
  }
};
Allocator g_alloc;

}  // namespace

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}
void clear_error() { g_err[0] = 0; }
hipStream_t stream() { return g_state.stream; }
bool initialized() { return g_state.init; }

void* scratch_alloc(size_t bytes) {
  void* p = nullptr;
  if (g_alloc.alloc(&p, bytes) != KH_OK) return nullptr;
  return p;
}
void scratch_free(void* p) { (void)g_alloc.free(p); }

}  // namespace kh

using namespace kh;

extern "C" {

int kh_device_count(int* count) {
  if (!count) {
    set_error("kh_device_count: null output pointer");
    return KH_ERR_INVALID;
  }
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    n = 0;
  }
  *count = n;
  return KH_OK;
}

int kh_init(int device) {
  if (g_state.init) {
    if (device == g_state.device) return KH_OK;
    set_error("kh_init: already initialised on device %d (asked for %d)", g_state.device, device);
    return KH_ERR_INVALID;
  }
  int n = 0;
  kh_device_count(&n);
  if (device < 0 || device >= n) {
    set_error("kh_init: device %d not available (%d HIP device(s) visible)", device, n);
    return KH_ERR_INVALID;
  }
  KH_CHECK_HIP(hipSetDevice(device));
  KH_CHECK_HIP(hipStreamCreateWithFlags(&g_state.stream, hipStreamNonBlocking));
  g_state.device = device;
  g_state.init = true;
  return KH_OK;
}

const char* kh_last_error(void) { return g_err; }

int kh_alloc(void** ptr, size_t bytes) {
  KH_REQUIRE_INIT();
  KH_REQUIRE(ptr != nullptr, "kh_alloc: null output pointer");
  return g_alloc.alloc(ptr, bytes);
}

int kh_free(void* ptr) {
  KH_REQUIRE_INIT();
  return g_alloc.free(ptr);
}

int kh_empty_cache(void) {
  KH_REQUIRE_INIT();
  std::lock_guard<std::mutex> lock(g_alloc.mu);
  g_alloc.release_cached_locked();
  return KH_OK;
}

int kh_get_alloc_stats(kh_alloc_stats* out) {
  KH_REQUIRE(out != nullptr, "kh_get_alloc_stats: null output pointer");
  std::lock_guard<std::mutex> lock(g_alloc.mu);
  *out = g_alloc.stats;
  return KH_OK;
}

int kh_memcpy_h2d(void* dst, const void* src, size_t bytes) {
  KH_REQUIRE_INIT();
  if (bytes == 0) return KH_OK;
  KH_REQUIRE(dst && src, "kh_memcpy_h2d: null pointer");
  KH_CHECK_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g_state.stream));
  // The host buffer may be pageable and owned by the caller: wait until it has been consumed.
  KH_CHECK_HIP(hipStreamSynchronize(g_state.stream));
  return KH_OK;
}

int kh_memcpy_d2h(void* dst, const void* src, size_t bytes) {
  KH_REQUIRE_INIT();
  if (bytes == 0) return KH_OK;
  KH_REQUIRE(dst && src, "kh_memcpy_d2h: null pointer");
  KH_CHECK_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g_state.stream));
  KH_CHECK_HIP(hipStreamSynchronize(g_state.stream));
  return KH_OK;
}

int kh_memcpy_d2d(void* dst, const void* src, size_t bytes) {
  KH_REQUIRE_INIT();
  if (bytes == 0) return KH_OK;
  KH_REQUIRE(dst && src, "kh_memcpy_d2d: null pointer");
  KH_CHECK_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, g_state.stream));
  return KH_OK;
}

int kh_synchronize(void) {
  KH_REQUIRE_INIT();
  KH_CHECK_HIP(hipStreamSynchronize(g_state.stream));
  return KH_OK;
}

int kh_event_create(void** event) {
  KH_REQUIRE_INIT();
  KH_REQUIRE(event != nullptr, "kh_event_create: null output pointer");
  hipEvent_t e;
  KH_CHECK_HIP(hipEventCreate(&e));
  *event = (void*)e;
  return KH_OK;
}

int kh_event_destroy(void* event) {
  KH_REQUIRE_INIT();
  if (event) KH_CHECK_HIP(hipEventDestroy((hipEvent_t)event));
  return KH_OK;
}

int kh_event_record(void* event) {
  KH_REQUIRE_INIT();
  KH_REQUIRE(event != nullptr, "kh_event_record: null event");
  KH_CHECK_HIP(hipEventRecord((hipEvent_t)event, g_state.stream));
  return KH_OK;
}

int kh_event_elapsed_ms(void* start, void* stop, float* ms) {
  KH_REQUIRE_INIT();
  KH_REQUIRE(start && stop && ms, "kh_event_elapsed_ms: null argument");
  KH_CHECK_HIP(hipEventSynchronize((hipEvent_t)stop));
  KH_CHECK_HIP(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop));
  return KH_OK;
}

}  // extern "C"
