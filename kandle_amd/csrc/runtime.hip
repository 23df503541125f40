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

struct Pool;
struct GraphObj;

struct State {
  bool init = false;
  int device = -1;
  hipStream_t stream = nullptr;
  GraphObj* capturing = nullptr;  // graph whose stream capture is open
  int debug = 0;                  // kh_set_debug flags
  int cus = 0;                    // compute units of the device
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

// Blocks that belong to one captured graph.  While a capture is open, every allocation comes from
// the capture's pool and every block freed (whoever allocated it) joins that pool, so no address a
// graph replays can be handed to other work before the graph is destroyed.
struct Pool {
  std::multimap<size_t, void*> free_blocks;
  std::unordered_map<void*, size_t> owned;  // every block of the pool, free or live
};

struct Allocator {
  std::mutex mu;
  std::multimap<size_t, void*> free_blocks;   // size -> block
  std::unordered_map<void*, size_t> live;     // block -> size
  std::unordered_map<void*, Pool*> pool_of;   // block -> graph pool (absent: global cache)
  Pool* capture = nullptr;                    // pool of the open capture, if any
  kh_alloc_stats stats{};

  static bool take(std::multimap<size_t, void*>& fl, size_t sz, void** p, size_t* bsz) {
    // The smallest cached block that fits and wastes at most half of itself.
    auto it = fl.lower_bound(sz);
    if (it == fl.end() || it->first > 2 * sz) return false;
    *p = it->second;
    *bsz = it->first;
    fl.erase(it);
    return true;
  }

  void note_live(void* p, size_t bsz) {
    live[p] = bsz;
    stats.live_bytes += bsz;
    if (stats.live_bytes > stats.peak_bytes) stats.peak_bytes = stats.live_bytes;
  }

  int alloc(void** out, size_t bytes) {
    std::lock_guard<std::mutex> lock(mu);
    const size_t sz = round_size(bytes);
    void* p = nullptr;
    size_t bsz = 0;
    if (take(capture ? capture->free_blocks : free_blocks, sz, &p, &bsz)) {
      stats.cached_bytes -= bsz;
      note_live(p, bsz);
      stats.n_cache_hits++;
      *out = p;
      return KH_OK;
    }
    hipError_t e = hipMalloc(&p, sz);
    if (e != hipSuccess && capture == nullptr) {
      (void)hipGetLastError();
      release_cached_locked();
      e = hipMalloc(&p, sz);
    }
    if (e != hipSuccess) {
      (void)hipGetLastError();
      set_error("kh_alloc: out of device memory for %zu bytes (%s)", sz, hipGetErrorString(e));
      return KH_ERR_OOM;
    }
    if (capture) {
      capture->owned[p] = sz;
      pool_of[p] = capture;
    }
    note_live(p, sz);
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
    stats.cached_bytes += sz;
    auto po = pool_of.find(p);
    Pool* pool = po != pool_of.end() ? po->second : capture;
    if (pool == nullptr) {
      free_blocks.emplace(sz, p);
      return KH_OK;
    }
    if (po == pool_of.end()) {  // a global block released inside a capture joins the capture's pool
      pool->owned[p] = sz;
      pool_of[p] = pool;
    }
    pool->free_blocks.emplace(sz, p);
    return KH_OK;
  }

  // Caller holds `mu`.  Waits for the stream so no queued kernel still uses a released block.
  void release_cached_locked() {
    if (g_state.stream) (void)hipStreamSynchronize(g_state.stream);
    for (auto& kv : free_blocks) {
      (void)hipFree(kv.second);
      stats.cached_bytes -= kv.first;
    }
    free_blocks.clear();
  }

  // Caller holds `mu` and has synchronised the stream.  Frees the pool's idle blocks; blocks still
  // live (tensors the caller kept) become ordinary blocks that a later kh_free returns to the cache.
  void release_pool_locked(Pool* pool) {
    for (auto& kv : pool->owned) {
      pool_of.erase(kv.first);
      if (live.find(kv.first) == live.end()) {
        (void)hipFree(kv.first);
        stats.cached_bytes -= kv.second;
      }
    }
    pool->owned.clear();
    pool->free_blocks.clear();
  }
};
Allocator g_alloc;

// A captured, instantiated sequence of library launches plus the device blocks it addresses.
struct GraphObj {
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  Pool pool;
};

#define KH_REQUIRE_NO_CAPTURE(name) \
  KH_REQUIRE(g_state.capturing == nullptr, name ": not allowed while a graph capture is open")

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
int cu_count() { return g_state.cus; }
int current_device() { return g_state.init ? g_state.device : -1; }

bool debug_sync() { return (g_state.debug & 1) != 0 && g_state.capturing == nullptr && g_state.stream != nullptr; }

int debug_check(const char* where, const char* file, int line) {
  const hipError_t e = hipStreamSynchronize(g_state.stream);
  const hipError_t e2 = hipGetLastError();
  if (e != hipSuccess || e2 != hipSuccess) {
    set_error("%s: a kernel it launched failed on the device: %s (%s:%d; debug mode)", where,
              hipGetErrorString(e != hipSuccess ? e : e2), file, line);
    return KH_ERR_HIP;
  }
  return KH_OK;
}

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
  KH_CHECK_HIP(hipDeviceGetAttribute(&g_state.cus, hipDeviceAttributeMultiprocessorCount, device));
  const int rc = attention_init(device);
  if (rc != KH_OK) return rc;
  KH_CHECK_HIP(hipStreamCreateWithFlags(&g_state.stream, hipStreamNonBlocking));
  g_state.device = device;
  g_state.init = true;
  return KH_OK;
}

const char* kh_last_error(void) { return g_err; }

int kh_set_debug(int flags) {
  KH_REQUIRE(flags >= 0 && flags <= 1, "kh_set_debug: unknown flags %d", flags);
  g_state.debug = flags;
  return KH_OK;
}

int kh_is_capturing(void) { return g_state.capturing != nullptr ? 1 : 0; }

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
  KH_REQUIRE_NO_CAPTURE("kh_empty_cache");
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
  KH_REQUIRE_NO_CAPTURE("kh_memcpy_h2d");
  if (bytes == 0) return KH_OK;
  KH_REQUIRE(dst && src, "kh_memcpy_h2d: null pointer");
  KH_CHECK_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g_state.stream));
  // The host buffer may be pageable and owned by the caller: wait until it has been consumed.
  KH_CHECK_HIP(hipStreamSynchronize(g_state.stream));
  return KH_OK;
}

int kh_memcpy_d2h(void* dst, const void* src, size_t bytes) {
  KH_REQUIRE_INIT();
  KH_REQUIRE_NO_CAPTURE("kh_memcpy_d2h");
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
  KH_REQUIRE_NO_CAPTURE("kh_synchronize");
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

int kh_graph_begin_capture(void) {
  KH_REQUIRE_INIT();
  KH_REQUIRE_NO_CAPTURE("kh_graph_begin_capture");
  GraphObj* g = new GraphObj();
  {
    std::lock_guard<std::mutex> lock(g_alloc.mu);
    g_alloc.capture = &g->pool;
  }
  const hipError_t e = hipStreamBeginCapture(g_state.stream, hipStreamCaptureModeRelaxed);
  if (e != hipSuccess) {
    std::lock_guard<std::mutex> lock(g_alloc.mu);
    g_alloc.capture = nullptr;
    delete g;
    set_error("kh_graph_begin_capture: hipStreamBeginCapture failed: %s", hipGetErrorString(e));
    return KH_ERR_HIP;
  }
  g_state.capturing = g;
  return KH_OK;
}

int kh_graph_end_capture(void** graph) {
  KH_REQUIRE_INIT();
  KH_REQUIRE(g_state.capturing != nullptr, "kh_graph_end_capture: no capture is open");
  GraphObj* g = g_state.capturing;
  g_state.capturing = nullptr;
  hipError_t e = hipStreamEndCapture(g_state.stream, &g->graph);
  {
    std::lock_guard<std::mutex> lock(g_alloc.mu);
    g_alloc.capture = nullptr;
  }
  if (e == hipSuccess && graph == nullptr) e = hipErrorInvalidValue;
  if (e == hipSuccess) e = hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    kh_graph_destroy(g);
    set_error("kh_graph_end_capture: capture or instantiation failed: %s", hipGetErrorString(e));
    return KH_ERR_HIP;
  }
  *graph = g;
  return KH_OK;
}

int kh_graph_launch(void* graph) {
  KH_REQUIRE_INIT();
  KH_REQUIRE_NO_CAPTURE("kh_graph_launch");
  KH_REQUIRE(graph != nullptr && ((GraphObj*)graph)->exec != nullptr, "kh_graph_launch: not an instantiated graph");
  KH_CHECK_HIP(hipGraphLaunch(((GraphObj*)graph)->exec, g_state.stream));
  return KH_OK;
}

int kh_graph_destroy(void* graph) {
  KH_REQUIRE_INIT();
  if (graph == nullptr) return KH_OK;
  KH_REQUIRE(graph != (void*)g_state.capturing, "kh_graph_destroy: the graph's capture is still open");
  GraphObj* g = (GraphObj*)graph;
  KH_CHECK_HIP(hipStreamSynchronize(g_state.stream));
  if (g->exec) (void)hipGraphExecDestroy(g->exec);
  if (g->graph) (void)hipGraphDestroy(g->graph);
  {
    std::lock_guard<std::mutex> lock(g_alloc.mu);
    g_alloc.release_pool_locked(&g->pool);
  }
  delete g;
  return KH_OK;
}

}  // extern "C"
