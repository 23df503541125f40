/*
 * addon.c — the N-API addon of Kandle's HIP backend (packages/backend-hip): one JavaScript function
 * per entry point of the C ABI in include/kandle_hip.h, for the TypeScript HipBackend that
 * registers the kernels with Kandle's operator registry (packages/types/src/backend/register.ts:
 * 102-144; the sibling plugin packages/backend-webgpu/src/index.ts:15-87).
 *
 * Conventions:
 *  - device pointers are BigInt (0n, null or undefined pass NULL where the C ABI allows it);
 *  - counts, extents and strides are Numbers (integers) or BigInts; stride lists are JS arrays;
 *  - host buffers are ArrayBuffers or typed arrays (memcpyH2D / memcpyD2H copy their bytes);
 *  - a non-zero return code throws a JS Error carrying kh_last_error() and a `code` property,
 *    the reference's convention of throwing from a kernel (packages/core/src/dispatch/handlers/
 *    normalize.ts:57-59); a wrong argument type throws a TypeError before any C call.
 * Built for Node 12 (N-API 8) with gcc against /usr/include/node; no node-gyp.
 */
#define NAPI_VERSION 8
#include <node_api.h>
#include <stdbool.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "kandle_hip.h"

#define MAX_ARGS 24
#define MAX_LIST 32

typedef struct {
  napi_env env;
  napi_value v[MAX_ARGS];
  size_t n;
  const char* fn;
  bool bad;
} Args;

static void type_error(Args* A, size_t i, const char* want) {
  if (A->bad) return;
  char msg[160];
  snprintf(msg, sizeof msg, "kandle_hip.%s: argument %zu must be %s", A->fn, i, want);
  napi_throw_type_error(A->env, NULL, msg);
  A->bad = true;
}

static napi_valuetype type_of(Args* A, size_t i) {
  napi_valuetype t = napi_undefined;
  if (i < A->n) napi_typeof(A->env, A->v[i], &t);
  return t;
}

/* A device pointer: BigInt, or null / undefined / 0 for NULL. */
static void* arg_ptr(Args* A, size_t i) {
  const napi_valuetype t = type_of(A, i);
  if (t == napi_null || t == napi_undefined) return NULL;
  if (t == napi_bigint) {
    uint64_t x = 0;
    bool lossless = false;
    napi_get_value_bigint_uint64(A->env, A->v[i], &x, &lossless);
    if (!lossless) type_error(A, i, "a device pointer (BigInt below 2^64)");
    return (void*)(uintptr_t)x;
  }
  if (t == napi_number) {
    double d = 0;
    napi_get_value_double(A->env, A->v[i], &d);
    if (d == 0) return NULL;
  }
  type_error(A, i, "a device pointer (BigInt, or null)");
  return NULL;
}

static int64_t arg_i64(Args* A, size_t i) {
  const napi_valuetype t = type_of(A, i);
  if (t == napi_number) {
    double d = 0;
    napi_get_value_double(A->env, A->v[i], &d);
    if (d == (double)(int64_t)d) return (int64_t)d;
  } else if (t == napi_bigint) {
    int64_t x = 0;
    bool lossless = false;
    napi_get_value_bigint_int64(A->env, A->v[i], &x, &lossless);
    if (lossless) return x;
  }
  type_error(A, i, "an integer (Number or BigInt)");
  return 0;
}

static int arg_int(Args* A, size_t i) {
  const int64_t x = arg_i64(A, i);
  if (x < INT32_MIN || x > INT32_MAX) type_error(A, i, "a 32-bit integer");
  return (int)x;
}

static uint64_t arg_u64(Args* A, size_t i) {
  if (type_of(A, i) == napi_bigint) {
    uint64_t x = 0;
    bool lossless = false;
    napi_get_value_bigint_uint64(A->env, A->v[i], &x, &lossless);
    if (lossless) return x;
  } else if (type_of(A, i) == napi_number) {
    const int64_t x = arg_i64(A, i);
    if (x >= 0) return (uint64_t)x;
  }
  type_error(A, i, "an unsigned 64-bit integer (Number or BigInt)");
  return 0;
}

static double arg_f64(Args* A, size_t i) {
  if (type_of(A, i) != napi_number) {
    type_error(A, i, "a number");
    return 0;
  }
  double d = 0;
  napi_get_value_double(A->env, A->v[i], &d);
  return d;
}

static int arg_flag(Args* A, size_t i) {
  const napi_valuetype t = type_of(A, i);
  if (t == napi_boolean) {
    bool b = false;
    napi_get_value_bool(A->env, A->v[i], &b);
    return b ? 1 : 0;
  }
  return arg_int(A, i) != 0;
}

/* A JS array of exactly n integers (n <= MAX_LIST) into out. */
static const int64_t* arg_list(Args* A, size_t i, int64_t* out, uint32_t n) {
  bool is_array = false;
  if (i < A->n) napi_is_array(A->env, A->v[i], &is_array);
  uint32_t len = 0;
  if (is_array) napi_get_array_length(A->env, A->v[i], &len);
  if (!is_array || len != n || n > MAX_LIST) {
    char want[64];
    snprintf(want, sizeof want, "an array of %u integers", n);
    type_error(A, i, want);
    return out;
  }
  for (uint32_t k = 0; k < n && !A->bad; ++k) {
    Args E = {A->env, {0}, 1, A->fn, false};
    napi_get_element(A->env, A->v[i], k, &E.v[0]);
    out[k] = arg_i64(&E, 0);
    if (E.bad) A->bad = true;
  }
  return out;
}

/* An array of at most `max` integers: returns its length, or -1 after a TypeError. */
static int arg_list_upto(Args* A, size_t i, int64_t* out, uint32_t max) {
  bool is_array = false;
  if (i < A->n) napi_is_array(A->env, A->v[i], &is_array);
  uint32_t len = 0;
  if (is_array) napi_get_array_length(A->env, A->v[i], &len);
  if (!is_array || len > max || max > MAX_LIST) {
    char want[64];
    snprintf(want, sizeof want, "an array of at most %u integers", max);
    type_error(A, i, want);
    return -1;
  }
  arg_list(A, i, out, len);
  return A->bad ? -1 : (int)len;
}

/* The bytes of an ArrayBuffer or of a typed array's view. */
static void* arg_host(Args* A, size_t i, size_t* len) {
  *len = 0;
  if (i >= A->n) {
    type_error(A, i, "an ArrayBuffer or typed array");
    return NULL;
  }
  bool yes = false;
  void* data = NULL;
  napi_is_arraybuffer(A->env, A->v[i], &yes);
  if (yes) {
    napi_get_arraybuffer_info(A->env, A->v[i], &data, len);
    return data;
  }
  napi_is_typedarray(A->env, A->v[i], &yes);
  if (yes) {
    napi_typedarray_type tt;
    size_t count = 0, off = 0;
    napi_value ab;
    napi_get_typedarray_info(A->env, A->v[i], &tt, &count, &data, &ab, &off);
    size_t es = 1;
    switch (tt) {
      case napi_int16_array: case napi_uint16_array: es = 2; break;
      case napi_int32_array: case napi_uint32_array: case napi_float32_array: es = 4; break;
      case napi_float64_array: case napi_bigint64_array: case napi_biguint64_array: es = 8; break;
      default: es = 1;
    }
    *len = count * es;
    return data;
  }
  type_error(A, i, "an ArrayBuffer or typed array");
  return NULL;
}

static bool begin(Args* A, napi_env env, napi_callback_info info, const char* fn, size_t want) {
  A->env = env;
  A->fn = fn;
  A->bad = false;
  A->n = MAX_ARGS;
  napi_get_cb_info(env, info, &A->n, A->v, NULL, NULL);
  /* napi reports the count the caller passed, which may exceed the capacity of v: only the first
     MAX_ARGS values were stored, so reads past them must see "no argument" */
  if (A->n > MAX_ARGS) A->n = MAX_ARGS;
  if (want > MAX_ARGS) {
    napi_throw_error(env, NULL, "kandle_hip: a binding declares more arguments than MAX_ARGS");
    return false;
  }
  if (A->n < want) {
    char msg[128];
    snprintf(msg, sizeof msg, "kandle_hip.%s: expected %zu arguments, got %zu", fn, want, A->n);
    napi_throw_type_error(env, NULL, msg);
    return false;
  }
  return true;
}

/* Throws an Error with kh_last_error() (and .code) for a non-zero return code. */
static napi_value done(Args* A, int rc) {
  if (rc == KH_OK) return NULL;
  char code[16];
  snprintf(code, sizeof code, "KH_%d", rc);
  napi_throw_error(A->env, code, kh_last_error());
  return NULL;
}

static napi_value big_ptr(napi_env env, void* p) {
  napi_value out;
  napi_create_bigint_uint64(env, (uint64_t)(uintptr_t)p, &out);
  return out;
}

#define FN(js, want) \
  static napi_value js_##js(napi_env env, napi_callback_info info) { \
    Args A_, *A = &A_; \
    if (!begin(A, env, info, #js, want)) return NULL;
#define CALL(expr) \
  if (A->bad) return NULL; \
  return done(A, (expr)); \
  }

/* ---------------------------------------------------------------- runtime ---------------------- */
FN(init, 1) int dev = arg_int(A, 0); CALL(kh_init(dev))

FN(setDebug, 1) int f = arg_int(A, 0); CALL(kh_set_debug(f))

static napi_value js_deviceCount(napi_env env, napi_callback_info info) {
  (void)info;
  int n = 0;
  kh_device_count(&n);
  napi_value out;
  napi_create_int32(env, n, &out);
  return out;
}

static napi_value js_isCapturing(napi_env env, napi_callback_info info) {
  (void)info;
  napi_value out;
  napi_get_boolean(env, kh_is_capturing() != 0, &out);
  return out;
}

static napi_value js_lastError(napi_env env, napi_callback_info info) {
  (void)info;
  napi_value out;
  napi_create_string_utf8(env, kh_last_error(), NAPI_AUTO_LENGTH, &out);
  return out;
}

static napi_value js_alloc(napi_env env, napi_callback_info info) {
  Args A_, *A = &A_;
  if (!begin(A, env, info, "alloc", 1)) return NULL;
  const int64_t bytes = arg_i64(A, 0);
  if (A->bad) return NULL;
  void* p = NULL;
  if (bytes < 0 || kh_alloc(&p, (size_t)bytes) != KH_OK) {
    if (bytes < 0) type_error(A, 0, "a byte count >= 0");
    else done(A, 1);
    return NULL;
  }
  return big_ptr(env, p);
}

FN(free, 1) void* p = arg_ptr(A, 0); CALL(kh_free(p))

/* Owned device blocks.  allocOwned(bytes) returns an external object that holds the block;
   freeOwned(ext) returns it to the allocator (once; later calls do nothing), and the object's
   finalizer -- run by the garbage collector after the object becomes unreachable -- returns a
   block that was never freed: the safety net of a storage whose dispose() was forgotten (Node 12
   has no FinalizationRegistry).  ownedPtr(ext) is the block's address as a BigInt.
   An external made elsewhere (another addon) is told apart by the tag and the self pointer
   written at creation: Node 12 has no napi_type_tag_object. */
#define OWNED_TAG 0x6b68426c6f636b31ULL /* "khBlock1" */
typedef struct {
  uint64_t tag;
  const void* self;
  void* p;
  int live;
} Owned;

static void owned_finalize(napi_env env, void* data, void* hint) {
  (void)env;
  (void)hint;
  Owned* o = (Owned*)data;
  if (o->live) kh_free(o->p);
  o->tag = 0;
  free(o);
}

static Owned* arg_owned(Args* A, size_t i) {
  void* d = NULL;
  if (type_of(A, i) != napi_external || napi_get_value_external(A->env, A->v[i], &d) != napi_ok || d == NULL ||
      ((Owned*)d)->tag != OWNED_TAG || ((Owned*)d)->self != d) {
    type_error(A, i, "an owned block (from allocOwned)");
    return NULL;
  }
  return (Owned*)d;
}

static napi_value js_allocOwned(napi_env env, napi_callback_info info) {
  Args A_, *A = &A_;
  if (!begin(A, env, info, "allocOwned", 1)) return NULL;
  const int64_t bytes = arg_i64(A, 0);
  if (A->bad) return NULL;
  if (bytes < 0) {
    type_error(A, 0, "a byte count >= 0");
    return NULL;
  }
  void* p = NULL;
  const int rc = kh_alloc(&p, (size_t)bytes);
  if (rc != KH_OK) return done(A, rc);
  Owned* o = (Owned*)malloc(sizeof(Owned));
  napi_value ext;
  if (o == NULL) {
    kh_free(p);
    napi_throw_error(env, NULL, "kandle_hip.allocOwned: out of host memory");
    return NULL;
  }
  o->tag = OWNED_TAG;
  o->self = o;
  o->p = p;
  o->live = 1;
  if (napi_create_external(env, o, owned_finalize, NULL, &ext) != napi_ok) {
    kh_free(p);
    free(o);
    napi_throw_error(env, NULL, "kandle_hip.allocOwned: napi_create_external failed");
    return NULL;
  }
  return ext;
}

static napi_value js_ownedPtr(napi_env env, napi_callback_info info) {
  Args A_, *A = &A_;
  if (!begin(A, env, info, "ownedPtr", 1)) return NULL;
  Owned* o = arg_owned(A, 0);
  if (A->bad) return NULL;
  return big_ptr(env, o->live ? o->p : NULL);
}

static napi_value js_freeOwned(napi_env env, napi_callback_info info) {
  Args A_, *A = &A_;
  if (!begin(A, env, info, "freeOwned", 1)) return NULL;
  Owned* o = arg_owned(A, 0);
  if (A->bad) return NULL;
  if (!o->live) return NULL;
  o->live = 0;
  return done(A, kh_free(o->p));
}
FN(emptyCache, 0) CALL(kh_empty_cache())
FN(synchronize, 0) CALL(kh_synchronize())

static napi_value js_allocStats(napi_env env, napi_callback_info info) {
  Args A_, *A = &A_;
  if (!begin(A, env, info, "allocStats", 0)) return NULL;
  kh_alloc_stats s;
  if (kh_get_alloc_stats(&s) != KH_OK) return done(A, KH_ERR_INVALID);
  napi_value o, v;
  napi_create_object(env, &o);
  const char* names[] = {"liveBytes", "cachedBytes", "peakBytes", "nDeviceAllocs", "nCacheHits"};
  const uint64_t vals[] = {s.live_bytes, s.cached_bytes, s.peak_bytes, s.n_device_allocs, s.n_cache_hits};
  for (int i = 0; i < 5; ++i) {
    napi_create_double(env, (double)vals[i], &v);
    napi_set_named_property(env, o, names[i], v);
  }
  return o;
}

/* memcpyH2D(dstPtr, hostBuffer) / memcpyD2H(hostBuffer, srcPtr): the host buffer's bytes. */
FN(memcpyH2D, 2) void* d = arg_ptr(A, 0); size_t n = 0; void* h = arg_host(A, 1, &n); CALL(kh_memcpy_h2d(d, h, n))
FN(memcpyD2H, 2) size_t n = 0; void* h = arg_host(A, 0, &n); void* s = arg_ptr(A, 1); CALL(kh_memcpy_d2h(h, s, n))
FN(memcpyD2D, 3)
  void* d = arg_ptr(A, 0); void* s = arg_ptr(A, 1); int64_t n = arg_i64(A, 2);
  CALL(kh_memcpy_d2d(d, s, (size_t)n))

static napi_value js_eventCreate(napi_env env, napi_callback_info info) {
  Args A_, *A = &A_;
  if (!begin(A, env, info, "eventCreate", 0)) return NULL;
  void* e = NULL;
  if (kh_event_create(&e) != KH_OK) return done(A, KH_ERR_HIP);
  return big_ptr(env, e);
}
FN(eventDestroy, 1) void* e = arg_ptr(A, 0); CALL(kh_event_destroy(e))
FN(eventRecord, 1) void* e = arg_ptr(A, 0); CALL(kh_event_record(e))

static napi_value js_eventElapsedMs(napi_env env, napi_callback_info info) {
  Args A_, *A = &A_;
  if (!begin(A, env, info, "eventElapsedMs", 2)) return NULL;
  void* a = arg_ptr(A, 0);
  void* b = arg_ptr(A, 1);
  if (A->bad) return NULL;
  float ms = 0.f;
  const int rc = kh_event_elapsed_ms(a, b, &ms);
  if (rc != KH_OK) return done(A, rc);
  napi_value out;
  napi_create_double(env, ms, &out);
  return out;
}

FN(graphBeginCapture, 0) CALL(kh_graph_begin_capture())

static napi_value js_graphEndCapture(napi_env env, napi_callback_info info) {
  Args A_, *A = &A_;
  if (!begin(A, env, info, "graphEndCapture", 0)) return NULL;
  void* g = NULL;
  const int rc = kh_graph_end_capture(&g);
  if (rc != KH_OK) return done(A, rc);
  return big_ptr(env, g);
}
FN(graphLaunch, 1) void* g = arg_ptr(A, 0); CALL(kh_graph_launch(g))
FN(graphDestroy, 1) void* g = arg_ptr(A, 0); CALL(kh_graph_destroy(g))

/* ---------------------------------------------------------------- support ops ------------------ */
FN(fill, 4)
  void* d = arg_ptr(A, 0); int64_t n = arg_i64(A, 1); double v = arg_f64(A, 2); int dt = arg_int(A, 3);
  CALL(kh_fill(d, n, (float)v, dt))
/* copyStrided(src, srcOffset, dst, shape[], srcStrides[], dtypeSrc, dtypeDst) */
FN(copyStrided, 7)
  int64_t shape[6], st[6];
  void* s = arg_ptr(A, 0); int64_t off = arg_i64(A, 1); void* d = arg_ptr(A, 2);
  uint32_t nd = 0;
  bool arr = false;
  if (A->n > 3) napi_is_array(env, A->v[3], &arr);
  if (arr) napi_get_array_length(env, A->v[3], &nd);
  if (!arr || nd > 6) type_error(A, 3, "an array of at most 6 extents");
  if (!A->bad) { arg_list(A, 3, shape, nd); arg_list(A, 4, st, nd); }
  int ds = arg_int(A, 5), dd = arg_int(A, 6);
  CALL(kh_copy_strided(s, off, d, (int)nd, shape, st, ds, dd))
FN(binary, 6)
  int op = arg_int(A, 0); void* a = arg_ptr(A, 1); void* b = arg_ptr(A, 2); void* o = arg_ptr(A, 3);
  int64_t n = arg_i64(A, 4); int dt = arg_int(A, 5);
  CALL(kh_binary(op, a, b, o, n, dt))
FN(silu, 4) void* x = arg_ptr(A, 0); void* o = arg_ptr(A, 1); int64_t n = arg_i64(A, 2); int dt = arg_int(A, 3);
  CALL(kh_silu(x, o, n, dt))
FN(unary, 5)
  int op = arg_int(A, 0); void* x = arg_ptr(A, 1); void* o = arg_ptr(A, 2); int64_t n = arg_i64(A, 3);
  int dt = arg_int(A, 4);
  CALL(kh_unary(op, x, o, n, dt))
FN(arange, 5)
  void* o = arg_ptr(A, 0); int64_t n = arg_i64(A, 1); double s0 = arg_f64(A, 2); double st = arg_f64(A, 3);
  int dt = arg_int(A, 4);
  CALL(kh_arange(o, n, s0, st, dt))
/* siluMul(gate, gateRowStride, up, upRowStride, out, outRowStride, rows, n, dtype) */
FN(siluMul, 9)
  void* g = arg_ptr(A, 0); int64_t gs = arg_i64(A, 1); void* u = arg_ptr(A, 2); int64_t us = arg_i64(A, 3);
  void* o = arg_ptr(A, 4); int64_t os = arg_i64(A, 5); int64_t rows = arg_i64(A, 6); int64_t n = arg_i64(A, 7);
  int dt = arg_int(A, 8);
  CALL(kh_silu_mul(g, gs, u, us, o, os, rows, n, dt))
/* indexSelect(table, nRows, idx, nIdx, rowElems, out, dtype, outDtype) */
FN(indexSelect, 8)
  void* t = arg_ptr(A, 0); int64_t nr = arg_i64(A, 1); void* idx = arg_ptr(A, 2); int64_t ni = arg_i64(A, 3);
  int64_t re = arg_i64(A, 4); void* o = arg_ptr(A, 5); int dt = arg_int(A, 6); int odt = arg_int(A, 7);
  CALL(kh_index_select(t, nr, (const int32_t*)idx, ni, re, o, dt, odt))
/* indexSelectDim(table, outer, nRows, inner, idx, nIdx, out, dtype, outDtype) */
FN(indexSelectDim, 9)
  void* t = arg_ptr(A, 0); int64_t outer = arg_i64(A, 1); int64_t nr = arg_i64(A, 2); int64_t inner = arg_i64(A, 3);
  void* idx = arg_ptr(A, 4); int64_t ni = arg_i64(A, 5); void* o = arg_ptr(A, 6); int dt = arg_int(A, 7);
  int odt = arg_int(A, 8);
  CALL(kh_index_select_dim(t, outer, nr, inner, (const int32_t*)idx, ni, o, dt, odt))
FN(argmax, 5)
  void* x = arg_ptr(A, 0); int64_t rows = arg_i64(A, 1); int64_t n = arg_i64(A, 2); void* o = arg_ptr(A, 3);
  int dt = arg_int(A, 4);
  CALL(kh_argmax(x, rows, n, (int32_t*)o, dt))
FN(greedyAdvance, 6)
  void* nt = arg_ptr(A, 0); void* pos = arg_ptr(A, 1); void* sl = arg_ptr(A, 2); void* log = arg_ptr(A, 3);
  int64_t base = arg_i64(A, 4); int64_t cap = arg_i64(A, 5);
  CALL(kh_greedy_advance((const int32_t*)nt, (int32_t*)pos, (int32_t*)sl, (int32_t*)log, base, cap))
/* sample(logits, vocab, doSample, temperature, topK, topP, seed, counter, token, logprob, displayK,
          displayIds, displayProbs) */
FN(sample, 13)
  void* lg = arg_ptr(A, 0); int64_t v = arg_i64(A, 1); int ds = arg_flag(A, 2); double t = arg_f64(A, 3);
  int tk = arg_int(A, 4); double tp = arg_f64(A, 5); uint64_t seed = arg_u64(A, 6); void* ctr = arg_ptr(A, 7);
  void* tok = arg_ptr(A, 8); void* lp = arg_ptr(A, 9); int dk = arg_int(A, 10); void* di = arg_ptr(A, 11);
  void* dp = arg_ptr(A, 12);
  CALL(kh_sample((const float*)lg, v, ds, t, tk, tp, seed, (const int32_t*)ctr, (int32_t*)tok, (float*)lp, dk,
                 (int32_t*)di, (float*)dp))
FN(sampleSetPath, 1) int p = arg_int(A, 0); CALL(kh_sample_set_path(p))
FN(philox4x32_10, 4)
  uint64_t seed = arg_u64(A, 0); void* c = arg_ptr(A, 1); int64_t n = arg_i64(A, 2); void* o = arg_ptr(A, 3);
  CALL(kh_philox4x32_10(seed, (const uint32_t*)c, n, (uint32_t*)o))
/* decodeAttentionBlock(qkv, qNormW, kNormW, invFreq, eps, position, kCache, vCache, hq, hkv, maxLen,
                        cacheStrides[4], scale, wO, ldw, nOut, x, dtype) */
FN(decodeAttentionBlock, 18)
  int64_t cs[4];
  void* qkv = arg_ptr(A, 0); void* qn = arg_ptr(A, 1); void* kn = arg_ptr(A, 2); void* inv = arg_ptr(A, 3);
  double eps = arg_f64(A, 4); void* pos = arg_ptr(A, 5); void* kc = arg_ptr(A, 6); void* vc = arg_ptr(A, 7);
  int hq = arg_int(A, 8); int hkv = arg_int(A, 9); int64_t ml = arg_i64(A, 10); arg_list(A, 11, cs, 4);
  double sc = arg_f64(A, 12); void* wo = arg_ptr(A, 13); int64_t ldw = arg_i64(A, 14); int64_t no = arg_i64(A, 15);
  void* x = arg_ptr(A, 16); int dt = arg_int(A, 17);
  CALL(kh_decode_attention_block(qkv, qn, kn, (const float*)inv, (float)eps, (const int32_t*)pos, kc, vc, hq, hkv,
                                 ml, cs, (float)sc, wo, ldw, no, (float*)x, dt))

/* mapStrided(op, shape[], out, outStrides[], outDtype, a, aStrides[], aDtype, b, bStrides[], bDtype, s0, s1):
   an elementwise op over `shape` with every operand addressed by its own element strides (Kandle's
   iterator kernel contract, tensor.ts:282-378); a / b may be null when the op does not read them */
FN(mapStrided, 13)
  int64_t sh[MAX_LIST], so[MAX_LIST], sa[MAX_LIST], sb[MAX_LIST];
  int op = arg_int(A, 0);
  const int nd = arg_list_upto(A, 1, sh, 8);
  const uint32_t n = nd < 0 ? 0 : (uint32_t)nd;
  void* o = arg_ptr(A, 2);
  arg_list(A, 3, so, n);
  int odt = arg_int(A, 4);
  void* a = arg_ptr(A, 5);
  if (a != NULL) arg_list(A, 6, sa, n);
  int adt = arg_int(A, 7);
  void* b = arg_ptr(A, 8);
  if (b != NULL) arg_list(A, 9, sb, n);
  int bdt = arg_int(A, 10);
  double s0 = arg_f64(A, 11), s1 = arg_f64(A, 12);
  CALL(kh_map_strided(op, (int)n, sh, o, so, odt, a, a != NULL ? sa : NULL, adt, b, b != NULL ? sb : NULL, bdt, s0,
                      s1))

/* ---------------------------------------------------------------- hot path --------------------- */
/* rmsNorm(x, xRowStride, w, y, yRowStride, rows, n, eps, dtype, outDtype) */
FN(rmsNorm, 10)
  void* x = arg_ptr(A, 0); int64_t xs = arg_i64(A, 1); void* w = arg_ptr(A, 2); void* y = arg_ptr(A, 3);
  int64_t ys = arg_i64(A, 4); int64_t rows = arg_i64(A, 5); int64_t n = arg_i64(A, 6); double eps = arg_f64(A, 7);
  int dt = arg_int(A, 8); int odt = arg_int(A, 9);
  CALL(kh_rms_norm(x, xs, w, y, ys, rows, n, (float)eps, dt, odt))
/* qkNormRope(q, k, qOut, kOut, v, vOut, wq, wk, invFreq, positions, nBatch, seqLen, nQHeads, nKvHeads,
              headDim, strides[12 or 18], eps, dtype, kvCacheLen) */
FN(qkNormRope, 19)
  int64_t st[18];
  void* q = arg_ptr(A, 0); void* k = arg_ptr(A, 1); void* qo = arg_ptr(A, 2); void* ko = arg_ptr(A, 3);
  void* v = arg_ptr(A, 4); void* vo = arg_ptr(A, 5); void* wq = arg_ptr(A, 6); void* wk = arg_ptr(A, 7);
  void* inv = arg_ptr(A, 8); void* pos = arg_ptr(A, 9); int64_t nb = arg_i64(A, 10); int64_t sl = arg_i64(A, 11);
  int hq = arg_int(A, 12); int hkv = arg_int(A, 13); int hd = arg_int(A, 14);
  arg_list(A, 15, st, v != NULL ? 18 : 12);
  double eps = arg_f64(A, 16); int dt = arg_int(A, 17); int64_t kvl = arg_i64(A, 18);
  CALL(kh_qk_norm_rope(q, k, qo, ko, v, vo, wq, wk, (const float*)inv, (const int32_t*)pos, nb, sl, hq, hkv, hd, st,
                       (float)eps, dt, kvl))
/* flashAttention(q, k, v, o, batch, hq, hkv, lq, lk, d, strides[12], scale, causal, dtype): the
   flash_attention kernel signature (q, k, v, out, scale, isCausal) of register.ts:102-109 with the
   shapes and element strides the TypeScript side reads from the handles */
FN(flashAttention, 14)
  int64_t st[12];
  void* q = arg_ptr(A, 0); void* k = arg_ptr(A, 1); void* v = arg_ptr(A, 2); void* o = arg_ptr(A, 3);
  int b = arg_int(A, 4); int hq = arg_int(A, 5); int hkv = arg_int(A, 6); int64_t lq = arg_i64(A, 7);
  int64_t lk = arg_i64(A, 8); int d = arg_int(A, 9); arg_list(A, 10, st, 12); double sc = arg_f64(A, 11);
  int causal = arg_flag(A, 12); int dt = arg_int(A, 13);
  CALL(kh_flash_attention(q, k, v, o, b, hq, hkv, lq, lk, d, st, (float)sc, causal, dt))
/* flashAttentionSplit(q, k, v, o, batch, hq, hkv, lq, lk, d, strides[12], scale, causal): fp32
   attention in split-bf16 form (kh_flash_attention_split) */
FN(flashAttentionSplit, 13)
  int64_t st[12];
  void* q = arg_ptr(A, 0); void* k = arg_ptr(A, 1); void* v = arg_ptr(A, 2); void* o = arg_ptr(A, 3);
  int b = arg_int(A, 4); int hq = arg_int(A, 5); int hkv = arg_int(A, 6); int64_t lq = arg_i64(A, 7);
  int64_t lk = arg_i64(A, 8); int d = arg_int(A, 9); arg_list(A, 10, st, 12); double sc = arg_f64(A, 11);
  int causal = arg_flag(A, 12);
  CALL(kh_flash_attention_split(q, k, v, o, b, hq, hkv, lq, lk, d, st, (float)sc, causal))
/* flashAttentionMasked(q, k, v, o, batch, hq, hkv, lq, lk, d, strides[12], scale, mask, maskStrides[4],
                        maskDtype, dtype): the attnMask route of composite.ts:279-300 in one call */
FN(flashAttentionMasked, 16)
  int64_t st[12], ms[4];
  void* q = arg_ptr(A, 0); void* k = arg_ptr(A, 1); void* v = arg_ptr(A, 2); void* o = arg_ptr(A, 3);
  int b = arg_int(A, 4); int hq = arg_int(A, 5); int hkv = arg_int(A, 6); int64_t lq = arg_i64(A, 7);
  int64_t lk = arg_i64(A, 8); int d = arg_int(A, 9); arg_list(A, 10, st, 12); double sc = arg_f64(A, 11);
  void* m = arg_ptr(A, 12); arg_list(A, 13, ms, 4); int mdt = arg_int(A, 14); int dt = arg_int(A, 15);
  CALL(kh_flash_attention_masked(q, k, v, o, b, hq, hkv, lq, lk, d, st, (float)sc, m, ms, mdt, dt))
/* decodeAttention(q, kCache, vCache, o, seqLens, batch, hq, hkv, d, maxLen, strides[10], scale, dtype) */
FN(decodeAttention, 13)
  int64_t st[10];
  void* q = arg_ptr(A, 0); void* kc = arg_ptr(A, 1); void* vc = arg_ptr(A, 2); void* o = arg_ptr(A, 3);
  void* sl = arg_ptr(A, 4); int b = arg_int(A, 5); int hq = arg_int(A, 6); int hkv = arg_int(A, 7);
  int d = arg_int(A, 8); int64_t ml = arg_i64(A, 9); arg_list(A, 10, st, 10); double sc = arg_f64(A, 11);
  int dt = arg_int(A, 12);
  CALL(kh_decode_attention(q, kc, vc, o, (const int32_t*)sl, b, hq, hkv, d, ml, st, (float)sc, dt))
/* decodeAttentionNoalloc: decodeAttention's arguments, no device allocation */
FN(decodeAttentionNoalloc, 13)
  int64_t st[10];
  void* q = arg_ptr(A, 0); void* kc = arg_ptr(A, 1); void* vc = arg_ptr(A, 2); void* o = arg_ptr(A, 3);
  void* sl = arg_ptr(A, 4); int b = arg_int(A, 5); int hq = arg_int(A, 6); int hkv = arg_int(A, 7);
  int d = arg_int(A, 8); int64_t ml = arg_i64(A, 9); arg_list(A, 10, st, 10); double sc = arg_f64(A, 11);
  int dt = arg_int(A, 12);
  CALL(kh_decode_attention_noalloc(q, kc, vc, o, (const int32_t*)sl, b, hq, hkv, d, ml, st, (float)sc, dt))
/* gemm(a, lda, b, ldb, c, ldc, cin, ldcin, bias, m, n, k, alpha, beta, transB, dtype, outDtype): the
   matmul kernel's mm path with its alpha / beta / C epilogue (matmulOps.ts:32-125) */
FN(gemm, 17)
  void* a = arg_ptr(A, 0); int64_t lda = arg_i64(A, 1); void* b = arg_ptr(A, 2); int64_t ldb = arg_i64(A, 3);
  void* c = arg_ptr(A, 4); int64_t ldc = arg_i64(A, 5); void* cin = arg_ptr(A, 6); int64_t ldcin = arg_i64(A, 7);
  void* bias = arg_ptr(A, 8); int64_t m = arg_i64(A, 9); int64_t n = arg_i64(A, 10); int64_t k = arg_i64(A, 11);
  double al = arg_f64(A, 12); double be = arg_f64(A, 13); int tb = arg_flag(A, 14); int dt = arg_int(A, 15);
  int odt = arg_int(A, 16);
  CALL(kh_gemm(a, lda, b, ldb, c, ldc, cin, ldcin, bias, m, n, k, (float)al, (float)be, tb, dt, odt))
/* gemmEx(a, lda, aDtype, b, ldb, bDtype, c, ldc, cin, ldcin, bias, m, n, k, alpha, beta, transB, outDtype):
   gemm with A and B of their own dtypes (float32 activations by bfloat16 weights) */
FN(gemmEx, 18)
  void* a = arg_ptr(A, 0); int64_t lda = arg_i64(A, 1); int adt = arg_int(A, 2); void* b = arg_ptr(A, 3);
  int64_t ldb = arg_i64(A, 4); int bdt = arg_int(A, 5); void* c = arg_ptr(A, 6); int64_t ldc = arg_i64(A, 7);
  void* cin = arg_ptr(A, 8); int64_t ldcin = arg_i64(A, 9); void* bias = arg_ptr(A, 10); int64_t m = arg_i64(A, 11);
  int64_t n = arg_i64(A, 12); int64_t k = arg_i64(A, 13); double al = arg_f64(A, 14); double be = arg_f64(A, 15);
  int tb = arg_flag(A, 16); int odt = arg_int(A, 17);
  CALL(kh_gemm_ex(a, lda, adt, b, ldb, bdt, c, ldc, cin, ldcin, bias, m, n, k, (float)al, (float)be, tb, odt))
/* gemmSwiglu(x, ldx, wGu, ldw, h, ldh, m, nHalf, k, xDtype): the SwiGLU gate/up projections with
   silu * mul in the epilogue (swiglu.ts:119-134), weight rows interleaved in blocks of 8 */
FN(gemmSwiglu, 10)
  void* x = arg_ptr(A, 0); int64_t ldx = arg_i64(A, 1); void* w = arg_ptr(A, 2); int64_t ldw = arg_i64(A, 3);
  void* h = arg_ptr(A, 4); int64_t ldh = arg_i64(A, 5); int64_t m = arg_i64(A, 6); int64_t nh = arg_i64(A, 7);
  int64_t k = arg_i64(A, 8); int xdt = arg_int(A, 9);
  CALL(kh_gemm_swiglu(x, ldx, w, ldw, h, ldh, m, nh, k, xdt))
/* gemmQkNormRope(x, ldx, wQkv, ldw, nBatch, seqLen, k, hq, hkv, headDim, wq, wk, invFreq, positions,
   qOut, kOut, vOut, strides[9], eps, kvCacheLen, dtype): the QKV projection with qk-norm, RoPE and the
   K/V cache write in its epilogue (gqa.ts:269-309, rope.ts:546-644, kv-cache.ts:164-212) */
FN(gemmQkNormRope, 21)
  int64_t st[9];
  void* x = arg_ptr(A, 0); int64_t ldx = arg_i64(A, 1); void* w = arg_ptr(A, 2); int64_t ldw = arg_i64(A, 3);
  int64_t nb = arg_i64(A, 4); int64_t sl = arg_i64(A, 5); int64_t k = arg_i64(A, 6);
  int hq = arg_int(A, 7); int hkv = arg_int(A, 8); int hd = arg_int(A, 9);
  void* wq = arg_ptr(A, 10); void* wk = arg_ptr(A, 11); void* inv = arg_ptr(A, 12); void* pos = arg_ptr(A, 13);
  void* qo = arg_ptr(A, 14); void* ko = arg_ptr(A, 15); void* vo = arg_ptr(A, 16);
  arg_list(A, 17, st, 9);
  double eps = arg_f64(A, 18); int64_t kvl = arg_i64(A, 19); int dt = arg_int(A, 20);
  CALL(kh_gemm_qk_norm_rope(x, ldx, w, ldw, nb, sl, k, hq, hkv, hd, wq, wk, (const float*)inv, (const int32_t*)pos,
                            qo, ko, vo, st, (float)eps, kvl, dt))
/* gemmQkNormRopeTable(..., dtype, ropeTable): gemmQkNormRope with the RoPE angles read from a
   ropeTable table (null: computed per tile) */
FN(gemmQkNormRopeTable, 22)
  int64_t st[9];
  void* x = arg_ptr(A, 0); int64_t ldx = arg_i64(A, 1); void* w = arg_ptr(A, 2); int64_t ldw = arg_i64(A, 3);
  int64_t nb = arg_i64(A, 4); int64_t sl = arg_i64(A, 5); int64_t k = arg_i64(A, 6);
  int hq = arg_int(A, 7); int hkv = arg_int(A, 8); int hd = arg_int(A, 9);
  void* wq = arg_ptr(A, 10); void* wk = arg_ptr(A, 11); void* inv = arg_ptr(A, 12); void* pos = arg_ptr(A, 13);
  void* qo = arg_ptr(A, 14); void* ko = arg_ptr(A, 15); void* vo = arg_ptr(A, 16);
  arg_list(A, 17, st, 9);
  double eps = arg_f64(A, 18); int64_t kvl = arg_i64(A, 19); int dt = arg_int(A, 20); void* tab = arg_ptr(A, 21);
  CALL(kh_gemm_qk_norm_rope_table(x, ldx, w, ldw, nb, sl, k, hq, hkv, hd, wq, wk, (const float*)inv,
                                  (const int32_t*)pos, qo, ko, vo, st, (float)eps, kvl, dt, (const float*)tab))
/* ropeTable(positions, n, invFreq, half, out): (cos, sin) of float(positions[t]) * invFreq[i] */
FN(ropeTable, 5)
  void* pos = arg_ptr(A, 0); int64_t n = arg_i64(A, 1); void* inv = arg_ptr(A, 2); int half = arg_int(A, 3);
  void* out = arg_ptr(A, 4);
  CALL(kh_rope_table((const int32_t*)pos, n, (const float*)inv, half, (float*)out))
/* gemmSplitCount(m, n, k) -> the split count gemm uses for a contiguous bf16 [m, k] x [n, k]^T */
static napi_value js_gemmSplitCount(napi_env env, napi_callback_info info) {
  Args A_, *A = &A_;
  if (!begin(A, env, info, "gemmSplitCount", 3)) return NULL;
  int64_t m = arg_i64(A, 0), n = arg_i64(A, 1), k = arg_i64(A, 2);
  if (A->bad) return NULL;
  int splits = 0;
  if (kh_gemm_split_count(m, n, k, &splits) != KH_OK) return done(A, KH_ERR_INVALID);
  napi_value out;
  napi_create_int32(env, splits, &out);
  return out;
}
/* gemmSplitkPartials(a, lda, b, ldb, part, m, n, k, splits, aDtype): gemm's split-K stage alone, fp32
   partials [splits][m][n] */
FN(gemmSplitkPartials, 10)
  void* a = arg_ptr(A, 0); int64_t lda = arg_i64(A, 1); void* b = arg_ptr(A, 2); int64_t ldb = arg_i64(A, 3);
  void* part = arg_ptr(A, 4); int64_t m = arg_i64(A, 5); int64_t n = arg_i64(A, 6); int64_t k = arg_i64(A, 7);
  int sp = arg_int(A, 8); int adt = arg_int(A, 9);
  CALL(kh_gemm_splitk_partials(a, lda, b, ldb, (float*)part, m, n, k, sp, adt))
/* addRmsNorm(part, splits, splitStride, x, w, y, rows, n, eps, outDtype): x += sum of the partials
   (residual add, decoder_layer.ts:224-238), then y = rms_norm(x) * w */
FN(addRmsNorm, 10)
  void* part = arg_ptr(A, 0); int sp = arg_int(A, 1); int64_t ss = arg_i64(A, 2); void* x = arg_ptr(A, 3);
  void* w = arg_ptr(A, 4); void* y = arg_ptr(A, 5); int64_t rows = arg_i64(A, 6); int64_t n = arg_i64(A, 7);
  double eps = arg_f64(A, 8); int odt = arg_int(A, 9);
  CALL(kh_add_rms_norm((const float*)part, sp, ss, (float*)x, w, y, rows, n, (float)eps, odt))
/* gemvFused(prologue, x, x2, normW, eps, w, ldw, c, cin, bias, n, k, alpha, beta, outDtype, xDtype) */
FN(gemvFused, 16)
  int pro = arg_int(A, 0); void* x = arg_ptr(A, 1); void* x2 = arg_ptr(A, 2); void* nw = arg_ptr(A, 3);
  double eps = arg_f64(A, 4); void* w = arg_ptr(A, 5); int64_t ldw = arg_i64(A, 6); void* c = arg_ptr(A, 7);
  void* cin = arg_ptr(A, 8); void* bias = arg_ptr(A, 9); int64_t n = arg_i64(A, 10); int64_t k = arg_i64(A, 11);
  double al = arg_f64(A, 12); double be = arg_f64(A, 13); int odt = arg_int(A, 14); int xdt = arg_int(A, 15);
  CALL(kh_gemv_fused(pro, x, x2, nw, (float)eps, w, ldw, c, cin, bias, n, k, (float)al, (float)be, odt, xdt))

/* gemvSwiglu(prologue, x, normW, eps, wGu, ldw, h, nHalf, k, xDtype) */
FN(gemvSwiglu, 10)
  int pro = arg_int(A, 0); void* x = arg_ptr(A, 1); void* nw = arg_ptr(A, 2); double eps = arg_f64(A, 3);
  void* w = arg_ptr(A, 4); int64_t ldw = arg_i64(A, 5); void* h = arg_ptr(A, 6); int64_t nh = arg_i64(A, 7);
  int64_t k = arg_i64(A, 8); int xdt = arg_int(A, 9);
  CALL(kh_gemv_swiglu(pro, x, nw, (float)eps, w, ldw, h, nh, k, xdt))

/* ---------------------------------------------------------------- module ----------------------- */
#define EXPORT(name) {#name, 0, js_##name, 0, 0, 0, napi_enumerable, 0}

static napi_value module_init(napi_env env, napi_value exports) {
  napi_property_descriptor d[] = {
      EXPORT(init), EXPORT(deviceCount), EXPORT(lastError), EXPORT(setDebug), EXPORT(isCapturing), EXPORT(alloc), EXPORT(free), EXPORT(emptyCache),
      EXPORT(allocOwned), EXPORT(ownedPtr), EXPORT(freeOwned),
      EXPORT(allocStats), EXPORT(memcpyH2D), EXPORT(memcpyD2H), EXPORT(memcpyD2D), EXPORT(synchronize),
      EXPORT(eventCreate), EXPORT(eventDestroy), EXPORT(eventRecord), EXPORT(eventElapsedMs),
      EXPORT(graphBeginCapture), EXPORT(graphEndCapture), EXPORT(graphLaunch), EXPORT(graphDestroy),
      EXPORT(fill), EXPORT(copyStrided), EXPORT(mapStrided), EXPORT(binary), EXPORT(silu), EXPORT(unary), EXPORT(arange),
      EXPORT(siluMul), EXPORT(indexSelect), EXPORT(indexSelectDim), EXPORT(argmax), EXPORT(greedyAdvance), EXPORT(sample),
      EXPORT(sampleSetPath), EXPORT(philox4x32_10), EXPORT(decodeAttentionBlock), EXPORT(rmsNorm),
      EXPORT(qkNormRope), EXPORT(flashAttention), EXPORT(flashAttentionSplit), EXPORT(flashAttentionMasked), EXPORT(decodeAttention),
      EXPORT(decodeAttentionNoalloc), EXPORT(gemm), EXPORT(gemmEx), EXPORT(gemmSwiglu), EXPORT(gemmQkNormRope), EXPORT(gemmQkNormRopeTable), EXPORT(ropeTable), EXPORT(gemmSplitCount),
      EXPORT(gemmSplitkPartials), EXPORT(addRmsNorm), EXPORT(gemvFused), EXPORT(gemvSwiglu),
  };
  napi_define_properties(env, exports, sizeof(d) / sizeof(d[0]), d);
  napi_value v;
  const int codes[] = {KH_F32, KH_BF16, KH_I32};
  const char* names[] = {"F32", "BF16", "I32"};
  for (int i = 0; i < 3; ++i) {
    napi_create_int32(env, codes[i], &v);
    napi_set_named_property(env, exports, names[i], v);
  }
  return exports;
}

NAPI_MODULE(kandle_hip, module_init)
