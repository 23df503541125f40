// Shared definitions for the gfx950 kernels and the C ABI of the Kandle HIP backend.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/kandle_hip.h"

namespace kh {

// ---- error reporting (thread-local text behind kh_last_error) --------------------------------
void set_error(const char* fmt, ...);
void clear_error();
hipStream_t stream();  // the library stream; nullptr before kh_init
bool initialized();
int current_device();  // the device kh_init selected (-1 before)
int cu_count();        // compute units of that device
int attention_init(int device);  // kh_init's set-up of attention.hip (device current)

// Internal scratch allocation through the caching allocator (stream-ordered on the library stream).
void* scratch_alloc(size_t bytes);
void scratch_free(void* p);

// Split-K decode attention partials of one sequence as the o_proj GEMV prologue reads them:
// o[hq][max_chunks][128] floats, then (m, l)[hq][max_chunks]; chunks of `chunk` keys, the sequence
// length position[0] + 1 clamped to [0, max_len].
struct AttnMerge {
  const int32_t* position = nullptr;
  int hq = 0, max_chunks = 0, max_len = 0, chunk = 0;
};
bool launch_gemv_attn_merge(const float* part, const AttnMerge& am, const uint16_t* W, int64_t ldw, float* C,
                            const float* cin, int N, int K, float alpha, float beta, bool exact);

#define KH_CHECK_HIP(expr)                                                              \
  do {                                                                                  \
    hipError_t _e = (expr);                                                             \
    if (_e != hipSuccess) {                                                             \
      ::kh::set_error("%s failed: %s (%s:%d)", #expr, hipGetErrorString(_e), __FILE__, \
                      __LINE__);                                                        \
      return KH_ERR_HIP;                                                                \
    }                                                                                   \
  } while (0)

#define KH_REQUIRE(cond, ...)         \
  do {                                \
    if (!(cond)) {                    \
      ::kh::set_error(__VA_ARGS__);   \
      return KH_ERR_INVALID;          \
    }                                 \
  } while (0)

#define KH_REQUIRE_INIT()                                              \
  do {                                                                 \
    if (!::kh::initialized()) {                                        \
      ::kh::set_error("kh_init has not been called");                  \
      return KH_ERR_NOT_INIT;                                          \
    }                                                                  \
  } while (0)

// Debug mode (kh_set_debug): after every launch, wait for the stream and report an asynchronous
// fault at the call that launched the kernel.  Off while a graph capture is open.
bool debug_sync();
int debug_check(const char* where, const char* file, int line);

#define KH_DEBUG_SYNC()                                                      \
  do {                                                                       \
    if (::kh::debug_sync()) {                                                \
      const int _rc = ::kh::debug_check(__func__, __FILE__, __LINE__);       \
      if (_rc != KH_OK) return _rc;                                          \
    }                                                                        \
  } while (0)

// After a launch: report launch-configuration errors immediately (and, in debug mode, faults).
#define KH_CHECK_LAUNCH()                 \
  do {                                    \
    KH_CHECK_HIP(hipGetLastError());      \
    KH_DEBUG_SYNC();                      \
  } while (0)

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ---- device helpers ------------------------------------------------------------------------
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// Exact widening of a bf16 bit pattern (the 16 high bits of a float32).
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// Two floats -> packed bf16x2 (lo in bits 0..15), round to nearest even, NaN stays NaN: one gfx950
// v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// float32 -> bf16 bits (low 16 bits of the result), rounded as pack_bf16x2.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) { return pack_bf16x2(f, 0.f) & 0xffffu; }

__device__ __forceinline__ float lo_bf16(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_bf16(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

template <typename T>
struct Elem;
template <>
struct Elem<float> {
  static __device__ __forceinline__ float load(const float* p, int64_t i) { return p[i]; }
  static __device__ __forceinline__ void store(float* p, int64_t i, float v) { p[i] = v; }
};
template <>
struct Elem<uint16_t> {
  static __device__ __forceinline__ float load(const uint16_t* p, int64_t i) {
    return bf16_bits_to_f32(p[i]);
  }
  static __device__ __forceinline__ void store(uint16_t* p, int64_t i, float v) {
    p[i] = (uint16_t)f32_to_bf16_bits(v);
  }
};

// Raw buffer access: a load at a byte offset >= `bytes` returns zero instead of touching memory,
// so bounds checks need no branch (and no divergent vmcnt bookkeeping).  0x00020000 is the gfx9
// family's buffer-resource word 3 (32-bit data format, no swizzle).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
// The same load with the non-temporal cache hint (the instruction's nt bit): for streams read once
// per launch -- decode weights, KV caches -- whose lines should not displace data that is reused.
__device__ __forceinline__ uint4 buf_load16_nt(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 2));
}
__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0));
}
// 2^x with the hardware instruction (denormal results flush to 0: fine for softmax weights <= 1).
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// silu(x) = x / (1 + exp(-clamp(x, -88, 88))), the reference's pointwise silu (the clamp keeps
// exp finite for large |x|; reference: packages/backend-webgpu/src/kernels/pointwise/ops.ts:299).
__device__ __forceinline__ float silu_ref(float x) {
  const float c = fminf(fmaxf(x, -88.0f), 88.0f);
  return x / (1.0f + expf(-c));
}

// Round a float to the nearest bf16 value (kept in a float register).
__device__ __forceinline__ float round_bf16(float v) { return __uint_as_float(f32_to_bf16_bits(v) << 16); }

// Eight bf16 values of one 16-byte load, in memory order, widened exactly; and eight floats rounded
// (as pack_bf16x2) into one 16-byte store.
__device__ __forceinline__ void unpack_bf16x8(const uint4& u, float (&f)[8]) {
  f[0] = __uint_as_float(u.x << 16); f[1] = __uint_as_float(u.x & 0xffff0000u);
  f[2] = __uint_as_float(u.y << 16); f[3] = __uint_as_float(u.y & 0xffff0000u);
  f[4] = __uint_as_float(u.z << 16); f[5] = __uint_as_float(u.z & 0xffff0000u);
  f[6] = __uint_as_float(u.w << 16); f[7] = __uint_as_float(u.w & 0xffff0000u);
}
__device__ __forceinline__ uint4 pack_bf16x8(const float (&f)[8]) {
  return make_uint4(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]),
                    pack_bf16x2(f[6], f[7]));
}

// ---- cross-lane reductions ------------------------------------------------------------------
// gfx9 DPP controls: quad_perm [1,0,3,2] (lane ^ 1), quad_perm [2,3,0,1] (lane ^ 2), row_half_mirror
// (lane i <-> 7 - i in each group of 8), row_mirror (lane i <-> 15 - i in each row of 16).  The
// callers below run with every lane of the wave active.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
// Sum over aligned groups of N lanes (N = 2, 4, 8 or 16); every lane of a group receives it.
template <int N>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(N == 2 || N == 4 || N == 8 || N == 16, "group of 2, 4, 8 or 16 lanes");
  v += dpp_f<0xB1>(v);
  if (N >= 4) v += dpp_f<0x4E>(v);
  if (N >= 8) v += dpp_f<0x141>(v);
  if (N >= 16) v += dpp_f<0x140>(v);
  return v;
}
// Sum over the 16 lanes of a DPP row; every lane of the row receives it.  VALU only (no LDS).
__device__ __forceinline__ float row16_sum(float v) { return group_sum<16>(v); }

// Wave-wide (64 lanes) sum: row sums by DPP, then the four row results read as scalars.
__device__ __forceinline__ float wave_sum(float v) {
  v = row16_sum(v);
  const int b = __builtin_bit_cast(int, v);
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
  return (r0 + r1) + (r2 + r3);
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

}  // namespace kh
