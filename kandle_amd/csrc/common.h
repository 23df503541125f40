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

// Internal scratch allocation through the caching allocator (stream-ordered on the library stream).
void* scratch_alloc(size_t bytes);
void scratch_free(void* p);

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

// After a launch: report launch-configuration errors immediately.
#define KH_CHECK_LAUNCH() KH_CHECK_HIP(hipGetLastError())

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ---- device helpers ------------------------------------------------------------------------
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// Exact widening of a bf16 bit pattern (the 16 high bits of a float32).
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// float32 -> bf16 bits, round to nearest even; NaN stays a quiet NaN.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

// Two floats -> packed bf16x2 (lo in bits 0..15).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
}

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

// Wave-wide (64 lanes) reductions via cross-lane shuffles.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

}  // namespace kh
