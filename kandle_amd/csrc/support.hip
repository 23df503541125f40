// Support kernels of the hot path: fill, strided copy/cast, binary add/mul/sub, silu, silu*mul,
// index_select (embedding rows) and argmax.  All are HBM-bound; contiguous ones move 16 bytes per
// lane per access when the pointers allow it.
#include <cfloat>

#include "common.h"

using namespace kh;

namespace {

constexpr int kThreads = 256;

inline int grid_for(int64_t work, int per_block = kThreads, int cap = 65536) {
  int64_t g = (work + per_block - 1) / per_block;
  if (g < 1) g = 1;
  if (g > cap) g = cap;
  return (int)g;
}

// ---- fill ---------------------------------------------------------------------------------
template <typename T>
__global__ void fill_kernel(T* dst, int64_t n, float value) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    Elem<T>::store(dst, i, value);
}
__global__ void fill_i32_kernel(int32_t* dst, int64_t n, int32_t value) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    dst[i] = value;
}

// ---- strided copy / cast ------------------------------------------------------------------
struct StridedDesc {
  int ndim;
  int64_t shape[6];
  int64_t stride[6];
};

template <typename S, typename D>
__global__ void copy_strided_kernel(const S* __restrict__ src, int64_t src_offset, D* __restrict__ dst,
                                    int64_t n, StridedDesc desc) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    int64_t rem = i, off = src_offset;
    for (int d = desc.ndim - 1; d >= 0; --d) {
      const int64_t c = rem % desc.shape[d];
      rem /= desc.shape[d];
      off += c * desc.stride[d];
    }
    Elem<D>::store(dst, i, Elem<S>::load(src, off));
  }
}
__global__ void copy_strided_i32_kernel(const int32_t* __restrict__ src, int64_t src_offset,
                                        int32_t* __restrict__ dst, int64_t n, StridedDesc desc) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    int64_t rem = i, off = src_offset;
    for (int d = desc.ndim - 1; d >= 0; --d) {
      const int64_t c = rem % desc.shape[d];
      rem /= desc.shape[d];
      off += c * desc.stride[d];
    }
    dst[i] = src[off];
  }
}

// ---- N-D strided map: the iterator kernels (kh_map_strided) -----------------------------------
// One output element per thread step; the element's offset in every operand is formed from its
// coordinates in the (coalesced) index space and that operand's element strides, so broadcast
// operands (stride 0), permuted and sliced views and strided outputs need no materialised copy.
constexpr int kMapMaxDims = 8;
struct MapDesc {
  int ndim;
  int64_t shape[kMapMaxDims];
  int64_t so[kMapMaxDims], sa[kMapMaxDims], sb[kMapMaxDims];
};

__device__ __forceinline__ float map_ld_f(const void* p, int64_t i, int dt) {
  if (dt == KH_F32) return reinterpret_cast<const float*>(p)[i];
  if (dt == KH_BF16) return bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
  return (float)reinterpret_cast<const int32_t*>(p)[i];
}
// int32 view of an element: ints as they are, floats truncated toward zero and saturated (NaN 0),
// the float -> i32 conversion of WGSL's i32(f).
__device__ __forceinline__ int32_t map_ld_i(const void* p, int64_t i, int dt) {
  if (dt == KH_I32) return reinterpret_cast<const int32_t*>(p)[i];
  const float f = map_ld_f(p, i, dt);
  if (!(f == f)) return 0;
  if (f >= 2147483647.f) return INT32_MAX;
  if (f <= -2147483648.f) return INT32_MIN;
  return (int32_t)f;
}
__device__ __forceinline__ void map_st_f(void* p, int64_t i, int dt, float v) {
  if (dt == KH_F32)
    reinterpret_cast<float*>(p)[i] = v;
  else
    reinterpret_cast<uint16_t*>(p)[i] = (uint16_t)f32_to_bf16_bits(v);
}

// INT: int32 output with int32 arithmetic (copy / add / sub / mul / neg / fill / arange, two's
// complement wrap-around as WGSL's i32); otherwise fp32 math stored in the output's float dtype.
template <bool INT>
__global__ void map_strided_kernel(int op, MapDesc d, int64_t n, void* out, int odt, const void* a, int adt,
                                   const void* b, int bdt, float s0, float s1, int32_t i0, int32_t i1) {
#pragma clang fp contract(off)  // arange's product and sum round separately, as the WGSL kernel's
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    int64_t rem = i, oo = 0, oa = 0, ob = 0;
    for (int k = d.ndim - 1; k >= 0; --k) {
      const int64_t c = rem % d.shape[k];
      rem /= d.shape[k];
      oo += c * d.so[k];
      oa += c * d.sa[k];
      ob += c * d.sb[k];
    }
    if constexpr (INT) {
      int32_t v = 0;
      switch (op) {
        case KH_MAP_COPY: v = map_ld_i(a, oa, adt); break;
        case KH_MAP_ADD: v = (int32_t)((uint32_t)map_ld_i(a, oa, adt) + (uint32_t)i0 * (uint32_t)map_ld_i(b, ob, bdt)); break;
        case KH_MAP_SUB: v = (int32_t)((uint32_t)map_ld_i(a, oa, adt) - (uint32_t)i0 * (uint32_t)map_ld_i(b, ob, bdt)); break;
        case KH_MAP_MUL: v = (int32_t)((uint32_t)map_ld_i(a, oa, adt) * (uint32_t)map_ld_i(b, ob, bdt)); break;
        case KH_MAP_NEG: v = (int32_t)(0u - (uint32_t)map_ld_i(a, oa, adt)); break;
        case KH_MAP_FILL: v = i0; break;
        case KH_MAP_ARANGE: v = (int32_t)((uint32_t)i0 + (uint32_t)i * (uint32_t)i1); break;
        default: break;
      }
      reinterpret_cast<int32_t*>(out)[oo] = v;
    } else {
      float v = 0.f;
      switch (op) {
        case KH_MAP_COPY: v = map_ld_f(a, oa, adt); break;
        case KH_MAP_ADD: v = map_ld_f(a, oa, adt) + s0 * map_ld_f(b, ob, bdt); break;
        case KH_MAP_SUB: v = map_ld_f(a, oa, adt) - s0 * map_ld_f(b, ob, bdt); break;
        case KH_MAP_MUL: v = map_ld_f(a, oa, adt) * map_ld_f(b, ob, bdt); break;
        case KH_MAP_DIV: v = map_ld_f(a, oa, adt) / map_ld_f(b, ob, bdt); break;
        case KH_MAP_NEG: v = -map_ld_f(a, oa, adt); break;
        case KH_MAP_COS: v = cosf(map_ld_f(a, oa, adt)); break;
        case KH_MAP_SIN: v = sinf(map_ld_f(a, oa, adt)); break;
        case KH_MAP_SILU: v = silu_ref(map_ld_f(a, oa, adt)); break;
        case KH_MAP_FILL: v = s0; break;
        case KH_MAP_ARANGE: {
          const float prod = (float)i * s1;
          v = s0 + prod;
          break;
        }
        default: break;
      }
      map_st_f(out, oo, odt, v);
    }
  }
}

// ---- binary / unary ---------------------------------------------------------------------------
__device__ __forceinline__ float apply_binary(int op, float a, float b) {
  return op == 0 ? a + b : (op == 1 ? a * b : a - b);
}


template <typename T>
__global__ void binary_kernel(int op, const T* __restrict__ a, const T* __restrict__ b, T* __restrict__ out,
                              int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    Elem<T>::store(out, i, apply_binary(op, Elem<T>::load(a, i), Elem<T>::load(b, i)));
}

// bf16, 8 elements per lane per step (16-byte accesses).
__global__ void binary_bf16x8_kernel(int op, const uint4* __restrict__ a, const uint4* __restrict__ b,
                                     uint4* __restrict__ out, int64_t n8) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n8;
       i += (int64_t)gridDim.x * blockDim.x) {
    const uint4 va = a[i], vb = b[i];
    const uint32_t wa[4] = {va.x, va.y, va.z, va.w};
    const uint32_t wb[4] = {vb.x, vb.y, vb.z, vb.w};
    uint32_t wo[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      wo[j] = pack_bf16x2(apply_binary(op, lo_bf16(wa[j]), lo_bf16(wb[j])),
                          apply_binary(op, hi_bf16(wa[j]), hi_bf16(wb[j])));
    out[i] = make_uint4(wo[0], wo[1], wo[2], wo[3]);
  }
}

template <typename T>
__global__ void silu_kernel(const T* __restrict__ x, T* __restrict__ out, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    Elem<T>::store(out, i, silu_ref(Elem<T>::load(x, i)));
}

// Unary map ops of the pointwise kernels: 0 = neg, 1 = cos, 2 = sin, computed in fp32 and stored
// in the tensor's dtype (reference: packages/backend-webgpu/src/kernels/pointwise/ops.ts:168 neg,
// :201 sin, :202 cos; WGSL evaluates them in f32).
template <typename T>
__global__ void unary_kernel(const T* __restrict__ x, T* __restrict__ out, int64_t n, int op) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const float v = Elem<T>::load(x, i);
    Elem<T>::store(out, i, op == 0 ? -v : (op == 1 ? cosf(v) : sinf(v)));
  }
}

// arange: out[i] = start + f32(i) * step in f32 for floating dtypes, start + i * step in i32 for int32
// (reference: packages/backend-webgpu/src/kernels/factory/arangeShaderBuilder.ts:66-78).
template <typename T>
__global__ void arange_kernel(T* __restrict__ out, int64_t n, float start, float step) {
#pragma clang fp contract(off)  // the product and the sum round separately (no fma)
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const float prod = (float)i * step;
    Elem<T>::store(out, i, start + prod);
  }
}
__global__ void arange_i32_kernel(int32_t* __restrict__ out, int64_t n, int32_t start, int32_t step) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    out[i] = (int32_t)((uint32_t)start + (uint32_t)i * (uint32_t)step);  // i32 wrap-around as WGSL
}

template <typename T>
__global__ void silu_mul_kernel(const T* __restrict__ g, int64_t gs, const T* __restrict__ u, int64_t us,
                                T* __restrict__ out, int64_t os, int64_t rows, int64_t n) {
  const int64_t total = rows * n;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / n, c = i - r * n;
    const float gv = Elem<T>::load(g, r * gs + c);
    const float uv = Elem<T>::load(u, r * us + c);
    Elem<T>::store(out, r * os + c, silu_ref(gv) * uv);
  }
}

// bf16 silu*mul with 8 elements per lane (n % 8 == 0, 16-byte aligned rows).
__global__ void silu_mul_bf16x8_kernel(const uint16_t* __restrict__ g, int64_t gs, const uint16_t* __restrict__ u,
                                       int64_t us, uint16_t* __restrict__ out, int64_t os, int64_t rows,
                                       int64_t n8) {
  const int64_t total = rows * n8;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / n8, c = (i - r * n8) * 8;
    const uint4 vg = *reinterpret_cast<const uint4*>(g + r * gs + c);
    const uint4 vu = *reinterpret_cast<const uint4*>(u + r * us + c);
    const uint32_t wg[4] = {vg.x, vg.y, vg.z, vg.w};
    const uint32_t wu[4] = {vu.x, vu.y, vu.z, vu.w};
    uint32_t wo[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      wo[j] = pack_bf16x2(silu_ref(lo_bf16(wg[j])) * lo_bf16(wu[j]), silu_ref(hi_bf16(wg[j])) * hi_bf16(wu[j]));
    *reinterpret_cast<uint4*>(out + r * os + c) = make_uint4(wo[0], wo[1], wo[2], wo[3]);
  }
}

// ---- index_select -------------------------------------------------------------------------
// Rows of `table` (element type T) gathered into `out` (element type D, converted through fp32);
// an id outside [0, n_rows) yields a zero row.
// The table is viewed as [outer, n_rows, row_elems] (outer = 1: rows of an embedding table):
// out[a, r, :] = table[a, idx[r], :].  Block (r, a-slice) copies one output row of row_elems.
template <typename T, typename D>
__global__ void index_select_kernel(const T* __restrict__ table, int64_t n_rows, const int32_t* __restrict__ idx,
                                    int64_t row_elems, D* __restrict__ out, int64_t outer, int64_t n_idx) {
  const int64_t r = blockIdx.x;
  const int32_t id = idx[r];
  const bool ok = id >= 0 && id < n_rows;
  for (int64_t a = blockIdx.y; a < outer; a += gridDim.y) {
    const T* src = table + (a * n_rows + (ok ? (int64_t)id : 0)) * row_elems;
    D* dst = out + (a * n_idx + r) * row_elems;
    for (int64_t c = threadIdx.x; c < row_elems; c += blockDim.x)
      Elem<D>::store(dst, c, ok ? Elem<T>::load(src, c) : 0.0f);
  }
}

int launch_index_select(const void* table, int64_t outer, int64_t n_rows, int64_t inner, const int32_t* idx,
                        int64_t n_idx, void* out, int dtype, int out_dtype, const char* name) {
  KH_REQUIRE(outer > 0 && n_rows > 0 && n_idx >= 0 && inner > 0, "%s: bad extents", name);
  if (n_idx == 0) return KH_OK;
  KH_REQUIRE(n_idx <= INT32_MAX, "%s: too many indices", name);
  KH_REQUIRE(table && idx && out, "%s: null pointer", name);
  const dim3 grid((unsigned)n_idx, (unsigned)(outer < 65535 ? outer : 65535)), block(kThreads);
  if (dtype == KH_BF16 && out_dtype == KH_BF16)
    index_select_kernel<uint16_t, uint16_t><<<grid, block, 0, stream()>>>((const uint16_t*)table, n_rows, idx, inner,
                                                                          (uint16_t*)out, outer, n_idx);
  else if (dtype == KH_BF16 && out_dtype == KH_F32)
    index_select_kernel<uint16_t, float><<<grid, block, 0, stream()>>>((const uint16_t*)table, n_rows, idx, inner,
                                                                       (float*)out, outer, n_idx);
  else if (dtype == KH_F32 && out_dtype == KH_F32)
    index_select_kernel<float, float><<<grid, block, 0, stream()>>>((const float*)table, n_rows, idx, inner,
                                                                    (float*)out, outer, n_idx);
  else if (dtype == KH_F32 && out_dtype == KH_BF16)
    index_select_kernel<float, uint16_t><<<grid, block, 0, stream()>>>((const float*)table, n_rows, idx, inner,
                                                                       (uint16_t*)out, outer, n_idx);
  else
    KH_REQUIRE(false, "%s: unsupported dtypes (table %d, out %d)", name, dtype, out_dtype);
  KH_CHECK_LAUNCH();
  return KH_OK;
}

// ---- greedy decode bookkeeping (one thread) ------------------------------------------------
__global__ void greedy_advance_kernel(const int32_t* __restrict__ next_token, int32_t* __restrict__ position,
                                      int32_t* __restrict__ seq_len, int32_t* __restrict__ token_log,
                                      int64_t log_base, int64_t log_cap) {
  const int32_t p = *position;
  const int64_t slot = (int64_t)p + 1 - log_base;
  if (token_log != nullptr && slot >= 0 && slot < log_cap) token_log[slot] = *next_token;
  *position = p + 1;
  *seq_len = p + 2;
}

// ---- argmax (lowest index among maxima; NaN never wins; init -FLT_MAX at index 0) ----------
// A candidate must be strictly greater than -FLT_MAX (the reference's initial value); a row with
// none yields index 0, as the reference's initial best_idx does.  Pass 1: block (c, r) scans
// columns [c * AM_CHUNK, (c + 1) * AM_CHUNK) of row r with all its loads issued up front; pass 2
// combines the per-chunk (value, index) pairs of a row.  A row of one chunk finishes in pass 1.
constexpr int AM_PER_THREAD = 16;
constexpr int AM_CHUNK = kThreads * AM_PER_THREAD;

__device__ __forceinline__ bool am_better(float v, int32_t i, float bv, int32_t bi) {
  return v > bv || (v == bv && i < bi);
}

// Block-wide (value, index) reduction; every thread returns the block's best pair.
__device__ __forceinline__ void am_block_reduce(float& best, int32_t& bidx) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(best, o, 64);
    const int32_t oi = __shfl_xor(bidx, o, 64);
    if (am_better(ov, oi, best, bidx)) {
      best = ov;
      bidx = oi;
    }
  }
  __shared__ float sv[kThreads / 64];
  __shared__ int32_t si[kThreads / 64];
  if ((threadIdx.x & 63) == 0) {
    sv[threadIdx.x >> 6] = best;
    si[threadIdx.x >> 6] = bidx;
  }
  __syncthreads();
  best = sv[0];
  bidx = si[0];
  for (int w = 1; w < (int)(blockDim.x >> 6); ++w)
    if (am_better(sv[w], si[w], best, bidx)) {
      best = sv[w];
      bidx = si[w];
    }
}

template <typename T>
__global__ __launch_bounds__(kThreads) void argmax_partial_kernel(const T* __restrict__ x, int64_t n,
                                                                  float* __restrict__ pv, int32_t* __restrict__ pi,
                                                                  int32_t* __restrict__ out) {
  const int64_t r = blockIdx.y;
  const int64_t c0 = (int64_t)blockIdx.x * AM_CHUNK;
  const T* row = x + r * n;
  float v[AM_PER_THREAD];
#pragma unroll
  for (int j = 0; j < AM_PER_THREAD; ++j) {
    const int64_t i = c0 + j * kThreads + threadIdx.x;
    v[j] = i < n ? Elem<T>::load(row, i) : -FLT_MAX;
  }
  float best = -FLT_MAX;
  int32_t bidx = INT32_MAX;
#pragma unroll
  for (int j = 0; j < AM_PER_THREAD; ++j)  // increasing column order: strict > keeps the first
    if (v[j] > best) {
      best = v[j];
      bidx = (int32_t)(c0 + j * kThreads + threadIdx.x);
    }
  am_block_reduce(best, bidx);
  if (threadIdx.x == 0) {
    if (gridDim.x == 1) {
      out[r] = bidx == INT32_MAX ? 0 : bidx;
    } else {
      pv[r * gridDim.x + blockIdx.x] = best;
      pi[r * gridDim.x + blockIdx.x] = bidx;
    }
  }
}

__global__ __launch_bounds__(kThreads) void argmax_final_kernel(const float* __restrict__ pv,
                                                                const int32_t* __restrict__ pi, int nchunks,
                                                                int32_t* __restrict__ out) {
  const int64_t r = blockIdx.x;
  float best = -FLT_MAX;
  int32_t bidx = INT32_MAX;
  for (int c = threadIdx.x; c < nchunks; c += blockDim.x) {
    const float v = pv[r * nchunks + c];
    const int32_t i = pi[r * nchunks + c];
    if (am_better(v, i, best, bidx)) {
      best = v;
      bidx = i;
    }
  }
  am_block_reduce(best, bidx);
  if (threadIdx.x == 0) out[r] = bidx == INT32_MAX ? 0 : bidx;
}

}  // namespace

extern "C" {

int kh_fill(void* dst, int64_t n, float value, int dtype) {
  KH_REQUIRE_INIT();
  KH_REQUIRE(n >= 0, "kh_fill: negative count");
  if (n == 0) return KH_OK;
  KH_REQUIRE(dst != nullptr, "kh_fill: null pointer");
  const int g = grid_for(n);
  if (dtype == KH_F32)
    fill_kernel<float><<<g, kThreads, 0, stream()>>>((float*)dst, n, value);
  else if (dtype == KH_BF16)
    fill_kernel<uint16_t><<<g, kThreads, 0, stream()>>>((uint16_t*)dst, n, value);
  else if (dtype == KH_I32)
    fill_i32_kernel<<<g, kThreads, 0, stream()>>>((int32_t*)dst, n, (int32_t)value);
  else
    KH_REQUIRE(false, "kh_fill: unsupported dtype %d", dtype);
  KH_CHECK_LAUNCH();
  return KH_OK;
}

int kh_copy_strided(const void* src, int64_t src_offset, void* dst, int ndim, const int64_t* shape,
                    const int64_t* src_strides, int dtype_src, int dtype_dst) {
  KH_REQUIRE_INIT();
  KH_REQUIRE(ndim >= 0 && ndim <= 6, "kh_copy_strided: ndim %d outside [0, 6]", ndim);
  KH_REQUIRE(ndim == 0 || (shape && src_strides), "kh_copy_strided: null shape/strides");
  StridedDesc desc{};
  desc.ndim = ndim;
  int64_t n = 1;
  for (int d = 0; d < ndim; ++d) {
    KH_REQUIRE(shape[d] >= 0, "kh_copy_strided: negative extent");
    desc.shape[d] = shape[d];
    desc.stride[d] = src_strides[d];
    n *= shape[d];
  }
  if (n == 0) return KH_OK;
  KH_REQUIRE(src && dst, "kh_copy_strided: null pointer");
  const int g = grid_for(n);
  if (dtype_src == KH_I32 || dtype_dst == KH_I32) {
    KH_REQUIRE(dtype_src == KH_I32 && dtype_dst == KH_I32, "kh_copy_strided: int32 copies cannot cast");
    copy_strided_i32_kernel<<<g, kThreads, 0, stream()>>>((const int32_t*)src, src_offset, (int32_t*)dst, n, desc);
  } else if (dtype_src == KH_F32 && dtype_dst == KH_F32) {
    copy_strided_kernel<float, float><<<g, kThreads, 0, stream()>>>((const float*)src, src_offset, (float*)dst, n, desc);
  } else if (dtype_src == KH_F32 && dtype_dst == KH_BF16) {
    copy_strided_kernel<float, uint16_t><<<g, kThreads, 0, stream()>>>((const float*)src, src_offset, (uint16_t*)dst, n, desc);
  } else if (dtype_src == KH_BF16 && dtype_dst == KH_F32) {
    copy_strided_kernel<uint16_t, float><<<g, kThreads, 0, stream()>>>((const uint16_t*)src, src_offset, (float*)dst, n, desc);
  } else if (dtype_src == KH_BF16 && dtype_dst == KH_BF16) {
    copy_strided_kernel<uint16_t, uint16_t><<<g, kThreads, 0, stream()>>>((const uint16_t*)src, src_offset, (uint16_t*)dst, n, desc);
  } else {
    KH_REQUIRE(false, "kh_copy_strided: unsupported dtypes %d -> %d", dtype_src, dtype_dst);
  }
  KH_CHECK_LAUNCH();
  return KH_OK;
}

int kh_map_strided(int op, int ndim, const int64_t* shape, void* out, const int64_t* out_strides, int out_dtype,
                   const void* a, const int64_t* a_strides, int a_dtype, const void* b, const int64_t* b_strides,
                   int b_dtype, double s0, double s1) {
  KH_REQUIRE_INIT();
  KH_REQUIRE(op >= KH_MAP_COPY && op <= KH_MAP_ARANGE, "kh_map_strided: unknown op %d", op);
  KH_REQUIRE(ndim >= 0 && ndim <= kMapMaxDims, "kh_map_strided: ndim %d outside [0, %d]", ndim, kMapMaxDims);
  KH_REQUIRE(ndim == 0 || shape != nullptr, "kh_map_strided: null shape");
  const int nin = op == KH_MAP_FILL || op == KH_MAP_ARANGE
                      ? 0
                      : (op == KH_MAP_ADD || op == KH_MAP_SUB || op == KH_MAP_MUL || op == KH_MAP_DIV ? 2 : 1);
  auto dtype_ok = [](int dt) { return dt == KH_F32 || dt == KH_BF16 || dt == KH_I32; };
  KH_REQUIRE(dtype_ok(out_dtype), "kh_map_strided: unsupported output dtype %d", out_dtype);
  KH_REQUIRE(nin < 1 || dtype_ok(a_dtype), "kh_map_strided: unsupported dtype %d of a", a_dtype);
  KH_REQUIRE(nin < 2 || dtype_ok(b_dtype), "kh_map_strided: unsupported dtype %d of b", b_dtype);
  const bool int_out = out_dtype == KH_I32;
  // int32 outputs take integer arithmetic (copy casts any dtype; the arithmetic ops need int32 inputs);
  // division and the transcendental ops produce floats
  KH_REQUIRE(!int_out || op == KH_MAP_COPY || op == KH_MAP_FILL || op == KH_MAP_ARANGE ||
                 ((op == KH_MAP_ADD || op == KH_MAP_SUB || op == KH_MAP_MUL || op == KH_MAP_NEG) &&
                  a_dtype == KH_I32 && (nin < 2 || b_dtype == KH_I32)),
             "kh_map_strided: op %d has no int32 form for these operands", op);
  int64_t n = 1;
  for (int k = 0; k < ndim; ++k) {
    KH_REQUIRE(shape[k] >= 0, "kh_map_strided: negative extent");
    n *= shape[k];
  }
  if (n == 0) return KH_OK;
  KH_REQUIRE(out && (ndim == 0 || out_strides), "kh_map_strided: null output");
  KH_REQUIRE(nin < 1 || (a && (ndim == 0 || a_strides)), "kh_map_strided: null operand a");
  KH_REQUIRE(nin < 2 || (b && (ndim == 0 || b_strides)), "kh_map_strided: null operand b");
  // Coalesce: drop extent-1 axes, then merge axis k into k + 1 wherever every operand steps
  // through k exactly as through a whole row of k + 1 (stride[k] == stride[k + 1] * shape[k + 1]).
  MapDesc d{};
  d.ndim = 0;
  for (int k = 0; k < ndim; ++k) {
    if (shape[k] == 1) continue;
    const int j = d.ndim++;
    d.shape[j] = shape[k];
    d.so[j] = out_strides[k];
    d.sa[j] = nin >= 1 ? a_strides[k] : 0;
    d.sb[j] = nin >= 2 ? b_strides[k] : 0;
  }
  int m = 0;
  for (int k = 0; k < d.ndim; ++k) {
    if (m > 0 && d.so[m - 1] == d.so[k] * d.shape[k] && d.sa[m - 1] == d.sa[k] * d.shape[k] &&
        d.sb[m - 1] == d.sb[k] * d.shape[k]) {
      d.shape[m - 1] *= d.shape[k];
      d.so[m - 1] = d.so[k];
      d.sa[m - 1] = d.sa[k];
      d.sb[m - 1] = d.sb[k];
    } else {
      d.shape[m] = d.shape[k];
      d.so[m] = d.so[k];
      d.sa[m] = d.sa[k];
      d.sb[m] = d.sb[k];
      ++m;
    }
  }
  d.ndim = m;
  const int g = grid_for(n);
  const float f0 = (float)s0, f1 = (float)s1;
  const int32_t i0 = (int32_t)(int64_t)s0, i1 = (int32_t)(int64_t)s1;
  // add / sub scale b by alpha (s0): 1 when the caller has none
  if (int_out)
    map_strided_kernel<true><<<g, kThreads, 0, stream()>>>(op, d, n, out, out_dtype, a, a_dtype, b, b_dtype, f0, f1,
                                                           i0, i1);
  else
    map_strided_kernel<false><<<g, kThreads, 0, stream()>>>(op, d, n, out, out_dtype, a, a_dtype, b, b_dtype, f0,
                                                            f1, i0, i1);
  KH_CHECK_LAUNCH();
  return KH_OK;
}

int kh_binary(int op, const void* a, const void* b, void* out, int64_t n, int dtype) {
  KH_REQUIRE_INIT();
  KH_REQUIRE(op >= 0 && op <= 2, "kh_binary: unknown op %d", op);
  KH_REQUIRE(n >= 0, "kh_binary: negative count");
  if (n == 0) return KH_OK;
  KH_REQUIRE(a && b && out, "kh_binary: null pointer");
  if (dtype == KH_BF16 && n % 8 == 0 && aligned16(a) && aligned16(b) && aligned16(out)) {
    binary_bf16x8_kernel<<<grid_for(n / 8), kThreads, 0, stream()>>>(op, (const uint4*)a, (const uint4*)b,
                                                                     (uint4*)out, n / 8);
  } else if (dtype == KH_BF16) {
    binary_kernel<uint16_t><<<grid_for(n), kThreads, 0, stream()>>>(op, (const uint16_t*)a, (const uint16_t*)b,
                                                                    (uint16_t*)out, n);
  } else if (dtype == KH_F32) {
    binary_kernel<float><<<grid_for(n), kThreads, 0, stream()>>>(op, (const float*)a, (const float*)b,
                                                                 (float*)out, n);
  } else {
    KH_REQUIRE(false, "kh_binary: unsupported dtype %d", dtype);
  }
  KH_CHECK_LAUNCH();
  return KH_OK;
}

int kh_silu(const void* x, void* out, int64_t n, int dtype) {
  KH_REQUIRE_INIT();
  KH_REQUIRE(n >= 0, "kh_silu: negative count");
  if (n == 0) return KH_OK;
  KH_REQUIRE(x && out, "kh_silu: null pointer");
  if (dtype == KH_F32)
    silu_kernel<float><<<grid_for(n), kThreads, 0, stream()>>>((const float*)x, (float*)out, n);
  else if (dtype == KH_BF16)
    silu_kernel<uint16_t><<<grid_for(n), kThreads, 0, stream()>>>((const uint16_t*)x, (uint16_t*)out, n);
  else
    KH_REQUIRE(false, "kh_silu: unsupported dtype %d", dtype);
  KH_CHECK_LAUNCH();
  return KH_OK;
}

int kh_unary(int op, const void* x, void* out, int64_t n, int dtype) {
  KH_REQUIRE_INIT();
  KH_REQUIRE(op >= 0 && op <= 2, "kh_unary: unknown op %d", op);
  KH_REQUIRE(n >= 0, "kh_unary: negative count");
  if (n == 0) return KH_OK;
  KH_REQUIRE(x && out, "kh_unary: null pointer");
  if (dtype == KH_F32)
    unary_kernel<float><<<grid_for(n), kThreads, 0, stream()>>>((const float*)x, (float*)out, n, op);
  else if (dtype == KH_BF16)
    unary_kernel<uint16_t><<<grid_for(n), kThreads, 0, stream()>>>((const uint16_t*)x, (uint16_t*)out, n, op);
  else
    KH_REQUIRE(false, "kh_unary: unsupported dtype %d", dtype);
  KH_CHECK_LAUNCH();
  return KH_OK;
}

int kh_arange(void* out, int64_t n, double start, double step, int dtype) {
  KH_REQUIRE_INIT();
  KH_REQUIRE(n >= 0, "kh_arange: negative count");
  if (n == 0) return KH_OK;
  KH_REQUIRE(out, "kh_arange: null pointer");
  if (dtype == KH_F32)
    arange_kernel<float><<<grid_for(n), kThreads, 0, stream()>>>((float*)out, n, (float)start, (float)step);
  else if (dtype == KH_BF16)
    arange_kernel<uint16_t><<<grid_for(n), kThreads, 0, stream()>>>((uint16_t*)out, n, (float)start, (float)step);
  else if (dtype == KH_I32)
    arange_i32_kernel<<<grid_for(n), kThreads, 0, stream()>>>((int32_t*)out, n, (int32_t)start, (int32_t)step);
  else
    KH_REQUIRE(false, "kh_arange: unsupported dtype %d", dtype);
  KH_CHECK_LAUNCH();
  return KH_OK;
}

int kh_silu_mul(const void* gate, int64_t gate_row_stride, const void* up, int64_t up_row_stride, void* out,
                int64_t out_row_stride, int64_t rows, int64_t n, int dtype) {
  KH_REQUIRE_INIT();
  KH_REQUIRE(rows >= 0 && n >= 0, "kh_silu_mul: negative extent");
  if (rows == 0 || n == 0) return KH_OK;
  KH_REQUIRE(gate && up && out, "kh_silu_mul: null pointer");
  KH_REQUIRE(gate_row_stride >= n && up_row_stride >= n && out_row_stride >= n,
             "kh_silu_mul: row strides must be >= n");
  if (dtype == KH_BF16) {
    const bool vec = n % 8 == 0 && gate_row_stride % 8 == 0 && up_row_stride % 8 == 0 && out_row_stride % 8 == 0 &&
                     aligned16(gate) && aligned16(up) && aligned16(out);
    if (vec)
      silu_mul_bf16x8_kernel<<<grid_for(rows * (n / 8)), kThreads, 0, stream()>>>(
          (const uint16_t*)gate, gate_row_stride, (const uint16_t*)up, up_row_stride, (uint16_t*)out, out_row_stride,
          rows, n / 8);
    else
      silu_mul_kernel<uint16_t><<<grid_for(rows * n), kThreads, 0, stream()>>>(
          (const uint16_t*)gate, gate_row_stride, (const uint16_t*)up, up_row_stride, (uint16_t*)out, out_row_stride,
          rows, n);
  } else if (dtype == KH_F32) {
    silu_mul_kernel<float><<<grid_for(rows * n), kThreads, 0, stream()>>>(
        (const float*)gate, gate_row_stride, (const float*)up, up_row_stride, (float*)out, out_row_stride, rows, n);
  } else {
    KH_REQUIRE(false, "kh_silu_mul: unsupported dtype %d", dtype);
  }
  KH_CHECK_LAUNCH();
  return KH_OK;
}

int kh_index_select(const void* table, int64_t n_rows, const int32_t* idx, int64_t n_idx, int64_t row_elems,
                    void* out, int dtype, int out_dtype) {
  KH_REQUIRE_INIT();
  return launch_index_select(table, 1, n_rows, row_elems, idx, n_idx, out, dtype, out_dtype, "kh_index_select");
}

int kh_index_select_dim(const void* table, int64_t outer, int64_t n_rows, int64_t inner, const int32_t* idx,
                        int64_t n_idx, void* out, int dtype, int out_dtype) {
  KH_REQUIRE_INIT();
  return launch_index_select(table, outer, n_rows, inner, idx, n_idx, out, dtype, out_dtype, "kh_index_select_dim");
}

int kh_greedy_advance(const int32_t* next_token, int32_t* position, int32_t* seq_len, int32_t* token_log,
                      int64_t log_base, int64_t log_cap) {
  KH_REQUIRE_INIT();
  KH_REQUIRE(next_token && position && seq_len, "kh_greedy_advance: null pointer");
  KH_REQUIRE(log_cap >= 0 && (log_cap == 0 || token_log != nullptr), "kh_greedy_advance: bad token log");
  greedy_advance_kernel<<<1, 1, 0, stream()>>>(next_token, position, seq_len, token_log, log_base, log_cap);
  KH_CHECK_LAUNCH();
  return KH_OK;
}

int kh_argmax(const void* x, int64_t rows, int64_t n, int32_t* out, int dtype) {
  KH_REQUIRE_INIT();
  KH_REQUIRE(rows >= 0 && n > 0, "kh_argmax: bad extents (rows %lld, n %lld)", (long long)rows, (long long)n);
  if (rows == 0) return KH_OK;
  KH_REQUIRE(rows <= INT32_MAX && n <= INT32_MAX, "kh_argmax: extents too large");
  KH_REQUIRE(x && out, "kh_argmax: null pointer");
  KH_REQUIRE(dtype == KH_F32 || dtype == KH_BF16, "kh_argmax: unsupported dtype %d", dtype);
  const int64_t nchunks = (n + AM_CHUNK - 1) / AM_CHUNK;
  float* pv = nullptr;
  int32_t* pi = nullptr;
  void* part = nullptr;
  if (nchunks > 1) {
    part = scratch_alloc((size_t)rows * nchunks * 8);
    KH_REQUIRE(part != nullptr, "kh_argmax: out of device memory for partials");
    pv = (float*)part;
    pi = (int32_t*)(pv + rows * nchunks);
  }
  const size_t esz = dtype == KH_F32 ? 4 : 2;
  for (int64_t r0 = 0; r0 < rows; r0 += 65535) {  // grid.y holds at most 65535 rows per launch
    const int64_t nr = rows - r0 < 65535 ? rows - r0 : 65535;
    const dim3 grid((unsigned)nchunks, (unsigned)nr);
    const void* xr = (const char*)x + (size_t)r0 * n * esz;
    float* pvr = pv ? pv + r0 * nchunks : nullptr;
    int32_t* pir = pi ? pi + r0 * nchunks : nullptr;
    if (dtype == KH_F32)
      argmax_partial_kernel<float><<<grid, kThreads, 0, stream()>>>((const float*)xr, n, pvr, pir, out + r0);
    else
      argmax_partial_kernel<uint16_t><<<grid, kThreads, 0, stream()>>>((const uint16_t*)xr, n, pvr, pir, out + r0);
    if (nchunks > 1)
      argmax_final_kernel<<<(unsigned)nr, kThreads, 0, stream()>>>(pvr, pir, (int)nchunks, out + r0);
  }
  if (part) scratch_free(part);  // stream-ordered reuse only
  KH_CHECK_LAUNCH();
  return KH_OK;
}

}  // extern "C"
