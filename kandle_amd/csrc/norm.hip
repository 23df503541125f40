// RMSNorm and the fused per-head qk-norm + rotary embedding (+ optional V copy) kernels.
//
// Both are HBM-bound single-pass kernels: each element is read once and written once, with
// 16-byte lane accesses.  Math is fp32 for both bf16 and fp32 storage.
//
// RMSNorm follows the reference formula exactly: rms = sqrt(sum(x^2)/N + eps), scale = 1/rms,
// y = (x * scale) * w   (reference: packages/backend-webgpu/src/kernels/normalize/shaderBuilder.ts:394-411).
#include <type_traits>

#include "common.h"
#include "qk_rope.h"

using namespace kh;

namespace {

// ---- 8-element vector access for float and bf16 -------------------------------------------
template <typename T>
struct Vec8;
template <>
struct Vec8<uint16_t> {
  // Raw form: the loaded bytes, converted later (so that several loads can be in flight).
  using Raw = uint4;
  static __device__ __forceinline__ Raw ld(const uint16_t* p) { return *reinterpret_cast<const uint4*>(p); }
  static __device__ __forceinline__ void cvt(const Raw& w, float (&v)[8]) {
    v[0] = lo_bf16(w.x); v[1] = hi_bf16(w.x); v[2] = lo_bf16(w.y); v[3] = hi_bf16(w.y);
    v[4] = lo_bf16(w.z); v[5] = hi_bf16(w.z); v[6] = lo_bf16(w.w); v[7] = hi_bf16(w.w);
  }
  static __device__ __forceinline__ void load(const uint16_t* p, float (&v)[8]) { cvt(ld(p), v); }
  static __device__ __forceinline__ void store(uint16_t* p, const float (&v)[8]) {
    *reinterpret_cast<uint4*>(p) = make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]),
                                              pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7]));
  }
};
template <>
struct Vec8<float> {
  struct Raw {
    float4 a, b;
  };
  static __device__ __forceinline__ Raw ld(const float* p) {
    return Raw{reinterpret_cast<const float4*>(p)[0], reinterpret_cast<const float4*>(p)[1]};
  }
  static __device__ __forceinline__ void cvt(const Raw& r, float (&v)[8]) {
    v[0] = r.a.x; v[1] = r.a.y; v[2] = r.a.z; v[3] = r.a.w; v[4] = r.b.x; v[5] = r.b.y; v[6] = r.b.z; v[7] = r.b.w;
  }
  static __device__ __forceinline__ void load(const float* p, float (&v)[8]) { cvt(ld(p), v); }
  static __device__ __forceinline__ void store(float* p, const float (&v)[8]) {
    reinterpret_cast<float4*>(p)[0] = make_float4(v[0], v[1], v[2], v[3]);
    reinterpret_cast<float4*>(p)[1] = make_float4(v[4], v[5], v[6], v[7]);
  }
};

// ---- RMSNorm: one wave per row, row kept in registers (n <= 64 * 8 * CPL) -----------------
// The row's math once its values v are in registers (lane chunk c holds elements 8 (lane + 64 c)
// .. + 7): sum of squares, 1 / rms, y = (v * inv) * w.  Shared by the plain and the fused
// residual kernels, so both round identically.
template <typename TO, int CPL>
__device__ __forceinline__ void rms_row(const float (&v)[CPL][8], const typename Vec8<TO>::Raw (&rw)[CPL],
                                       bool has_w, int lane, int nchunks, int n, float eps, TO* yr) {
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    if (lane + 64 * c < nchunks) {
#pragma unroll
      for (int j = 0; j < 8; ++j) ss += v[c][j] * v[c][j];
    }
  }
  ss = wave_sum(ss);
  const float rms = sqrtf(ss / (float)n + eps);
  const float inv = 1.0f / rms;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int ch = lane + 64 * c;
    if (ch < nchunks) {
      float o[8];
      if (has_w) {
        float wv[8];
        Vec8<TO>::cvt(rw[c], wv);
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = (v[c][j] * inv) * wv[j];
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = v[c][j] * inv;
      }
      Vec8<TO>::store(yr + ch * 8, o);
    }
  }
}

// x has element type TI; w and y have TO (e.g. a float32 residual stream normalised into bf16).
// Every load of the row and of the weights is issued before any math (lanes past the row end load
// the last chunk again and ignore it), so a wave waits for one memory round trip, not one per chunk.
template <typename TI, typename TO, int CPL>
__global__ __launch_bounds__(256) void rms_norm_vec_kernel(const TI* __restrict__ x, int64_t xs,
                                                            const TO* __restrict__ w, TO* __restrict__ y,
                                                            int64_t ys, int64_t rows, int n, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * (blockDim.x >> 6) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (row >= rows) return;
  const int nchunks = n >> 3;
  const TI* xr = x + row * xs;
  typename Vec8<TI>::Raw rx[CPL];
  typename Vec8<TO>::Raw rw[CPL];
#pragma unroll
  for (int c = 0; c < CPL; ++c) rx[c] = Vec8<TI>::ld(xr + min(lane + 64 * c, nchunks - 1) * 8);
  if (w != nullptr) {
#pragma unroll
    for (int c = 0; c < CPL; ++c) rw[c] = Vec8<TO>::ld(w + min(lane + 64 * c, nchunks - 1) * 8);
  }
  float v[CPL][8];
#pragma unroll
  for (int c = 0; c < CPL; ++c) Vec8<TI>::cvt(rx[c], v[c]);
  rms_row<TO, CPL>(v, rw, w != nullptr, lane, nchunks, n, eps, y + row * ys);
}

// ---- Split-K residual add + RMSNorm (kh_add_rms_norm) ----------------------------------------
// x[row] = (sum over splits s, in order from 0, of part[s][row]) + x[row] -- the fp32 result the
// GEMM's split reduction with a beta = 1 residual writes -- then y[row] = RMSNorm(x[row]) * w as
// rms_norm_vec_kernel computes it.  Rows are contiguous (stride n); part[s] starts s * pstride
// elements after part.
constexpr int kAddNormMaxSplits = 8;
template <typename TO, int CPL>
__global__ __launch_bounds__(256) void add_rms_norm_kernel(const float* __restrict__ part, int splits,
                                                            int64_t pstride, float* x, const TO* __restrict__ w,
                                                            TO* __restrict__ y, int64_t rows, int n, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * (blockDim.x >> 6) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (row >= rows) return;
  const int nchunks = n >> 3;
  float* xr = x + row * n;
  const float* pr = part + row * n;
  typename Vec8<float>::Raw rx[CPL], rp[kAddNormMaxSplits][CPL];
  typename Vec8<TO>::Raw rw[CPL];
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int off = min(lane + 64 * c, nchunks - 1) * 8;
#pragma unroll
    for (int s2 = 0; s2 < kAddNormMaxSplits; ++s2)
      if (s2 < splits) rp[s2][c] = Vec8<float>::ld(pr + s2 * pstride + off);
    rx[c] = Vec8<float>::ld(xr + off);
    rw[c] = Vec8<TO>::ld(w + off);
  }
  float v[CPL][8];
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    float xo[8], pv[8];
    Vec8<float>::cvt(rx[c], xo);
#pragma unroll
    for (int j = 0; j < 8; ++j) v[c][j] = 0.f;
#pragma unroll
    for (int s2 = 0; s2 < kAddNormMaxSplits; ++s2)
      if (s2 < splits) {
        Vec8<float>::cvt(rp[s2][c], pv);
#pragma unroll
        for (int j = 0; j < 8; ++j) v[c][j] += pv[j];
      }
#pragma unroll
    for (int j = 0; j < 8; ++j) v[c][j] += xo[j];
    if (lane + 64 * c < nchunks) Vec8<float>::store(xr + (lane + 64 * c) * 8, v[c]);
  }
  rms_row<TO, CPL>(v, rw, true, lane, nchunks, n, eps, y + row * n);
}

// Generic RMSNorm (any n, any alignment): one wave per row, two passes over the row.
template <typename TI, typename TO>
__global__ __launch_bounds__(256) void rms_norm_generic_kernel(const TI* __restrict__ x, int64_t xs,
                                                                const TO* __restrict__ w, TO* __restrict__ y,
                                                                int64_t ys, int64_t rows, int64_t n, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (row >= rows) return;
  const TI* xr = x + row * xs;
  float ss = 0.f;
  for (int64_t i = lane; i < n; i += 64) {
    const float v = Elem<TI>::load(xr, i);
    ss += v * v;
  }
  ss = wave_sum(ss);
  const float rms = sqrtf(ss / (float)n + eps);
  const float inv = 1.0f / rms;
  TO* yr = y + row * ys;
  for (int64_t i = lane; i < n; i += 64) {
    const float nv = Elem<TI>::load(xr, i) * inv;
    Elem<TO>::store(yr, i, w != nullptr ? nv * Elem<TO>::load(w, i) : nv);
  }
}

// ---- fused qk-norm + RoPE ---------------------------------------------------------------
// One wave per token.  A head row of D elements is owned by LPR = D/16 lanes; lane t of a row holds
// elements [8t, 8t+8) and [D/2 + 8t, D/2 + 8t + 8), so rotate_half pairs stay inside the lane and
// each lane needs cos/sin for frequencies 8t..8t+7 only.  Each frequency's sincosf is evaluated by
// one lane and read by the others (a full-range sincosf is ~200 VALU instructions; eight per lane
// made the kernel VALU bound).
struct QkStrides {
  int64_t s[18];
};

// A wave handles `spw` consecutive row steps of one token: steps [0, qk_steps) are RPW q/k head
// rows each (q heads first), steps [qk_steps, qk_steps + v_steps) copy RPW V rows each.  The host
// gives a long sequence one wave per token (spw = all steps: the angles are computed once per
// token) and a short one (decode) one step per wave, so a single token still spreads over waves.
// Token and step indices are wave-uniform (scalar registers); the host bounds them below 2^32.
template <typename T, int D, int NB>
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(
    const T* __restrict__ q, const T* __restrict__ k, T* __restrict__ qo, T* __restrict__ ko,
    const T* __restrict__ v, T* __restrict__ vo, const T* __restrict__ wq, const T* __restrict__ wk,
    const float* __restrict__ inv_freq, const int32_t* __restrict__ positions, uint32_t n_tokens,
    uint32_t seq_len, int hq, int hkv, QkStrides st, float eps, int64_t kv_cache_len, int spw) {
  constexpr int LPR = D / 16;        // lanes per row
  constexpr int RPW = 64 / LPR;      // rows per wave step
  constexpr int HALF = D / 2;
  const int lane = threadIdx.x & 63;
  const int qk_steps = (hq + hkv + RPW - 1) / RPW;
  const int v_steps = v != nullptr ? (hkv + RPW - 1) / RPW : 0;
  const int total_steps = qk_steps + v_steps;
  const uint32_t groups = (uint32_t)((total_steps + spw - 1) / spw);
  const uint32_t gw = blockIdx.x * (blockDim.x >> 6) + (uint32_t)__builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t tok = gw / groups;
  if (tok >= n_tokens) return;
  const int step0 = (int)(gw - tok * groups) * spw;
  const int step1 = min(step0 + spw, total_steps);
  const uint32_t b = tok / seq_len, s = tok - b * seq_len;
  const int t = lane % LPR;          // chunk index inside the row
  const int rsub = lane / LPR;       // row slot inside the step
  const int total_rows = hq + hkv;

  // K/V destination row: the token's index in its sequence, or (cache addressing) its position,
  // in which case a position outside the cache writes no K/V row.
  const int32_t ipos = positions[tok];
  const bool cache_mode = kv_cache_len > 0;
  const int64_t kv_row = cache_mode ? (int64_t)ipos : (int64_t)s;
  const bool kv_ok = !cache_mode || (ipos >= 0 && (int64_t)ipos < kv_cache_len);
  const T* qt = q + b * st.s[0] + s * st.s[1];
  const T* kt = k + b * st.s[3] + s * st.s[4];
  const T* vt = v ? v + b * st.s[12] + s * st.s[13] : v;
  T* qot = qo + b * st.s[6] + s * st.s[7];
  T* kot = ko + b * st.s[9] + kv_row * st.s[10];
  T* vot = vo ? vo + b * st.s[15] + kv_row * st.s[16] : vo;

  // Row steps are processed in batches of NB: every load of a batch is issued, unconditionally,
  // before any math, so a wave keeps NB * 32 bytes per lane in flight.  Rows past the end of a
  // partial step or batch load a valid clamped row and store nothing.  The host uses NB = 1: at
  // NB = 3 the kernel needs 142 VGPRs (3 waves per SIMD), at NB = 1 106 (4 waves), and the extra
  // resident waves hide more latency than the deeper batch (C2: 4.97 -> 5.28 TB/s).
  float cs[8], sn[8];
  // The frequencies are loaded before the rows (loads complete in order, so the angles can then be
  // computed while the row loads are in flight); the weights after them.
  float f0 = 0.f, f1 = 0.f;
  if (step0 < qk_steps) {
    if (lane < HALF) f0 = inv_freq[lane];
    if (HALF > 64 && lane + 64 < HALF) f1 = inv_freq[lane + 64];
  }
  for (int base = step0; base < step1; base += NB) {
    typename Vec8<T>::Raw ra[NB], rc[NB], rwa[NB], rwb[NB];
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      const int step = min(base + u, step1 - 1);
      const T* src;
      if (step < qk_steps) {
        const int r = min(step * RPW + rsub, total_rows - 1);
        src = r < hq ? qt + (int64_t)r * st.s[2] : kt + (int64_t)(r - hq) * st.s[5];
        // this lane's row weights (q_norm or k_norm), loaded with the row
        const T* wsrc = r < hq ? wq : wk;
        rwa[u] = Vec8<T>::ld(wsrc + 8 * t);
        rwb[u] = Vec8<T>::ld(wsrc + HALF + 8 * t);
      } else {
        const int h = min((step - qk_steps) * RPW + rsub, hkv - 1);
        src = vt + (int64_t)h * st.s[14];
      }
      ra[u] = Vec8<T>::ld(src + 8 * t);
      rc[u] = Vec8<T>::ld(src + HALF + 8 * t);
    }
    if (base == step0 && step0 < qk_steps) {
      // Keeps the angle computation below the row loads (the compiler would otherwise hoist it,
      // and its wait for the frequencies, above them).
      asm volatile("" : "+v"(f0), "+v"(f1));
      // cos/sin of f = float(pos) * inv_freq[i]: lane i evaluates frequencies i and i + 64 once,
      // then each lane gathers its eight (i = 8t .. 8t+7) from the lanes that hold them.
      const float pos = (float)ipos;
      float c0 = 1.f, s0 = 0.f;
      if (lane < HALF) sincosf(pos * f0, &s0, &c0);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int i = 8 * t + j;
        cs[j] = __shfl(c0, i & 63, 64);
        sn[j] = __shfl(s0, i & 63, 64);
      }
      if (HALF > 64) {
        float c1 = 1.f, s1 = 0.f;
        if (lane + 64 < HALF) sincosf(pos * f1, &s1, &c1);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int i = 8 * t + j;
          const float c1j = __shfl(c1, i & 63, 64), s1j = __shfl(s1, i & 63, 64);
          if (i >= 64) {
            cs[j] = c1j;
            sn[j] = s1j;
          }
        }
      }
    }
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      const int step = base + u;
      if (step >= step1) break;
      float a[8], c[8];
      Vec8<T>::cvt(ra[u], a);
      Vec8<T>::cvt(rc[u], c);
      if (step < qk_steps) {
        const int r = step * RPW + rsub;
        const bool isq = r < hq;
        const bool active = r < total_rows && (isq || kv_ok);
        float wa[8], wb[8];
        Vec8<T>::cvt(rwa[u], wa);
        Vec8<T>::cvt(rwb[u], wb);
        float oa[8], oc[8];
        qk_norm_rope_row<D>(a, c, wa, wb, cs, sn, eps, oa, oc);
        if (active) {
          T* dst = isq ? qot + (int64_t)r * st.s[8] : kot + (int64_t)(r - hq) * st.s[11];
          Vec8<T>::store(dst + 8 * t, oa);
          Vec8<T>::store(dst + HALF + 8 * t, oc);
        }
      } else {
        // Fused KV-cache write of V rows (unchanged values).
        const int h = (step - qk_steps) * RPW + rsub;
        if (h < hkv && kv_ok) {
          T* dst = vot + (int64_t)h * st.s[17];
          Vec8<T>::store(dst + 8 * t, a);
          Vec8<T>::store(dst + HALF + 8 * t, c);
        }
      }
    }
  }
}

template <typename T, int D, typename... Args>
void launch_qk_norm_rope_d(int nb, int grid, int block, Args... args) {
  (void)nb;  // one row step per load batch (see the kernel)
  qk_norm_rope_kernel<T, D, 1><<<grid, block, 0, stream()>>>(args...);
}
template <typename T, typename... Args>
void launch_qk_norm_rope(int head_dim, int nb, int grid, int block, Args... args) {
  switch (head_dim) {
    case 32: launch_qk_norm_rope_d<T, 32>(nb, grid, block, args...); break;
    case 64: launch_qk_norm_rope_d<T, 64>(nb, grid, block, args...); break;
    case 128: launch_qk_norm_rope_d<T, 128>(nb, grid, block, args...); break;
    default: launch_qk_norm_rope_d<T, 256>(nb, grid, block, args...); break;
  }
}

template <typename TI, typename TO>
int launch_rms_norm(const void* x, int64_t xs, const void* w, void* y, int64_t ys, int64_t rows, int64_t n,
                    float eps) {
  const int waves = 4;
  const int64_t grid = (rows + waves - 1) / waves;
  KH_REQUIRE(grid <= INT32_MAX, "kh_rms_norm: too many rows");
  const bool vec = n % 8 == 0 && xs % 8 == 0 && ys % 8 == 0 && aligned16(x) && aligned16(y) &&
                   (w == nullptr || aligned16(w));
  const TI* xp = (const TI*)x;
  const TO* wp = (const TO*)w;
  TO* yp = (TO*)y;
  if (vec && n <= 64 * 8 * 1)
    rms_norm_vec_kernel<TI, TO, 1><<<(int)grid, 64 * waves, 0, stream()>>>(xp, xs, wp, yp, ys, rows, (int)n, eps);
  else if (vec && n <= 64 * 8 * 2)
    rms_norm_vec_kernel<TI, TO, 2><<<(int)grid, 64 * waves, 0, stream()>>>(xp, xs, wp, yp, ys, rows, (int)n, eps);
  else if (vec && n <= 64 * 8 * 4)
    rms_norm_vec_kernel<TI, TO, 4><<<(int)grid, 64 * waves, 0, stream()>>>(xp, xs, wp, yp, ys, rows, (int)n, eps);
  else if (vec && n <= 64 * 8 * 8)
    rms_norm_vec_kernel<TI, TO, 8><<<(int)grid, 64 * waves, 0, stream()>>>(xp, xs, wp, yp, ys, rows, (int)n, eps);
  else
    rms_norm_generic_kernel<TI, TO><<<(int)grid, 64 * waves, 0, stream()>>>(xp, xs, wp, yp, ys, rows, n, eps);
  KH_CHECK_LAUNCH();
  return KH_OK;
}

}  // namespace

extern "C" {

int kh_rms_norm(const void* x, int64_t x_row_stride, const void* w, void* y, int64_t y_row_stride, int64_t rows,
                int64_t n, float eps, int dtype, int out_dtype) {
  KH_REQUIRE_INIT();
  KH_REQUIRE(rows >= 0 && n > 0, "kh_rms_norm: bad extents (rows %lld, n %lld)", (long long)rows, (long long)n);
  if (rows == 0) return KH_OK;
  KH_REQUIRE(x && y, "kh_rms_norm: null pointer");
  KH_REQUIRE(x_row_stride >= n && y_row_stride >= n, "kh_rms_norm: row strides must be >= n");
  if (dtype == KH_BF16 && out_dtype == KH_BF16)
    return launch_rms_norm<uint16_t, uint16_t>(x, x_row_stride, w, y, y_row_stride, rows, n, eps);
  if (dtype == KH_F32 && out_dtype == KH_F32)
    return launch_rms_norm<float, float>(x, x_row_stride, w, y, y_row_stride, rows, n, eps);
  if (dtype == KH_F32 && out_dtype == KH_BF16)
    return launch_rms_norm<float, uint16_t>(x, x_row_stride, w, y, y_row_stride, rows, n, eps);
  if (dtype == KH_BF16 && out_dtype == KH_F32)
    return launch_rms_norm<uint16_t, float>(x, x_row_stride, w, y, y_row_stride, rows, n, eps);
  KH_REQUIRE(false, "kh_rms_norm: unsupported dtypes (in %d, out %d)", dtype, out_dtype);
}

int kh_add_rms_norm(const float* part, int splits, int64_t split_stride, float* x, const void* w, void* y,
                    int64_t rows, int64_t n, float eps, int out_dtype) {
  KH_REQUIRE_INIT();
  KH_REQUIRE(rows >= 0 && n > 0, "kh_add_rms_norm: bad extents (rows %lld, n %lld)", (long long)rows, (long long)n);
  if (rows == 0) return KH_OK;
  KH_REQUIRE(part && x && w && y, "kh_add_rms_norm: null pointer");
  KH_REQUIRE(splits >= 1 && splits <= kAddNormMaxSplits, "kh_add_rms_norm: splits %d outside [1, %d]", splits,
             kAddNormMaxSplits);
  KH_REQUIRE(split_stride >= rows * n, "kh_add_rms_norm: split_stride below rows * n");
  KH_REQUIRE(n % 8 == 0 && n <= 64 * 8 * 4 && split_stride % 8 == 0,
             "kh_add_rms_norm: n must be a multiple of 8 up to 2048 (and split_stride a multiple of 8)");
  KH_REQUIRE(aligned16(part) && aligned16(x) && aligned16(w) && aligned16(y),
             "kh_add_rms_norm: pointers must be 16-byte aligned");
  KH_REQUIRE(out_dtype == KH_BF16 || out_dtype == KH_F32, "kh_add_rms_norm: unsupported output dtype %d", out_dtype);
  // One row (one wave) per workgroup: a C5 prefill's 512 rows then spread over every CU instead of
  // 128 four-wave workgroups (prefill 2.528 -> 2.514 ms over three runs).
  const int waves = 1;
  const int64_t grid = (rows + waves - 1) / waves;
  KH_REQUIRE(grid <= INT32_MAX, "kh_add_rms_norm: too many rows");
  auto run = [&](auto* wp, auto* yp) {
    using TO = std::remove_const_t<std::remove_pointer_t<decltype(wp)>>;
    if (n <= 64 * 8)
      add_rms_norm_kernel<TO, 1><<<(int)grid, 64 * waves, 0, stream()>>>(part, splits, split_stride, x, wp, yp, rows,
                                                                         (int)n, eps);
    else if (n <= 64 * 8 * 2)
      add_rms_norm_kernel<TO, 2><<<(int)grid, 64 * waves, 0, stream()>>>(part, splits, split_stride, x, wp, yp, rows,
                                                                         (int)n, eps);
    else
      add_rms_norm_kernel<TO, 4><<<(int)grid, 64 * waves, 0, stream()>>>(part, splits, split_stride, x, wp, yp, rows,
                                                                         (int)n, eps);
  };
  if (out_dtype == KH_BF16)
    run((const uint16_t*)w, (uint16_t*)y);
  else
    run((const float*)w, (float*)y);
  KH_CHECK_LAUNCH();
  return KH_OK;
}

int kh_qk_norm_rope(const void* q, const void* k, void* q_out, void* k_out, const void* v, void* v_out,
                    const void* wq, const void* wk, const float* inv_freq, const int32_t* positions,
                    int64_t n_batch, int64_t seq_len, int n_q_heads, int n_kv_heads, int head_dim,
                    const int64_t* strides, float eps, int dtype, int64_t kv_cache_len) {
  KH_REQUIRE_INIT();
  KH_REQUIRE(n_batch >= 0 && seq_len >= 0, "kh_qk_norm_rope: negative extent");
  KH_REQUIRE(kv_cache_len >= 0, "kh_qk_norm_rope: negative kv_cache_len");
  KH_REQUIRE(n_q_heads > 0 && n_kv_heads > 0, "kh_qk_norm_rope: head counts must be positive");
  KH_REQUIRE(head_dim == 32 || head_dim == 64 || head_dim == 128 || head_dim == 256,
             "kh_qk_norm_rope: head_dim %d not in {32, 64, 128, 256}", head_dim);
  KH_REQUIRE(dtype == KH_BF16 || dtype == KH_F32, "kh_qk_norm_rope: unsupported dtype %d", dtype);
  const int64_t n_tokens = n_batch * seq_len;
  if (n_tokens == 0) return KH_OK;
  KH_REQUIRE(q && k && q_out && k_out && wq && wk && inv_freq && positions && strides,
             "kh_qk_norm_rope: null pointer");
  KH_REQUIRE((v == nullptr) == (v_out == nullptr), "kh_qk_norm_rope: v and v_out must both be set or both NULL");
  QkStrides st{};
  const int ns = v ? 18 : 12;
  const int64_t vec_elems = 16 / (dtype == KH_BF16 ? 2 : 4);
  for (int i = 0; i < ns; ++i) {
    st.s[i] = strides[i];
    KH_REQUIRE(strides[i] % vec_elems == 0, "kh_qk_norm_rope: stride %d (%lld) breaks 16-byte alignment", i,
               (long long)strides[i]);
  }
  const void* ptrs[8] = {q, k, q_out, k_out, wq, wk, v, v_out};
  for (int i = 0; i < 8; ++i)
    KH_REQUIRE(ptrs[i] == nullptr || aligned16(ptrs[i]), "kh_qk_norm_rope: pointer %d not 16-byte aligned", i);
  // Long sequences: one wave per token (angles once per token).  Short ones: one row step per wave.
  const int rpw = 64 / (head_dim / 16);
  const int total_steps = (n_q_heads + n_kv_heads + rpw - 1) / rpw + (v ? (n_kv_heads + rpw - 1) / rpw : 0);
  const int spw = n_tokens >= 2048 ? total_steps : 1;
  const int groups = (total_steps + spw - 1) / spw;
  const int nb = 1;
  const int waves = 4;
  const int64_t grid = (n_tokens * groups + waves - 1) / waves;
  KH_REQUIRE(grid * waves <= (int64_t)UINT32_MAX && seq_len <= (int64_t)UINT32_MAX,
             "kh_qk_norm_rope: too many tokens");
  if (dtype == KH_BF16)
    launch_qk_norm_rope<uint16_t>(head_dim, nb, (int)grid, 64 * waves, (const uint16_t*)q, (const uint16_t*)k,
                                  (uint16_t*)q_out, (uint16_t*)k_out, (const uint16_t*)v, (uint16_t*)v_out,
                                  (const uint16_t*)wq, (const uint16_t*)wk, inv_freq, positions, (uint32_t)n_tokens,
                                  (uint32_t)seq_len, n_q_heads, n_kv_heads, st, eps, kv_cache_len, spw);
  else
    launch_qk_norm_rope<float>(head_dim, nb, (int)grid, 64 * waves, (const float*)q, (const float*)k, (float*)q_out,
                               (float*)k_out, (const float*)v, (float*)v_out, (const float*)wq, (const float*)wk,
                               inv_freq, positions, (uint32_t)n_tokens, (uint32_t)seq_len, n_q_heads, n_kv_heads, st,
                               eps, kv_cache_len, spw);
  KH_CHECK_LAUNCH();
  return KH_OK;
}

}  // extern "C"
