// RMSNorm and the fused per-head qk-norm + rotary embedding (+ optional V copy) kernels.
//
// Both are HBM-bound single-pass kernels: each element is read once and written once, with
// 16-byte lane accesses.  Math is fp32 for both bf16 and fp32 storage.
//
// RMSNorm follows the reference formula exactly: rms = sqrt(sum(x^2)/N + eps), scale = 1/rms,
// y = (x * scale) * w   (reference: packages/backend-webgpu/src/kernels/normalize/shaderBuilder.ts:394-411).
#include "common.h"

using namespace kh;

namespace {

// ---- 8-element vector access for float and bf16 -------------------------------------------
template <typename T>
struct Vec8;
template <>
struct Vec8<uint16_t> {
  static __device__ __forceinline__ void load(const uint16_t* p, float (&v)[8]) {
    const uint4 w = *reinterpret_cast<const uint4*>(p);
    v[0] = lo_bf16(w.x); v[1] = hi_bf16(w.x); v[2] = lo_bf16(w.y); v[3] = hi_bf16(w.y);
    v[4] = lo_bf16(w.z); v[5] = hi_bf16(w.z); v[6] = lo_bf16(w.w); v[7] = hi_bf16(w.w);
  }
  static __device__ __forceinline__ void store(uint16_t* p, const float (&v)[8]) {
    *reinterpret_cast<uint4*>(p) = make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]),
                                              pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7]));
  }
};
template <>
struct Vec8<float> {
  static __device__ __forceinline__ void load(const float* p, float (&v)[8]) {
    const float4 a = reinterpret_cast<const float4*>(p)[0];
    const float4 b = reinterpret_cast<const float4*>(p)[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  }
  static __device__ __forceinline__ void store(float* p, const float (&v)[8]) {
    reinterpret_cast<float4*>(p)[0] = make_float4(v[0], v[1], v[2], v[3]);
    reinterpret_cast<float4*>(p)[1] = make_float4(v[4], v[5], v[6], v[7]);
  }
};

// ---- RMSNorm: one wave per row, row kept in registers (n <= 64 * 8 * CPL) -----------------
// x has element type TI; w and y have TO (e.g. a float32 residual stream normalised into bf16).
template <typename TI, typename TO, int CPL>
__global__ __launch_bounds__(256) void rms_norm_vec_kernel(const TI* __restrict__ x, int64_t xs,
                                                            const TO* __restrict__ w, TO* __restrict__ y,
                                                            int64_t ys, int64_t rows, int n, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int nchunks = n >> 3;
  const TI* xr = x + row * xs;
  float v[CPL][8];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int ch = lane + 64 * c;
    if (ch < nchunks) {
      Vec8<TI>::load(xr + ch * 8, v[c]);
#pragma unroll
      for (int j = 0; j < 8; ++j) ss += v[c][j] * v[c][j];
    }
  }
  ss = wave_sum(ss);
  const float rms = sqrtf(ss / (float)n + eps);
  const float inv = 1.0f / rms;
  TO* yr = y + row * ys;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int ch = lane + 64 * c;
    if (ch < nchunks) {
      float o[8];
      if (w != nullptr) {
        float wv[8];
        Vec8<TO>::load(w + ch * 8, wv);
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
// each lane needs cos/sin for frequencies 8t..8t+7 only (computed once per token).
struct QkStrides {
  int64_t s[18];
};

// A wave handles `spw` consecutive row steps of one token: steps [0, qk_steps) are RPW q/k head
// rows each (q heads first), steps [qk_steps, qk_steps + v_steps) copy RPW V rows each.  The host
// gives a long sequence one wave per token (spw = all steps: the angles are computed once per
// token) and a short one (decode) one step per wave, so a single token still spreads over waves.
template <typename T>
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(
    const T* __restrict__ q, const T* __restrict__ k, T* __restrict__ qo, T* __restrict__ ko,
    const T* __restrict__ v, T* __restrict__ vo, const T* __restrict__ wq, const T* __restrict__ wk,
    const float* __restrict__ inv_freq, const int32_t* __restrict__ positions, int64_t n_tokens, int64_t seq_len,
    int hq, int hkv, int D, QkStrides st, float eps, int64_t kv_cache_len, int spw) {
  const int lane = threadIdx.x & 63;
  const int LPR = D >> 4;            // lanes per row
  const int RPW = 64 / LPR;          // rows per wave step
  const int qk_steps = (hq + hkv + RPW - 1) / RPW;
  const int v_steps = v != nullptr ? (hkv + RPW - 1) / RPW : 0;
  const int total_steps = qk_steps + v_steps;
  const int groups = (total_steps + spw - 1) / spw;
  const int64_t gw = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int64_t tok = gw / groups;
  if (tok >= n_tokens) return;
  const int step0 = (int)(gw - tok * groups) * spw;
  const int step1 = min(step0 + spw, total_steps);
  const int64_t b = tok / seq_len, s = tok - b * seq_len;
  const int t = lane % LPR;          // chunk index inside the row
  const int rsub = lane / LPR;       // row slot inside the step
  const int half = D >> 1;

  // K/V destination row: the token's index in its sequence, or (cache addressing) its position,
  // in which case a position outside the cache writes no K/V row.
  const int32_t ipos = positions[tok];
  const bool cache_mode = kv_cache_len > 0;
  const int64_t kv_row = cache_mode ? (int64_t)ipos : s;
  const bool kv_ok = !cache_mode || (ipos >= 0 && (int64_t)ipos < kv_cache_len);

  if (step0 < qk_steps) {
    // cos/sin of f = float(pos) * inv_freq[i] for i = 8t..8t+7.
    const float pos = (float)ipos;
    float cs[8], sn[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float f = pos * inv_freq[8 * t + j];
      sincosf(f, &sn[j], &cs[j]);
    }
    float wqa[8], wqb[8], wka[8], wkb[8];
    Vec8<T>::load(wq + 8 * t, wqa);
    Vec8<T>::load(wq + half + 8 * t, wqb);
    Vec8<T>::load(wk + 8 * t, wka);
    Vec8<T>::load(wk + half + 8 * t, wkb);

    const int total_rows = hq + hkv;
    const int qk_end = min(step1, qk_steps);
    for (int step = step0; step < qk_end; ++step) {
      const int r = step * RPW + rsub;
      const bool isq = r < hq;
      const bool active = r < total_rows && (isq || kv_ok);
      const int h = isq ? r : r - hq;
      const T* src;
      T* dst;
      if (isq) {
        src = q + b * st.s[0] + s * st.s[1] + (int64_t)h * st.s[2];
        dst = qo + b * st.s[6] + s * st.s[7] + (int64_t)h * st.s[8];
      } else {
        src = k + b * st.s[3] + s * st.s[4] + (int64_t)h * st.s[5];
        dst = ko + b * st.s[9] + kv_row * st.s[10] + (int64_t)h * st.s[11];
      }
      float a[8], c[8];
      float ss = 0.f;
      if (active) {
        Vec8<T>::load(src + 8 * t, a);
        Vec8<T>::load(src + half + 8 * t, c);
#pragma unroll
        for (int j = 0; j < 8; ++j) ss += a[j] * a[j] + c[j] * c[j];
      }
      // Reduce over the LPR lanes of this row (LPR is a power of two <= 16).
      for (int o = LPR >> 1; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
      if (active) {
        const float inv = 1.0f / sqrtf(ss / (float)D + eps);
        float oa[8], oc[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float na = (a[j] * inv) * (isq ? wqa[j] : wka[j]);
          const float nc = (c[j] * inv) * (isq ? wqb[j] : wkb[j]);
          oa[j] = na * cs[j] + (-nc) * sn[j];
          oc[j] = nc * cs[j] + na * sn[j];
        }
        Vec8<T>::store(dst + 8 * t, oa);
        Vec8<T>::store(dst + half + 8 * t, oc);
      }
    }
  }
  if (kv_ok) {
    // Fused KV-cache write of V rows (unchanged values).
    for (int step = max(step0, qk_steps); step < step1; ++step) {
      const int h = (step - qk_steps) * RPW + rsub;
      if (h < hkv) {
        const T* src = v + b * st.s[12] + s * st.s[13] + (int64_t)h * st.s[14];
        T* dst = vo + b * st.s[15] + kv_row * st.s[16] + (int64_t)h * st.s[17];
        float a[8], c[8];
        Vec8<T>::load(src + 8 * t, a);
        Vec8<T>::load(src + half + 8 * t, c);
        Vec8<T>::store(dst + 8 * t, a);
        Vec8<T>::store(dst + half + 8 * t, c);
      }
    }
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
  const int waves = 4;
  const int64_t grid = (n_tokens * groups + waves - 1) / waves;
  KH_REQUIRE(grid <= INT32_MAX, "kh_qk_norm_rope: too many tokens");
  if (dtype == KH_BF16)
    qk_norm_rope_kernel<uint16_t><<<(int)grid, 64 * waves, 0, stream()>>>(
        (const uint16_t*)q, (const uint16_t*)k, (uint16_t*)q_out, (uint16_t*)k_out, (const uint16_t*)v,
        (uint16_t*)v_out, (const uint16_t*)wq, (const uint16_t*)wk, inv_freq, positions, n_tokens, seq_len,
        n_q_heads, n_kv_heads, head_dim, st, eps, kv_cache_len, spw);
  else
    qk_norm_rope_kernel<float><<<(int)grid, 64 * waves, 0, stream()>>>(
        (const float*)q, (const float*)k, (float*)q_out, (float*)k_out, (const float*)v, (float*)v_out,
        (const float*)wq, (const float*)wk, inv_freq, positions, n_tokens, seq_len, n_q_heads, n_kv_heads, head_dim,
        st, eps, kv_cache_len, spw);
  KH_CHECK_LAUNCH();
  return KH_OK;
}

}  // extern "C"
