// Scaled dot-product attention entry points for gfx950: routing to the bf16 MFMA flash prefill
// (flash_prefill.hip), the fp32 MFMA flash kernel (flash_f32.hip), the split-K decode kernels and a
// generic fp32-math kernel (this file).
//
// Semantics (reference: packages/backend-webgpu/src/kernels/attention/builder.ts:138-329):
//   S = (Q K^T) * scale, causal masks key j > query i (top-left aligned), GQA query head h reads
//   kv head h / (hq / hkv), online softmax in fp32, O = P V / l.
#include <cfloat>
#include <cmath>

#include <type_traits>

#include "attention.h"

using namespace kh;

namespace {

// =============================================================================================
// Generic attention (f32 or bf16 storage, d <= 256, any lq/lk): one wave per query row, 64 keys
// per step (lane j scores key k0 + j), fp32 online softmax, each lane accumulates d/64 output
// columns.  Used for masked fp32 calls and shapes the MFMA kernels do not take.
// =============================================================================================
//
// With a mask M (mdt KH_F32 or KH_BF16; the reference's explicit-mask route, composite.ts:279-300)
// a score is s = (q . k) * scale + M[b, h, i, j], causal is not applied, the running max starts at
// f32(-1e38) as in the reference softmax (normalize/shaderBuilder.ts:190-195), and a row whose
// exponentials sum to 0 stores NaN (0 / 0).
template <typename T>
__global__ __launch_bounds__(256) void attn_generic_kernel(const T* __restrict__ Q, const T* __restrict__ K,
                                                           const T* __restrict__ V, T* __restrict__ O, int batch,
                                                           int hq, int hkv, int lq, int lk, int D, AttnStrides st,
                                                           float scale, int causal, const void* __restrict__ M,
                                                           int mdt, MaskArgs ma) {
  __shared__ float qs[4][256];
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int64_t row = (int64_t)blockIdx.x * 4 + w;  // flattened (b, h, i)
  const int64_t total = (int64_t)batch * hq * lq;
  const bool valid = row < total;
  const int i = valid ? (int)(row % lq) : 0;
  const int h = valid ? (int)((row / lq) % hq) : 0;
  const int b = valid ? (int)(row / ((int64_t)lq * hq)) : 0;
  const int hk = h / (hq / hkv);
  const T* qrow = Q + b * st.qb + h * st.qh + (int64_t)i * st.qs;
  for (int d = lane; d < D; d += 64) qs[w][d] = valid ? Elem<T>::load(qrow, d) : 0.f;
  __syncthreads();
  if (!valid) return;
  const T* Kb = K + b * st.kb + hk * st.kh;
  const T* Vb = V + b * st.vb + hk * st.vh;
  const int kend = causal ? min(lk, i + 1) : lk;
  const int64_t mrow = M ? b * ma.sb + h * ma.sh + (int64_t)i * ma.sq : 0;
  float m = M ? -1e38f : -INFINITY, l = 0.f;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};  // columns lane, lane+64, lane+128, lane+192
  for (int k0 = 0; k0 < kend; k0 += 64) {
    const int key = k0 + lane;
    float s = -INFINITY;
    if (key < kend) {
      const T* kr = Kb + (int64_t)key * st.ks;
      float dot = 0.f;
      for (int d = 0; d < D; ++d) dot += qs[w][d] * Elem<T>::load(kr, d);
      s = dot * scale;
      if (M) {
        const int64_t mi = mrow + (int64_t)key * ma.sk;
        s += mdt == KH_F32 ? static_cast<const float*>(M)[mi]
                           : bf16_bits_to_f32(static_cast<const uint16_t*>(M)[mi]);
      }
    }
    const float mx = fmaxf(m, wave_max(s));
    const float alpha = expf(m - mx);
    const float p = (key < kend) ? expf(s - mx) : 0.f;
    l = l * alpha + wave_sum(p);
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[c] *= alpha;
    const int nk = min(64, kend - k0);
    for (int j = 0; j < nk; ++j) {
      const float pj = __shfl(p, j, 64);
      const T* vr = Vb + (int64_t)(k0 + j) * st.vs;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int d = lane + 64 * c;
        if (d < D) acc[c] += pj * Elem<T>::load(vr, d);
      }
    }
    m = mx;
  }
  T* orow = O + b * st.ob + h * st.oh + (int64_t)i * st.os;
  const float inv = l > 0.f ? 1.0f / l : (M ? __builtin_nanf("") : 0.f);
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int d = lane + 64 * c;
    if (d < D) Elem<T>::store(orow, d, acc[c] * inv);
  }
}

// Copies a strided mask into rows of ldm elements (unit key stride, 16-byte aligned 8-key runs)
// for the MFMA kernel: dst[((b' nh + h') nq + q') ldm + j] = src[b' sb + h' sh + q' sq + j sk] for
// j < lk, 0 for lk <= j < ldm.  Broadcast axes (stride 0) keep extent 1.
template <typename T>
__global__ __launch_bounds__(256) void mask_pack_kernel(const T* __restrict__ src, T* __restrict__ dst, int nh,
                                                        int nq, int lk, int ldm, int64_t sb, int64_t sh, int64_t sq,
                                                        int64_t sk, int64_t rows) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int q = (int)(row % nq), h = (int)((row / nq) % nh);
  const int64_t b = row / ((int64_t)nq * nh);
  const T* s = src + b * sb + h * sh + (int64_t)q * sq;
  T* d = dst + row * ldm;
  for (int j = threadIdx.x & 63; j < ldm; j += 64) d[j] = j < lk ? s[(int64_t)j * sk] : T(0);
}

// Attention operands staged in rows of ld elements (rows of a multiple of 16 bytes, 16-byte aligned),
// from and back to strided views with a unit column stride and any alignment.  Thread i handles
// the 16 bytes of V = 16 / sizeof(T) consecutive elements of one row with one 16-byte access on the
// staged side and element accesses on the caller's side.
// rows_pad_kernel: dst[((b' nh + h') nq + q') ld + j] = src[b' sb + h' sh + q' sq + j] for j < d, 0 for
// d <= j < ld.
template <typename T>
__global__ __launch_bounds__(256) void rows_pad_kernel(const T* __restrict__ src, T* __restrict__ dst, int nh, int nq,
                                                       int d, int ld, int64_t sb, int64_t sh, int64_t sq,
                                                       int64_t rows) {
  constexpr int V = 16 / sizeof(T);
  const int per_row = ld / V;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t row = i / per_row;
  if (row >= rows) return;
  const int j0 = (int)(i - row * per_row) * V;
  const int q = (int)(row % nq), h = (int)((row / nq) % nh);
  const int64_t b = row / ((int64_t)nq * nh);
  const T* s = src + b * sb + h * sh + (int64_t)q * sq;
  union {
    T e[V];
    uint4 u;
  } w;
#pragma unroll
  for (int e = 0; e < V; ++e) w.e[e] = j0 + e < d ? s[j0 + e] : T(0);
  *reinterpret_cast<uint4*>(dst + row * ld + j0) = w.u;
}

// rows_unpack_kernel: dst[b' sb + h' sh + q' sq + j] = src[((b' nh + h') nq + q') ld + j] for j < d.
template <typename T>
__global__ __launch_bounds__(256) void rows_unpack_kernel(const T* __restrict__ src, T* __restrict__ dst, int nh,
                                                          int nq, int d, int ld, int64_t sb, int64_t sh, int64_t sq,
                                                          int64_t rows) {
  constexpr int V = 16 / sizeof(T);
  const int per_row = (d + V - 1) / V;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t row = i / per_row;
  if (row >= rows) return;
  const int j0 = (int)(i - row * per_row) * V;
  const int q = (int)(row % nq), h = (int)((row / nq) % nh);
  const int64_t b = row / ((int64_t)nq * nh);
  T* o = dst + b * sb + h * sh + (int64_t)q * sq;
  union {
    T e[V];
    uint4 u;
  } w;
  w.u = *reinterpret_cast<const uint4*>(src + row * ld + j0);
#pragma unroll
  for (int e = 0; e < V; ++e)
    if (j0 + e < d) o[j0 + e] = w.e[e];
}

// =============================================================================================
// Split-K decode: one query token per sequence, per-sequence KV length.
//
// Work unit = (b, kv head, chunk of CHUNK keys); the G query heads of the kv head are served from
// the same K/V bytes.  A row of 128 elements is read by 16 (bf16) or 32 (f32) lanes with 16-byte
// buffer loads, so a wave covers 4 (2) keys per load instruction; all K and V loads of a wave's
// keys are issued before any math so the bytes in flight per lane stay high, and rows past the
// sequence end read as zero without a branch.  Each unit writes (m, l, o[d]) per query head; the
// merge kernel combines the chunks of a head with the log-sum-exp rule.
// =============================================================================================
constexpr int DC_WAVES = 4;
// Keys per wave per unit: 16 load instructions of 16 B per lane for K and for V in both dtypes.
template <typename T>
constexpr int dc_kpw() { return sizeof(T) == 2 ? 64 : 32; }
// Keys per split-K chunk.  Head dim 64 halves the bytes of a key row, so a chunk holds twice the
// keys and moves the same 64 KiB of K (and of V) per workgroup.
template <typename T, int DH = 128>
constexpr int dc_chunk() { return DC_WAVES * dc_kpw<T>() * (128 / DH); }

// Key count of sequence b: seq_lens[b] (or the uniform length when seq_lens is NULL), clamped to
// [0, max_len] so that a bad device-side length can never index past the cache.
__device__ __forceinline__ int decode_len(const int32_t* lens, int uniform_len, int b, int max_len) {
  const int L = lens ? lens[b] : uniform_len;
  return L < 0 ? 0 : (L > max_len ? max_len : L);
}

// Split-K partials: the column sums o of a (sequence, query head, chunk) as one row of DH floats
// (512 bytes at head dim 128), so the merge reads whole 128-byte lines of it, and the (max,
// denominator) pairs in an array of their own.  Both kernels run on a grid whose z extent is the
// batch.
__device__ __forceinline__ float* decode_part_o(float* part) { return part; }
__device__ __forceinline__ const float* decode_part_o(const float* part) { return part; }
template <int DH = 128>
__device__ __forceinline__ float2* decode_part_ml(float* part, int hq, int max_chunks) {
  return reinterpret_cast<float2*>(part + (int64_t)gridDim.z * hq * max_chunks * DH);
}
template <int DH = 128>
__device__ __forceinline__ const float2* decode_part_ml(const float* part, int hq, int max_chunks) {
  return reinterpret_cast<const float2*>(part + (int64_t)gridDim.z * hq * max_chunks * DH);
}

template <typename T, int G, int DH = 128>
__global__ __launch_bounds__(256) void decode_partial_kernel(const T* __restrict__ Q, const T* __restrict__ K,
                                                             const T* __restrict__ V, const int32_t* __restrict__ lens,
                                                             int uniform_len, int max_len, int hq, int nsub,
                                                             AttnStrides st, float scale, int max_chunks,
                                                             float* __restrict__ part) {
  // Layout of `part` (decode_part_o / decode_part_ml): o[b][hq][max_chunks][DH] floats, then
  // (m, l)[b][hq][max_chunks] float pairs; valid chunks only.  decode_merge_cols_kernel combines them.
  // Head dim 64 halves the lanes of a key row and doubles the keys of a chunk.
  constexpr int D = DH;
  constexpr int EPL = 16 / (int)sizeof(T);            // elements per 16-byte load
  constexpr int LPK = D / EPL;                        // lanes per key row (16 bf16, 32 f32 at D = 128)
  constexpr int KPI = 64 / LPK;                       // keys per load instruction (4 bf16, 2 f32 at 128)
  constexpr int KPW = dc_kpw<T>() * (128 / DH);
  constexpr int CHUNK = dc_chunk<T, DH>();
  constexpr int NI = KPW / KPI;                       // load instructions per wave (16)
  static_assert(DH == 128 || DH == 64, "head dim 64 or 128");
  __shared__ float red_m[DC_WAVES][G];
  __shared__ float red_l[DC_WAVES][G];
  __shared__ float red_o[DC_WAVES][G][D];

  const int chunk = blockIdx.x;
  const int vg = blockIdx.y;      // group of G query heads: vg G .. vg G + G - 1
  const int hk = vg / nsub;       // their kv head (nsub groups per kv head)
  const int b = blockIdx.z;
  const int L = decode_len(lens, uniform_len, b, max_len);
  if (chunk * CHUNK >= L) return;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int sub = lane % LPK;          // 16-byte column inside the row
  const int kk = lane / LPK;           // key slot inside a load instruction
  const int key0 = chunk * CHUNK + w * KPW;

  // q for the G heads, this lane's EPL columns, pre-multiplied by the scale.
  float qv[G][EPL];
#pragma unroll
  for (int gi = 0; gi < G; ++gi) {
    const T* qr = Q + b * st.qb + (int64_t)(vg * G + gi) * st.qh + sub * EPL;
#pragma unroll
    for (int e = 0; e < EPL; ++e) qv[gi][e] = Elem<T>::load(qr, e) * scale;
  }

  // Byte ranges end at the sequence length: keys >= L read as zero.
  const auto rk = make_rsrc(K + b * st.kb + hk * st.kh, (uint32_t)(((int64_t)(L - 1) * st.ks + D) * sizeof(T)));
  const auto rv = make_rsrc(V + b * st.vb + hk * st.vh, (uint32_t)(((int64_t)(L - 1) * st.vs + D) * sizeof(T)));
  uint4 kr[NI], vr[NI];
#pragma unroll
  for (int it = 0; it < NI; ++it) {
    const int key = key0 + it * KPI + kk;
    kr[it] = buf_load16_nt(rk, (uint32_t)(((int64_t)key * st.ks + sub * EPL) * sizeof(T)));
  }
#pragma unroll
  for (int it = 0; it < NI; ++it) {
    const int key = key0 + it * KPI + kk;
    vr[it] = buf_load16_nt(rv, (uint32_t)(((int64_t)key * st.vs + sub * EPL) * sizeof(T)));
  }

  auto unpack = [](const uint4& u, float (&f)[EPL]) {
    if constexpr (sizeof(T) == 2) {
      f[0] = lo_bf16(u.x); f[1] = hi_bf16(u.x); f[2] = lo_bf16(u.y); f[3] = hi_bf16(u.y);
      f[4] = lo_bf16(u.z); f[5] = hi_bf16(u.z); f[6] = lo_bf16(u.w); f[7] = hi_bf16(u.w);
    } else {
      f[0] = __uint_as_float(u.x); f[1] = __uint_as_float(u.y);
      f[2] = __uint_as_float(u.z); f[3] = __uint_as_float(u.w);
    }
  };

  // Scores: partial dot over this lane's columns, reduced over the LPK lanes of the key row.
  float sc[G][NI];
#pragma unroll
  for (int it = 0; it < NI; ++it) {
    float kf[EPL];
    unpack(kr[it], kf);
#pragma unroll
    for (int gi = 0; gi < G; ++gi) {
      float d = 0.f;
#pragma unroll
      for (int e = 0; e < EPL; ++e) d += qv[gi][e] * kf[e];
#pragma unroll
      for (int o = LPK / 2; o > 0; o >>= 1) d += __shfl_xor(d, o, 64);
      const int key = key0 + it * KPI + kk;
      sc[gi][it] = key < L ? d : -INFINITY;
    }
  }
  float mw[G], lw[G], ow[G][EPL];
#pragma unroll
  for (int gi = 0; gi < G; ++gi) {
    float mx = -INFINITY;
#pragma unroll
    for (int it = 0; it < NI; ++it) mx = fmaxf(mx, sc[gi][it]);
    // lanes with different kk hold different keys; lanes with the same kk hold the same scores
    for (int o = LPK; o < 64; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    mw[gi] = mx;
    const float mu = mx == -INFINITY ? 0.f : mx;
    float ls = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) ow[gi][e] = 0.f;
#pragma unroll
    for (int it = 0; it < NI; ++it) {
      const float p = __expf(sc[gi][it] - mu);
      ls += p;
      float vf[EPL];
      unpack(vr[it], vf);
#pragma unroll
      for (int e = 0; e < EPL; ++e) ow[gi][e] += p * vf[e];
    }
    for (int o = LPK; o < 64; o <<= 1) {
      ls += __shfl_xor(ls, o, 64);
#pragma unroll
      for (int e = 0; e < EPL; ++e) ow[gi][e] += __shfl_xor(ow[gi][e], o, 64);
    }
    lw[gi] = ls;  // each key's p enters once: lanes of one key row (same kk) are not summed together
  }
  if (kk == 0) {
#pragma unroll
    for (int gi = 0; gi < G; ++gi) {
      if (sub == 0) {
        red_m[w][gi] = mw[gi];
        red_l[w][gi] = lw[gi];
      }
#pragma unroll
      for (int e = 0; e < EPL; ++e) red_o[w][gi][sub * EPL + e] = ow[gi][e];
    }
  }
  __syncthreads();
  // Combine the 4 waves: thread t < G*128 handles (head t/128, column t%128).
  for (int t = threadIdx.x; t < G * D; t += blockDim.x) {
    const int gi = t / D, d = t % D;
    float M = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < DC_WAVES; ++ww) M = fmaxf(M, red_m[ww][gi]);
    const float mu = M == -INFINITY ? 0.f : M;
    float Ls = 0.f, Os = 0.f;
#pragma unroll
    for (int ww = 0; ww < DC_WAVES; ++ww) {
      const float f = __expf(red_m[ww][gi] - mu);
      Ls += red_l[ww][gi] * f;
      Os += red_o[ww][gi][d] * f;
    }
    const int64_t row = ((int64_t)b * hq + vg * G + gi) * max_chunks + chunk;
    if (d == 0) decode_part_ml<DH>(part, hq, max_chunks)[row] = make_float2(M, Ls);
    decode_part_o(part)[row * D + d] = Os;
  }
}

// ---- bf16 decode partials with in-row DPP reductions ------------------------------------------

// The fused decode block merges the split-K partials inside the o_proj GEMV's prologue (every
// workgroup reads all of them) up to this many 256-key chunks; longer caches use the merge kernel.
constexpr int kMergeInPrologueMaxChunks = 8;

// The decode step's q/k/v as the fused attention block takes them: raw projection rows (before
// qk-norm and RoPE) of one sequence whose new token sits at cache position *position.
struct DecodeFuse {
  const uint16_t* wq = nullptr;       // q_norm weight [128], bf16
  const uint16_t* wk = nullptr;       // k_norm weight [128], bf16
  const float* inv_freq = nullptr;    // RoPE inverse frequencies [64]
  const int32_t* position = nullptr;  // the new token's position p; the sequence has p + 1 keys
  const void* k_new = nullptr;        // raw k rows of the new token [hkv][128] (the caches' type)
  const void* v_new = nullptr;        // raw v rows [hkv][128]
  float eps = 0.f;
};

// RMSNorm (weight w, eps) then RoPE of one 128-wide head row held by the 16 lanes of a DPP row,
// lane `sub` holding columns 8 sub .. 8 sub + 7 (a[]); cs/sn are the lane's cos/sin.  The same
// arithmetic, term for term, as qk_norm_rope_kernel: x * (1 / sqrt(mean x^2 + eps)) * w, then
// (first half) x cos - partner sin, (second half) x cos + partner sin, the partner 64 columns away
// (lane sub ^ 8, row_ror:8).
__device__ __forceinline__ void norm_rope_row(float (&a)[8], const float (&wv)[8], const float (&cs)[8],
                                              const float (&sn)[8], int sub, float eps) {
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) ss += a[j] * a[j];
  ss = row16_sum(ss);
  const float inv = 1.0f / sqrtf(ss / 128.0f + eps);
  float n[8], pn[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) n[j] = (a[j] * inv) * wv[j];
#pragma unroll
  for (int j = 0; j < 8; ++j) pn[j] = dpp_f<0x128>(n[j]);
  const bool first = sub < 8;
#pragma unroll
  for (int j = 0; j < 8; ++j) a[j] = first ? n[j] * cs[j] + (-pn[j]) * sn[j] : n[j] * cs[j] + pn[j] * sn[j];
}

__device__ __forceinline__ void unpack8(const uint4& u, float (&f)[8]) {
  f[0] = lo_bf16(u.x); f[1] = hi_bf16(u.x); f[2] = lo_bf16(u.y); f[3] = hi_bf16(u.y);
  f[4] = lo_bf16(u.z); f[5] = hi_bf16(u.z); f[6] = lo_bf16(u.w); f[7] = hi_bf16(u.w);
}
__device__ __forceinline__ uint4 pack8(const float (&f)[8]) {
  return make_uint4(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]),
                    pack_bf16x2(f[6], f[7]));
}

// Eight consecutive elements of a row as raw 16-byte words: one for bf16, two for fp32.
template <typename T>
struct Row8 {
  static constexpr int NV = (int)sizeof(T) / 2;
  uint4 u[NV];
  __device__ __forceinline__ void to_f32(float (&f)[8]) const {
    if constexpr (NV == 1) {
      unpack8(u[0], f);
    } else {
      f[0] = __uint_as_float(u[0].x); f[1] = __uint_as_float(u[0].y);
      f[2] = __uint_as_float(u[0].z); f[3] = __uint_as_float(u[0].w);
      f[4] = __uint_as_float(u[1].x); f[5] = __uint_as_float(u[1].y);
      f[6] = __uint_as_float(u[1].z); f[7] = __uint_as_float(u[1].w);
    }
  }
  // the row as T stores it: rounded to bf16, or the fp32 values
  __device__ __forceinline__ void from_f32(const float (&f)[8]) {
    if constexpr (NV == 1) {
      u[0] = pack8(f);
    } else {
      u[0] = make_uint4(__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]), __float_as_uint(f[3]));
      u[1] = make_uint4(__float_as_uint(f[4]), __float_as_uint(f[5]), __float_as_uint(f[6]), __float_as_uint(f[7]));
    }
  }
  __device__ __forceinline__ void load(const T* p) {
#pragma unroll
    for (int i = 0; i < NV; ++i) u[i] = reinterpret_cast<const uint4*>(p)[i];
  }
  __device__ __forceinline__ void store(T* p) const {
#pragma unroll
    for (int i = 0; i < NV; ++i) reinterpret_cast<uint4*>(p)[i] = u[i];
  }
  // raw buffer loads (non-temporal) at byte offset off of range r
  __device__ __forceinline__ void load_nt(__amdgpu_buffer_rsrc_t r, uint32_t off) {
#pragma unroll
    for (int i = 0; i < NV; ++i) u[i] = buf_load16_nt(r, off + 16u * i);
  }
};

// Same unit of work and output as decode_partial_kernel: the 16 lanes of a DPP row hold one key
// row (8 columns each: one 16-byte load for bf16, two for fp32), so a score is an in-lane dot
// product plus a 4-step DPP row sum, and the 4 rows of a wave (key slots kk) keep separate softmax
// states (m, l, o) -- no cross-row shuffles.  The 16 states of the workgroup (4 waves x 4 rows)
// are combined once through LDS.  A wave covers 16 key rows per slot with bf16 (64 keys, chunks
// of 256) and 8 with fp32 (32 keys, chunks of 128), so both keep 16 KiB of K and V in flight.
// Head dim DH = 64: 8 lanes (half a DPP row) hold a key row and sum by a 3-step DPP reduction, so
// a load instruction covers 8 keys, a wave 128 (bf16) or 64 (fp32) and the workgroup keeps 32
// softmax states; the bytes in flight per lane are the same as at 128.
// FUSE (decode attention block, one sequence): Q holds the raw q heads; each workgroup applies
// qk-norm + RoPE to its G heads (rounded to bf16 as the unfused path stores them, or kept in fp32
// with fp32 caches).  The wave whose keys include the new token p normalises and rotates that
// token's k row, writes it and the v row into the caches at row p, and scores it from registers
// (the stale cache row it loaded is masked): the new key joins the softmax state of the DPP row
// that owns it, with no data dependence on the cache write.  Only this workgroup reads row p in
// this launch (when a kv head's query heads span several groups, each group's workgroup scores
// row p from its own registers and only the first group's writes it).
// Both decode kernels take G query heads per workgroup; blockIdx.y is the group, and a kv head
// whose ratio hq / hkv is above 8 (or not a multiple of the G chosen) is served by nsub groups.
template <typename T, int G, bool FUSE = false, int DH = 128>
__global__ __launch_bounds__(256) void decode_partial_rows_kernel(const T* __restrict__ Q, const T* __restrict__ K,
                                                                  const T* __restrict__ V,
                                                                  const int32_t* __restrict__ lens, int uniform_len,
                                                                  int max_len, int hq, int nsub, AttnStrides st,
                                                                  float scale, int max_chunks,
                                                                  float* __restrict__ part, DecodeFuse fz) {
  constexpr bool F32 = sizeof(T) == 4;
  static_assert(DH == 128 || (DH == 64 && !FUSE), "head dim 128, or 64 without the fused block");
  constexpr int D = DH, LPR = D / 8, NI = F32 ? 8 : 16, KPI = 64 / LPR, KPW = NI * KPI, CHUNK = DC_WAVES * KPW,
                NS = DC_WAVES * KPI;
  static_assert(CHUNK == dc_chunk<T, DH>(), "chunk size shared with the merge");
  __shared__ float red_m[NS][G];
  __shared__ float red_l[NS][G];
  __shared__ float red_o[NS][G][D];

  const int chunk = blockIdx.x;
  const int vg = blockIdx.y;      // group of G query heads: vg G .. vg G + G - 1
  const int hk = vg / nsub;       // their kv head (nsub groups per kv head)
  const int b = blockIdx.z;
  int praw = 0;
  int L;
  if constexpr (FUSE) {
    praw = *fz.position;
    L = praw + 1 < 0 ? 0 : (praw + 1 > max_len ? max_len : praw + 1);
  } else {
    L = decode_len(lens, uniform_len, b, max_len);
  }
  if (chunk * CHUNK >= L) return;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int sub = lane & (LPR - 1);  // 8-column group of the key row
  const int kk = lane / LPR;         // key slot (group of LPR lanes) inside a load instruction
  const int key0 = chunk * CHUNK + w * KPW;

  float qv[G][8];
  Row8<T> qraw[G], knr, vnr, kn;
  uint4 wqr, wkr;
  float f0 = 0.f;
  bool newkey = false;  // FUSE: this lane's DPP row scores the new key from registers
#pragma unroll
  for (int gi = 0; gi < G; ++gi) qraw[gi].load(Q + b * st.qb + (int64_t)(vg * G + gi) * st.qh + sub * 8);
  if constexpr (FUSE) {
    // everything the norm and rotation need is requested before the cache rows (loads return in order)
    wqr = *reinterpret_cast<const uint4*>(fz.wq + sub * 8);
    wkr = *reinterpret_cast<const uint4*>(fz.wk + sub * 8);
    knr.load((const T*)fz.k_new + hk * D + sub * 8);
    vnr.load((const T*)fz.v_new + hk * D + sub * 8);
    f0 = fz.inv_freq[lane];
  }
  // Byte ranges end at the sequence length: keys >= L read as zero.
  const auto rk = make_rsrc(K + b * st.kb + hk * st.kh, (uint32_t)(((int64_t)(L - 1) * st.ks + D) * sizeof(T)));
  const auto rv = make_rsrc(V + b * st.vb + hk * st.vh, (uint32_t)(((int64_t)(L - 1) * st.vs + D) * sizeof(T)));
  Row8<T> kr[NI], vr[NI];
#pragma unroll
  for (int it = 0; it < NI; ++it) {
    const int key = key0 + it * KPI + kk;
    kr[it].load_nt(rk, (uint32_t)(((int64_t)key * st.ks + sub * 8) * sizeof(T)));
  }
#pragma unroll
  for (int it = 0; it < NI; ++it) {
    const int key = key0 + it * KPI + kk;
    vr[it].load_nt(rv, (uint32_t)(((int64_t)key * st.vs + sub * 8) * sizeof(T)));
  }
  if constexpr (FUSE) {
    // cos/sin of float(p) * inv_freq[i] for this lane's columns (i = (8 sub + j) mod 64): lane l
    // evaluates frequency l once and the lanes gather theirs.
    float c0, s0;
    sincosf((float)praw * f0, &s0, &c0);
    float cs[8], sn[8], wv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int i = (8 * sub + j) & 63;
      cs[j] = __shfl(c0, i, 64);
      sn[j] = __shfl(s0, i, 64);
    }
    unpack8(wqr, wv);
#pragma unroll
    for (int gi = 0; gi < G; ++gi) {
      float a[8];
      qraw[gi].to_f32(a);
      norm_rope_row(a, wv, cs, sn, sub, fz.eps);
#pragma unroll
      for (int j = 0; j < 8; ++j) qv[gi][j] = (F32 ? a[j] : round_bf16(a[j])) * scale;
    }
    // The new key's row, normalised and rotated (every wave computes it: one row), and the DPP row
    // of this wave that owns key p (if any) writes it and the v row into the caches.
    const int rel = praw - key0;  // the new key relative to this wave's first key
    newkey = praw < max_len && rel >= 0 && rel < KPW && kk == (rel & (KPI - 1));
    float a[8];
    knr.to_f32(a);
    unpack8(wkr, wv);
    norm_rope_row(a, wv, cs, sn, sub, fz.eps);
    kn.from_f32(a);
    if (newkey && vg % nsub == 0) {  // the first group of the kv head writes the cache rows
      T* kc = const_cast<T*>(K) + b * st.kb + hk * st.kh + (int64_t)praw * st.ks + sub * 8;
      T* vc = const_cast<T*>(V) + b * st.vb + hk * st.vh + (int64_t)praw * st.vs + sub * 8;
      kn.store(kc);
      vnr.store(vc);
    }
  } else {
#pragma unroll
    for (int gi = 0; gi < G; ++gi) {
      float a[8];
      qraw[gi].to_f32(a);
#pragma unroll
      for (int j = 0; j < 8; ++j) qv[gi][j] = a[j] * scale;
    }
  }

  // FUSE: cache row p is read stale (this launch writes it) and masked; the new key is scored from
  // its registers below, as one more key of the DPP row that owns it.
  const int Lc = FUSE && praw < max_len ? praw : L;
  float sc[G][NI];
#pragma unroll
  for (int it = 0; it < NI; ++it) {
    float kf[8];
    kr[it].to_f32(kf);
    const bool valid = key0 + it * KPI + kk < Lc;
#pragma unroll
    for (int gi = 0; gi < G; ++gi) {
      float d = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) d += qv[gi][j] * kf[j];
      d = group_sum<LPR>(d);
      sc[gi][it] = valid ? d : -INFINITY;
    }
  }
  float sn_new[G];
#pragma unroll
  for (int gi = 0; gi < G; ++gi) sn_new[gi] = -INFINITY;
  if constexpr (FUSE) {
    float kf[8];
    kn.to_f32(kf);
#pragma unroll
    for (int gi = 0; gi < G; ++gi) {
      float d = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) d += qv[gi][j] * kf[j];
      d = group_sum<LPR>(d);
      sn_new[gi] = newkey ? d : -INFINITY;
    }
  }
  const int s_id = w * KPI + kk;
#pragma unroll
  for (int gi = 0; gi < G; ++gi) {
    float mx = sc[gi][0];
#pragma unroll
    for (int it = 1; it < NI; ++it) mx = fmaxf(mx, sc[gi][it]);
    if constexpr (FUSE) mx = fmaxf(mx, sn_new[gi]);
    const float mu = mx == -INFINITY ? 0.f : mx;
    float ls = 0.f, o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if constexpr (FUSE) {
      const float p = __expf(sn_new[gi] - mu);
      ls += p;
      float vf[8];
      vnr.to_f32(vf);
#pragma unroll
      for (int j = 0; j < 8; ++j) o[j] += p * vf[j];
    }
#pragma unroll
    for (int it = 0; it < NI; ++it) {
      const float p = __expf(sc[gi][it] - mu);
      ls += p;
      float vf[8];
      vr[it].to_f32(vf);
#pragma unroll
      for (int j = 0; j < 8; ++j) o[j] += p * vf[j];
    }
    if (sub == 0) {
      red_m[s_id][gi] = mx;
      red_l[s_id][gi] = ls;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) red_o[s_id][gi][sub * 8 + e] = o[e];
  }
  __syncthreads();
  for (int t = threadIdx.x; t < G * D; t += blockDim.x) {
    const int gi = t / D, d = t % D;
    float M = -INFINITY;
#pragma unroll
    for (int s2 = 0; s2 < NS; ++s2) M = fmaxf(M, red_m[s2][gi]);
    const float mu = M == -INFINITY ? 0.f : M;
    float Ls = 0.f, Os = 0.f;
#pragma unroll
    for (int s2 = 0; s2 < NS; ++s2) {
      const float f = __expf(red_m[s2][gi] - mu);
      Ls += red_l[s2][gi] * f;
      Os += red_o[s2][gi][d] * f;
    }
    const int64_t row = ((int64_t)b * hq + vg * G + gi) * max_chunks + chunk;
    if (d == 0) decode_part_ml<DH>(part, hq, max_chunks)[row] = make_float2(M, Ls);
    decode_part_o(part)[row * D + d] = Os;
  }
}

// Merge by column groups: workgroup (cg, h, b) produces columns 32 cg .. 32 cg + 31 of query head
// h.  8 groups of 32 threads (one per column) each run one online log-sum-exp pass over every 8th
// chunk (running max, denominator and column sum, rescaled when the max grows), and the 8 group
// states are combined through LDS.  The grid's x extent is DH / 32.
template <typename T, int DH = 128>
__device__ __forceinline__ void decode_merge_cols_body(const float* __restrict__ part, int L, int hq, int max_chunks,
                                                       const AttnStrides& st, T* __restrict__ O) {
  constexpr int D = DH, COLS = 32, NG = 8;
  __shared__ float gm[NG], gl[NG];
  __shared__ float gacc[NG][COLS];
  const int cg = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x;
  const int col = tid & (COLS - 1), grp = tid >> 5;
  const int d = cg * COLS + col;
  const int nch = (L + dc_chunk<T, DH>() - 1) / dc_chunk<T, DH>();
  const int64_t row0 = ((int64_t)b * hq + h) * max_chunks;
  const float* po = decode_part_o(part) + row0 * D + d;
  const float2* pml = decode_part_ml<DH>(part, hq, max_chunks) + row0;

  float m = -INFINITY, l = 0.f, acc = 0.f;
  // Fold chunk (mc, lc, oc) into the running state.
  auto fold = [&](float mc, float lc, float oc) {
    const float mn = fmaxf(m, mc);
    const float mu = mn == -INFINITY ? 0.f : mn;
    const float a = __expf(m - mu), p = __expf(mc - mu);
    l = l * a + lc * p;
    acc = acc * a + oc * p;
    m = mn;
  };
  // Up to 16 chunks per thread and pass, all loads issued first; indices past the last chunk are
  // clamped to it and folded as empty (max -inf, weight 0).
  constexpr int U = 16;
  for (int c = grp; c < nch; c += U * NG) {
    float mc[U], lc[U], oc[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int cc = min(c + u * NG, nch - 1);
      const float2 mlc = pml[cc];
      mc[u] = mlc.x;
      lc[u] = mlc.y;
      oc[u] = po[(int64_t)cc * D];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) fold(c + u * NG < nch ? mc[u] : -INFINITY, lc[u], oc[u]);
  }
  if (col == 0) {
    gm[grp] = m;
    gl[grp] = l;
  }
  gacc[grp][col] = acc;
  __syncthreads();
  if (grp == 0) {
    float M = -INFINITY;
#pragma unroll
    for (int g2 = 0; g2 < NG; ++g2) M = fmaxf(M, gm[g2]);
    const float mu = M == -INFINITY ? 0.f : M;
    float Ls = 0.f, tot = 0.f;
#pragma unroll
    for (int g2 = 0; g2 < NG; ++g2) {
      const float f = __expf(gm[g2] - mu);
      Ls += gl[g2] * f;
      tot += gacc[g2][col] * f;
    }
    Elem<T>::store(O + b * st.ob + h * st.oh, d, Ls > 0.f ? tot / Ls : 0.f);
  }
}

template <typename T, int DH = 128>
__global__ __launch_bounds__(256) void decode_merge_cols_kernel(const float* __restrict__ part,
                                                                const int32_t* __restrict__ lens, int uniform_len,
                                                                int max_len, int hq, int max_chunks, AttnStrides st,
                                                                T* __restrict__ O) {
  decode_merge_cols_body<T, DH>(part, decode_len(lens, uniform_len, blockIdx.z, max_len), hq, max_chunks, st, O);
}

// The merge of the fused decode block (one sequence, length *position + 1): the same kernel body
// with the length taken from the position.
template <typename T>
__global__ __launch_bounds__(256) void decode_merge_cols_pos_kernel(const float* __restrict__ part,
                                                                   const int32_t* __restrict__ position, int max_len,
                                                                   int hq, int max_chunks, AttnStrides st,
                                                                   T* __restrict__ O) {
  const int p = *position;
  const int L = p + 1 < 0 ? 0 : (p + 1 > max_len ? max_len : p + 1);
  decode_merge_cols_body<T>(part, L, hq, max_chunks, st, O);
}

// ---- scratch of the allocation-free decode entry point (kh_decode_attention_noalloc) ----------
// The split-K partials of one call live in this file-scope device array instead of the caching
// allocator.  Every GPU the library runs on holds its own copy until the process ends; host code
// uses only the device address hipGetSymbolAddress returns for it (the array's name is a
// host-side stand-in, not a device address).  Calls on one GPU share the array, so calls that
// overlap on one GPU (another thread's stream) race; on the library's single stream they are
// ordered.  Nothing in it needs to start at zero: the merge reads only the chunks this call's
// partial kernel wrote.
constexpr size_t kNoAllocScratchBytes = size_t(16) << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];
constexpr int kMaxDevices = 64;
void* g_scratch_ptr[kMaxDevices] = {};

AttnStrides load_strides(const int64_t* s) {
  AttnStrides a;
  a.qb = s[0]; a.qh = s[1]; a.qs = s[2];
  a.kb = s[3]; a.kh = s[4]; a.ks = s[5];
  a.vb = s[6]; a.vh = s[7]; a.vs = s[8];
  a.ob = s[9]; a.oh = s[10]; a.os = s[11];
  return a;
}

// Bytes of split-K partials launch_decode needs: o rows + (m, l) per (sequence, head, chunk).
template <typename T, int DH = 128>
size_t decode_part_bytes(int batch, int hq, int64_t max_len) {
  const int64_t max_chunks = (max_len + dc_chunk<T, DH>() - 1) / dc_chunk<T, DH>();
  return (size_t)batch * hq * max_chunks * (DH + 2) * sizeof(float);
}

size_t decode_part_bytes_for(int dtype, int d, int batch, int hq, int64_t max_len) {
  if (dtype == KH_BF16)
    return d == 64 ? decode_part_bytes<uint16_t, 64>(batch, hq, max_len) : decode_part_bytes<uint16_t>(batch, hq, max_len);
  return d == 64 ? decode_part_bytes<float, 64>(batch, hq, max_len) : decode_part_bytes<float>(batch, hq, max_len);
}

// Query heads per decode workgroup for GQA ratio G: G itself up to 8, else its largest divisor
// up to 8 (G / that many workgroups then share each kv head's chunk, each reading its K/V rows).
inline int decode_group_heads(int G) {
  if (G <= 8) return G;
  int gc = 8;
  while (G % gc != 0) --gc;
  return gc;
}

// part_in: the partials buffer (at least decode_part_bytes), or nullptr to take one from the
// caching allocator for the duration of the call.
template <typename T, int DH = 128>
int launch_decode(const void* q, const void* k, const void* v, void* o, const int32_t* lens, int uniform_len,
                  int batch, int hq, int hkv, int64_t max_len, const AttnStrides& st, float scale,
                  float* part_in = nullptr) {
  const int GC = decode_group_heads(hq / hkv), nsub = hq / hkv / GC;
  KH_REQUIRE((int64_t)hkv * nsub <= 65535, "kh_decode_attention: %d query heads need too many workgroup groups", hq);
  const int64_t lim = int64_t(1) << 31;
  constexpr int CH = dc_chunk<T, DH>();
  KH_REQUIRE((max_len + CH) * st.ks * (int64_t)sizeof(T) < lim && (max_len + CH) * st.vs * (int64_t)sizeof(T) < lim,
             "kh_decode_attention: one head of the cache spans more than 2 GiB");
  const int ml = (int)max_len;
  const int max_chunks = (ml + CH - 1) / CH;
  KH_REQUIRE(max_chunks <= 65535 * 64, "kh_decode_attention: max_len too large");
  float* part = part_in ? part_in : (float*)scratch_alloc(decode_part_bytes<T, DH>(batch, hq, max_len));
  if (!part) return KH_ERR_OOM;
  dim3 grid(max_chunks, hkv * nsub, batch);
  const T* Q = (const T*)q;
  const T* K = (const T*)k;
  const T* V = (const T*)v;
  // bf16 takes the DPP-row kernel, fp32 the shuffle one (each measured the faster for its type).
#define KH_DECODE_CASE(GG)                                                                                 \
  case GG:                                                                                                 \
    if constexpr (sizeof(T) == 2)                                                                          \
      decode_partial_rows_kernel<T, GG, false, DH><<<grid, 256, 0, stream()>>>(                            \
          Q, K, V, lens, uniform_len, ml, hq, nsub, st, scale, max_chunks, part, DecodeFuse{});            \
    else                                                                                                   \
      decode_partial_kernel<T, GG, DH><<<grid, 256, 0, stream()>>>(Q, K, V, lens, uniform_len, ml, hq, nsub, st, \
                                                                scale, max_chunks, part);                  \
    break;
  switch (GC) {
    KH_DECODE_CASE(1)
    KH_DECODE_CASE(2)
    KH_DECODE_CASE(3)
    KH_DECODE_CASE(4)
    KH_DECODE_CASE(5)
    KH_DECODE_CASE(6)
    KH_DECODE_CASE(7)
    KH_DECODE_CASE(8)
  }
#undef KH_DECODE_CASE
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) {
    decode_merge_cols_kernel<T, DH><<<dim3(DH / 32, hq, batch), 256, 0, stream()>>>(part, lens, uniform_len, ml,
                                                                                    hq, max_chunks, st, (T*)o);
    e = hipGetLastError();
  }
  if (!part_in) scratch_free(part);  // stream-ordered: the block is reused only by later work on the same stream
  if (e != hipSuccess) {
    set_error("kh_decode_attention: launch failed: %s", hipGetErrorString(e));
    return KH_ERR_HIP;
  }
  KH_DEBUG_SYNC();
  return KH_OK;
}

// launch_decode for the element type `dtype` and head dim d (64 or 128).
int launch_decode_for(int dtype, int d, const void* q, const void* k, const void* v, void* o, const int32_t* lens,
                      int uniform_len, int batch, int hq, int hkv, int64_t max_len, const AttnStrides& st,
                      float scale, float* part_in = nullptr) {
  if (dtype == KH_BF16)
    return d == 64 ? launch_decode<uint16_t, 64>(q, k, v, o, lens, uniform_len, batch, hq, hkv, max_len, st, scale,
                                                 part_in)
                   : launch_decode<uint16_t>(q, k, v, o, lens, uniform_len, batch, hq, hkv, max_len, st, scale,
                                             part_in);
  return d == 64 ? launch_decode<float, 64>(q, k, v, o, lens, uniform_len, batch, hq, hkv, max_len, st, scale, part_in)
                 : launch_decode<float>(q, k, v, o, lens, uniform_len, batch, hq, hkv, max_len, st, scale, part_in);
}

// q, the caches and their batch / head / row strides on 16-byte boundaries (the decode kernels
// read 16-byte words of q, K and V rows).
bool decode_aligned(const void* q, const void* k, const void* v, const AttnStrides& st, int dtype) {
  const int64_t vec = dtype == KH_BF16 ? 8 : 4;
  return aligned16(q) && aligned16(k) && aligned16(v) && st.qb % vec == 0 && st.qh % vec == 0 && st.kb % vec == 0 &&
         st.kh % vec == 0 && st.ks % vec == 0 && st.vb % vec == 0 && st.vh % vec == 0 && st.vs % vec == 0;
}

int launch_generic(const void* q, const void* k, const void* v, void* o, int batch, int hq, int hkv, int lq, int lk,
                   int d, const AttnStrides& st, float scale, int causal, const void* mask, int mask_dtype,
                   const MaskArgs& ma, int dtype) {
  KH_REQUIRE(d <= 256, "kh_flash_attention: head_dim %d > 256 is not supported", d);
  const int64_t rows = (int64_t)batch * hq * lq;
  const int64_t grid = (rows + 3) / 4;
  KH_REQUIRE(grid <= INT32_MAX, "kh_flash_attention: grid too large");
  if (dtype == KH_BF16)
    attn_generic_kernel<uint16_t><<<(int)grid, 256, 0, stream()>>>((const uint16_t*)q, (const uint16_t*)k,
                                                                   (const uint16_t*)v, (uint16_t*)o, batch, hq, hkv,
                                                                   lq, lk, d, st, scale, causal, mask, mask_dtype,
                                                                   ma);
  else
    attn_generic_kernel<float><<<(int)grid, 256, 0, stream()>>>((const float*)q, (const float*)k, (const float*)v,
                                                                (float*)o, batch, hq, hkv, lq, lk, d, st, scale,
                                                                causal, mask, mask_dtype, ma);
  KH_CHECK_LAUNCH();
  return KH_OK;
}

}  // namespace

namespace kh {

// Called by kh_init with `device` current: records this GPU's address of the scratch array.
int attention_init(int device) {
  KH_REQUIRE(device >= 0 && device < kMaxDevices, "kh_init: device %d beyond the %d the library tracks", device,
             kMaxDevices);
  void* ptr = nullptr;
  KH_CHECK_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
  KH_REQUIRE(ptr != nullptr, "kh_init: no device address for the decode scratch array");
  g_scratch_ptr[device] = ptr;
  return KH_OK;
}

}  // namespace kh

extern "C" {

// Calls the MFMA attention kernels have no tiles or layout for -- bf16 head dims below 128 other
// than 64, fp32 head dims other than 32, 64, 96 and 128 up to 128, or views a kernel cannot read in
// place (unaligned pointers or strides) -- run them on staged copies: Q, K and V are copied into
// contiguous rows of dp elements (bf16: 64 or 128; fp32: the next multiple of 32) whose columns past
// d are zero, so each q.k sum is the sum over the d columns plus exact zeros, and the output's
// columns past d (P times zero V columns) are dropped when the rows are copied into the caller's o.
// The scale stays the caller's.  Staging costs one read and one write of Q, K, V and O.
namespace {
struct StagedAttn {
  void* block = nullptr;
  void *q = nullptr, *k = nullptr, *v = nullptr, *o = nullptr;
  AttnStrides st{};
  int dp = 0;
};

void launch_rows_pad(bool f32, const void* src, void* dst, int nh, int64_t n, int d, int dp, int64_t sb, int64_t sh,
                     int64_t ss, int64_t rows) {
  const int64_t grid = (rows * (dp * (f32 ? 4 : 2) / 16) + 255) / 256;
  if (f32)
    rows_pad_kernel<float><<<(int)grid, 256, 0, stream()>>>(static_cast<const float*>(src), static_cast<float*>(dst),
                                                            nh, (int)n, d, dp, sb, sh, ss, rows);
  else
    rows_pad_kernel<uint16_t><<<(int)grid, 256, 0, stream()>>>(static_cast<const uint16_t*>(src),
                                                               static_cast<uint16_t*>(dst), nh, (int)n, d, dp, sb, sh,
                                                               ss, rows);
}

// Returns KH_OK with p.block set when staged, KH_OK with p.block null when the staged shapes are
// outside the kernel's limits too (the caller takes the generic kernel), or an error.
int stage_attn(StagedAttn& p, int dtype, const void* q, const void* k, const void* v, int batch, int hq, int hkv,
               int64_t lq, int64_t lk, int d, const AttnStrides& st) {
  p = StagedAttn{};
  if (d > 128) return KH_OK;
  const bool f32 = dtype == KH_F32;
  const int es = f32 ? 4 : 2;
  const int dp = f32 ? (d + 31) / 32 * 32 : (d <= 64 ? 64 : 128);
  const int64_t rq = (int64_t)batch * hq * lq, rk = (int64_t)batch * hkv * lk;
  AttnStrides ps{};
  ps.qb = ps.ob = hq * lq * dp;
  ps.qh = ps.oh = lq * dp;
  ps.qs = ps.os = dp;
  ps.kb = ps.vb = hkv * lk * dp;
  ps.kh = ps.vh = lk * dp;
  ps.ks = ps.vs = dp;
  const void* a16 = reinterpret_cast<const void*>(uintptr_t(256));  // the block's parts are 256-byte aligned
  if (f32 ? !flash_f32_supported(a16, a16, a16, a16, lq, lk, dp, ps)
          : !flash_prefill_supported(a16, a16, a16, a16, hq, hkv, lq, lk, dp, ps))
    return KH_OK;
  const int64_t per = dp * es / 16;  // threads per staged row
  if ((rq * per + 255) / 256 > INT32_MAX || (rk * per + 255) / 256 > INT32_MAX) return KH_OK;
  const size_t bq = (size_t)rq * dp * es, bk = (size_t)rk * dp * es;  // multiples of 64 bytes
  const size_t align = 256, oq = (bq + align - 1) / align * align, ok = (bk + align - 1) / align * align;
  p.block = scratch_alloc(2 * oq + 2 * ok);
  if (!p.block) return KH_ERR_OOM;
  char* base = static_cast<char*>(p.block);
  p.q = base;
  p.k = base + oq;
  p.v = base + oq + ok;
  p.o = base + oq + 2 * ok;
  p.st = ps;
  p.dp = dp;
  launch_rows_pad(f32, q, p.q, hq, lq, d, dp, st.qb, st.qh, st.qs, rq);
  launch_rows_pad(f32, k, p.k, hkv, lk, d, dp, st.kb, st.kh, st.ks, rk);
  launch_rows_pad(f32, v, p.v, hkv, lk, d, dp, st.vb, st.vh, st.vs, rk);
  return KH_OK;
}

// Copies the staged output into the caller's o (after a successful launch) and releases the block.
int unstage_attn(StagedAttn& p, int rc, int dtype, void* o, int batch, int hq, int64_t lq, int d,
                 const AttnStrides& st) {
  if (rc == KH_OK) {
    const int64_t rq = (int64_t)batch * hq * lq;
    const int V = dtype == KH_F32 ? 4 : 8;
    const int64_t grid = (rq * ((d + V - 1) / V) + 255) / 256;  // <= the staging grid, checked at staging
    if (dtype == KH_F32)
      rows_unpack_kernel<float><<<(int)grid, 256, 0, stream()>>>(static_cast<const float*>(p.o), static_cast<float*>(o),
                                                                 hq, (int)lq, d, p.dp, st.ob, st.oh, st.os, rq);
    else
      rows_unpack_kernel<uint16_t><<<(int)grid, 256, 0, stream()>>>(static_cast<const uint16_t*>(p.o),
                                                                    static_cast<uint16_t*>(o), hq, (int)lq, d, p.dp,
                                                                    st.ob, st.oh, st.os, rq);
  }
  scratch_free(p.block);  // stream-ordered: reused only by later work on the same stream
  p.block = nullptr;
  return rc;
}
}  // namespace

int kh_flash_attention(const void* q, const void* k, const void* v, void* o, int batch, int hq, int hkv, int64_t lq,
                       int64_t lk, int d, const int64_t* strides, float scale, int causal, int dtype) {
  KH_REQUIRE_INIT();
  KH_REQUIRE(batch >= 0 && hq > 0 && hkv > 0 && lq >= 0 && lk >= 0 && d > 0, "kh_flash_attention: bad extents");
  KH_REQUIRE(hq % hkv == 0, "kh_flash_attention: numHeadsQ (%d) must be divisible by numHeadsKV (%d)", hq, hkv);
  KH_REQUIRE(dtype == KH_BF16 || dtype == KH_F32, "kh_flash_attention: unsupported dtype %d", dtype);
  KH_REQUIRE(lq <= INT32_MAX && lk <= INT32_MAX, "kh_flash_attention: sequence too long");
  if (batch == 0 || lq == 0) return KH_OK;
  KH_REQUIRE(q && k && v && o && strides, "kh_flash_attention: null pointer");
  const AttnStrides st = load_strides(strides);
  KH_REQUIRE(lk > 0, "kh_flash_attention: the key sequence is empty (softmax over no keys is undefined)");

  // One query row, no mask: split-K decode over the keys (the caller's 1-token decode step).
  const bool decode_ok = lq == 1 && !causal && (d == 128 || d == 64) && batch <= 65535 &&
                         decode_aligned(q, k, v, st, dtype);
  if (decode_ok) {
    AttnStrides ds = st;
    ds.qs = 0;
    ds.os = 0;
    return launch_decode_for(dtype, d, q, k, v, o, nullptr, (int)lk, batch, hq, hkv, lk, ds, scale);
  }
  // The MFMA kernel's softmax takes the raw q.k maximum as its reference, which is only the largest
  // scaled score for scale > 0; other scales take the generic kernel.
  if (dtype == KH_BF16 && lq > 1 && scale > 0.f) {
    if (flash_prefill_supported(q, k, v, o, hq, hkv, lq, lk, d, st))
      return launch_flash_prefill_bf16(q, k, v, o, batch, hq, hkv, (int)lq, (int)lk, d, st, scale, causal != 0);
    StagedAttn p;
    const int rs = stage_attn(p, KH_BF16, q, k, v, batch, hq, hkv, lq, lk, d, st);
    if (rs != KH_OK) return rs;
    if (p.block) {
      const int rc = launch_flash_prefill_bf16(p.q, p.k, p.v, p.o, batch, hq, hkv, (int)lq, (int)lk, p.dp, p.st,
                                               scale, causal != 0);
      return unstage_attn(p, rc, KH_BF16, o, batch, hq, lq, d, st);
    }
  }
  if (dtype == KH_F32) {
    if (flash_f32_supported(q, k, v, o, lq, lk, d, st))
      return launch_flash_f32(q, k, v, o, batch, hq, hkv, (int)lq, (int)lk, d, st, scale, causal != 0);
    StagedAttn p;
    const int rs = stage_attn(p, KH_F32, q, k, v, batch, hq, hkv, lq, lk, d, st);
    if (rs != KH_OK) return rs;
    if (p.block) {
      const int rc = launch_flash_f32(p.q, p.k, p.v, p.o, batch, hq, hkv, (int)lq, (int)lk, p.dp, p.st, scale,
                                      causal != 0);
      return unstage_attn(p, rc, KH_F32, o, batch, hq, lq, d, st);
    }
  }
  return launch_generic(q, k, v, o, batch, hq, hkv, (int)lq, (int)lk, d, st, scale, causal, nullptr, 0, MaskArgs{},
                        dtype);
}

int kh_flash_attention_split(const void* q, const void* k, const void* v, void* o, int batch, int hq, int hkv,
                             int64_t lq, int64_t lk, int d, const int64_t* strides, float scale, int causal) {
  KH_REQUIRE_INIT();
  KH_REQUIRE(batch >= 0 && hq > 0 && hkv > 0 && lq >= 0 && lk >= 0 && d > 0, "kh_flash_attention_split: bad extents");
  KH_REQUIRE(hq % hkv == 0, "kh_flash_attention_split: numHeadsQ (%d) must be divisible by numHeadsKV (%d)", hq,
             hkv);
  KH_REQUIRE(lq <= INT32_MAX && lk <= INT32_MAX, "kh_flash_attention_split: sequence too long");
  if (batch == 0 || lq == 0) return KH_OK;
  KH_REQUIRE(q && k && v && o && strides, "kh_flash_attention_split: null pointer");
  KH_REQUIRE(lk > 0, "kh_flash_attention_split: the key sequence is empty (softmax over no keys is undefined)");
  const AttnStrides st = load_strides(strides);
  if (lq > 1 && flash_split_supported(q, k, v, o, hq, hkv, lq, lk, d, st, scale))
    return launch_flash_split_f32(q, k, v, o, batch, hq, hkv, (int)lq, (int)lk, st, scale, causal != 0);
  // outside the split kernel's shapes: the fp32 route of kh_flash_attention
  return kh_flash_attention(q, k, v, o, batch, hq, hkv, lq, lk, d, strides, scale, causal, KH_F32);
}

int kh_flash_attention_masked(const void* q, const void* k, const void* v, void* o, int batch, int hq, int hkv,
                              int64_t lq, int64_t lk, int d, const int64_t* strides, float scale, const void* mask,
                              const int64_t* mask_strides, int mask_dtype, int dtype) {
  KH_REQUIRE_INIT();
  KH_REQUIRE(batch >= 0 && hq > 0 && hkv > 0 && lq >= 0 && lk >= 0 && d > 0,
             "kh_flash_attention_masked: bad extents");
  KH_REQUIRE(hq % hkv == 0, "kh_flash_attention_masked: numHeadsQ (%d) must be divisible by numHeadsKV (%d)", hq,
             hkv);
  KH_REQUIRE(dtype == KH_BF16 || dtype == KH_F32, "kh_flash_attention_masked: unsupported dtype %d", dtype);
  KH_REQUIRE(mask_dtype == KH_BF16 || mask_dtype == KH_F32, "kh_flash_attention_masked: unsupported mask dtype %d",
             mask_dtype);
  KH_REQUIRE(lq <= INT32_MAX && lk <= INT32_MAX, "kh_flash_attention_masked: sequence too long");
  if (batch == 0 || lq == 0) return KH_OK;
  KH_REQUIRE(q && k && v && o && strides && mask && mask_strides, "kh_flash_attention_masked: null pointer");
  KH_REQUIRE(lk > 0, "kh_flash_attention_masked: the key sequence is empty (softmax over no keys is undefined)");
  const AttnStrides st = load_strides(strides);
  MaskArgs ma{};
  ma.sb = mask_strides[0];
  ma.sh = mask_strides[1];
  ma.sq = mask_strides[2];
  ma.sk = mask_strides[3];
  ma.inv_scale = 1.0f / scale;
  // The reference softmax's max floor f32(-1e38) in raw q.k units (scores carry 1 / scale).
  const double fl = (double)-1e38f / (double)scale;
  ma.floor_raw = (scale > 0.f && fl >= -(double)FLT_MAX) ? (float)fl : -INFINITY;

  if (!(dtype == KH_BF16 && scale > 0.f))
    return launch_generic(q, k, v, o, batch, hq, hkv, (int)lq, (int)lk, d, st, scale, 0, mask, mask_dtype, ma, dtype);
  // Q, K and V the kernel cannot read in place are staged (stage_attn) once the mask is ready.
  const bool direct_qkv = flash_prefill_supported(q, k, v, o, hq, hkv, lq, lk, d, st);
  if (!direct_qkv && d > 128)
    return launch_generic(q, k, v, o, batch, hq, hkv, (int)lq, (int)lk, d, st, scale, 0, mask, mask_dtype, ma, dtype);

  // MFMA path: the mask must have a unit key stride and 16-byte aligned 8-key runs; otherwise it is
  // packed into rows of ldm = lk rounded up to 8 elements (broadcast axes stay broadcast).
  const int es = mask_dtype == KH_F32 ? 4 : 2;
  const bool direct = ma.sk == 1 && ((uintptr_t)mask % 16) == 0 && ma.sb % 8 == 0 && ma.sh % 8 == 0 &&
                      ma.sq % 8 == 0 && ma.sb >= 0 && ma.sh >= 0 && ma.sq >= 0;
  const void* mp = mask;
  void* packed = nullptr;
  int64_t extent;
  if (direct) {
    extent = ((int64_t)(batch - 1) * ma.sb + (int64_t)(hq - 1) * ma.sh + (lq - 1) * ma.sq + lk) * es;
  } else {
    const int nb = ma.sb ? batch : 1, nh = ma.sh ? hq : 1, nq = ma.sq ? (int)lq : 1;
    const int ldm = (int)((lk + 7) / 8 * 8);
    const int64_t rows = (int64_t)nb * nh * nq;
    extent = rows * ldm * es;
    KH_REQUIRE(extent < (int64_t(1) << 31), "kh_flash_attention_masked: mask larger than 2 GiB");
    packed = scratch_alloc((size_t)extent);
    if (!packed) return KH_ERR_OOM;
    const int64_t grid = (rows + 3) / 4;
    KH_REQUIRE(grid <= INT32_MAX, "kh_flash_attention_masked: mask grid too large");
    if (mask_dtype == KH_F32)
      mask_pack_kernel<float><<<(int)grid, 256, 0, stream()>>>((const float*)mask, (float*)packed, nh, nq, (int)lk,
                                                                ldm, ma.sb, ma.sh, ma.sq, ma.sk, rows);
    else
      mask_pack_kernel<uint16_t><<<(int)grid, 256, 0, stream()>>>((const uint16_t*)mask, (uint16_t*)packed, nh, nq,
                                                                   (int)lk, ldm, ma.sb, ma.sh, ma.sq, ma.sk, rows);
    ma.sb = ma.sb ? (int64_t)nh * nq * ldm : 0;
    ma.sh = ma.sh ? (int64_t)nq * ldm : 0;
    ma.sq = ma.sq ? ldm : 0;
    ma.sk = 1;
    mp = packed;
  }
  int rc = KH_OK;
  StagedAttn sp;
  if (extent < (int64_t(1) << 31) && !direct_qkv) rc = stage_attn(sp, KH_BF16, q, k, v, batch, hq, hkv, lq, lk, d, st);
  if (rc != KH_OK) {
  } else if (extent >= (int64_t(1) << 31) || (!direct_qkv && !sp.block)) {
    // The generic kernel reads the caller's mask (its strides, not the packed copy's).
    MaskArgs mg = ma;
    mg.sb = mask_strides[0];
    mg.sh = mask_strides[1];
    mg.sq = mask_strides[2];
    mg.sk = mask_strides[3];
    rc = launch_generic(q, k, v, o, batch, hq, hkv, (int)lq, (int)lk, d, st, scale, 0, mask, mask_dtype, mg, dtype);
  } else {
    ma.bytes = (uint32_t)extent;
    if (sp.block)
      rc = unstage_attn(sp,
                        launch_flash_prefill_bf16_masked(sp.q, sp.k, sp.v, sp.o, batch, hq, hkv, (int)lq, (int)lk,
                                                         sp.dp, sp.st, scale, mp, ma, mask_dtype),
                        KH_BF16, o, batch, hq, lq, d, st);
    else
      rc = launch_flash_prefill_bf16_masked(q, k, v, o, batch, hq, hkv, (int)lq, (int)lk, d, st, scale, mp, ma,
                                            mask_dtype);
  }
  if (packed) scratch_free(packed);  // stream-ordered: reused only by later work on the same stream
  return rc;
}

int kh_decode_attention(const void* q, const void* k_cache, const void* v_cache, void* o, const int32_t* seq_lens,
                        int batch, int hq, int hkv, int d, int64_t max_len, const int64_t* strides, float scale,
                        int dtype) {
  KH_REQUIRE_INIT();
  KH_REQUIRE(batch >= 0 && hq > 0 && hkv > 0 && max_len > 0, "kh_decode_attention: bad extents");
  KH_REQUIRE(hq % hkv == 0, "kh_decode_attention: numHeadsQ (%d) must be divisible by numHeadsKV (%d)", hq, hkv);
  KH_REQUIRE(d == 128 || d == 64, "kh_decode_attention: head_dim %d not supported (64 or 128)", d);
  KH_REQUIRE(dtype == KH_BF16 || dtype == KH_F32, "kh_decode_attention: unsupported dtype %d", dtype);
  KH_REQUIRE(max_len <= INT32_MAX, "kh_decode_attention: max_len too large");
  if (batch == 0) return KH_OK;
  KH_REQUIRE(batch <= 65535, "kh_decode_attention: batch too large");
  KH_REQUIRE(q && k_cache && v_cache && o && seq_lens && strides, "kh_decode_attention: null pointer");
  AttnStrides st{};
  st.qb = strides[0]; st.qh = strides[1]; st.qs = 0;
  st.kb = strides[2]; st.kh = strides[3]; st.ks = strides[4];
  st.vb = strides[5]; st.vh = strides[6]; st.vs = strides[7];
  st.ob = strides[8]; st.oh = strides[9]; st.os = 0;
  KH_REQUIRE(decode_aligned(q, k_cache, v_cache, st, dtype),
             "kh_decode_attention: q and the caches must be 16-byte aligned with 16-byte aligned strides");
  return launch_decode_for(dtype, d, q, k_cache, v_cache, o, seq_lens, 0, batch, hq, hkv, max_len, st, scale);
}

int kh_decode_attention_noalloc(const void* q, const void* k_cache, const void* v_cache, void* o,
                                const int32_t* seq_lens, int batch, int hq, int hkv, int d, int64_t max_len,
                                const int64_t* strides, float scale, int dtype) {
  KH_REQUIRE_INIT();
  KH_REQUIRE(batch >= 0 && hq > 0 && hkv > 0 && max_len > 0, "kh_decode_attention_noalloc: bad extents");
  KH_REQUIRE(hq % hkv == 0, "kh_decode_attention_noalloc: numHeadsQ (%d) must be divisible by numHeadsKV (%d)", hq,
             hkv);
  KH_REQUIRE(d == 128 || d == 64, "kh_decode_attention_noalloc: head_dim %d not supported (64 or 128)", d);
  KH_REQUIRE(dtype == KH_BF16 || dtype == KH_F32, "kh_decode_attention_noalloc: unsupported dtype %d", dtype);
  KH_REQUIRE(max_len <= INT32_MAX, "kh_decode_attention_noalloc: max_len too large");
  if (batch == 0) return KH_OK;
  KH_REQUIRE(batch <= 65535, "kh_decode_attention_noalloc: batch too large");
  KH_REQUIRE(q && k_cache && v_cache && o && seq_lens && strides, "kh_decode_attention_noalloc: null pointer");
  const size_t need = decode_part_bytes_for(dtype, d, batch, hq, max_len);
  KH_REQUIRE(need <= kNoAllocScratchBytes,
             "kh_decode_attention_noalloc: batch %d x %d heads x %lld keys needs %zu bytes of split-K partials, "
             "more than the %zu-byte scratch array (use kh_decode_attention)",
             batch, hq, (long long)max_len, need, kNoAllocScratchBytes);
  const int dev = current_device();
  KH_REQUIRE(dev >= 0 && dev < kMaxDevices && g_scratch_ptr[dev] != nullptr,
             "kh_decode_attention_noalloc: the scratch array of device %d has no address (kh_init)", dev);
  AttnStrides st{};
  st.qb = strides[0]; st.qh = strides[1]; st.qs = 0;
  st.kb = strides[2]; st.kh = strides[3]; st.ks = strides[4];
  st.vb = strides[5]; st.vh = strides[6]; st.vs = strides[7];
  st.ob = strides[8]; st.oh = strides[9]; st.os = 0;
  KH_REQUIRE(decode_aligned(q, k_cache, v_cache, st, dtype),
             "kh_decode_attention_noalloc: q and the caches must be 16-byte aligned with 16-byte aligned strides");
  float* part = (float*)g_scratch_ptr[dev];
  return launch_decode_for(dtype, d, q, k_cache, v_cache, o, seq_lens, 0, batch, hq, hkv, max_len, st, scale, part);
}

int kh_decode_attention_block(const void* qkv, const void* q_norm_w, const void* k_norm_w, const float* inv_freq,
                              float eps, const int32_t* position, void* k_cache, void* v_cache, int hq, int hkv,
                              int64_t max_len, const int64_t* cache_strides, float scale, const void* w_o, int64_t ldw,
                              int64_t n_out, float* x, int dtype) {
  KH_REQUIRE_INIT();
  KH_REQUIRE(hq > 0 && hkv > 0 && hq % hkv == 0, "kh_decode_attention_block: bad head counts %d / %d", hq, hkv);
  const int GC = decode_group_heads(hq / hkv), nsub = hq / hkv / GC;
  KH_REQUIRE((int64_t)hkv * nsub <= 65535, "kh_decode_attention_block: %d query heads need too many workgroup groups",
             hq);
  KH_REQUIRE(dtype == KH_BF16 || dtype == KH_F32, "kh_decode_attention_block: unsupported dtype %d", dtype);
  KH_REQUIRE(max_len > 0 && max_len <= INT32_MAX && n_out > 0 && n_out <= INT32_MAX,
             "kh_decode_attention_block: bad extents");
  KH_REQUIRE(qkv && q_norm_w && k_norm_w && inv_freq && position && k_cache && v_cache && cache_strides && w_o && x,
             "kh_decode_attention_block: null pointer");
  const bool f32 = dtype == KH_F32;
  const int64_t eb = f32 ? 4 : 2, vec = 16 / eb;
  const int64_t kh_s = cache_strides[0], ks = cache_strides[1], vh_s = cache_strides[2], vs = cache_strides[3];
  KH_REQUIRE(aligned16(qkv) && aligned16(q_norm_w) && aligned16(k_norm_w) && aligned16(k_cache) &&
                 aligned16(v_cache) && kh_s % vec == 0 && ks % vec == 0 && vh_s % vec == 0 && vs % vec == 0,
             "kh_decode_attention_block: operands must be 16-byte aligned with 16-byte aligned strides");
  const int64_t lim = int64_t(1) << 31;
  KH_REQUIRE((max_len + 256) * ks * eb < lim && (max_len + 256) * vs * eb < lim,
             "kh_decode_attention_block: one head of the cache spans more than 2 GiB");
  const int ml = (int)max_len;
  const int CH = f32 ? dc_chunk<float>() : dc_chunk<uint16_t>();  // keys per split-K chunk
  const int max_chunks = (ml + CH - 1) / CH;
  KH_REQUIRE(max_chunks <= 65535, "kh_decode_attention_block: max_len too large");
  const size_t part_bytes = (size_t)hq * max_chunks * (128 + 2) * sizeof(float);
  float* part = (float*)scratch_alloc(part_bytes);
  if (!part) return KH_ERR_OOM;
  AttnStrides st{};
  st.qh = 128;
  st.kh = kh_s; st.ks = ks; st.vh = vh_s; st.vs = vs;
  DecodeFuse fz;
  fz.wq = (const uint16_t*)q_norm_w;
  fz.wk = (const uint16_t*)k_norm_w;
  fz.inv_freq = inv_freq;
  fz.position = position;
  fz.k_new = (const char*)qkv + (int64_t)hq * 128 * eb;
  fz.v_new = (const char*)qkv + (int64_t)(hq + hkv) * 128 * eb;
  fz.eps = eps;
  const dim3 grid(max_chunks, hkv * nsub, 1);
  auto partial = [&](auto* tp) {
    using T = std::remove_pointer_t<decltype(tp)>;
    const T* Q = (const T*)qkv;
    const T* K = (const T*)k_cache;
    const T* V = (const T*)v_cache;
#define KH_BLOCK_CASE(GG)                                                                                   \
  case GG:                                                                                                  \
    decode_partial_rows_kernel<T, GG, true><<<grid, 256, 0, stream()>>>(Q, K, V, nullptr, 0, ml, hq, nsub, st,  \
                                                                        scale, max_chunks, part, fz);        \
    break;
    switch (GC) {
      KH_BLOCK_CASE(1)
      KH_BLOCK_CASE(2)
      KH_BLOCK_CASE(3)
      KH_BLOCK_CASE(4)
      KH_BLOCK_CASE(5)
      KH_BLOCK_CASE(6)
      KH_BLOCK_CASE(7)
      KH_BLOCK_CASE(8)
    }
#undef KH_BLOCK_CASE
  };
  if (f32)
    partial((float*)nullptr);
  else
    partial((uint16_t*)nullptr);
  // Launch errors are recorded, and the scratch blocks returned, before any return.
  hipError_t e = hipGetLastError();
  const int K_in = hq * 128;
  int rc = KH_OK;
  AttnMerge am;
  am.position = position;
  am.hq = hq;
  am.max_chunks = max_chunks;
  am.max_len = ml;
  am.chunk = CH;
  if (e != hipSuccess) {
    // nothing more is launched
  } else if (max_chunks <= kMergeInPrologueMaxChunks &&
             launch_gemv_attn_merge(part, am, (const uint16_t*)w_o, ldw, x, x, (int)n_out, K_in, 1.f, 1.f, f32)) {
    e = hipGetLastError();
  } else {
    // long caches: a separate merge into a row of the caches' type, then the plain GEMV with the residual
    void* o = scratch_alloc((size_t)K_in * eb);
    if (!o) {
      scratch_free(part);
      return KH_ERR_OOM;
    }
    AttnStrides so{};
    so.oh = 128;
    if (f32)
      decode_merge_cols_pos_kernel<float><<<dim3(4, hq, 1), 256, 0, stream()>>>(part, position, ml, hq, max_chunks, so,
                                                                                (float*)o);
    else
      decode_merge_cols_pos_kernel<uint16_t><<<dim3(4, hq, 1), 256, 0, stream()>>>(part, position, ml, hq, max_chunks,
                                                                                   so, (uint16_t*)o);
    e = hipGetLastError();
    if (e == hipSuccess)
      rc = kh_gemv_fused(0, o, nullptr, nullptr, 0.f, w_o, ldw, x, x, nullptr, n_out, K_in, 1.f, 1.f, KH_F32, dtype);
    scratch_free(o);
  }
  scratch_free(part);  // stream-ordered: reused only by later work on the same stream
  if (e != hipSuccess) {
    set_error("kh_decode_attention_block: launch failed: %s", hipGetErrorString(e));
    return KH_ERR_HIP;
  }
  if (rc == KH_OK) KH_DEBUG_SYNC();
  return rc;
}

}  // extern "C"
