// Scaled dot-product attention for gfx950: bf16 MFMA flash prefill, split-K decode, and a generic
// fp32-math kernel for every other case.
//
// Semantics (reference: packages/backend-webgpu/src/kernels/attention/builder.ts:138-329):
//   S = (Q K^T) * scale, causal masks key j > query i (top-left aligned), GQA query head h reads
//   kv head h / (hq / hkv), online softmax in fp32, O = P V / l.
#include <cfloat>
#include <cmath>

#include "common.h"

using namespace kh;

namespace {

constexpr float kLog2e = 1.4426950408889634f;

struct AttnStrides {
  int64_t qb, qh, qs, kb, kh, ks, vb, vh, vs, ob, oh, os;
};

// =============================================================================================
// bf16 flash prefill, head_dim 128.
//
// Workgroup = 8 waves sharing one kv head: wave w serves query head g = w / (8/G) of the G query
// heads that read this kv head (G = hq / hkv in {1, 2, 4, 8}) and 32 query rows of a BMQ = 256/G
// row block.  K/V tiles of 64 keys are staged in LDS (double buffered) and shared by all 8 waves.
//
// Per wave and tile, with v_mfma_f32_32x32x16_bf16:
//   S^T (keys x queries) = K Q^T : A = K rows from LDS, B = Q held in registers for the whole loop.
//   O^T (d x queries)   += V^T P^T: A = V^T rows from LDS (V is transposed when staged), B = P.
// Each lane thus owns one query column: the row max / sum of the softmax are in-lane over 32
// scores plus one exchange with lane ^ 32.  K rows are loaded into the A operand in the order
// "swap bits 2 and 3 of the row index", which makes the S^T accumulator registers j = 0..7 of lane
// group g hold keys 8g + j (and j = 8..15 keys 16 + 8g + j - 8): exactly the B-operand layout the
// PV product needs, so P never leaves registers.
// =============================================================================================
constexpr int FA_D = 128;
constexpr int FA_BN = 64;                 // keys per tile
constexpr int FA_WAVES = 8;
constexpr int FA_THREADS = FA_WAVES * 64;
constexpr int FA_KSTR = FA_D + 8;         // K row stride in LDS (elements), 16B-aligned, padded
constexpr int FA_VSTR = FA_BN + 8;        // V^T row stride in LDS (elements)
constexpr int FA_KTILE = FA_BN * FA_KSTR; // elements
constexpr int FA_VTILE = FA_D * FA_VSTR;  // elements

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

__global__ __launch_bounds__(FA_THREADS, 1) void flash_fwd_bf16_d128_kernel(
    const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K, const uint16_t* __restrict__ V,
    uint16_t* __restrict__ O, int batch, int hq, int hkv, int lq, int lk, AttnStrides st, float scale, int causal,
    int n_qblocks) {
  __shared__ __attribute__((aligned(16))) uint16_t smem[2 * (FA_KTILE + FA_VTILE)];

  const int G = hq / hkv;
  const int wpg = FA_WAVES / G;           // waves per query head
  const int BMQ = 32 * wpg;               // query rows per head in this workgroup
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int r = lane & 31;                // query column owned by this lane
  const int g = lane >> 5;                // lane group

  // Heaviest (last) query blocks first for causal load balance; (b, kv head) fastest-varying.
  const int bh = blockIdx.x % (batch * hkv);
  const int qblk = n_qblocks - 1 - blockIdx.x / (batch * hkv);
  const int b = bh / hkv;
  const int hk = bh % hkv;
  const int hqi = hk * G + wave / wpg;
  const int q0 = qblk * BMQ;                      // first query row of the workgroup
  const int qw0 = q0 + (wave % wpg) * 32;         // first query row of this wave
  const int qi = qw0 + r;                         // this lane's query row

  const uint16_t* Kb = K + b * st.kb + hk * st.kh;
  const uint16_t* Vb = V + b * st.vb + hk * st.vh;

  // ---- Q operand (B of S^T = K Q^T): lane holds query qi, d = 16c + 8g + [0, 8) ----
  bf16x8 qreg[8];
  {
    const uint16_t* qrow = Q + b * st.qb + hqi * st.qh + (int64_t)qi * st.qs;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      uint4 v = make_uint4(0, 0, 0, 0);
      if (qi < lq) v = *reinterpret_cast<const uint4*>(qrow + 16 * c + 8 * g);
      qreg[c] = as_bf16x8(v);
    }
  }

  // ---- key range ----
  int kv_end = lk;
  if (causal) kv_end = min(lk, q0 + BMQ);
  const int ntiles = (kv_end + FA_BN - 1) / FA_BN;
  const int wave_last_q = min(qw0 + 31, lq - 1);  // last valid query of the wave

  // ---- staging of one K/V tile: global -> registers -> LDS ----
  // K: 1024 chunks of 16 B per tile, 2 per thread: chunk id = tid + 512 i -> key id/16, d 8*(id%16).
  // V: thread owns keys 2p, 2p+1 (p = tid/16) and d 8*(tid%16)..+8, written transposed as bf16 pairs.
  uint4 kst[2], vst[2];
  auto load_tile = [&](int t) {
    const int kt = t * FA_BN;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int id = tid + FA_THREADS * i;
      const int key = kt + (id >> 4);
      kst[i] = make_uint4(0, 0, 0, 0);
      if (key < lk) kst[i] = *reinterpret_cast<const uint4*>(Kb + (int64_t)key * st.ks + 8 * (id & 15));
    }
    const int p = tid >> 4;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int key = kt + 2 * p + i;
      vst[i] = make_uint4(0, 0, 0, 0);
      if (key < lk) vst[i] = *reinterpret_cast<const uint4*>(Vb + (int64_t)key * st.vs + 8 * (tid & 15));
    }
  };
  auto store_tile = [&](int buf) {
    uint16_t* ks = smem + buf * (FA_KTILE + FA_VTILE);
    uint16_t* vts = ks + FA_KTILE;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int id = tid + FA_THREADS * i;
      *reinterpret_cast<uint4*>(ks + (id >> 4) * FA_KSTR + 8 * (id & 15)) = kst[i];
    }
    const int p = tid >> 4;
    const int d0 = 8 * (tid & 15);
    const uint32_t a[4] = {vst[0].x, vst[0].y, vst[0].z, vst[0].w};
    const uint32_t c[4] = {vst[1].x, vst[1].y, vst[1].z, vst[1].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      // d = d0 + 2e: (V[2p][d], V[2p+1][d]);  d = d0 + 2e + 1: (V[2p][d+1], V[2p+1][d+1])
      const uint32_t lo = (a[e] & 0xffffu) | (c[e] << 16);
      const uint32_t hi = (a[e] >> 16) | (c[e] & 0xffff0000u);
      *reinterpret_cast<uint32_t*>(vts + (d0 + 2 * e) * FA_VSTR + 2 * p) = lo;
      *reinterpret_cast<uint32_t*>(vts + (d0 + 2 * e + 1) * FA_VSTR + 2 * p) = hi;
    }
  };

  // ---- accumulators ----
  f32x16 oacc[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int j = 0; j < 16; ++j) oacc[dt][j] = 0.f;
  float m_run = -INFINITY;  // running max of raw scores (q.k) for this lane's query
  float l_run = 0.f;        // this lane's partial softmax denominator
  const float c2 = scale * kLog2e;

  // A-operand row of K for this lane: row index r with bits 2 and 3 swapped.
  const int krow = (r & ~12) | ((r & 4) << 1) | ((r & 8) >> 1);

  if (ntiles > 0) {
    load_tile(0);
    store_tile(0);
  }
  __syncthreads();

  for (int t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    const bool has_next = t + 1 < ntiles;
    if (has_next) load_tile(t + 1);

    const int kt = t * FA_BN;
    const uint16_t* ks = smem + buf * (FA_KTILE + FA_VTILE);
    const uint16_t* vts = ks + FA_KTILE;

    // Skip compute when every key of the tile is masked for every query of this wave.
    const bool wave_active = qw0 < lq && (!causal || kt <= wave_last_q);
    if (wave_active) {
      // ---- S^T = K Q^T over two 32-key subtiles ----
      f32x16 sacc[2];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
#pragma unroll
        for (int j = 0; j < 16; ++j) sacc[s][j] = 0.f;
        const uint16_t* krp = ks + (32 * s + krow) * FA_KSTR + 8 * g;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          const bf16x8 kv = as_bf16x8(*reinterpret_cast<const uint4*>(krp + 16 * c));
          sacc[s] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kv, qreg[c], sacc[s], 0, 0, 0);
        }
      }
      // ---- mask: register j of subtile s holds key kt + 32s + 16(j/8) + 8g + j%8 ----
      const bool need_mask = (kt + FA_BN > lk) || (causal && kt + FA_BN - 1 > qw0);
      if (need_mask) {
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            const int key = kt + 32 * s + 16 * (j >> 3) + 8 * g + (j & 7);
            if (key >= lk || (causal && key > qi)) sacc[s][j] = -INFINITY;
          }
      }
      // ---- online softmax ----
      float mx = m_run;
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int j = 0; j < 16; ++j) mx = fmaxf(mx, sacc[s][j]);
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float m_use = (mx == -INFINITY) ? 0.f : mx;
      const float alpha = exp2f((m_run - m_use) * c2);
      m_run = mx;
      const float mb = m_use * c2;
      float psum = 0.f;
      bf16x8 pk[4];
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          bf16x8 pv;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float p = exp2f(sacc[s][8 * h + e] * c2 - mb);
            psum += p;
            pv[e] = (__bf16)p;
          }
          pk[2 * s + h] = pv;
        }
      l_run = l_run * alpha + psum;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int j = 0; j < 16; ++j) oacc[dt][j] *= alpha;
      // ---- O^T += V^T P^T ----
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        const uint16_t* vrp = vts + (32 * dt + r) * FA_VSTR + 8 * g;
#pragma unroll
        for (int kc = 0; kc < 4; ++kc) {
          const bf16x8 vv = as_bf16x8(*reinterpret_cast<const uint4*>(vrp + 16 * kc));
          oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vv, pk[kc], oacc[dt], 0, 0, 0);
        }
      }
    }

    if (has_next) store_tile(buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue: O[qi][d] = oacc / l, lane holds d = 32dt + 8(j/4) + 4g + j%4 ----
  const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
  if (qi < lq) {
    const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
    uint16_t* orow = O + b * st.ob + hqi * st.oh + (int64_t)qi * st.os;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const int d = 32 * dt + 8 * a + 4 * g;
        uint2 w;
        w.x = pack_bf16x2(oacc[dt][4 * a + 0] * inv, oacc[dt][4 * a + 1] * inv);
        w.y = pack_bf16x2(oacc[dt][4 * a + 2] * inv, oacc[dt][4 * a + 3] * inv);
        *reinterpret_cast<uint2*>(orow + d) = w;
      }
  }
}

// =============================================================================================
// Generic attention (any dtype in {f32, bf16}, d <= 256, any lq/lk): one wave per query row,
// 64 keys per step (lane j scores key k0 + j), fp32 online softmax, each lane accumulates
// d/64 output columns.  Used for fp32 (C1-style) calls and shapes the MFMA kernel does not take.
// =============================================================================================
template <typename T>
__global__ __launch_bounds__(256) void attn_generic_kernel(const T* __restrict__ Q, const T* __restrict__ K,
                                                           const T* __restrict__ V, T* __restrict__ O, int batch,
                                                           int hq, int hkv, int lq, int lk, int D, AttnStrides st,
                                                           float scale, int causal) {
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
  float m = -INFINITY, l = 0.f;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};  // columns lane, lane+64, lane+128, lane+192
  for (int k0 = 0; k0 < kend; k0 += 64) {
    const int key = k0 + lane;
    float s = -INFINITY;
    if (key < kend) {
      const T* kr = Kb + (int64_t)key * st.ks;
      float dot = 0.f;
      for (int d = 0; d < D; ++d) dot += qs[w][d] * Elem<T>::load(kr, d);
      s = dot * scale;
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
  const float inv = l > 0.f ? 1.0f / l : 0.f;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int d = lane + 64 * c;
    if (d < D) Elem<T>::store(orow, d, acc[c] * inv);
  }
}

// =============================================================================================
// Split-K decode: one query token per sequence, per-sequence KV length.
//
// Work unit = (b, kv head, chunk of DC_CHUNK keys); the G query heads of the kv head are served
// from the same K/V bytes.  A row of 128 bf16 (256 B) is read by 16 lanes with 16-byte loads, so a
// wave covers 4 keys per load instruction; all K and V loads of a wave's keys are issued before any
// math so the bytes in flight per lane stay high.  Each unit writes (m, l, o[d]) per query head;
// a merge kernel combines chunks with the log-sum-exp rule.
// =============================================================================================
constexpr int DC_WAVES = 4;
// Keys per wave per unit: 16 load instructions of 16 B per lane for K and for V in both dtypes.
template <typename T>
constexpr int dc_kpw() { return sizeof(T) == 2 ? 64 : 32; }
template <typename T>
constexpr int dc_chunk() { return DC_WAVES * dc_kpw<T>(); }

// Key count of sequence b: seq_lens[b] (or the uniform length when seq_lens is NULL), clamped to
// [0, max_len] so that a bad device-side length can never index past the cache.
__device__ __forceinline__ int decode_len(const int32_t* lens, int uniform_len, int b, int max_len) {
  const int L = lens ? lens[b] : uniform_len;
  return L < 0 ? 0 : (L > max_len ? max_len : L);
}

template <typename T, int G>
__global__ __launch_bounds__(256) void decode_partial_kernel(const T* __restrict__ Q, const T* __restrict__ K,
                                                             const T* __restrict__ V, const int32_t* __restrict__ lens,
                                                             int uniform_len, int max_len, int hq, int hkv,
                                                             AttnStrides st, float scale, int max_chunks,
                                                             float* __restrict__ part) {
  // Layout of `part`: [b][hq][max_chunks][2 + 128] floats (m, l, o[0..127]), valid chunks only.
  constexpr int D = 128;
  constexpr int EPL = (sizeof(T) == 2) ? 8 : 4;      // elements per 16-byte load
  constexpr int LPK = D / EPL;                        // lanes per key row (16 bf16, 32 f32)
  constexpr int KPI = 64 / LPK;                       // keys per load instruction (4 bf16, 2 f32)
  constexpr int KPW = dc_kpw<T>();
  constexpr int CHUNK = dc_chunk<T>();
  constexpr int NI = KPW / KPI;                       // load instructions per wave (16)
  __shared__ float red_m[DC_WAVES][G];
  __shared__ float red_l[DC_WAVES][G];
  __shared__ float red_o[DC_WAVES][G][D];

  const int chunk = blockIdx.x;
  const int hk = blockIdx.y;
  const int b = blockIdx.z;
  // Device-side lengths are clamped to [0, max_chunks * CHUNK] and the caller sizes max_chunks from
  // the cache length, so no key beyond the cache is ever read.
  const int L = decode_len(lens, uniform_len, b, max_len);
  if (chunk * CHUNK >= L) return;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int sub = lane % LPK;          // 16-byte column inside the row
  const int kk = lane / LPK;           // key slot inside a load instruction
  const int key0 = chunk * CHUNK + w * KPW;

  // q for the G heads, this lane's EPL columns.
  float qv[G][EPL];
#pragma unroll
  for (int gi = 0; gi < G; ++gi) {
    const T* qr = Q + b * st.qb + (int64_t)(hk * G + gi) * st.qh + sub * EPL;
#pragma unroll
    for (int e = 0; e < EPL; ++e) qv[gi][e] = Elem<T>::load(qr, e) * scale;
  }

  const T* Kb = K + b * st.kb + hk * st.kh + sub * EPL;
  const T* Vb = V + b * st.vb + hk * st.vh + sub * EPL;
  uint4 kr[NI], vr[NI];
#pragma unroll
  for (int it = 0; it < NI; ++it) {
    const int key = key0 + it * KPI + kk;
    kr[it] = make_uint4(0, 0, 0, 0);
    vr[it] = make_uint4(0, 0, 0, 0);
    if (key < L) {
      kr[it] = *reinterpret_cast<const uint4*>(Kb + (int64_t)key * st.ks);
      vr[it] = *reinterpret_cast<const uint4*>(Vb + (int64_t)key * st.vs);
    }
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
  // Per-head max over the wave's keys.
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
    float* pp = part + (((int64_t)b * hq + hk * G + gi) * max_chunks + chunk) * (2 + D);
    if (d == 0) {
      pp[0] = M;
      pp[1] = Ls;
    }
    pp[2 + d] = Os;
  }
}

template <typename T>
__global__ __launch_bounds__(128) void decode_merge_kernel(const float* __restrict__ part,
                                                           const int32_t* __restrict__ lens, int uniform_len,
                                                           int max_len, int hq, int max_chunks, AttnStrides st,
                                                           T* __restrict__ O) {
  constexpr int D = 128;
  const int h = blockIdx.x, b = blockIdx.y;
  const int d = threadIdx.x;
  const int L = decode_len(lens, uniform_len, b, max_len);
  const int nch = (L + dc_chunk<T>() - 1) / dc_chunk<T>();
  const float* pp = part + ((int64_t)b * hq + h) * max_chunks * (2 + D);
  float M = -INFINITY;
  for (int c = 0; c < nch; ++c) M = fmaxf(M, pp[c * (2 + D)]);
  const float mu = M == -INFINITY ? 0.f : M;
  float Ls = 0.f, Os = 0.f;
  for (int c = 0; c < nch; ++c) {
    const float f = __expf(pp[c * (2 + D)] - mu);
    Ls += pp[c * (2 + D) + 1] * f;
    Os += pp[c * (2 + D) + 2 + d] * f;
  }
  Elem<T>::store(O + b * st.ob + h * st.oh, d, Ls > 0.f ? Os / Ls : 0.f);
}

AttnStrides load_strides(const int64_t* s) {
  AttnStrides a;
  a.qb = s[0]; a.qh = s[1]; a.qs = s[2];
  a.kb = s[3]; a.kh = s[4]; a.ks = s[5];
  a.vb = s[6]; a.vh = s[7]; a.vs = s[8];
  a.ob = s[9]; a.oh = s[10]; a.os = s[11];
  return a;
}

template <typename T>
int launch_decode(const void* q, const void* k, const void* v, void* o, const int32_t* lens, int uniform_len,
                  int batch, int hq, int hkv, int64_t max_len, const AttnStrides& st, float scale) {
  const int G = hq / hkv;
  KH_REQUIRE(G == 1 || G == 2 || G == 4 || G == 8, "kh_decode_attention: hq/hkv = %d not in {1, 2, 4, 8}", G);
  const int ml = (int)max_len;
  const int max_chunks = (ml + dc_chunk<T>() - 1) / dc_chunk<T>();
  const size_t part_bytes = (size_t)batch * hq * max_chunks * (2 + 128) * sizeof(float);
  float* part = (float*)scratch_alloc(part_bytes);
  if (!part) return KH_ERR_OOM;
  dim3 grid(max_chunks, hkv, batch);
  const T* Q = (const T*)q;
  const T* K = (const T*)k;
  const T* V = (const T*)v;
#define KH_DECODE_CASE(GG)                                                                        \
  case GG:                                                                                        \
    decode_partial_kernel<T, GG><<<grid, 256, 0, stream()>>>(Q, K, V, lens, uniform_len, ml, hq, hkv, st, \
                                                              scale, max_chunks, part);           \
    break;
  switch (G) {
    KH_DECODE_CASE(1)
    KH_DECODE_CASE(2)
    KH_DECODE_CASE(4)
    KH_DECODE_CASE(8)
  }
#undef KH_DECODE_CASE
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) {
    decode_merge_kernel<T><<<dim3(hq, batch), 128, 0, stream()>>>(part, lens, uniform_len, ml, hq, max_chunks, st,
                                                                  (T*)o);
    e = hipGetLastError();
  }
  scratch_free(part);  // stream-ordered: the block is reused only by later work on the same stream
  if (e != hipSuccess) {
    set_error("kh_decode_attention: launch failed: %s", hipGetErrorString(e));
    return KH_ERR_HIP;
  }
  return KH_OK;
}

}  // namespace

extern "C" {

int kh_flash_attention(const void* q, const void* k, const void* v, void* o, int batch, int hq, int hkv, int64_t lq,
                       int64_t lk, int d, const int64_t* strides, float scale, int causal, int dtype) {
  KH_REQUIRE_INIT();
  KH_REQUIRE(batch >= 0 && hq > 0 && hkv > 0 && lq >= 0 && lk >= 0 && d > 0,
             "kh_flash_attention: bad extents");
  KH_REQUIRE(hq % hkv == 0, "kh_flash_attention: numHeadsQ (%d) must be divisible by numHeadsKV (%d)", hq, hkv);
  KH_REQUIRE(dtype == KH_BF16 || dtype == KH_F32, "kh_flash_attention: unsupported dtype %d", dtype);
  KH_REQUIRE(lq <= INT32_MAX && lk <= INT32_MAX, "kh_flash_attention: sequence too long");
  if (batch == 0 || lq == 0) return KH_OK;
  KH_REQUIRE(q && k && v && o && strides, "kh_flash_attention: null pointer");
  const AttnStrides st = load_strides(strides);
  const int G = hq / hkv;
  KH_REQUIRE(lk > 0, "kh_flash_attention: the key sequence is empty (softmax over no keys is undefined)");

  // One query row, no mask: split-K decode over the keys (the caller's 1-token decode step).
  const int64_t vec = dtype == KH_BF16 ? 8 : 4;
  const bool decode_ok = lq == 1 && !causal && d == 128 && (G == 1 || G == 2 || G == 4 || G == 8) && aligned16(k) &&
                         aligned16(v) && st.kb % vec == 0 && st.kh % vec == 0 && st.ks % vec == 0 &&
                         st.vb % vec == 0 && st.vh % vec == 0 && st.vs % vec == 0;
  if (decode_ok) {
    AttnStrides ds = st;
    ds.qs = 0;
    ds.os = 0;
    if (dtype == KH_BF16) return launch_decode<uint16_t>(q, k, v, o, nullptr, (int)lk, batch, hq, hkv, lk, ds, scale);
    return launch_decode<float>(q, k, v, o, nullptr, (int)lk, batch, hq, hkv, lk, ds, scale);
  }

  const bool mfma_ok = dtype == KH_BF16 && d == FA_D && (G == 1 || G == 2 || G == 4 || G == 8) && aligned16(q) &&
                       aligned16(k) && aligned16(v) && aligned16(o) && st.qs % 8 == 0 && st.ks % 8 == 0 &&
                       st.vs % 8 == 0 && st.os % 4 == 0 && st.qb % 8 == 0 && st.qh % 8 == 0 && st.kb % 8 == 0 &&
                       st.kh % 8 == 0 && st.vb % 8 == 0 && st.vh % 8 == 0 && st.ob % 4 == 0 && st.oh % 4 == 0;
  if (mfma_ok && lq > 1) {
    const int BMQ = 32 * (FA_WAVES / G);
    const int nqb = (int)((lq + BMQ - 1) / BMQ);
    const int64_t nblk = (int64_t)nqb * batch * hkv;
    KH_REQUIRE(nblk <= INT32_MAX, "kh_flash_attention: grid too large");
    flash_fwd_bf16_d128_kernel<<<(int)nblk, FA_THREADS, 0, stream()>>>(
        (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v, (uint16_t*)o, batch, hq, hkv, (int)lq, (int)lk,
        st, scale, causal, nqb);
    KH_CHECK_LAUNCH();
    return KH_OK;
  }
  KH_REQUIRE(d <= 256, "kh_flash_attention: head_dim %d > 256 is not supported", d);
  const int64_t rows = (int64_t)batch * hq * lq;
  const int64_t grid = (rows + 3) / 4;
  KH_REQUIRE(grid <= INT32_MAX, "kh_flash_attention: grid too large");
  if (dtype == KH_BF16)
    attn_generic_kernel<uint16_t><<<(int)grid, 256, 0, stream()>>>((const uint16_t*)q, (const uint16_t*)k,
                                                                   (const uint16_t*)v, (uint16_t*)o, batch, hq, hkv,
                                                                   (int)lq, (int)lk, d, st, scale, causal);
  else
    attn_generic_kernel<float><<<(int)grid, 256, 0, stream()>>>((const float*)q, (const float*)k, (const float*)v,
                                                                (float*)o, batch, hq, hkv, (int)lq, (int)lk, d, st,
                                                                scale, causal);
  KH_CHECK_LAUNCH();
  return KH_OK;
}

int kh_decode_attention(const void* q, const void* k_cache, const void* v_cache, void* o, const int32_t* seq_lens,
                        int batch, int hq, int hkv, int d, int64_t max_len, const int64_t* strides, float scale,
                        int dtype) {
  KH_REQUIRE_INIT();
  KH_REQUIRE(batch >= 0 && hq > 0 && hkv > 0 && max_len > 0, "kh_decode_attention: bad extents");
  KH_REQUIRE(hq % hkv == 0, "kh_decode_attention: numHeadsQ (%d) must be divisible by numHeadsKV (%d)", hq, hkv);
  KH_REQUIRE(d == 128, "kh_decode_attention: head_dim %d not supported (128 only)", d);
  KH_REQUIRE(dtype == KH_BF16 || dtype == KH_F32, "kh_decode_attention: unsupported dtype %d", dtype);
  KH_REQUIRE(max_len <= INT32_MAX, "kh_decode_attention: max_len too large");
  if (batch == 0) return KH_OK;
  KH_REQUIRE(q && k_cache && v_cache && o && seq_lens && strides, "kh_decode_attention: null pointer");
  AttnStrides st{};
  st.qb = strides[0]; st.qh = strides[1]; st.qs = 0;
  st.kb = strides[2]; st.kh = strides[3]; st.ks = strides[4];
  st.vb = strides[5]; st.vh = strides[6]; st.vs = strides[7];
  st.ob = strides[8]; st.oh = strides[9]; st.os = 0;
  const int64_t vec = dtype == KH_BF16 ? 8 : 4;
  KH_REQUIRE(aligned16(k_cache) && aligned16(v_cache) && st.kb % vec == 0 && st.kh % vec == 0 && st.ks % vec == 0 &&
                 st.vb % vec == 0 && st.vh % vec == 0 && st.vs % vec == 0,
             "kh_decode_attention: caches must be 16-byte aligned with 16-byte aligned strides");
  if (dtype == KH_BF16)
    return launch_decode<uint16_t>(q, k_cache, v_cache, o, seq_lens, 0, batch, hq, hkv, max_len, st, scale);
  return launch_decode<float>(q, k_cache, v_cache, o, seq_lens, 0, batch, hq, hkv, max_len, st, scale);
}

}  // extern "C"
