// Flash attention in fp32 for gfx950: fp32 storage, fp32 MFMA products and accumulation
// (v_mfma_f32_32x32x2_f32), online softmax in fp32.  Config C1 (fp32 SDPA) runs here.
//
// Semantics as kh_flash_attention (reference: packages/backend-webgpu/src/kernels/attention/
// builder.ts:138-329): S = (Q K^T) * scale, causal masks key j > query i (top-left aligned), GQA
// query head h reads kv head h / (hq / hkv), O = softmax(S) V.
//
// One workgroup per (batch, query head, block of 32 queries), NW waves (8 at head_dim 128; at 64, 8
// for grids with fewer than two workgroups per CU; else 4).  Wave w takes the block's 32-key tiles w, w + NW, ... (with the
// causal mask only tiles up to the block's last query), so a short prompt still spreads each block
// over every SIMD of its CU.  Per tile the wave
// forms S^T = K Q^T in D/2 MFMA steps (step s pairs head-dim element s on lanes 0-31 with s + D/2
// on lanes 32-63): lane (r, g) = (lane & 31, lane >> 5) then holds query r's scores against keys
// 8(v/4) + 4g + v%4, v < 16, so a query's maximum and sum are an in-lane reduction plus one
// exchange with lane r ^ 32.  O^T = V^T P^T follows in 16 MFMA steps per 32 head-dim columns; the
// probabilities enter as the B operand straight from the score registers (step s uses key
// 8(s/4) + 4g + s%4, the key that lane's score s belongs to).  All of a lane's outputs belong to one
// query, so the online-softmax rescale is a per-lane multiply.  At the end the waves' (m, l, O)
// are combined through LDS, in wave order.  Inputs at head dim 128 whose 32-query blocks give
// fewer workgroups than CUs take 16-query blocks (flash_f32_q16_kernel, below).
#include <cmath>

#include "attention.h"

using namespace kh;

namespace {

constexpr int kF32Waves = 4;  // waves per workgroup of the default (register-prefetching) variant
constexpr int kQ16Waves = 4;  // waves per workgroup of the 16-query-block kernel
constexpr float kLog2e = 1.4426950408889634f;
constexpr uint32_t kOut = 0xffffffffu;  // a byte offset past every buffer range: the load reads 0

__device__ __forceinline__ float buf_load4f(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}
__device__ __forceinline__ float4 buf_load16f(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

// c = scale * log2(e): scores are kept in log2 units (softmax by exp2).  NW waves per workgroup;
// with NW = 4 (one wave per SIMD) the next tile's K is loaded during the current tile's softmax and
// PV and V during QK^T; with NW = 8 (two per SIMD, for short inputs whose blocks would otherwise
// give each SIMD a chain of tiles; 256 registers per wave) the other wave on the SIMD hides the
// latency: K loads at the tile start and V after QK^T, into the registers K has left.
// V16 (head dim 128, V rows 16-byte aligned): row m of output block db is head-dim column 4 m + db
// instead of 32 db + m -- a permutation of the MFMA rows, which changes no sum -- so the V^T
// operands of one key for the four blocks are 16 contiguous bytes of its row: one 16-byte load per
// key instead of four 4-byte ones.
template <int D, bool CAUSAL, int NW = kF32Waves, bool V16 = false>
__global__ __launch_bounds__(NW * 64) void flash_f32_kernel(const float* __restrict__ Q,
                                                                   const float* __restrict__ K,
                                                                   const float* __restrict__ V, float* __restrict__ O,
                                                                   int hq, int hkv, int lq, int lk, AttnStrides st,
                                                                   float c, int nqb) {
  constexpr int HALF = D / 2, NH4 = HALF / 4, NDB = D / 32;
  constexpr int OSTR = D + 4;  // LDS row stride (floats) of the wave partial outputs
  constexpr bool PREFETCH_K = NW <= 4;
  __shared__ float2 ml_s[NW][32];
  __shared__ __attribute__((aligned(16))) float o_s[NW][32 * OSTR];

  const int lane = threadIdx.x & 63, r = lane & 31, g = lane >> 5;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int bid = blockIdx.x;
  const int qb = nqb - 1 - bid % nqb;  // the longest causal blocks start first
  const int bh = bid / nqb;
  const int h = bh % hq, b = bh / hq;
  const int hk = h / (hq / hkv);
  const int q0 = qb * 32;
  const int kend = CAUSAL ? min(lk, q0 + 32) : lk;
  const int nt = (kend + 31) >> 5;

  const float* Qh = Q + (int64_t)b * st.qb + (int64_t)h * st.qh;
  const float* Kh = K + (int64_t)b * st.kb + (int64_t)hk * st.kh;
  const float* Vh = V + (int64_t)b * st.vb + (int64_t)hk * st.vh;
  const auto rq = make_rsrc(Qh, (uint32_t)(((int64_t)(lq - 1) * st.qs + D) * 4));
  const auto rk = make_rsrc(Kh, (uint32_t)(((int64_t)(lk - 1) * st.ks + D) * 4));
  const auto rv = make_rsrc(Vh, (uint32_t)(((int64_t)(lk - 1) * st.vs + D) * 4));
  const uint32_t qs = (uint32_t)st.qs, ks = (uint32_t)st.ks, vs = (uint32_t)st.vs;

  // This lane's query row, half g of the head dim, pre-scaled (rows past lq read as zero).
  const int qi = q0 + r;
  float qv[HALF];
#pragma unroll
  for (int i = 0; i < NH4; ++i) {
    const uint32_t off = qi < lq ? ((uint32_t)qi * qs + g * HALF + 4 * i) * 4u : kOut;
    const float4 t = buf_load16f(rq, off);
    qv[4 * i] = t.x * c;
    qv[4 * i + 1] = t.y * c;
    qv[4 * i + 2] = t.z * c;
    qv[4 * i + 3] = t.w * c;
  }
  // Key row k0 + r, half g (rows past lk read as zero and are masked).
  auto load_k = [&](float (&kv)[HALF], int k0) {
    const int kr = k0 + r;
#pragma unroll
    for (int i = 0; i < NH4; ++i) {
      const uint32_t off = kr < lk ? ((uint32_t)kr * ks + g * HALF + 4 * i) * 4u : kOut;
      const float4 t = buf_load16f(rk, off);
      kv[4 * i] = t.x;
      kv[4 * i + 1] = t.y;
      kv[4 * i + 2] = t.z;
      kv[4 * i + 3] = t.w;
    }
  };
  // V[key(s)][32 db + r] (V16: [4 r + db]) for the 16 keys key(s) = k0 + 8(s/4) + 4g + s%4 of the
  // PV steps.
  auto load_v = [&](float (&vv)[NDB][16], int k0) {
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      const int kr = k0 + 8 * (s >> 2) + 4 * g + (s & 3);
      if constexpr (V16) {
        static_assert(NDB == 4, "one 16-byte load per key");
        const float4 x = buf_load16f(rv, kr < lk ? ((uint32_t)kr * vs + 4 * r) * 4u : kOut);
        vv[0][s] = x.x;
        vv[1][s] = x.y;
        vv[2][s] = x.z;
        vv[3][s] = x.w;
      } else {
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
          const uint32_t off = kr < lk ? ((uint32_t)kr * vs + 32 * db + r) * 4u : kOut;
          vv[db][s] = buf_load4f(rv, off);
        }
      }
    }
  };

  f32x16 oacc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int v = 0; v < 16; ++v) oacc[db][v] = 0.f;
  float m = -INFINITY, l = 0.f;
  float kv[HALF];
  if (PREFETCH_K && w < nt) load_k(kv, w * 32);
  for (int t = w; t < nt; t += NW) {
    const int k0 = t * 32;
    if (!PREFETCH_K) load_k(kv, k0);
    float vv[NDB][16];
    if (PREFETCH_K) load_v(vv, k0);  // in flight during QK^T
    f32x16 sacc;
#pragma unroll
    for (int v = 0; v < 16; ++v) sacc[v] = 0.f;
#pragma unroll
    for (int s = 0; s < HALF; ++s) sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(kv[s], qv[s], sacc, 0, 0, 0);
    if (PREFETCH_K && t + NW < nt) load_k(kv, k0 + 32 * NW);  // next tile's keys, during softmax and PV
    if (!PREFETCH_K) load_v(vv, k0);  // into the registers K has left
    float tmax = -INFINITY;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int key = k0 + 8 * (v >> 2) + 4 * g + (v & 3);
      const bool ok = key < lk && (!CAUSAL || key <= qi);
      sacc[v] = ok ? sacc[v] : -INFINITY;
      tmax = fmaxf(tmax, sacc[v]);
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float mn = fmaxf(m, tmax);
    const float mu = mn == -INFINITY ? 0.f : mn;  // no key seen yet: every weight is exp2(-inf) = 0
    const float alpha = fast_exp2(m - mu);
    float ps = 0.f;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      sacc[v] = fast_exp2(sacc[v] - mu);
      ps += sacc[v];
    }
    ps += __shfl_xor(ps, 32, 64);
    l = l * alpha + ps;
    m = mn;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
#pragma unroll
      for (int v = 0; v < 16; ++v) oacc[db][v] *= alpha;
#pragma unroll
      for (int s = 0; s < 16; ++s)
        oacc[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv[db][s], sacc[s], oacc[db], 0, 0, 0);
    }
  }

  // Combine the waves: O = sum_w exp2(m_w - M) O_w / sum_w exp2(m_w - M) l_w, M = max_w m_w.
  // Register v of block db holds MFMA row 8 (v / 4) + 4 g + v % 4: column 32 db + that row, or
  // with V16 4 (that row) + db (the four blocks' registers v are then 16 contiguous bytes).
  if (g == 0) ml_s[w][r] = make_float2(m, l);
  if constexpr (V16) {
#pragma unroll
    for (int v = 0; v < 16; ++v)
      *reinterpret_cast<float4*>(&o_s[w][r * OSTR + 4 * (8 * (v >> 2) + 4 * g + (v & 3))]) =
          make_float4(oacc[0][v], oacc[1][v], oacc[2][v], oacc[3][v]);
  } else {
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int v4 = 0; v4 < 4; ++v4)
        *reinterpret_cast<float4*>(&o_s[w][r * OSTR + 32 * db + 8 * v4 + 4 * g]) =
            make_float4(oacc[db][4 * v4], oacc[db][4 * v4 + 1], oacc[db][4 * v4 + 2], oacc[db][4 * v4 + 3]);
  }
  __syncthreads();
  constexpr int TPQ = NW * 64 / 32;  // threads per query
  constexpr int CPT = D / TPQ;      // output columns per thread
  static_assert(CPT % 4 == 0, "whole float4 columns per thread");
  const int tq = threadIdx.x / TPQ, c0 = (threadIdx.x % TPQ) * CPT;
  float2 mlw[NW];
  float M = -INFINITY;
#pragma unroll
  for (int u = 0; u < NW; ++u) {
    mlw[u] = ml_s[u][tq];
    M = fmaxf(M, mlw[u].x);
  }
  const float mu = M == -INFINITY ? 0.f : M;
  float f[NW], L = 0.f;
#pragma unroll
  for (int u = 0; u < NW; ++u) {
    f[u] = fast_exp2(mlw[u].x - mu);
    L += mlw[u].y * f[u];
  }
  const float inv = L > 0.f ? 1.0f / L : 0.f;
  const int qo = q0 + tq;
  if (qo < lq) {
    float* orow = O + (int64_t)b * st.ob + (int64_t)h * st.oh + (int64_t)qo * st.os + c0;
#pragma unroll
    for (int j = 0; j < CPT; j += 4) {
      float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
      for (int u = 0; u < NW; ++u) {
        const float4 x = *reinterpret_cast<const float4*>(&o_s[u][tq * OSTR + c0 + j]);
        a0 += x.x * f[u];
        a1 += x.y * f[u];
        a2 += x.z * f[u];
        a3 += x.w * f[u];
      }
      *reinterpret_cast<float4*>(orow + j) = make_float4(a0 * inv, a1 * inv, a2 * inv, a3 * inv);
    }
  }
}

// 16-query blocks for inputs whose 32-query blocks give fewer workgroups than CUs (C1: 16 heads x 8
// blocks = 128 workgroups on 256 CUs): twice the workgroups and half of the heaviest block's MFMA
// work, which bounds the call.  Same online softmax with v_mfma_f32_16x16x4_f32: per 32-key tile
// the wave forms S^T = K Q^T as two 16-key blocks kb in D/4 steps (step s pairs head-dim element
// j D/4 + s of lane group j = lane >> 4), so lane (r, j) = (lane & 15, lane >> 4) holds query r's
// scores against keys 16 kb + 4 j + i (i < 4): a query's maximum and sum are an in-lane reduction
// plus exchanges with lanes ^ 16 and ^ 32.  O^T = V^T P^T follows in 8 steps per 16 head-dim
// columns; step (kb, i) takes key 16 kb + 4 j + i from lane group j, the score that lane holds in
// its register (kb, i).  Every output of a lane belongs to query r (columns 16 db + 4 j + i).
// NW waves split a block's tiles (kQ16Waves: four, one per SIMD; eight, two per SIMD, took C1
// 11.1 -> 11.5 us once V loads were 16 bytes wide); K loads at the tile start, V during QK^T.
// V16 (V rows 16-byte aligned): row m of output block db is head-dim column 8 m + db instead of
// 16 db + m -- a permutation of the MFMA rows, which changes no sum -- so the V^T operands of one
// key for all eight blocks are 32 contiguous bytes of its row: two 16-byte loads per key instead
// of eight 4-byte ones, and a tile's loads fit the 63 a wave's load counter tracks (16 K + 64 V
// 4-byte loads did not, and the wave stalled at issue).
template <int D, bool CAUSAL, int NW, bool V16 = false>
__global__ __launch_bounds__(NW * 64) void flash_f32_q16_kernel(const float* __restrict__ Q,
                                                                const float* __restrict__ K,
                                                                const float* __restrict__ V, float* __restrict__ O,
                                                                int hq, int hkv, int lq, int lk, AttnStrides st,
                                                                float c, int nqb) {
  constexpr int QD = D / 4, NQ4 = QD / 4, NDB = D / 16;
  constexpr int OSTR = D + 4;  // LDS row stride (floats) of the wave partial outputs
  __shared__ float2 ml_s[NW][16];
  __shared__ __attribute__((aligned(16))) float o_s[NW][16 * OSTR];

  const int lane = threadIdx.x & 63, r = lane & 15, j = lane >> 4;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int bid = blockIdx.x;
  const int qb = nqb - 1 - bid % nqb;  // the longest causal blocks start first
  const int bh = bid / nqb;
  const int h = bh % hq, b = bh / hq;
  const int hk = h / (hq / hkv);
  const int q0 = qb * 16;
  const int kend = CAUSAL ? min(lk, q0 + 16) : lk;
  const int nt = (kend + 31) >> 5;

  const float* Qh = Q + (int64_t)b * st.qb + (int64_t)h * st.qh;
  const float* Kh = K + (int64_t)b * st.kb + (int64_t)hk * st.kh;
  const float* Vh = V + (int64_t)b * st.vb + (int64_t)hk * st.vh;
  const auto rq = make_rsrc(Qh, (uint32_t)(((int64_t)(lq - 1) * st.qs + D) * 4));
  const auto rk = make_rsrc(Kh, (uint32_t)(((int64_t)(lk - 1) * st.ks + D) * 4));
  const auto rv = make_rsrc(Vh, (uint32_t)(((int64_t)(lk - 1) * st.vs + D) * 4));
  const uint32_t qs = (uint32_t)st.qs, ks = (uint32_t)st.ks, vs = (uint32_t)st.vs;

  // This lane's query row, quarter j of the head dim, pre-scaled (rows past lq read as zero).
  const int qi = q0 + r;
  float qv[QD];
#pragma unroll
  for (int i = 0; i < NQ4; ++i) {
    const uint32_t off = qi < lq ? ((uint32_t)qi * qs + j * QD + 4 * i) * 4u : kOut;
    const float4 t = buf_load16f(rq, off);
    qv[4 * i] = t.x * c;
    qv[4 * i + 1] = t.y * c;
    qv[4 * i + 2] = t.z * c;
    qv[4 * i + 3] = t.w * c;
  }

  f32x4 oacc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int v = 0; v < 4; ++v) oacc[db][v] = 0.f;
  float m = -INFINITY, l = 0.f;
  for (int t = w; t < nt; t += NW) {
    const int k0 = t * 32;
    // Key rows k0 + 16 kb + r, quarter j (rows past lk read as zero and are masked).
    float kv[2][QD];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const int kr = k0 + 16 * kb + r;
#pragma unroll
      for (int i = 0; i < NQ4; ++i) {
        const uint32_t off = kr < lk ? ((uint32_t)kr * ks + j * QD + 4 * i) * 4u : kOut;
        const float4 x = buf_load16f(rk, off);
        kv[kb][4 * i] = x.x;
        kv[kb][4 * i + 1] = x.y;
        kv[kb][4 * i + 2] = x.z;
        kv[kb][4 * i + 3] = x.w;
      }
    }
    // V[key(s)][16 db + r] for the keys key(s) = k0 + 16 (s / 4) + 4 j + s % 4 of the PV steps,
    // requested before QK^T so that they arrive during it.
    float vv[NDB][8];
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const int kr = k0 + 16 * (s >> 2) + 4 * j + (s & 3);
      if constexpr (V16) {
        static_assert(NDB == 8, "two 16-byte loads per key");
        const uint32_t off = kr < lk ? ((uint32_t)kr * vs + 8 * r) * 4u : kOut;
        const float4 x0 = buf_load16f(rv, off), x1 = buf_load16f(rv, off == kOut ? kOut : off + 16);
        vv[0][s] = x0.x; vv[1][s] = x0.y; vv[2][s] = x0.z; vv[3][s] = x0.w;
        vv[4][s] = x1.x; vv[5][s] = x1.y; vv[6][s] = x1.z; vv[7][s] = x1.w;
      } else {
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
          const uint32_t off = kr < lk ? ((uint32_t)kr * vs + 16 * db + r) * 4u : kOut;
          vv[db][s] = buf_load4f(rv, off);
        }
      }
    }
    f32x4 sacc[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int v = 0; v < 4; ++v) sacc[kb][v] = 0.f;
#pragma unroll
      for (int s = 0; s < QD; ++s) sacc[kb] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[kb][s], qv[s], sacc[kb], 0, 0, 0);
    }
    float tmax = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = k0 + 16 * kb + 4 * j + i;
        const bool ok = key < lk && (!CAUSAL || key <= qi);
        sacc[kb][i] = ok ? sacc[kb][i] : -INFINITY;
        tmax = fmaxf(tmax, sacc[kb][i]);
      }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float mn = fmaxf(m, tmax);
    const float mu = mn == -INFINITY ? 0.f : mn;  // no key seen yet: every weight is exp2(-inf) = 0
    const float alpha = fast_exp2(m - mu);
    float ps = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sacc[kb][i] = fast_exp2(sacc[kb][i] - mu);
        ps += sacc[kb][i];
      }
    ps += __shfl_xor(ps, 16, 64);
    ps += __shfl_xor(ps, 32, 64);
    l = l * alpha + ps;
    m = mn;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
#pragma unroll
      for (int v = 0; v < 4; ++v) oacc[db][v] *= alpha;
#pragma unroll
      for (int s = 0; s < 8; ++s)
        oacc[db] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv[db][s], sacc[s >> 2][s & 3], oacc[db], 0, 0, 0);
    }
  }

  // Combine the waves: O = sum_w exp2(m_w - M) O_w / sum_w exp2(m_w - M) l_w, M = max_w m_w.
  // Register i of block db holds MFMA row 4 j + i: column 16 db + 4 j + i, or with V16
  // 8 (4 j + i) + db (the eight blocks' registers i are then 32 contiguous columns).
  if (j == 0) ml_s[w][r] = make_float2(m, l);
  if constexpr (V16) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      *reinterpret_cast<float4*>(&o_s[w][r * OSTR + 32 * j + 8 * i]) =
          make_float4(oacc[0][i], oacc[1][i], oacc[2][i], oacc[3][i]);
      *reinterpret_cast<float4*>(&o_s[w][r * OSTR + 32 * j + 8 * i + 4]) =
          make_float4(oacc[4][i], oacc[5][i], oacc[6][i], oacc[7][i]);
    }
  } else {
#pragma unroll
    for (int db = 0; db < NDB; ++db)
      *reinterpret_cast<float4*>(&o_s[w][r * OSTR + 16 * db + 4 * j]) =
          make_float4(oacc[db][0], oacc[db][1], oacc[db][2], oacc[db][3]);
  }
  __syncthreads();
  constexpr int TPQ = NW * 64 / 16;  // threads per query
  constexpr int CPT = D / TPQ;       // output columns per thread
  static_assert(CPT % 4 == 0, "whole float4 columns per thread");
  const int tq = threadIdx.x / TPQ, c0 = (threadIdx.x % TPQ) * CPT;
  float2 mlw[NW];
  float M = -INFINITY;
#pragma unroll
  for (int u = 0; u < NW; ++u) {
    mlw[u] = ml_s[u][tq];
    M = fmaxf(M, mlw[u].x);
  }
  const float mu = M == -INFINITY ? 0.f : M;
  float f[NW], L = 0.f;
#pragma unroll
  for (int u = 0; u < NW; ++u) {
    f[u] = fast_exp2(mlw[u].x - mu);
    L += mlw[u].y * f[u];
  }
  const float inv = L > 0.f ? 1.0f / L : 0.f;
  const int qo = q0 + tq;
  if (qo < lq) {
    float* orow = O + (int64_t)b * st.ob + (int64_t)h * st.oh + (int64_t)qo * st.os + c0;
#pragma unroll
    for (int jj = 0; jj < CPT; jj += 4) {
      float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
      for (int u = 0; u < NW; ++u) {
        const float4 x = *reinterpret_cast<const float4*>(&o_s[u][tq * OSTR + c0 + jj]);
        a0 += x.x * f[u];
        a1 += x.y * f[u];
        a2 += x.z * f[u];
        a3 += x.w * f[u];
      }
      *reinterpret_cast<float4*>(orow + jj) = make_float4(a0 * inv, a1 * inv, a2 * inv, a3 * inv);
    }
  }
}

template <int D, int NW>
void launch_f32_dw(const float* q, const float* k, const float* v, float* o, int grid, int hq, int hkv, int lq,
                   int lk, const AttnStrides& st, float c, int nqb, bool causal) {
  if constexpr (D == 128) {
    if (aligned16(v) && st.vb % 4 == 0 && st.vh % 4 == 0 && st.vs % 4 == 0) {
      if (causal)
        flash_f32_kernel<D, true, NW, true><<<grid, NW * 64, 0, stream()>>>(q, k, v, o, hq, hkv, lq, lk, st, c, nqb);
      else
        flash_f32_kernel<D, false, NW, true><<<grid, NW * 64, 0, stream()>>>(q, k, v, o, hq, hkv, lq, lk, st, c, nqb);
      return;
    }
  }
  if (causal)
    flash_f32_kernel<D, true, NW><<<grid, NW * 64, 0, stream()>>>(q, k, v, o, hq, hkv, lq, lk, st, c, nqb);
  else
    flash_f32_kernel<D, false, NW><<<grid, NW * 64, 0, stream()>>>(q, k, v, o, hq, hkv, lq, lk, st, c, nqb);
}

// Eight-wave workgroups (two waves per SIMD, the tiles of a block over twice the waves): always at
// head_dim 128 (with 16-byte V loads, grids of 512 and 2048 workgroups too: B=2, 16/8 heads, S=512
// 53.3 -> 50.6 us; B=4, S=1024 347.5 -> 326.3 us), and at 64 when the grid leaves CUs without a
// second workgroup.
template <int D>
void launch_f32_d(const float* q, const float* k, const float* v, float* o, int grid, int hq, int hkv, int lq, int lk,
                  const AttnStrides& st, float c, int nqb, bool causal) {
  if constexpr (D == 64 || D == 128) {
    if (D == 128 || grid < 2 * cu_count()) {
      launch_f32_dw<D, 8>(q, k, v, o, grid, hq, hkv, lq, lk, st, c, nqb, causal);
      return;
    }
  }
  launch_f32_dw<D, kF32Waves>(q, k, v, o, grid, hq, hkv, lq, lk, st, c, nqb, causal);
}

}  // namespace

namespace kh {

bool flash_f32_supported(const void* q, const void* k, const void* v, const void* o, int64_t lq, int64_t lk, int d,
                         const AttnStrides& st) {
  if (!(d == 32 || d == 64 || d == 96 || d == 128)) return false;
  if (!aligned16(q) || !aligned16(k) || !aligned16(o) || (reinterpret_cast<uintptr_t>(v) & 3u) != 0) return false;
  const int64_t vec[] = {st.qb, st.qh, st.qs, st.kb, st.kh, st.ks, st.ob, st.oh, st.os};
  for (int64_t s : vec)
    if (s < 0 || s % 4 != 0) return false;  // 16-byte q / k loads and o stores
  if (st.vb < 0 || st.vh < 0 || st.vs < 0) return false;
  // Offsets within one head are 32-bit byte offsets.
  const int64_t lim = int64_t(1) << 31;
  return (lq * st.qs + d) * 4 < lim && (lk * st.ks + d) * 4 < lim && (lk * st.vs + d) * 4 < lim;
}

int launch_flash_f32(const void* q, const void* k, const void* v, void* o, int batch, int hq, int hkv, int lq, int lk,
                     int d, const AttnStrides& st, float scale, bool causal) {
  const int nqb = (lq + 31) / 32;
  const int64_t grid = (int64_t)batch * hq * nqb;
  KH_REQUIRE(grid <= INT32_MAX, "kh_flash_attention: grid too large");
  const float c = scale * kLog2e;
  const float *Q = (const float*)q, *K = (const float*)k, *V = (const float*)v;
  float* Out = (float*)o;
  if (d == 128 && grid < cu_count()) {
    // fewer 32-query blocks than CUs: 16-query blocks (twice the workgroups)
    const int nqb16 = (lq + 15) / 16;
    const int grid16 = (int)(grid / nqb * nqb16);
    const bool v16 = aligned16(v) && st.vb % 4 == 0 && st.vh % 4 == 0 && st.vs % 4 == 0;
#define KH_Q16(CAUSAL, V16) \
  flash_f32_q16_kernel<128, CAUSAL, kQ16Waves, V16><<<grid16, kQ16Waves * 64, 0, stream()>>>(Q, K, V, Out, hq, hkv, lq, lk, st, c, nqb16)
    if (causal) {
      if (v16) KH_Q16(true, true);
      else KH_Q16(true, false);
    } else {
      if (v16) KH_Q16(false, true);
      else KH_Q16(false, false);
    }
#undef KH_Q16
    KH_CHECK_LAUNCH();
    return KH_OK;
  }
  switch (d) {
    case 32: launch_f32_d<32>(Q, K, V, Out, (int)grid, hq, hkv, lq, lk, st, c, nqb, causal); break;
    case 64: launch_f32_d<64>(Q, K, V, Out, (int)grid, hq, hkv, lq, lk, st, c, nqb, causal); break;
    case 96: launch_f32_d<96>(Q, K, V, Out, (int)grid, hq, hkv, lq, lk, st, c, nqb, causal); break;
    default: launch_f32_d<128>(Q, K, V, Out, (int)grid, hq, hkv, lq, lk, st, c, nqb, causal); break;
  }
  KH_CHECK_LAUNCH();
  return KH_OK;
}

}  // namespace kh
