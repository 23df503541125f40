// One-row projection (decode GEMV) building blocks shared by the kernels of gemm.hip and the
// fused decode kernels: the epilogue, the prologues that form the activation row x' in LDS, and
// the weight-row streamer.  Header-only device code (each translation unit gets its own copy).
#pragma once

#include <type_traits>

#include "common.h"

namespace kh {
namespace gemv {

// out = alpha * acc + beta * cin[m, n] (+ bias[n]) -- the matmul epilogue
// (packages/backend-webgpu/src/kernels/matrix/builder.ts:152-218).
template <typename TO>
__device__ __forceinline__ float epilogue(float acc, float alpha, float beta, const TO* cin, int64_t ldcin,
                                          const TO* bias, int64_t m, int64_t n) {
  float v = alpha * acc;
  if (cin != nullptr && beta != 0.f) v += beta * Elem<TO>::load(cin, m * ldcin + n);
  if (bias != nullptr) v += Elem<TO>::load(bias, n);
  return v;
}

constexpr int PRO_NONE = 0, PRO_RMSNORM = 1, PRO_SILU_MUL = 2, PRO_SILU_MUL_IL = 3, PRO_ATTN_MERGE = 4;
constexpr int kAttnMergeMaxChunks = 8;   // split-K chunks the attention-merge prologue accepts
constexpr int GV_CHUNK = 512;  // columns per wave-wide 16-byte load (64 lanes x 8 bf16)

// EX (exact): x' keeps the fp32 value of every element instead of rounding it to bf16, and the
// inputs of prologues 0, 2 and 3 (x, x2) are fp32 instead of bf16 -- the float32 activations of
// the reference's arithmetic.
template <int PRO, bool EX = false>
__device__ __forceinline__ void gemv_prologue(float* xs, const void* x, const void* x2v, const uint16_t* nw,
                                              float eps, int K, int kpad, const AttnMerge& am) {
  const int tid = threadIdx.x;
  // x' as stored by the producer: rounded to bf16, or kept whole (EX)
  auto rnd = [](float v) { return EX ? v : round_bf16(v); };
  using TX = std::conditional_t<EX, float, uint16_t>;
  if constexpr (PRO == PRO_ATTN_MERGE) {
    // Thread t merges columns 8 (t mod 16) .. + 7 of head t / 16 (then t + 256, ...): the chunks'
    // (m, l, o) combined with weights exp(m_c - M), M the largest chunk max.  Up to kAttnMergeMaxChunks
    // chunks, every load issued before any math (indices past the last chunk clamped, weight 0).
    constexpr int MC = kAttnMergeMaxChunks;
    const float* po = (const float*)x;
    const float2* pml = reinterpret_cast<const float2*>(po + (int64_t)am.hq * am.max_chunks * 128);
    const int p = *am.position;
    const int L = p + 1 < 0 ? 0 : (p + 1 > am.max_len ? am.max_len : p + 1);
    const int nch = (L + am.chunk - 1) / am.chunk;
    for (int g = tid; g < (kpad >> 3); g += blockDim.x) {
      const int h = g >> 4, d0 = (g & 15) * 8;
      float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      if (h < am.hq && nch > 0) {
        float2 ml[MC];
        float4 oa[MC], ob[MC];
#pragma unroll
        for (int c = 0; c < MC; ++c) {
          const int cc = min(c, nch - 1);
          ml[c] = pml[(int64_t)h * am.max_chunks + cc];
          const float4* o4 = reinterpret_cast<const float4*>(po + ((int64_t)h * am.max_chunks + cc) * 128 + d0);
          oa[c] = o4[0];
          ob[c] = o4[1];
        }
        if (nch > 0) {
          float M = -INFINITY;
#pragma unroll
          for (int c = 0; c < MC; ++c)
            if (c < nch) M = fmaxf(M, ml[c].x);
          const float mu = M == -INFINITY ? 0.f : M;
          float Ls = 0.f, t[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int c = 0; c < MC; ++c) {
            const float f = c < nch ? __expf(ml[c].x - mu) : 0.f;
            Ls += ml[c].y * f;
            t[0] += oa[c].x * f; t[1] += oa[c].y * f; t[2] += oa[c].z * f; t[3] += oa[c].w * f;
            t[4] += ob[c].x * f; t[5] += ob[c].y * f; t[6] += ob[c].z * f; t[7] += ob[c].w * f;
          }
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] = rnd(Ls > 0.f ? t[e] / Ls : 0.f);
        }
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) xs[g * 8 + e] = (g * 8 + e) < K ? v[e] : 0.f;
    }
  } else if constexpr (PRO == PRO_RMSNORM) {
    // Rows of up to 8 * blockDim elements stay in registers between the two passes.
    constexpr int PR = 8;
    __shared__ float red[4];
    const float* xf = (const float*)x;
    const bool in_regs = kpad <= PR * (int)blockDim.x;
    float xv[PR], wv[PR];
    float ss = 0.f;
    if (in_regs) {
#pragma unroll
      for (int j = 0; j < PR; ++j) {
        const int i = tid + j * blockDim.x;
        xv[j] = i < K ? xf[i] : 0.f;
        wv[j] = i < K ? bf16_bits_to_f32(nw[i]) : 0.f;
      }
#pragma unroll
      for (int j = 0; j < PR; ++j) ss += xv[j] * xv[j];
    } else {
      for (int i = tid; i < K; i += blockDim.x) ss += xf[i] * xf[i];
    }
    ss = wave_sum(ss);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    ss = red[0] + red[1] + red[2] + red[3];
    const float inv = 1.0f / sqrtf(ss / (float)K + eps);
    if (in_regs) {
#pragma unroll
      for (int j = 0; j < PR; ++j) {
        const int i = tid + j * blockDim.x;
        if (i < kpad) xs[i] = i < K ? rnd((xv[j] * inv) * wv[j]) : 0.f;
      }
    } else {
      for (int i = tid; i < kpad; i += blockDim.x)
        xs[i] = i < K ? rnd((xf[i] * inv) * bf16_bits_to_f32(nw[i])) : 0.f;
    }
  } else if constexpr (PRO == PRO_SILU_MUL) {
    const TX* g = (const TX*)x;
    const TX* x2 = (const TX*)x2v;
    for (int i = tid; i < kpad; i += blockDim.x)
      xs[i] = i < K ? rnd(silu_ref(Elem<TX>::load(g, i)) * Elem<TX>::load(x2, i)) : 0.f;
  } else if constexpr (PRO == PRO_SILU_MUL_IL) {
    const TX* gu = (const TX*)x;
    for (int i = tid; i < kpad; i += blockDim.x) {
      const int gi = 16 * (i >> 3) + (i & 7);
      xs[i] = i < K ? rnd(silu_ref(Elem<TX>::load(gu, gi)) * Elem<TX>::load(gu, gi + 8)) : 0.f;
    }
  } else {
    const TX* xb = (const TX*)x;
    for (int i = tid; i < kpad; i += blockDim.x) xs[i] = i < K ? Elem<TX>::load(xb, i) : 0.f;
  }
  __syncthreads();
}

// The weight-streaming part of the one-row projection: wave w of workgroup b owns row groups
// n0 = (b * waves + w) * U, then n0 + stride, ...; each lane accumulates 8 columns of every 512-column
// chunk of U rows, in chunk order, then a wave sum gives each row's dot product with x' (in LDS).
// issue_first() requests the first batch of weights (it may run long before x' exists); run()
// streams the rest with the next batch always in flight.  Every caller goes through this code, so
// a row's sum is formed the same way in every kernel that uses it.
// PAIR8 (U = 2, SwiGLU): the weight interleaves gate and up rows in blocks of 8 (rows 16i .. 16i+7
// gate rows 8i .. 8i+7, rows 16i+8 .. 16i+15 the matching up rows); row group q = n0 / 2 is gate row
// 16 (q / 8) + q % 8 and its up row 8 later, and the output is feature q:
// bf16(silu(bf16(gate)) * bf16(up)), the value the silu * mul prologue of the next projection forms
// (EX: silu(gate) * up of the fp32 sums, unrounded).
template <int U, bool PAIR8 = false, bool EX = false>
struct GemvRows {
  static_assert(!PAIR8 || U == 2, "paired gate/up rows take two rows per group");
  static constexpr int CB = 8 / U;  // 16-byte loads in flight per row per lane
  __amdgpu_buffer_rsrc_t rsrc;
  int64_t ldw, n0, stride;
  uint32_t w_bytes;
  int N, K, nch, lane;
  uint4 wv[U][CB];

  __device__ __forceinline__ void init(const uint16_t* W, int64_t ldw_, uint32_t w_bytes_, int N_, int K_, int nch_,
                                       int64_t first_wave, int64_t total_waves) {
    rsrc = make_rsrc(W, w_bytes_);
    ldw = ldw_;
    w_bytes = w_bytes_;
    N = N_;
    K = K_;
    nch = nch_;
    lane = threadIdx.x & 63;
    n0 = first_wave * U;
    stride = total_waves * U;
  }
  // Weight loads of batch (row group n, chunks [c0, c0 + CB)); columns past K (row padding when
  // ldw > K) and rows past N read as zero (offset w_bytes is out of range).
  // Weight row u of row group n.
  static __device__ __forceinline__ int64_t row_of(int64_t n, int u) {
    if constexpr (PAIR8) {
      const int64_t q = n >> 1;
      return 16 * (q >> 3) + (q & 7) + 8 * u;
    } else {
      return n + u;
    }
  }
  __device__ __forceinline__ void issue(int64_t n, int c0) {
#pragma unroll
    for (int cc = 0; cc < CB; ++cc)
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = c0 + cc;
        const int k = c * GV_CHUNK + lane * 8;
        const uint32_t off = k < K ? (uint32_t)((row_of(n, u) * ldw + k) * 2) : w_bytes;
        wv[u][cc] = c < nch ? buf_load16_nt(rsrc, off) : make_uint4(0, 0, 0, 0);  // every weight byte once
      }
  }
  __device__ __forceinline__ void issue_first() {
    if (n0 < N) issue(n0, 0);
  }
  template <typename TO>
  __device__ __forceinline__ void run(const float* xs, TO* C, const TO* cin, const TO* bias, float alpha, float beta) {
    for (; n0 < N; n0 += stride) {
      float acc[U];
#pragma unroll
      for (int u = 0; u < U; ++u) acc[u] = 0.f;
      for (int c0 = 0; c0 < nch; c0 += CB) {
        uint4 cur[U][CB];
#pragma unroll
        for (int cc = 0; cc < CB; ++cc)
#pragma unroll
          for (int u = 0; u < U; ++u) cur[u][cc] = wv[u][cc];
        // prefetch the next batch: the rest of this row group, else the next row group
        if (c0 + CB < nch)
          issue(n0, c0 + CB);
        else if (n0 + stride < N)
          issue(n0 + stride, 0);
#pragma unroll
        for (int cc = 0; cc < CB; ++cc) {
          if (c0 + cc < nch) {
            const float4* xp = reinterpret_cast<const float4*>(xs + (c0 + cc) * GV_CHUNK + lane * 8);
            const float4 xa = xp[0], xb = xp[1];
#pragma unroll
            for (int u = 0; u < U; ++u) {
              const uint4 q = cur[u][cc];
              float s = acc[u];
              s += lo_bf16(q.x) * xa.x;
              s += hi_bf16(q.x) * xa.y;
              s += lo_bf16(q.y) * xa.z;
              s += hi_bf16(q.y) * xa.w;
              s += lo_bf16(q.z) * xb.x;
              s += hi_bf16(q.z) * xb.y;
              s += lo_bf16(q.w) * xb.z;
              s += hi_bf16(q.w) * xb.w;
              acc[u] = s;
            }
          }
        }
      }
      if constexpr (PAIR8) {
        const float gsum = wave_sum(acc[0]), usum = wave_sum(acc[1]);
        if (lane == 0) {
          if constexpr (EX)
            Elem<TO>::store(C, n0 >> 1, silu_ref(gsum) * usum);
          else
            Elem<TO>::store(C, n0 >> 1, silu_ref(round_bf16(gsum)) * round_bf16(usum));
        }
      } else {
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const float sum = wave_sum(acc[u]);
          const int64_t n = n0 + u;
          if (lane == 0 && n < N) Elem<TO>::store(C, n, epilogue<TO>(sum, alpha, beta, cin, 0, bias, 0, n));
        }
      }
    }
  }
};

}  // namespace gemv
}  // namespace kh
