// On-device sampling of one token from a row of logits: temperature, top-k, top-p (nucleus), and a
// draw with a counter-based random number -- the sample() of Kandle's model-utils, without the
// logits readback and the JavaScript sort (reference: packages/model-utils/src/sampling/index.ts).
//
// Semantics, step by step as the reference (sampling/index.ts):
//   order   token ids sorted by logit, descending, stable (ties keep the lower id first)  (:132)
//   scale   s_i = f32(logit_i * (1 / T)), the product in f64 (JavaScript numbers)             (:169-176)
//   softmax e_i = f32(exp(f64(s_i) - f64(max s)));  Z = sum_i e_i in f64;  p_i = f32(e_i / Z) (:268-291)
//   top-k   keep the first K ids of the order (K = vocab when top_k <= 0 or >= vocab)      (:183-194)
//   top-p   keep the order's prefix up to the first position where the f64 running sum of p
//           reaches top_p (only when top_p < 1), within the top-k prefix                  (:197-215)
//   norm    q_i = f32(p_i / P) over the kept ids, P = f64 sum of their p (when P > 0)     (:218-223)
//   draw    r in [0, 1); the first id i, in id order, whose f64 running sum of q exceeds r;
//           if none, the last id with q > 0                                               (:294-311)
//   result  token, log(q_token + 1e-10), and the first display_k ids of the order with q  (:228-243)
// Greedy (do_sample = 0, :138-160): the token is the first id of the order, and the reported
// probabilities are softmaxCPU(logits, T) unfiltered: e_i = f32(exp((f64(l_i) - f64(max l)) * (1 / T))),
// the temperature applied to the f64 difference rather than to the stored logit.
// Logits equal to -0.0 sort as +0.0 (the reference's comparator b - a treats them as equal).
// The reference draws r with Math.random(); here r = bits(philox4x32-10(seed, counter)) / 2^32 at 24
// bits (word 0 >> 8, times 2^-24), with the counter read from device memory so a generation loop can
// advance it on the device.
//
// Running sums.  Sums over a kept set of at most 1024 ids (top-k) run sequentially in f64 in the
// reference's order, as the JavaScript loops do.  Sums over a larger set (the unfiltered draw, top-p
// without top-k) run in exact 2^-62 fixed point, in any order; they differ from the reference's
// sequential f64 sums by rounding only (about 1e-16 per term).  Z and P over large sets are f64 tree
// sums in a fixed order, so every result is deterministic.
//
// Two implementations give the same results.  The selection path (greedy, top-k <= 1024 with or
// without top-p, the unfiltered draw; display_k <= 1024) builds only the needed prefix of the order
// by bitonic selection and runs under graph capture.  Top-p without top-k may cut anywhere in the
// order, so it (and longer prefixes) takes the full-sort path: rocPRIM's stable radix sort, then
// the top-p cut and the draw found from the fixed-point block sums; rocPRIM may clear its temporary
// storage with memsets, so that path refuses to run under stream capture.
#include <rocprim/device/device_radix_sort.hpp>

#include "common.h"

using namespace kh;

namespace {

// ---- Philox4x32-10 (Salmon, Moraes, Dror, Shaw: "Parallel random numbers: as easy as 1, 2, 3",
// SC'11): ten rounds of two 32x32->64 multiplies, key bumped by the Weyl constants between rounds.
__device__ __forceinline__ void philox4x32_10(uint32_t (&c)[4], uint32_t k0, uint32_t k1) {
  constexpr uint32_t M0 = 0xD2511F53u, M1 = 0xCD9E8D57u, W0 = 0x9E3779B9u, W1 = 0xBB67AE85u;
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    if (r > 0) {
      k0 += W0;
      k1 += W1;
    }
    const uint64_t p0 = (uint64_t)M0 * c[0], p1 = (uint64_t)M1 * c[2];
    const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c[1] ^ k0;
    const uint32_t n2 = (uint32_t)(p0 >> 32) ^ c[3] ^ k1;
    c[0] = n0;
    c[1] = (uint32_t)p1;
    c[2] = n2;
    c[3] = (uint32_t)p0;
  }
}

__global__ void philox_kernel(uint64_t seed, const uint32_t* __restrict__ ctr, int64_t n, uint32_t* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  uint32_t c[4] = {ctr[4 * i], ctr[4 * i + 1], ctr[4 * i + 2], ctr[4 * i + 3]};
  philox4x32_10(c, (uint32_t)seed, (uint32_t)(seed >> 32));
#pragma unroll
  for (int j = 0; j < 4; ++j) out[4 * i + j] = c[j];
}

constexpr int kThreads = 256;

__device__ __forceinline__ double block_sum_f64(double v, double* red) {
  // deterministic: fixed shuffle tree inside each wave, then the waves in order
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  double t = 0.0;
  for (int w = 0; w < (int)(blockDim.x >> 6); ++w) t += red[w];
  __syncthreads();
  return t;
}

// ids 0..n-1 and the sort keys: the logits with -0.0 replaced by +0.0, so that the radix sort (which
// orders bit patterns) keeps the two zeros in id order as the reference's comparator does.
__global__ void iota_keys_kernel(const float* __restrict__ logits, int n, float* __restrict__ keys,
                                 int32_t* __restrict__ v) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) {
    const float x = logits[i];
    keys[i] = x == 0.f ? 0.f : x;
    v[i] = i;
  }
}

// Sampling: s = f32(logit * (1 / T)) with the product in f64 (T == 1: s = logit), then
// e (sorted order) = f32(exp(f64(s_j) - f64(s_0))).  Greedy: e = f32(exp((f64(l_j) - f64(l_0)) * (1 / T))).
// Per-block f64 sums of e.
__device__ __forceinline__ float scaled_logit(float x, double inv_t) { return (float)((double)x * inv_t); }
__global__ __launch_bounds__(kThreads) void exp_kernel(const float* __restrict__ sorted_logits, int n, double inv_t,
                                                       int greedy, float* __restrict__ e, double* __restrict__ part) {
  __shared__ double red[kThreads / 64];
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  const float x0 = sorted_logits[0];
  double v = 0.0;
  if (i < n) {
    const float x = sorted_logits[i];
    const double arg = greedy ? ((double)x - (double)x0) * inv_t
                              : (double)scaled_logit(x, inv_t) - (double)scaled_logit(x0, inv_t);
    const float ef = (float)exp(arg);
    e[i] = ef;
    v = (double)ef;
  }
  v = block_sum_f64(v, red);
  if (threadIdx.x == 0) part[blockIdx.x] = v;
}

// One block: total of part[0..nb) in f64 (fixed order), written to *out.
__global__ __launch_bounds__(kThreads) void final_sum_kernel(const double* __restrict__ part, int nb,
                                                             double* __restrict__ out) {
  __shared__ double red[kThreads / 64];
  double v = 0.0;
  for (int i = threadIdx.x; i < nb; i += blockDim.x) v += part[i];
  v = block_sum_f64(v, red);
  if (threadIdx.x == 0) *out = v;
}

inline size_t align256(size_t b) { return (b + 255) & ~size_t(255); }

int g_sample_path = 0;   // 0: selection path where it applies; 1: always the full sort (kh_sample_set_path)

// ---- selection path: the sorted prefix of length m <= kMaxPrefix without sorting the row --------
//
// Each id gets a 64-bit key whose descending order is the reference's order: the logit mapped to an
// order-preserving uint32 in the high word (-0.0 as +0.0), 0xffffffff - id in the low word (lower id
// first among equal logits).  Keys are distinct, so any sort yields the same order.  A block sorts
// 1024 or 4096 keys (bitonic, in registers) and keeps its first m; blocks of those survivors are reduced the same
// way until one block remains: its first m keys are the first m ids of the order.

// Selection blocks sort 1024 keys with 256 threads while m <= 256 (many blocks, short sorts), and
// 4096 keys with 1024 threads for longer prefixes; each level shrinks the key count 4x or more.
constexpr int kSelSmall = 1024, kSelSmallThreads = 256;
constexpr int kSelLarge = 4096, kSelLargeThreads = 1024;
constexpr int kMaxPrefix = 1024;    // longest prefix the selection path produces
constexpr int kIdThreads = 512;     // id-order passes: ids per block

__device__ __forceinline__ uint32_t order_bits(float x) {
  const uint32_t b = __float_as_uint(x == 0.f ? 0.f : x);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float order_value(uint32_t u) {
  return __uint_as_float((u & 0x80000000u) ? (u & 0x7fffffffu) : ~u);
}
__device__ __forceinline__ uint64_t order_key(float x, int id) {
  return ((uint64_t)order_bits(x) << 32) | (uint64_t)(0xffffffffu - (uint32_t)id);
}
__device__ __forceinline__ int key_id(uint64_t k) { return (int)(0xffffffffu - (uint32_t)k); }
__device__ __forceinline__ float key_logit(uint64_t k) { return order_value((uint32_t)(k >> 32)); }

// x of lane (lane ^ X) within the wave.  Distances 1, 2, 4 and 8 stay inside a 16-lane row and use
// DPP moves (quad_perm, row_half_mirror then a quad reversal, row_ror:8), which do not occupy the
// LDS crossbar; 16 and 32 use ds_bpermute.
template <int X>
__device__ __forceinline__ uint32_t lane_xor_u32(uint32_t x) {
  if constexpr (X == 1) {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)x, (int)x, 0xB1, 0xF, 0xF, false);   // quad_perm [1,0,3,2]
  } else if constexpr (X == 2) {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)x, (int)x, 0x4E, 0xF, 0xF, false);   // quad_perm [2,3,0,1]
  } else if constexpr (X == 4) {
    // row_half_mirror: lane i reads 7 - i (within 8); then quad_perm [3,2,1,0]: lane i reads
    // i ^ 3; composed, lane i reads 7 - (i ^ 3) = i ^ 4 (within 8)
    const int h = __builtin_amdgcn_update_dpp((int)x, (int)x, 0x141, 0xF, 0xF, false);
    return (uint32_t)__builtin_amdgcn_update_dpp(h, h, 0x1B, 0xF, 0xF, false);
  } else if constexpr (X == 8) {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)x, (int)x, 0x128, 0xF, 0xF, false);  // row_ror:8
  } else {
    return (uint32_t)__shfl_xor((int)x, X, 64);
  }
}

template <int X>
__device__ __forceinline__ uint64_t lane_xor_u64(uint64_t x) {
  return ((uint64_t)lane_xor_u32<X>((uint32_t)(x >> 32)) << 32) | lane_xor_u32<X>((uint32_t)x);
}

// One compare-exchange against the partner value p: the lower index of the pair keeps the larger
// value when the pair ends larger-first, the upper index the smaller (branch-free selects).
template <bool DESC>
__device__ __forceinline__ uint64_t cx_keep(uint64_t a, uint64_t p, int i, int j, int k) {
  const bool keep_max = ((i & j) == 0) == (((i & k) == 0) == DESC);
  return ((a > p) == keep_max) ? a : p;   // one 64-bit compare, two selects
}

// The in-register and lane-shuffle steps of one (k, j) stage.
template <int E, int T, bool DESC, int K, int J>
__device__ __forceinline__ void bitonic_step(uint64_t (&v)[E], uint64_t* lds, int t, int& half) {
  if constexpr (J < E) {
#pragma unroll
    for (int e = 0; e < E; ++e) {
      if (e & J) continue;
      const bool up = (((t * E + e) & K) == 0) == DESC;   // the pair ends larger-first
      const uint64_t a = v[e], b = v[e | J];
      const bool swap = (a < b) == up;
      v[e] = swap ? b : a;
      v[e | J] = swap ? a : b;
    }
  } else if constexpr (J < 64 * E) {
    uint64_t p[E];
#pragma unroll
    for (int e = 0; e < E; ++e) p[e] = lane_xor_u64<J / E>(v[e]);
#pragma unroll
    for (int e = 0; e < E; ++e) v[e] = cx_keep<DESC>(v[e], p[e], t * E + e, J, K);
  } else {
    constexpr int N = E * T;
    uint64_t* sb = lds + half * N;
#pragma unroll
    for (int e = 0; e < E; ++e) sb[t * E + e] = v[e];
    __syncthreads();
    uint64_t p[E];
#pragma unroll
    for (int e = 0; e < E; ++e) p[e] = sb[(t * E + e) ^ J];
    half ^= 1;
#pragma unroll
    for (int e = 0; e < E; ++e) v[e] = cx_keep<DESC>(v[e], p[e], t * E + e, J, K);
  }
}

template <int E, int T, bool DESC, int K, int J>
__device__ __forceinline__ void bitonic_merge(uint64_t (&v)[E], uint64_t* lds, int t, int& half) {
  bitonic_step<E, T, DESC, K, J>(v, lds, t, half);
  if constexpr (J > 1) bitonic_merge<E, T, DESC, K, J / 2>(v, lds, t, half);
}

template <int E, int T, bool DESC, int K>
__device__ __forceinline__ void bitonic_phases(uint64_t (&v)[E], uint64_t* lds, int t, int& half) {
  bitonic_merge<E, T, DESC, K, K / 2>(v, lds, t, half);
  if constexpr (K < E * T) bitonic_phases<E, T, DESC, K * 2>(v, lds, t, half);
}

// Bitonic sort of N = E * T distinct 64-bit values, descending when DESC, by T threads holding E
// values each in registers (element i = t * E + e in v[e]).  Partners within a thread are swapped in
// registers, partners within a wave exchanged across lanes, and only partners in other waves
// (j >= 64 E) go through LDS (lds: 2 N values; consecutive LDS steps alternate halves, so one
// barrier per step suffices).  When N <= 64 E no barrier is executed and a single wave may call it.
template <int E, int T, bool DESC>
__device__ __forceinline__ void bitonic_sort(uint64_t (&v)[E], uint64_t* lds) {
  int half = 0;
  bitonic_phases<E, T, DESC, 2>(v, lds, (int)(threadIdx.x % T), half);
}

// out[blockIdx.x * m + t] (t < m): the m largest keys of chunk blockIdx.x (CHUNK keys), in order.
// The chunk is logits[base, base + CHUNK) (FROM_LOGITS) or in[base, base + CHUNK); missing entries
// are key 0, which is below every real key (a real key's low word is 0xffffffff - id > 0).
template <bool FROM_LOGITS, int CHUNK, int THREADS>
__global__ __launch_bounds__(THREADS) void select_kernel(const float* __restrict__ logits,
                                                         const uint64_t* __restrict__ in, int n, int m,
                                                         uint64_t* __restrict__ out) {
  constexpr int E = CHUNK / THREADS;
  __shared__ uint64_t s[2 * CHUNK];
  const int base = blockIdx.x * CHUNK + threadIdx.x * E;
  uint64_t v[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int i = base + e;
    v[e] = 0;
    if (i < n) v[e] = FROM_LOGITS ? order_key(logits[i], i) : in[i];
  }
  bitonic_sort<E, THREADS, true>(v, s);
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int r = threadIdx.x * E + e;
    if (r < m) out[(size_t)blockIdx.x * m + r] = v[e];
  }
}

// e_i in id order (stored when e != nullptr) and per-block f64 sums of e, with the largest logit
// taken from the selected prefix (top[0]).
__global__ __launch_bounds__(kIdThreads) void exp_ids_kernel(const float* __restrict__ logits, int n,
                                                             const uint64_t* __restrict__ top, double inv_t,
                                                             int greedy, float* __restrict__ e,
                                                             double* __restrict__ part) {
  __shared__ double red[kIdThreads / 64];
  const int i = blockIdx.x * kIdThreads + threadIdx.x;
  const float x0 = key_logit(top[0]);
  double v = 0.0;
  if (i < n) {
    const float x = logits[i];
    const double arg = greedy ? ((double)x - (double)x0) * inv_t
                              : (double)scaled_logit(x, inv_t) - (double)scaled_logit(x0, inv_t);
    const float ef = (float)exp(arg);
    if (e) e[i] = ef;
    v = (double)ef;
  }
  v = block_sum_f64(v, red);
  if (threadIdx.x == 0) part[blockIdx.x] = v;
}

// Sum of part[0..nb) in a fixed order (the same in every block that calls it).
__device__ __forceinline__ double sum_parts(const double* __restrict__ part, int nb, double* red) {
  double v = 0.0;
  for (int i = threadIdx.x; i < nb; i += blockDim.x) v += part[i];
  return block_sum_f64(v, red);
}

// Top-k (with or without top-p) and greedy on the selected prefix, one block of kMaxPrefix threads.
// Every sum the reference runs sequentially is run sequentially here, in the reference's order:
// the top-p running sum over the order, the kept mass and the draw over ids (ids outside the kept
// set add exact zeros in the reference).  Only the softmax total Z is a tree sum.
__global__ __launch_bounds__(kMaxPrefix) void finish_prefix_kernel(
    const uint64_t* __restrict__ top, int m, const double* __restrict__ part, int nb, double inv_t, int greedy,
    int k_eff, double top_p, uint64_t seed, const int32_t* __restrict__ counter, int display_k,
    int32_t* __restrict__ token, float* __restrict__ logprob, int32_t* __restrict__ disp_ids,
    float* __restrict__ disp_p) {
  __shared__ double red[kMaxPrefix / 64];
  __shared__ float p_s[kMaxPrefix];
  __shared__ int id_s[kMaxPrefix];
  __shared__ uint64_t by_id[kMaxPrefix];
  __shared__ uint64_t sort_lds[2 * kMaxPrefix];
  __shared__ float v_s[kMaxPrefix];
  __shared__ int cut_s;
  __shared__ double P_s;
  const int t = threadIdx.x;
  const double Z = sum_parts(part, nb, red);
  const float x0 = key_logit(top[0]);
  if (t < m) {
    const uint64_t k = top[t];
    const float x = key_logit(k);
    const double arg = greedy ? ((double)x - (double)x0) * inv_t
                              : (double)scaled_logit(x, inv_t) - (double)scaled_logit(x0, inv_t);
    const float ef = (float)exp(arg);
    p_s[t] = (float)((double)ef / Z);
    id_s[t] = key_id(k);
  }
  __syncthreads();
  if (greedy) {
    if (t == 0) {
      *token = id_s[0];
      if (logprob) *logprob = (float)log((double)p_s[0] + 1e-10);
    }
    if (t < display_k) {
      if (disp_ids) disp_ids[t] = id_s[t];
      if (disp_p) disp_p[t] = p_s[t];
    }
    return;
  }
  if (t == 0) {
    int cut = k_eff;
    if (top_p < 1.0) {
      double cum = 0.0;
#pragma unroll 8
      for (int j = 0; j < k_eff; ++j) {
        cum += (double)p_s[j];
        if (cum >= top_p) {
          cut = j + 1;
          break;
        }
      }
    }
    cut_s = cut;
  }
  __syncthreads();
  const int cut = cut_s;
  // the kept positions in id order: by_id[j] = (id << 32) | position, ascending; the rest after
  {
    uint64_t kv[1] = {t < cut ? (((uint64_t)(uint32_t)id_s[t] << 32) | (uint32_t)t) : ~0ull};
    if (cut <= 64) {
      if (t < 64) bitonic_sort<1, 64, false>(kv, nullptr);
    } else {
      bitonic_sort<1, kMaxPrefix, false>(kv, sort_lds);
    }
    by_id[t] = kv[0];
  }
  __syncthreads();
  // p of the kept ids in id order, summed sequentially (the reference's probs.reduce)
  if (t < cut) v_s[t] = p_s[(uint32_t)by_id[t]];
  __syncthreads();
  if (t == 0) {
    double P = 0.0;
#pragma unroll 8
    for (int j = 0; j < cut; ++j) P += (double)v_s[j];
    P_s = P;
  }
  __syncthreads();
  const double P = P_s;
  float q = 0.f;
  if (t < cut) q = P > 0.0 ? (float)((double)p_s[t] / P) : p_s[t];
  __syncthreads();   // every p_s read above is done before q replaces it
  if (t < m) p_s[t] = t < cut ? q : 0.f;
  __syncthreads();
  if (t < cut) v_s[t] = p_s[(uint32_t)by_id[t]];   // q of the kept ids in id order
  __syncthreads();
  if (t == 0) {
    uint32_t c[4] = {(uint32_t)*counter, 0u, 0u, 0u};
    philox4x32_10(c, (uint32_t)seed, (uint32_t)(seed >> 32));
    const double r = (double)(c[0] >> 8) * (1.0 / 16777216.0);
    int pick = -1;
    double cum = 0.0;
#pragma unroll 8
    for (int j = 0; j < cut; ++j) {
      cum += (double)v_s[j];
      if (r < cum) {
        pick = j;
        break;
      }
    }
    if (pick < 0)   // the last kept id with q > 0
      for (int j = cut - 1; j >= 0; --j)
        if (v_s[j] > 0.f) {
          pick = j;
          break;
        }
    // nothing kept with q > 0: id 0, whose q is then 0 (id 0 is kept only with q == 0)
    const int pos = pick >= 0 ? (int)(uint32_t)by_id[pick] : -1;
    *token = pos >= 0 ? id_s[pos] : 0;
    if (logprob) *logprob = (float)log((double)(pos >= 0 ? p_s[pos] : 0.f) + 1e-10);
  }
  if (t < display_k) {
    if (disp_ids) disp_ids[t] = id_s[t];
    if (disp_p) disp_p[t] = p_s[t];
  }
}

// No filter (top_k off, top_p >= 1): every id is kept, so the renormalisation and the draw run
// over the whole row in id order.
// p_i = f32(e_i / Z) in place, per-block f64 sums of p.
__global__ __launch_bounds__(kIdThreads) void prob_ids_kernel(float* e, int n, const double* __restrict__ zpart,
                                                              int nb, double* __restrict__ part) {
  __shared__ double red[kIdThreads / 64];
  const double Z = sum_parts(zpart, nb, red);
  const int i = blockIdx.x * kIdThreads + threadIdx.x;
  double v = 0.0;
  if (i < n) {
    const float p = (float)((double)e[i] / Z);
    e[i] = p;
    v = (double)p;
  }
  v = block_sum_f64(v, red);
  if (threadIdx.x == 0) part[blockIdx.x] = v;
}

// q_i = f32(p_i / P) in place; per block the exact sum of q in 2^-62 fixed point (the draw's running
// sum, exact in any order) and the last id with q > 0 (-1 if none).
constexpr double kFix = 4611686018427387904.0;   // 2^62
__device__ __forceinline__ unsigned long long fix62(float x) { return (unsigned long long)((double)x * kFix); }
// (ppart == nullptr: p already holds the final q; only the sums are formed.)
__global__ __launch_bounds__(kIdThreads) void q_ids_kernel(float* p, int n, const double* __restrict__ ppart, int nb,
                                                           unsigned long long* __restrict__ qfix_sum,
                                                           int* __restrict__ last_pos) {
  __shared__ double red[kIdThreads / 64];
  __shared__ unsigned long long ured[kIdThreads / 64];
  __shared__ int lred[kIdThreads / 64];
  const double P = ppart ? sum_parts(ppart, nb, red) : 0.0;
  const int i = blockIdx.x * kIdThreads + threadIdx.x;
  unsigned long long f = 0;
  int last = -1;
  if (i < n) {
    float q = p[i];
    if (ppart) {
      q = P > 0.0 ? (float)((double)q / P) : q;
      p[i] = q;
    }
    f = fix62(q);
    if (q > 0.f) last = i;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    f += __shfl_xor(f, o, 64);
    last = max(last, __shfl_xor(last, o, 64));
  }
  if ((threadIdx.x & 63) == 0) {
    ured[threadIdx.x >> 6] = f;
    lred[threadIdx.x >> 6] = last;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long tot = 0;
    int l = -1;
    for (int w = 0; w < kIdThreads / 64; ++w) {
      tot += ured[w];
      l = max(l, lred[w]);
    }
    qfix_sum[blockIdx.x] = tot;
    last_pos[blockIdx.x] = l;
  }
}

// One block of 1024 threads: over the values load(0 .. count) (nonnegative integers), the first
// index at which base plus the inclusive running sum exceeds target (STRICT) or reaches it; count
// if none.  *before gets base plus the running sum ahead of that index (the total if none).  Exact
// integer sums make the running sum monotone, so the first crossing is unique.  pre: 1024 LDS
// words, res: one LDS int.  Every thread returns the same values.
template <bool STRICT, typename Load>
__device__ int first_crossing(Load load, int count, unsigned long long base, unsigned long long target,
                              unsigned long long* pre, int* res, unsigned long long* before) {
  const int t = threadIdx.x;
  unsigned long long carry = base;
  int found = -1;
  for (int c0 = 0; c0 < count && found < 0; c0 += 1024) {
    const int i = c0 + t;
    pre[t] = i < count ? load(i) : 0ull;
    if (t == 0) *res = -1;
    __syncthreads();
    for (int o = 1; o < 1024; o <<= 1) {   // inclusive Hillis-Steele scan
      const unsigned long long v = t >= o ? pre[t - o] : 0ull;
      __syncthreads();
      pre[t] += v;
      __syncthreads();
    }
    const unsigned long long incl = carry + pre[t], excl = carry + (t ? pre[t - 1] : 0ull);
    const bool hit = STRICT ? incl > target : incl >= target;
    const bool hit_before = STRICT ? excl > target : excl >= target;
    if (i < count && hit && !hit_before) *res = i;
    __syncthreads();
    found = *res;
    carry += found >= 0 ? (found == c0 ? 0ull : pre[found - c0 - 1]) : pre[1023];
    __syncthreads();
  }
  *before = carry;
  return found < 0 ? count : found;
}

// The draw over the whole row in id order (q: kIdThreads-id blocks with fixed-point totals
// qfix_sum and last positive ids last_pos): the first id whose running fixed-point sum of q exceeds
// r * 2^62, else the last id with q > 0, else 0.  Greedy: the first id of the order.  Display: the
// first display_k ids of the order (top keys or sorted ids) with q.  One block of 1024 threads.
__global__ __launch_bounds__(1024) void draw_ids_kernel(const float* __restrict__ q, int n,
                                                        const unsigned long long* __restrict__ qfix_sum,
                                                        const int* __restrict__ last_pos, int nb, int greedy,
                                                        const uint64_t* __restrict__ top,
                                                        const int32_t* __restrict__ sorted_ids, uint64_t seed,
                                                        const int32_t* __restrict__ counter, int display_k,
                                                        int32_t* __restrict__ token, float* __restrict__ logprob,
                                                        int32_t* __restrict__ disp_ids, float* __restrict__ disp_p) {
  __shared__ unsigned long long pre[1024];
  __shared__ int res_s, last_s;
  const int t = threadIdx.x;
  auto order_id = [&](int j) { return top ? key_id(top[j]) : sorted_ids[j]; };
  int tok = 0;
  if (greedy) {
    tok = order_id(0);
  } else {
    uint32_t c[4] = {(uint32_t)*counter, 0u, 0u, 0u};
    philox4x32_10(c, (uint32_t)seed, (uint32_t)(seed >> 32));
    const unsigned long long R = (unsigned long long)(c[0] >> 8) << 38;   // r * 2^62, exact
    unsigned long long carry = 0;
    const int blk = first_crossing<true>([&](int b) { return qfix_sum[b]; }, nb, 0ull, R, pre, &res_s, &carry);
    if (blk < nb) {
      const int base = blk * kIdThreads, cnt = min(kIdThreads, n - base);
      unsigned long long unused = 0;
      tok = base + first_crossing<true>([&](int u) { return fix62(q[base + u]); }, cnt, carry, R, pre, &res_s,
                                        &unused);
    } else {   // r beyond the total: the last id with q > 0, else 0
      if (t == 0) last_s = -1;
      __syncthreads();
      int l = -1;
      for (int b = t; b < nb; b += 1024) l = max(l, last_pos[b]);
      atomicMax(&last_s, l);
      __syncthreads();
      tok = last_s >= 0 ? last_s : 0;
    }
  }
  if (t == 0) {
    *token = tok;
    if (logprob) *logprob = (float)log((double)q[tok] + 1e-10);
  }
  for (int j = t; j < display_k; j += 1024) {
    const int id = order_id(j);
    if (disp_ids) disp_ids[j] = id;
    if (disp_p) disp_p[j] = q[id];
  }
}

// ---- full-sort path kernels (positions j index the descending order) ----------------------------

// p_j = f32(e_j / Z) in place; per kThreads-position block, over positions j < k_eff, the exact
// 2^-62 fixed-point sum of p (the top-p search) and the f64 tree sum (the kept mass).
__global__ __launch_bounds__(kThreads) void prob_sorted_kernel(float* e, int n, int k_eff, const double* __restrict__ Z,
                                                               unsigned long long* __restrict__ pfix_sum,
                                                               double* __restrict__ p_sum) {
  __shared__ double red[kThreads / 64];
  __shared__ unsigned long long ured[kThreads / 64];
  const int j = blockIdx.x * kThreads + threadIdx.x;
  double v = 0.0;
  unsigned long long f = 0;
  if (j < n) {
    const float p = (float)((double)e[j] / *Z);
    e[j] = p;
    if (j < k_eff) {
      v = (double)p;
      f = fix62(p);
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) f += __shfl_xor(f, o, 64);
  if ((threadIdx.x & 63) == 0) ured[threadIdx.x >> 6] = f;
  v = block_sum_f64(v, red);   // (its barriers also publish ured)
  if (threadIdx.x == 0) {
    unsigned long long tot = 0;
    for (int w = 0; w < kThreads / 64; ++w) tot += ured[w];
    pfix_sum[blockIdx.x] = tot;
    p_sum[blockIdx.x] = v;
  }
}

// One block of 1024 threads: cut = 1 + the first position j < k_eff whose running sum of p reaches
// top_p (k_eff if none, or when top_p >= 1), and the kept mass P = sum of p over j < cut (f64:
// whole blocks' tree sums, then the partial block, in a fixed order).
__global__ __launch_bounds__(1024) void cut_kernel(const float* __restrict__ p, int k_eff, double top_p,
                                                   const unsigned long long* __restrict__ pfix_sum,
                                                   const double* __restrict__ p_sum, int nb, int* __restrict__ cut_out,
                                                   double* __restrict__ P_out) {
  __shared__ unsigned long long pre[1024];
  __shared__ double red[1024 / 64];
  __shared__ int res_s;
  const int t = threadIdx.x;
  int cut = k_eff;
  if (top_p <= 0.0) {
    // The reference's `cum >= topP` holds at i = 0: exactly the first id is kept.
    cut = min(1, k_eff);
  } else if (top_p < 1.0) {
    const unsigned long long target = (unsigned long long)ceil(top_p * kFix);
    unsigned long long carry = 0, unused = 0;
    const int blk = first_crossing<false>([&](int b) { return pfix_sum[b]; }, nb, 0ull, target, pre, &res_s, &carry);
    if (blk < nb) {
      const int base = blk * kThreads, cnt = min(kThreads, k_eff - base);
      const int j = first_crossing<false>([&](int u) { return fix62(p[base + u]); }, cnt, carry, target, pre, &res_s,
                                          &unused);
      if (j < cnt) cut = base + j + 1;
    }
  }
  const int full = cut / kThreads;
  double v = 0.0;
  for (int b = t; b < full; b += 1024) v += p_sum[b];
  for (int j = full * kThreads + t; j < cut; j += 1024) v += (double)p[j];
  v = block_sum_f64(v, red);
  if (t == 0) {
    *cut_out = cut;
    *P_out = v;
  }
}

// q in id order: q[id] = f32(p_j / P) for kept positions j < cut (p itself when P == 0 or when not
// renormalising), 0 otherwise.
__global__ void scatter_q_kernel(const float* __restrict__ p, const int32_t* __restrict__ sorted_ids, int n,
                                 const int* __restrict__ cut, const double* __restrict__ P, int renorm,
                                 float* __restrict__ q) {
  const int j = blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= n) return;
  float v = 0.f;
  if (j < *cut) v = (renorm && *P > 0.0) ? (float)((double)p[j] / *P) : p[j];
  q[sorted_ids[j]] = v;
}

// rocPRIM's stable radix sort with its default configuration (for a 151,936-id row: a block sort
// and merge passes, measured faster here than forcing onesweep).
inline hipError_t sort_desc(void* tmp, size_t& bytes, const float* k_in, float* k_out, const int32_t* v_in,
                            int32_t* v_out, int n, hipStream_t s) {
  return rocprim::radix_sort_pairs_desc(tmp, bytes, k_in, k_out, v_in, v_out, n, 0, 32, s);
}

}  // namespace

extern "C" {

int kh_sample_set_path(int path) {
  KH_REQUIRE(path == 0 || path == 1, "kh_sample_set_path: path must be 0 (automatic) or 1 (full sort)");
  g_sample_path = path;
  return KH_OK;
}

int kh_philox4x32_10(uint64_t seed, const uint32_t* counters, int64_t n, uint32_t* out) {
  KH_REQUIRE_INIT();
  KH_REQUIRE(n >= 0, "kh_philox4x32_10: negative count");
  if (n == 0) return KH_OK;
  KH_REQUIRE(counters && out, "kh_philox4x32_10: null pointer");
  KH_REQUIRE(n <= (int64_t)INT32_MAX * 256, "kh_philox4x32_10: too many counters");
  philox_kernel<<<(unsigned)((n + 255) / 256), 256, 0, stream()>>>(seed, counters, n, out);
  KH_CHECK_LAUNCH();
  return KH_OK;
}

// The selection path (prefix of m <= kMaxPrefix ids; see select_kernel): greedy, top-k with or
// without top-p, and the unfiltered draw.
static int sample_selected(const float* logits, int n, int greedy, double inv_t, int k_eff, double top_p, int m,
                           uint64_t seed, const int32_t* counter, int32_t* token_out, float* logprob_out,
                           int display_k, int32_t* display_ids, float* display_probs) {
  const bool small = m <= kSelSmall / 4;
  const int chunk = small ? kSelSmall : kSelLarge;
  const int nsel = (n + chunk - 1) / chunk;
  const int nb = (n + kIdThreads - 1) / kIdThreads;
  const bool plain = !greedy && k_eff == n && top_p >= 1.0;
  const size_t sz_sel = align256((size_t)nsel * m * 8), sz_nb = align256((size_t)nb * 8);
  const size_t total = 2 * sz_sel + (plain ? align256((size_t)n * 4) + 3 * sz_nb + align256((size_t)nb * 4) : sz_nb);
  char* ws = (char*)scratch_alloc(total);
  if (!ws) return KH_ERR_OOM;
  char* cur = ws;
  auto take = [&](size_t b) { char* p = cur; cur += b; return p; };
  uint64_t* src = (uint64_t*)take(sz_sel);
  uint64_t* dst = (uint64_t*)take(sz_sel);
  double* zpart = (double*)take(sz_nb);

  if (small)
    select_kernel<true, kSelSmall, kSelSmallThreads><<<nsel, kSelSmallThreads, 0, stream()>>>(logits, nullptr, n, m,
                                                                                              src);
  else
    select_kernel<true, kSelLarge, kSelLargeThreads><<<nsel, kSelLargeThreads, 0, stream()>>>(logits, nullptr, n, m,
                                                                                              src);
  for (int blocks = nsel; blocks > 1;) {
    const int cnt = blocks * m;
    blocks = (cnt + chunk - 1) / chunk;
    if (small)
      select_kernel<false, kSelSmall, kSelSmallThreads><<<blocks, kSelSmallThreads, 0, stream()>>>(nullptr, src, cnt,
                                                                                                   m, dst);
    else
      select_kernel<false, kSelLarge, kSelLargeThreads><<<blocks, kSelLargeThreads, 0, stream()>>>(nullptr, src, cnt,
                                                                                                   m, dst);
    uint64_t* t = src;
    src = dst;
    dst = t;
  }
  const uint64_t* top = src;   // the first m ids of the order
  if (!plain) {
    exp_ids_kernel<<<nb, kIdThreads, 0, stream()>>>(logits, n, top, inv_t, greedy, nullptr, zpart);
    finish_prefix_kernel<<<1, kMaxPrefix, 0, stream()>>>(top, m, zpart, nb, inv_t, greedy, k_eff, top_p, seed, counter,
                                                         display_k, token_out, logprob_out, display_ids,
                                                         display_probs);
  } else {
    float* e = (float*)take(align256((size_t)n * 4));   // e, then p, then q (id order)
    double* ppart = (double*)take(sz_nb);
    unsigned long long* qfix = (unsigned long long*)take(sz_nb);
    int* last = (int*)take(align256((size_t)nb * 4));
    exp_ids_kernel<<<nb, kIdThreads, 0, stream()>>>(logits, n, top, inv_t, 0, e, zpart);
    prob_ids_kernel<<<nb, kIdThreads, 0, stream()>>>(e, n, zpart, nb, ppart);
    q_ids_kernel<<<nb, kIdThreads, 0, stream()>>>(e, n, ppart, nb, qfix, last);
    draw_ids_kernel<<<1, 1024, 0, stream()>>>(e, n, qfix, last, nb, 0, top, nullptr, seed, counter, display_k,
                                              token_out, logprob_out, display_ids, display_probs);
  }
  const hipError_t err = hipGetLastError();
  scratch_free(ws);  // stream-ordered: reused only by later work on the same stream
  if (err != hipSuccess) {
    set_error("kh_sample: launch failed: %s", hipGetErrorString(err));
    return KH_ERR_HIP;
  }
  KH_DEBUG_SYNC();
  return KH_OK;
}

int kh_sample(const float* logits, int64_t vocab, int do_sample, double temperature, int top_k, double top_p,
              uint64_t seed, const int32_t* counter, int32_t* token_out, float* logprob_out, int display_k, int32_t* display_ids,
              float* display_probs) {
  KH_REQUIRE_INIT();
  KH_REQUIRE(vocab > 0 && vocab <= (int64_t)INT32_MAX / 2, "kh_sample: vocab %lld out of range", (long long)vocab);
  KH_REQUIRE(logits && token_out && (counter || !do_sample), "kh_sample: null pointer");
  KH_REQUIRE(temperature > 0.0, "kh_sample: temperature must be positive (got %g)", temperature);
  KH_REQUIRE(display_k >= 0 && display_k <= vocab, "kh_sample: display_k %d out of [0, vocab]", display_k);
  const int n = (int)vocab;
  const int nb = (n + kThreads - 1) / kThreads;
  const int greedy = do_sample ? 0 : 1;
  const int k_eff = (!greedy && top_k > 0 && top_k < n) ? top_k : n;
  const double inv_t = 1.0 / temperature;
  // The selection path needs the order only up to m = max(display_k, 1, top-k); top-p without
  // top-k may cut anywhere in the order and takes the full sort below.
  int m = display_k > 1 ? display_k : 1;
  if (k_eff < n && k_eff > m) m = k_eff;
  const bool topp_only = !greedy && k_eff == n && top_p < 1.0;
  if (!topp_only && m <= kMaxPrefix && g_sample_path != 1)
    return sample_selected(logits, n, greedy, inv_t, k_eff, top_p, m, seed, counter, token_out, logprob_out,
                           display_k, display_ids, display_probs);
  // The full-sort path calls rocPRIM's sort, which may clear its temporary storage with memsets:
  // it is not captured into graphs.
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  KH_CHECK_HIP(hipStreamIsCapturing(stream(), &cap));
  KH_REQUIRE(cap == hipStreamCaptureStatusNone,
             "kh_sample: top-p without top-k, top-k > 1024 or display_k > 1024 is not supported under stream "
             "capture");

  size_t sort_bytes = 0;
  KH_CHECK_HIP(sort_desc(nullptr, sort_bytes, nullptr, nullptr, nullptr, nullptr, n, stream()));
  const int nbi = (n + kIdThreads - 1) / kIdThreads;
  const size_t sz_f = align256((size_t)n * 4);
  const size_t total = 6 * sz_f + 3 * align256((size_t)nb * 8) + 2 * align256((size_t)nbi * 8) + 256 +
                       align256(sort_bytes);
  char* ws = (char*)scratch_alloc(total);
  if (!ws) return KH_ERR_OOM;
  char* cur = ws;
  auto take = [&](size_t b) { char* p = cur; cur += b; return p; };
  float* keys = (float*)take(sz_f);
  float* sorted_logits = (float*)take(sz_f);
  int32_t* ids = (int32_t*)take(sz_f);
  int32_t* sorted_ids = (int32_t*)take(sz_f);
  float* e = (float*)take(sz_f);          // then p (sorted order), in place
  float* q = (float*)take(sz_f);          // id order
  double* part = (double*)take(align256((size_t)nb * 8));
  unsigned long long* pfix = (unsigned long long*)take(align256((size_t)nb * 8));
  double* psum = (double*)take(align256((size_t)nb * 8));
  unsigned long long* qfix = (unsigned long long*)take(align256((size_t)nbi * 8));
  int* last = (int*)take(align256((size_t)nbi * 8));
  char* small = take(256);
  double* Z = (double*)small;
  double* P = (double*)(small + 8);
  int* cut = (int*)(small + 16);
  void* sort_tmp = take(align256(sort_bytes));

  hipError_t err = hipSuccess;
  auto ok = [&](hipError_t x) { if (err == hipSuccess) err = x; };
  iota_keys_kernel<<<nb, kThreads, 0, stream()>>>(logits, n, keys, ids);
  ok(hipGetLastError());
  size_t sb = sort_bytes;
  ok(sort_desc(sort_tmp, sb, keys, sorted_logits, ids, sorted_ids, n, stream()));
  exp_kernel<<<nb, kThreads, 0, stream()>>>(sorted_logits, n, inv_t, greedy, e, part);
  final_sum_kernel<<<1, kThreads, 0, stream()>>>(part, nb, Z);
  prob_sorted_kernel<<<nb, kThreads, 0, stream()>>>(e, n, k_eff, Z, pfix, psum);
  cut_kernel<<<1, 1024, 0, stream()>>>(e, k_eff, greedy ? 1.0 : top_p, pfix, psum, nb, cut, P);
  scatter_q_kernel<<<nb, kThreads, 0, stream()>>>(e, sorted_ids, n, cut, P, greedy ? 0 : 1, q);
  q_ids_kernel<<<nbi, kIdThreads, 0, stream()>>>(q, n, nullptr, nbi, qfix, last);
  draw_ids_kernel<<<1, 1024, 0, stream()>>>(q, n, qfix, last, nbi, greedy, nullptr, sorted_ids, seed, counter,
                                            display_k, token_out, logprob_out, display_ids, display_probs);
  ok(hipGetLastError());
  scratch_free(ws);  // stream-ordered: reused only by later work on the same stream
  if (err != hipSuccess) {
    set_error("kh_sample: launch failed: %s", hipGetErrorString(err));
    return KH_ERR_HIP;
  }
  KH_DEBUG_SYNC();
  return KH_OK;
}

}  // extern "C"
