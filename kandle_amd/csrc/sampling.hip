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
// The sort is rocPRIM's stable radix sort; the f64 sums are two-pass block reductions
// and hipCUB inclusive scans (deterministic for a given size).  hipCUB may clear its temporary storage
// with memsets, so kh_sample refuses to run under stream capture.
#include <hipcub/hipcub.hpp>
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

// p (sorted order) = f32(e / Z), stored as f64 for the top-p scan.
// (p may be e itself: each element is read, then overwritten.)
__global__ void prob_kernel(const float* e, int n, const double* __restrict__ Z, float* p, double* __restrict__ p64) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) {
    const float pf = (float)((double)e[i] / *Z);
    p[i] = pf;
    p64[i] = (double)pf;
  }
}

// cut[0] = number of kept sorted positions: the first j < k_eff with cum[j] >= top_p gives j + 1
// (minimum over threads); k_eff when no position reaches top_p.  cut[0] starts at k_eff.
__global__ void topp_cut_kernel(const double* __restrict__ cum, int k_eff, double top_p, int* __restrict__ cut) {
  const int j = blockIdx.x * blockDim.x + threadIdx.x;
  if (j < k_eff && cum[j] >= top_p) atomicMin(cut, j + 1);
}

__global__ void fill_int_kernel(int* __restrict__ p, int v) { *p = v; }

// Per-block f64 sums of the kept p (sorted positions < cut).
__global__ __launch_bounds__(kThreads) void kept_sum_kernel(const float* __restrict__ p, int n,
                                                            const int* __restrict__ cut, double* __restrict__ part) {
  __shared__ double red[kThreads / 64];
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  const double v = (i < n && i < *cut) ? (double)p[i] : 0.0;
  const double s = block_sum_f64(v, red);
  if (threadIdx.x == 0) part[blockIdx.x] = s;
}

// q in id order: q[id] = f32(p / P) for kept sorted positions (p itself when P == 0 or when not
// renormalising), 0 otherwise; also the f64 copy for the id-order scan.
__global__ void scatter_q_kernel(const float* __restrict__ p, const int32_t* __restrict__ sorted_ids, int n,
                                 const int* __restrict__ cut, const double* __restrict__ P, int renorm,
                                 float* __restrict__ q, double* __restrict__ q64) {
  const int j = blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= n) return;
  const int id = sorted_ids[j];
  float v = 0.f;
  if (j < *cut) v = (renorm && *P > 0.0) ? (float)((double)p[j] / *P) : p[j];
  q[id] = v;
  q64[id] = (double)v;
}

// sel[0] = min id with r < cum[id]; sel[1] = max id with q[id] > 0 (the fallback); r from Philox.
// One atomic per wave: the wave's lowest (highest) qualifying id, found from a ballot.
__global__ void draw_kernel(const double* __restrict__ cum, const float* __restrict__ q, int n, uint64_t seed,
                            const int32_t* __restrict__ counter, int* __restrict__ sel) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  const int lane = threadIdx.x & 63;
  uint32_t c[4] = {(uint32_t)*counter, 0u, 0u, 0u};
  philox4x32_10(c, (uint32_t)seed, (uint32_t)(seed >> 32));
  const double r = (double)(c[0] >> 8) * (1.0 / 16777216.0);
  const bool in = i < n;
  const uint64_t hit = __ballot(in && r < cum[in ? i : 0]);
  const uint64_t pos = __ballot(in && q[in ? i : 0] > 0.f);
  const int base = i - lane;
  if (lane == 0 && hit) atomicMin(&sel[0], base + __ffsll((unsigned long long)hit) - 1);
  if (lane == 0 && pos) atomicMax(&sel[1], base + 63 - __clzll((unsigned long long)pos));
}

// token: greedy -> the first id of the order; sampling -> the draw, else the fallback, else 0.
__global__ void finish_kernel(const int* __restrict__ sel, const float* __restrict__ q,
                              const int32_t* __restrict__ sorted_ids, int n, int greedy, int display_k,
                              int32_t* __restrict__ token, float* __restrict__ logprob, int32_t* __restrict__ disp_ids,
                              float* __restrict__ disp_p) {
  const int t = threadIdx.x;
  if (t == 0) {
    const int tok = greedy ? sorted_ids[0] : (sel[0] < n ? sel[0] : (sel[1] >= 0 ? sel[1] : 0));
    *token = tok;
    if (logprob) *logprob = (float)log((double)q[tok] + 1e-10);
  }
  for (int j = t; j < display_k; j += blockDim.x) {
    const int id = sorted_ids[j];
    if (disp_ids) disp_ids[j] = id;
    if (disp_p) disp_p[j] = q[id];
  }
}

__global__ void init_sel_kernel(int* __restrict__ sel, int n) {
  sel[0] = n;   // "no id yet" for the min
  sel[1] = -1;  // "no id yet" for the max
}

inline size_t align256(size_t b) { return (b + 255) & ~size_t(255); }

// rocPRIM's stable radix sort with its default configuration (for a 151,936-id row: a block sort
// and merge passes, measured faster here than forcing onesweep).
inline hipError_t sort_desc(void* tmp, size_t& bytes, const float* k_in, float* k_out, const int32_t* v_in,
                            int32_t* v_out, int n, hipStream_t s) {
  return rocprim::radix_sort_pairs_desc(tmp, bytes, k_in, k_out, v_in, v_out, n, 0, 32, s);
}

}  // namespace

extern "C" {

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

int kh_sample(const float* logits, int64_t vocab, int do_sample, double temperature, int top_k, double top_p,
              uint64_t seed, const int32_t* counter, int32_t* token_out, float* logprob_out, int display_k, int32_t* display_ids,
              float* display_probs) {
  KH_REQUIRE_INIT();
  KH_REQUIRE(vocab > 0 && vocab <= (int64_t)INT32_MAX / 2, "kh_sample: vocab %lld out of range", (long long)vocab);
  KH_REQUIRE(logits && token_out && (counter || !do_sample), "kh_sample: null pointer");
  KH_REQUIRE(temperature > 0.0, "kh_sample: temperature must be positive (got %g)", temperature);
  KH_REQUIRE(display_k >= 0 && display_k <= vocab, "kh_sample: display_k %d out of [0, vocab]", display_k);
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  KH_CHECK_HIP(hipStreamIsCapturing(stream(), &cap));
  KH_REQUIRE(cap == hipStreamCaptureStatusNone, "kh_sample: not supported under stream capture");
  const int n = (int)vocab;
  const int nb = (n + kThreads - 1) / kThreads;
  const int greedy = do_sample ? 0 : 1;
  const int k_eff = (!greedy && top_k > 0 && top_k < n) ? top_k : n;
  const double inv_t = 1.0 / temperature;

  // temporary storage sizes of the hipCUB calls
  size_t sort_bytes = 0, scan_bytes = 0;
  KH_CHECK_HIP(sort_desc(nullptr, sort_bytes, nullptr, nullptr, nullptr, nullptr, n, stream()));
  KH_CHECK_HIP(hipcub::DeviceScan::InclusiveSum(nullptr, scan_bytes, (const double*)nullptr, (double*)nullptr, n,
                                                stream()));
  const size_t cub_bytes = sort_bytes > scan_bytes ? sort_bytes : scan_bytes;
  const size_t sz_f = align256((size_t)n * 4), sz_d = align256((size_t)n * 8);
  const size_t total = 6 * sz_f + 3 * sz_d + align256((size_t)nb * 8) + 256 + align256(cub_bytes);
  char* ws = (char*)scratch_alloc(total);
  if (!ws) return KH_ERR_OOM;
  char* cur = ws;
  auto take = [&](size_t b) { char* p = cur; cur += b; return p; };
  float* keys = (float*)take(sz_f);
  float* sorted_logits = (float*)take(sz_f);
  int32_t* ids = (int32_t*)take(sz_f);
  int32_t* sorted_ids = (int32_t*)take(sz_f);
  float* e = (float*)take(sz_f);          // then p (sorted order), in place
  double* p64 = (double*)take(sz_d);
  double* cum = (double*)take(sz_d);      // top-p scan, then the id-order scan
  double* q64 = (double*)take(sz_d);
  double* part = (double*)take(align256((size_t)nb * 8));
  char* small = take(256);
  double* Z = (double*)small;             // softmax total, then P
  double* P = (double*)(small + 8);
  int* cut = (int*)(small + 16);
  int* sel = (int*)(small + 24);
  void* cub_tmp = take(align256(cub_bytes));
  float* q = (float*)take(sz_f);

  hipError_t err = hipSuccess;
  auto ok = [&](hipError_t x) { if (err == hipSuccess) err = x; };
  iota_keys_kernel<<<nb, kThreads, 0, stream()>>>(logits, n, keys, ids);
  ok(hipGetLastError());
  size_t sb = sort_bytes;
  ok(sort_desc(cub_tmp, sb, keys, sorted_logits, ids, sorted_ids, n, stream()));
  exp_kernel<<<nb, kThreads, 0, stream()>>>(sorted_logits, n, inv_t, greedy, e, part);
  final_sum_kernel<<<1, kThreads, 0, stream()>>>(part, nb, Z);
  prob_kernel<<<nb, kThreads, 0, stream()>>>(e, n, Z, e, p64);
  fill_int_kernel<<<1, 1, 0, stream()>>>(cut, k_eff);
  ok(hipGetLastError());
  if (greedy) {
    scatter_q_kernel<<<nb, kThreads, 0, stream()>>>(e, sorted_ids, n, cut, Z, 0, q, q64);
    finish_kernel<<<1, kThreads, 0, stream()>>>(sel, q, sorted_ids, n, 1, display_k, token_out, logprob_out,
                                                display_ids, display_probs);
    ok(hipGetLastError());
    scratch_free(ws);
    if (err != hipSuccess) {
      set_error("kh_sample: launch failed: %s", hipGetErrorString(err));
      return KH_ERR_HIP;
    }
    return KH_OK;
  }
  if (top_p < 1.0) {
    size_t cb = scan_bytes;
    ok(hipcub::DeviceScan::InclusiveSum(cub_tmp, cb, p64, cum, k_eff, stream()));
    topp_cut_kernel<<<(k_eff + kThreads - 1) / kThreads, kThreads, 0, stream()>>>(cum, k_eff, top_p, cut);
    ok(hipGetLastError());
  }
  kept_sum_kernel<<<nb, kThreads, 0, stream()>>>(e, n, cut, part);
  final_sum_kernel<<<1, kThreads, 0, stream()>>>(part, nb, P);
  scatter_q_kernel<<<nb, kThreads, 0, stream()>>>(e, sorted_ids, n, cut, P, 1, q, q64);
  ok(hipGetLastError());
  size_t cb = scan_bytes;
  ok(hipcub::DeviceScan::InclusiveSum(cub_tmp, cb, q64, cum, n, stream()));
  init_sel_kernel<<<1, 1, 0, stream()>>>(sel, n);
  draw_kernel<<<nb, kThreads, 0, stream()>>>(cum, q, n, seed, counter, sel);
  finish_kernel<<<1, kThreads, 0, stream()>>>(sel, q, sorted_ids, n, 0, display_k, token_out, logprob_out,
                                              display_ids, display_probs);
  ok(hipGetLastError());
  scratch_free(ws);  // stream-ordered: reused only by later work on the same stream
  if (err != hipSuccess) {
    set_error("kh_sample: launch failed: %s", hipGetErrorString(err));
    return KH_ERR_HIP;
  }
  return KH_OK;
}

}  // extern "C"
