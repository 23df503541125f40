/*
 * oracle.c — CPU restatement of Kandle's transformer hot-path math, used ONLY as test
 * infrastructure: by tests/, by __graft_entry__.smoke() as the checker, and by bench.py's
 * cpu_baseline leg.  The product (kandle_amd) never links or calls it.
 *
 * All functions take float32 inputs (bf16 data is widened exactly by the caller), accumulate in
 * double unless stated, and write float32 outputs.  Single-threaded scalar code.
 *
 * Reference citations are relative to the Kandle repository root.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* bf16 <-> f32.  Widening: packages/core/src/io/safetensor/dtypes.ts:82-94 (bits << 16).
 * Narrowing: round to nearest even on the upper 16 bits; NaN kept quiet. */
void or_f32_to_bf16(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    uint32_t u;
    memcpy(&u, &in[i], 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) {
      out[i] = (uint16_t)((u >> 16) | 0x40u);
      continue;
    }
    u += 0x7fffu + ((u >> 16) & 1u);
    out[i] = (uint16_t)(u >> 16);
  }
}

void or_bf16_to_f32(const uint16_t* in, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    uint32_t u = ((uint32_t)in[i]) << 16;
    memcpy(&out[i], &u, 4);
  }
}

/*
 * Scaled dot-product attention, reference semantics:
 *   packages/core/src/dispatch/handlers/composite.ts:247-316 (scale default 1/sqrt(E) is the caller's),
 *   packages/backend-webgpu/src/kernels/attention/builder.ts:138-329:
 *     score = (q . k) * scale  (scale applied after the dot, :253-256),
 *     causal: key j > query i is masked (top-left, :247-249),
 *     GQA: query head h reads kv head h / (Hq / Hkv) (:143),
 *     softmax over the unmasked keys, O = sum p_j v_j / sum p_j (:270-329).
 * Layouts: q/o [B][Hq][Lq][D], k/v [B][Hkv][Lk][D], contiguous.
 * kv_len (may be NULL) gives a per-batch key count <= Lk (decode against a KV cache with
 * per-sequence lengths; keys beyond it are ignored).
 */
void or_sdpa(const float* q, const float* k, const float* v, float* o, int B, int Hq, int Hkv, int64_t Lq,
             int64_t Lk, int D, float scale, int causal, const int32_t* kv_len, double* work /* Lk doubles */) {
  const int G = Hq / Hkv;
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < Hq; ++h) {
      const int hk = h / G;
      const float* kb = k + ((int64_t)b * Hkv + hk) * Lk * D;
      const float* vb = v + ((int64_t)b * Hkv + hk) * Lk * D;
      const int64_t L = kv_len ? kv_len[b] : Lk;
      for (int64_t i = 0; i < Lq; ++i) {
        const float* qi = q + (((int64_t)b * Hq + h) * Lq + i) * D;
        float* oi = o + (((int64_t)b * Hq + h) * Lq + i) * D;
        const int64_t kend = causal ? (i + 1 < L ? i + 1 : L) : L;
        double m = -INFINITY;
        for (int64_t j = 0; j < kend; ++j) {
          const float* kj = kb + j * D;
          double dot = 0.0;
          for (int d = 0; d < D; ++d) dot += (double)qi[d] * (double)kj[d];
          work[j] = dot * (double)scale;
          if (work[j] > m) m = work[j];
        }
        double l = 0.0;
        for (int64_t j = 0; j < kend; ++j) {
          work[j] = exp(work[j] - m);
          l += work[j];
        }
        for (int d = 0; d < D; ++d) {
          double acc = 0.0;
          for (int64_t j = 0; j < kend; ++j) acc += work[j] * (double)vb[j * D + d];
          oi[d] = kend > 0 ? (float)(acc / l) : 0.0f;
        }
      }
    }
}

/*
 * SDPA with an explicit additive mask: the reference's naive route for attnMask
 * (packages/core/src/dispatch/handlers/composite.ts:279-300), which ignores isCausal:
 *   W = matmul(q, k^T) * scale            (dispatchMatmul alpha = scale, transposeB),
 *   W = W + mask                          (add_Tensor with broadcasting),
 *   P = softmax(W, -1)                    (packages/backend-webgpu/src/kernels/normalize/
 *                                          shaderBuilder.ts:143-213: the row max starts at
 *                                          f32(-1e38), p = exp(x - max), P = p / sum p, so a row whose
 *                                          sum is 0 -- every x <= -1e38 far enough -- is 0/0 = NaN),
 *   O = matmul(P, v).
 * GQA as in or_sdpa.  The mask is float32 with element strides (msb, msh, msq, msk) over (batch,
 * query head, query, key); a stride of 0 broadcasts that axis.  work: Lk doubles.
 */
void or_sdpa_masked(const float* q, const float* k, const float* v, float* o, int B, int Hq, int Hkv, int64_t Lq,
                    int64_t Lk, int D, float scale, const float* mask, int64_t msb, int64_t msh, int64_t msq,
                    int64_t msk, double* work) {
  const int G = Hq / Hkv;
  const double floor_max = (double)(float)-1e38;
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < Hq; ++h) {
      const int hk = h / G;
      const float* kb = k + ((int64_t)b * Hkv + hk) * Lk * D;
      const float* vb = v + ((int64_t)b * Hkv + hk) * Lk * D;
      for (int64_t i = 0; i < Lq; ++i) {
        const float* qi = q + (((int64_t)b * Hq + h) * Lq + i) * D;
        float* oi = o + (((int64_t)b * Hq + h) * Lq + i) * D;
        const float* mrow = mask + b * msb + h * msh + i * msq;
        double m = floor_max;
        for (int64_t j = 0; j < Lk; ++j) {
          const float* kj = kb + j * D;
          double dot = 0.0;
          for (int d = 0; d < D; ++d) dot += (double)qi[d] * (double)kj[d];
          work[j] = dot * (double)scale + (double)mrow[j * msk];
          if (work[j] > m) m = work[j];
        }
        double l = 0.0;
        for (int64_t j = 0; j < Lk; ++j) {
          work[j] = exp(work[j] - m);
          l += work[j];
        }
        for (int d = 0; d < D; ++d) {
          double acc = 0.0;
          for (int64_t j = 0; j < Lk; ++j) acc += work[j] * (double)vb[j * D + d];
          oi[d] = (float)(acc / l); /* l == 0: 0/0 = NaN, as the reference's softmax */
        }
      }
    }
}

/*
 * RMSNorm over rows of n: y = x * (1 / sqrt(mean(x^2) + eps)) * w
 * (packages/backend-webgpu/src/kernels/normalize/shaderBuilder.ts:394-411; normalizedShape = trailing
 * dims, packages/backend-webgpu/src/kernels/normalize/executor.ts:280-293).  w may be NULL.
 */
void or_rms_norm(const float* x, const float* w, float* y, int64_t rows, int64_t n, float eps) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * n;
    double ss = 0.0;
    for (int64_t i = 0; i < n; ++i) ss += (double)xr[i] * (double)xr[i];
    const double inv = 1.0 / sqrt(ss / (double)n + (double)eps);
    for (int64_t i = 0; i < n; ++i) y[r * n + i] = (float)((double)xr[i] * inv * (w ? (double)w[i] : 1.0));
  }
}

/*
 * Rotary inverse frequencies exactly as RotaryEmbedding._computeInvFreqDirect
 * (packages/model-utils/src/rope.ts:159-171): computed in double, stored as float32.
 */
void or_rope_inv_freq(float* inv_freq, int head_dim, double theta) {
  const int half = head_dim / 2;
  for (int i = 0; i < half; ++i) inv_freq[i] = (float)(1.0 / pow(theta, (double)i / (double)half));
}

/*
 * Per-head RMSNorm (qk-norm) then RoPE on rows [T][H][D] in place of out:
 *   n = rms_norm(x, w, eps) over D                    (packages/model-utils/src/attention/gqa.ts:279-286)
 *   f_i = float32(float32(pos) * inv_freq[i mod D/2])  (packages/model-utils/src/rope.ts:226,244: f32 mul)
 *   emb = cat(f, f); out = n * cos(emb) + rotate_half(n) * sin(emb),
 *   rotate_half(n) = cat(-n2, n1)                      (packages/model-utils/src/rope.ts:251-255, :590-630)
 * The normed value is kept in full precision between the norm and the rotation (fused op).
 * w may be NULL (plain RoPE).
 */
void or_qk_norm_rope(const float* x, const float* w, float* out, int64_t T, int H, int D, const int32_t* positions,
                     const float* inv_freq, float eps, int do_norm) {
  const int half = D / 2;
  double nbuf[512];
  for (int64_t t = 0; t < T; ++t) {
    const float posf = (float)positions[t];
    for (int h = 0; h < H; ++h) {
      const float* xr = x + (t * H + h) * D;
      float* orow = out + (t * H + h) * D;
      if (do_norm) {
        double ss = 0.0;
        for (int i = 0; i < D; ++i) ss += (double)xr[i] * (double)xr[i];
        const double inv = 1.0 / sqrt(ss / (double)D + (double)eps);
        for (int i = 0; i < D; ++i) nbuf[i] = (double)xr[i] * inv * (w ? (double)w[i] : 1.0);
      } else {
        for (int i = 0; i < D; ++i) nbuf[i] = (double)xr[i];
      }
      for (int i = 0; i < half; ++i) {
        const float f = posf * inv_freq[i]; /* float32 product, as the reference's f32 mul */
        const double c = cos((double)f), s = sin((double)f);
        const double a = nbuf[i], bb = nbuf[i + half];
        orow[i] = (float)(a * c - bb * s);
        orow[i + half] = (float)(bb * c + a * s);
      }
    }
  }
}

/* silu(x) = x / (1 + exp(-clamp(x, -88, 88)))  (packages/backend-webgpu/src/kernels/pointwise/ops.ts:299);
 * SwiGLU h = silu(g) * u  (packages/model-utils/src/mlp/swiglu.ts:119-134). */
void or_silu_mul(const float* g, const float* u, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    double x = g[i];
    double c = x < -88.0 ? -88.0 : (x > 88.0 ? 88.0 : x);
    double s = x / (1.0 + exp(-c));
    out[i] = (float)(u ? s * (double)u[i] : s);
  }
}

/*
 * C[m][n] = alpha * sum_k A[m][k] * W[n][k] + beta * Cin[m][n] + bias[n]   (nn.Linear: y = x W^T + b,
 * packages/core/src/dispatch/handlers/composite.ts:55-77; alpha/beta/C epilogue
 * packages/core/src/dispatch/matmulOps.ts:32-125).  Cin and bias may be NULL.
 */
void or_linear(const float* A, const float* W, const float* cin, const float* bias, float* C, int64_t M, int64_t N,
               int64_t K, float alpha, float beta) {
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n = 0; n < N; ++n) {
      const float* a = A + m * K;
      const float* w = W + n * K;
      double acc = 0.0;
      for (int64_t k = 0; k < K; ++k) acc += (double)a[k] * (double)w[k];
      double v = (double)alpha * acc;
      if (cin && beta != 0.0f) v += (double)beta * (double)cin[m * N + n];
      if (bias) v += (double)bias[n];
      C[m * N + n] = (float)v;
    }
}

/* Lowest index among the maxima of each row: the greedy rule of sample()
 * (packages/model-utils/src/sampling/index.ts:132,138: first id of a stable descending sort).
 * Values are compared with strict '>' from -FLT_MAX as the reference argmax kernel does
 * (packages/backend-webgpu/src/kernels/reduction/argShaderBuilder.ts:214-228), so NaN never wins
 * and a row with no value above -FLT_MAX yields 0.  Ties are NOT resolved as that kernel resolves
 * them: its thread t scans indices t, t + W, t + 2W, ... (W = the device's workgroup size) and
 * keeps its first maximum, and its tree reduction (:86-98) lets position p take position
 * p + stride's value only when strictly greater, so among tied maxima the result depends on W
 * (W = 4, maxima at 1 and 2: index 2; W = 256, maxima at 1 and 256: index 256).  This restatement
 * and the GPU kernel use the device-independent lowest-index rule. */
void or_argmax(const float* x, int64_t rows, int64_t n, int32_t* out) {
  for (int64_t r = 0; r < rows; ++r) {
    float best = -3.4028234663852886e38f;
    int32_t bi = 0;
    for (int64_t i = 0; i < n; ++i)
      if (x[r * n + i] > best) {
        best = x[r * n + i];
        bi = (int32_t)i;
      }
    out[r] = bi;
  }
}

/*
 * The reference's own flash algorithm in float32, block by block (packages/backend-webgpu/src/kernels/
 * attention/builder.ts:187-329: Br x Bc tiles, running max m and sum l initialised to -1e20 and 0, O
 * rescaled by exp(m_old - m_new), masked scores set to -1e20).  Used as the timed CPU baseline; its
 * results agree with or_sdpa to float32 rounding.
 */
void or_flash_f32(const float* q, const float* k, const float* v, float* o, int B, int Hq, int Hkv, int64_t Lq,
                  int64_t Lk, int D, float scale, int causal, int64_t heads_limit) {
  const int G = Hq / Hkv;
  const int BC = 4;
  float sblk[4];
  float acc[512];
  int64_t done = 0;
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < Hq; ++h) {
      if (heads_limit > 0 && done >= heads_limit) return;
      ++done;
      const int hk = h / G;
      const float* kb = k + ((int64_t)b * Hkv + hk) * Lk * D;
      const float* vb = v + ((int64_t)b * Hkv + hk) * Lk * D;
      for (int64_t i = 0; i < Lq; ++i) {
        const float* qi = q + (((int64_t)b * Hq + h) * Lq + i) * D;
        float* oi = o + (((int64_t)b * Hq + h) * Lq + i) * D;
        float m = -1e20f, l = 0.0f;
        for (int d = 0; d < D; ++d) acc[d] = 0.0f;
        for (int64_t j0 = 0; j0 < Lk; j0 += BC) {
          if (causal && j0 > i) break; /* block entirely after the query row */
          float mnew = m;
          for (int jj = 0; jj < BC; ++jj) {
            const int64_t j = j0 + jj;
            float s = -1e20f;
            if (j < Lk && !(causal && j > i)) {
              float dot = 0.0f;
              for (int d = 0; d < D; ++d) dot += qi[d] * kb[j * D + d];
              s = dot * scale;
            }
            sblk[jj] = s;
            if (s > mnew) mnew = s;
          }
          const float sf = expf(m - mnew);
          float p[4];
          l *= sf;
          for (int jj = 0; jj < BC; ++jj) {
            p[jj] = expf(sblk[jj] - mnew); /* the reference re-evaluates this per d; same value */
            l += p[jj];
          }
          for (int d = 0; d < D; ++d) {
            float ov = acc[d] * sf;
            for (int jj = 0; jj < BC; ++jj) {
              const int64_t j = j0 + jj;
              if (j < Lk) ov += p[jj] * vb[j * D + d];
            }
            acc[d] = ov;
          }
          m = mnew;
        }
        for (int d = 0; d < D; ++d) oi[d] = acc[d] / l;
      }
    }
}
