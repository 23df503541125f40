/*
 * kandle_hip.h — C ABI of the MI355X (gfx950) backend for Kandle's transformer hot path.
 *
 * Every entry point takes plain device pointers, element counts and element strides (no torch or
 * Node types), enqueues its work on the library's single HIP stream and returns 0 on success or a
 * non-zero error code whose text `kh_last_error()` returns.  Work is asynchronous: only
 * `kh_memcpy_d2h` and `kh_synchronize` wait for the device, mirroring Kandle's "kernels enqueue,
 * readback syncs" contract (reference: packages/backend-webgpu/src/kernels/attention/executor.ts:162-168
 * submits without waiting; packages/backend-webgpu/src/base/storage.ts:191-229 is the only wait).
 *
 * Strides and offsets are in ELEMENTS, as in Kandle's ITensorHandle
 * (reference: packages/types/src/tensor.ts:6-55; packages/backend-webgpu/src/kernels/matrix/executor.ts:141).
 * The innermost dimension of every tensor argument is contiguous (stride 1): host code materialises
 * any other view with kh_copy_strided first.
 *
 * dtype codes: KH_F32 = 0, KH_BF16 = 1, KH_I32 = 2.  bf16 is an extension of the reference API,
 * which has no bfloat16 DType (reference: packages/types/src/base.ts:5-25); it is the 16 high bits
 * of an IEEE float32, rounded to nearest even.
 */
#ifndef KANDLE_HIP_H
#define KANDLE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KH_F32 0
#define KH_BF16 1
#define KH_I32 2

#define KH_OK 0
#define KH_ERR_INVALID 1   /* bad argument: shape, dtype, stride or pointer */
#define KH_ERR_HIP 2       /* a HIP runtime call failed */
#define KH_ERR_NOT_INIT 3  /* kh_init was not called */
#define KH_ERR_OOM 4       /* device allocation failed even after emptying the cache */

/* ------------------------------------------------------------------ runtime ------------------ */

/* Selects `device`, creates the library stream (default priority) and its events.
 * Replaces WebGPUDeviceManager.init (reference: packages/backend-webgpu/src/base/device.ts:95-176)
 * as called from WebGPUBackend.create (packages/backend-webgpu/src/index.ts:73-85). */
int kh_init(int device);

/* Number of visible HIP devices (0 on a host without a GPU; never fails for lack of a GPU). */
int kh_device_count(int* count);

/* Text of the most recent error on the calling thread ("" when none). */
const char* kh_last_error(void);

/* Debug mode (flags bit 0): every entry point waits for the stream after each kernel it launches
 * and returns KH_ERR_HIP naming itself if the kernel faulted, instead of the fault surfacing at a
 * later synchronising call; skipped while a graph capture is open.  0 turns it off (the default).
 * The reference's knownIssues/shader.md:151-175 proposes the same per-dispatch check for WGSL. */
int kh_set_debug(int flags);

/* 1 while a graph capture (kh_graph_begin_capture) is open on the library stream, else 0.  Host
 * code that reads device memory after a kernel (debug mode's NaN/Inf scan) skips the read then:
 * the runtime refuses copies into a stream under capture.  No counterpart in the reference (WebGPU
 * has no graph capture). */
int kh_is_capturing(void);

/* Caching device allocator (size classes, stream-ordered reuse on the single library stream).
 * Replaces WebGPUStorage's GPUBuffer creation/destroy and its buffer pooling
 * (reference: packages/backend-webgpu/src/base/storage.ts:68-106, :114-143). */
int kh_alloc(void** ptr, size_t bytes);
int kh_free(void* ptr);
int kh_empty_cache(void);

typedef struct kh_alloc_stats {
  uint64_t live_bytes;    /* bytes handed out and not yet freed */
  uint64_t cached_bytes;  /* bytes held in the free lists */
  uint64_t peak_bytes;    /* maximum of live_bytes */
  uint64_t n_device_allocs;  /* hipMalloc calls made */
  uint64_t n_cache_hits;     /* kh_alloc calls served from the free lists */
} kh_alloc_stats;
/* Mirrors the live-bytes statistics of the reference storage (packages/backend-webgpu/src/base/storage.ts:16-58). */
int kh_get_alloc_stats(kh_alloc_stats* out);

/* Copies on the library stream.  h2d returns after the source may be reused; d2h waits for the
 * stream (replaces WebGPUStorage.toRawDataAsync, packages/backend-webgpu/src/base/storage.ts:191-229). */
int kh_memcpy_h2d(void* dst, const void* src, size_t bytes);
int kh_memcpy_d2h(void* dst, const void* src, size_t bytes);
int kh_memcpy_d2d(void* dst, const void* src, size_t bytes);
int kh_synchronize(void);

/* Stream events for timing (the reference has none; its timing is wall-clock only,
 * playground-node/src/qwen3/index.ts:253-261). */
int kh_event_create(void** event);
int kh_event_destroy(void* event);
int kh_event_record(void* event);
int kh_event_elapsed_ms(void* start, void* stop, float* ms);

/* Graphs of library launches.  Between kh_graph_begin_capture and kh_graph_end_capture, calls
 * that enqueue work are recorded instead of run; kh_graph_launch replays the recording on the
 * library stream.  Device blocks allocated or freed while the capture is open belong to the
 * graph until kh_graph_destroy (which waits for the stream), so a replay never touches memory
 * handed to other work.  Host-synchronous calls (kh_memcpy_h2d/d2h, kh_synchronize,
 * kh_empty_cache) fail while a capture is open.  No counterpart in the reference, whose decode
 * loop dispatches every op from the host per token (reference:
 * packages/model-utils/src/qwen3/for_causal_lm.ts:475-508); this replaces that per-token dispatch. */
int kh_graph_begin_capture(void);
int kh_graph_end_capture(void** graph);
int kh_graph_launch(void* graph);
int kh_graph_destroy(void* graph);

/* ------------------------------------------------------------------ support ops -------------- */

/* dst[i] = value for n elements of `dtype` (a fill kernel, never hipMemsetAsync).
 * Replaces the `zeros`/`fill` factory kernels (reference: packages/backend-webgpu/src/kernels/factory/index.ts:22-46). */
int kh_fill(void* dst, int64_t n, float value, int dtype);

/* Gathers a strided view of up to 6 dims into a contiguous buffer, converting dtype_src→dtype_dst
 * (f32/bf16 either way; i32→i32).  `src` points at storage element 0; `src_offset` is the view offset.
 * Replaces the `copy` kernel behind contiguous/clone/cast/copy_
 * (reference: packages/core/src/dispatch/handlers/copy.ts:40-71, :123-138; packages/backend-webgpu/src/kernels/copy/index.ts:13-33). */
int kh_copy_strided(const void* src, int64_t src_offset, void* dst, int ndim, const int64_t* shape,
                    const int64_t* src_strides, int dtype_src, int dtype_dst);

/* Ops of kh_map_strided. */
#define KH_MAP_COPY 0    /* out = a (cast to out's dtype) */
#define KH_MAP_ADD 1     /* out = a + s0 * b   (s0: add's alpha) */
#define KH_MAP_SUB 2     /* out = a - s0 * b   (s0: sub's alpha) */
#define KH_MAP_MUL 3     /* out = a * b */
#define KH_MAP_DIV 4     /* out = a / b */
#define KH_MAP_NEG 5     /* out = -a */
#define KH_MAP_COS 6     /* out = cos(a) */
#define KH_MAP_SIN 7     /* out = sin(a) */
#define KH_MAP_SILU 8    /* out = a / (1 + exp(-clamp(a, -88, 88))) */
#define KH_MAP_FILL 9    /* out = s0 */
#define KH_MAP_ARANGE 10 /* out = s0 + f32(i) * s1, i the element's row-major index in `shape` */

/* An elementwise op over the index space `shape` (ndim <= 8) in which every operand is addressed by
 * its own element strides from its pointer (the view's first element; a stride of 0 broadcasts an
 * axis, negative strides walk backwards): out[idx . out_strides] = op(a[idx . a_strides],
 * b[idx . b_strides]).  This is Kandle's iterator kernel contract (ITensorIterator operands carry
 * broadcast-aligned element strides and offsets: reference packages/types/src/tensor.ts:282-378,
 * built by packages/core/src/dispatch/TensorIterator.ts:660-725 computeBroadcastStrides) and
 * replaces the strided pointwise executor (packages/backend-webgpu/src/kernels/pointwise/
 * executor.ts:60-130) and the copy / cast / contiguous / clone / copy_ kernels (kernels/copy/
 * index.ts:13-33, called from packages/core/src/dispatch/handlers/copy.ts:175-206), the zeros /
 * full fills (handlers/factory.ts:50-61) and arange (kernels/factory/arangeExecutor.ts:37-44).
 * Math is fp32 with float (f32 or bf16) outputs, int32 two's-complement with an int32 output (copy
 * casts floats by truncation toward zero, saturated, NaN -> 0); inputs of any of the three dtypes.
 * Operands not used by the op may be NULL.  Nothing is read or written outside the element offsets
 * the strides give: the caller checks they lie in its buffers.  The output must not overlap an input
 * except element for element (identical strides). */
int kh_map_strided(int op, int ndim, const int64_t* shape, void* out, const int64_t* out_strides, int out_dtype,
                   const void* a, const int64_t* a_strides, int a_dtype, const void* b, const int64_t* b_strides,
                   int b_dtype, double s0, double s1);

/* out[i] = a[i] (op) b[i] for contiguous same-shape operands; op 0 = add, 1 = mul, 2 = sub.
 * Replaces the `add`/`mul`/`sub` pointwise iterator kernels for the contiguous case
 * (reference: packages/backend-webgpu/src/kernels/pointwise/ops.ts:329 mul, :437 add). */
int kh_binary(int op, const void* a, const void* b, void* out, int64_t n, int dtype);

/* out[i] = silu(x[i]) with silu(x) = x / (1 + exp(-clamp(x, -88, 88))).
 * Replaces the `silu` pointwise kernel (reference: packages/backend-webgpu/src/kernels/pointwise/ops.ts:299). */
int kh_silu(const void* x, void* out, int64_t n, int dtype);

/* out[i] = op(x[i]) for contiguous operands, computed in fp32: op 0 = neg, 1 = cos, 2 = sin.
 * Replaces the `neg`/`cos`/`sin` pointwise iterator kernels that Kandle's composite RoPE calls
 * (reference: packages/backend-webgpu/src/kernels/pointwise/ops.ts:168 neg, :201 sin, :202 cos;
 * callers packages/model-utils/src/rope.ts:254-255,590-630). */
int kh_unary(int op, const void* x, void* out, int64_t n, int dtype);

/* out[i] = start + f32(i) * step (f32/bf16) or start + i * step in int32 arithmetic (KH_I32), n
 * elements.  Replaces the `arange` factory kernel (reference:
 * packages/backend-webgpu/src/kernels/factory/arangeExecutor.ts:30-80, arangeShaderBuilder.ts:66-78). */
int kh_arange(void* out, int64_t n, double start, double step, int dtype);

/* out[r, i] = silu(gate[r, i]) * up[r, i] over rows x n, rows strided by the given element strides.
 * Fuses SwiGLUMLP's silu and mul (reference: packages/model-utils/src/mlp/swiglu.ts:119-134;
 * ops.ts:299 silu, :329 mul). */
int kh_silu_mul(const void* gate, int64_t gate_row_stride, const void* up, int64_t up_row_stride,
                void* out, int64_t out_row_stride, int64_t rows, int64_t n, int dtype);

/* out[i, :] = table[idx[i], :] for n_idx rows of row_elems elements; idx is device int32; an id
 * outside [0, n_rows) yields a zero row (checked on device, never read out of bounds).  The table
 * has `dtype`, the output `out_dtype` (the same, or float32 from bfloat16).
 * Replaces index_select behind embedding (reference: packages/core/src/dispatch/handlers/composite.ts:149-245;
 * packages/backend-webgpu/src/kernels/gather/index.ts:14-23). */
int kh_index_select(const void* table, int64_t n_rows, const int32_t* idx, int64_t n_idx, int64_t row_elems,
                    void* out, int dtype, int out_dtype);

/* index_select along any axis: a contiguous table viewed as [outer, n_rows, inner] (the axis of
 * length n_rows selected), out [outer, n_idx, inner] with out[a, i, :] = table[a, idx[i], :]; an id
 * outside [0, n_rows) yields zeros.  dtypes as kh_index_select.  Replaces the gather kernel's
 * index_select for every dim (reference: packages/core/src/dispatch/handlers/gather.ts:121,190;
 * packages/backend-webgpu/src/kernels/gather/index.ts:14-23). */
int kh_index_select_dim(const void* table, int64_t outer, int64_t n_rows, int64_t inner, const int32_t* idx,
                        int64_t n_idx, void* out, int dtype, int out_dtype);

/* out[r] = the lowest index of the maximum of row r (rows x n, contiguous), int32.
 * Replaces argmax (reference: packages/backend-webgpu/src/kernels/reduction/argShaderBuilder.ts:205-240)
 * with the greedy tie rule of sample() (packages/model-utils/src/sampling/index.ts:132,138). */
int kh_argmax(const void* x, int64_t rows, int64_t n, int32_t* out, int dtype);

/* Device-side bookkeeping of one greedy decode step, one thread: with p = *position,
 *   token_log[p + 1 - log_base] = *next_token  (if that index lies in [0, log_cap)),
 *   *position = p + 1,  *seq_len = p + 2.
 * next_token is the argmax just written for position p + 1; seq_len is the KV length the next
 * step attends over.  Keeps generateWithKVCache's loop state (reference:
 * packages/model-utils/src/qwen3/for_causal_lm.ts:475-508: append the token, advance the
 * position) on the device, so a captured decode step replays with no host round trip. */
int kh_greedy_advance(const int32_t* next_token, int32_t* position, int32_t* seq_len, int32_t* token_log,
                      int64_t log_base, int64_t log_cap);

/* One token chosen from a row of float32 logits [vocab] on the device.  do_sample != 0: temperature,
 * top-k (top_k <= 0: off), top-p (top_p >= 1: off), renormalisation, and a draw that walks the kept
 * probabilities in id order against r = (word 0 of philox4x32-10(key = seed, counter = (*counter, 0,
 * 0, 0)) >> 8) * 2^-24.  do_sample == 0 (greedy): the lowest id of the largest logit, with the
 * unfiltered softmax(logits / T) as its probabilities (counter may then be NULL).
 * Writes the token (int32), log(q_token + 1e-10) (logprob_out may be NULL) and the first display_k
 * ids of the descending logit order with their probabilities (NULL to skip).
 * counter is a device int32 (a generation loop advances it on the device).  Capturable into a
 * graph except for top-p without top-k, top_k > 1024 or display_k > 1024 (full-sort path).
 * Replaces sample() (reference: packages/model-utils/src/sampling/index.ts:103-243, softmaxCPU
 * :268-291, sampleFromProbs :294-311); the reference draws r with Math.random(). */
int kh_sample(const float* logits, int64_t vocab, int do_sample, double temperature, int top_k, double top_p,
              uint64_t seed, const int32_t* counter, int32_t* token_out, float* logprob_out, int display_k, int32_t* display_ids,
              float* display_probs);

/* Which kh_sample implementation runs: 0 (default) the selection path wherever it applies (greedy,
 * top-k <= 1024 with or without top-p, no filter; display_k <= 1024), 1 the full-sort path for
 * every call.  Both give the same results; the switch lets tests compare them.  No reference
 * counterpart.  Process-wide, not thread-safe. */
int kh_sample_set_path(int path);

/* out[4i .. 4i+3] = philox4x32-10(counters[4i .. 4i+3], key = (low, high 32 bits of seed)) for n
 * counters (device arrays).  The generator kh_sample draws from (Salmon et al., SC'11); no
 * reference counterpart (the reference draws with Math.random). */
int kh_philox4x32_10(uint64_t seed, const uint32_t* counters, int64_t n, uint32_t* out);

/* The attention block of one decode step of one sequence, from the raw q/k/v projection row to the
 * residual update: qk-norm + RoPE of the q heads and of the new token's k row (per-head RMSNorm with
 * q_norm_w / k_norm_w (bf16 [128]) and eps, angles float(p) * inv_freq[i]); the new k and v rows
 * written into the caches at row p = *position; split-K attention of the q heads over cache rows
 * [0, p] (GQA, any ratio hq / hkv, scale); the merge; then x += o W_o^T (w_o bf16 [n_out, hq*128] with row stride ldw,
 * x fp32 [n_out]).  qkv: [hq*128 + 2*hkv*128] (q heads, then k, then v) and the caches
 * [hkv][max_len][128] (element strides cache_strides = {k head, k row, v head, v row}) have `dtype`:
 * KH_BF16 (q and the new k row rounded to bf16 after RoPE, the merged row rounded to bf16 before
 * o_proj, as the unfused launches store them) or KH_F32 (every value kept in fp32: the reference's
 * float32 activations).  The position is read from device memory, so a captured step replays at
 * every position.  Two kernels (three when the cache exceeds 8 split-K chunks: 256 keys each for
 * bf16, 128 for fp32).  Fuses the decode path of GroupedQueryAttention.forward
 * (reference: packages/model-utils/src/attention/gqa.ts:246-430: projections, q_norm/k_norm,
 * RoPE, KV-cache update, SDPA, o_proj; kv-cache.ts:164-212) with the o_proj residual add of
 * Qwen3DecoderLayer.forward (qwen3/decoder_layer.ts:191-241). */
int kh_decode_attention_block(const void* qkv, const void* q_norm_w, const void* k_norm_w, const float* inv_freq,
                              float eps, const int32_t* position, void* k_cache, void* v_cache, int hq, int hkv,
                              int64_t max_len, const int64_t* cache_strides, float scale, const void* w_o,
                              int64_t ldw, int64_t n_out, float* x, int dtype);

/* ------------------------------------------------------------------ hot path ----------------- */

/* y[r, :] = x[r, :] * (1 / sqrt(mean(x[r, :]^2) + eps)) * w[:] (w may be NULL), fp32 math,
 * rows x n, x and y row-strided (contiguous rows).  x has `dtype`; y and w have `out_dtype` (the
 * same, or bfloat16 from a float32 residual stream).  Replaces the `rms_norm` kernel
 * (reference: packages/core/src/dispatch/handlers/normalize.ts:46-95;
 * packages/backend-webgpu/src/kernels/normalize/executor.ts:26-183; shaderBuilder.ts:343-414). */
int kh_rms_norm(const void* x, int64_t x_row_stride, const void* w, void* y, int64_t y_row_stride,
                int64_t rows, int64_t n, float eps, int dtype, int out_dtype);

/* Per-head RMSNorm (qk-norm) followed by rotary embedding, for q and k in one launch.
 * Token t of a [n_batch, seq_len] grid has position positions[t]; head h of q is read at
 *   q + b*s[0] + t_in_seq*s[1] + h*s[2]   and written at   q_out + b*s[6] + t_in_seq*s[7] + h*s[8],
 * k likewise with s[3..5] (read) and s[9..11] (write) — `strides` holds these 12 element strides.
 * Math per head row x (head_dim D): n = x / sqrt(mean(x^2)+eps) * w; then, with
 * f_i = float(positions[t]) * inv_freq[i mod D/2] (float32 product) and rotate_half(n) = cat(-n2, n1),
 *   out = n * cos(f) + rotate_half(n) * sin(f).
 * If v/v_out are non-NULL, v rows (k's head count and strides s[12..14] read, s[15..17] write;
 * `strides` then holds 18 values) are copied unchanged in the same launch (fused KV-cache write).
 * kv_cache_len > 0 selects cache addressing for k_out and v_out: token t is written at sequence
 * index positions[t] instead of t_in_seq, and a token whose position lies outside
 * [0, kv_cache_len) writes no K/V row; q_out keeps t_in_seq.  With positions held on the device,
 * one captured launch then serves every decode step.
 * Replaces q_norm/k_norm + _permuteToHeadsFirst + applyRotaryPosEmbDirect + kvCache.update
 * (reference: packages/model-utils/src/attention/gqa.ts:279-309; packages/model-utils/src/rope.ts:159-261, :546-644;
 * packages/model-utils/src/kv-cache.ts:164-212). */
int kh_qk_norm_rope(const void* q, const void* k, void* q_out, void* k_out,
                    const void* v, void* v_out,
                    const void* wq, const void* wk, const float* inv_freq, const int32_t* positions,
                    int64_t n_batch, int64_t seq_len, int n_q_heads, int n_kv_heads, int head_dim,
                    const int64_t* strides, float eps, int dtype, int64_t kv_cache_len);

/* Scaled dot-product attention O = softmax(scale * Q K^T + causal) V with GQA
 * (query head h reads kv head h / (hq / hkv)); causal masks key j > query i (top-left aligned).
 * Shapes q [batch, hq, lq, d], k/v [batch, hkv, lk, d], o [batch, hq, lq, d]; `strides` holds 12
 * element strides: q (batch, head, seq), k (…), v (…), o (…); the d axis is contiguous.
 * bf16 with d == 64 or 128 runs the MFMA flash kernel; fp32 with d in {32, 64, 96, 128} the fp32
 * MFMA flash kernel; lq == 1 without causal masking, d == 64 or 128 and 16-byte aligned q / k / v
 * rows runs split-K decode; any GQA ratio hq / hkv on every route; otherwise a LDS-tiled fp32-math kernel
 * (d <= 256).  Replaces the `flash_attention` kernel
 * (reference signature packages/types/src/backend/register.ts:102-109; semantics
 * packages/backend-webgpu/src/kernels/attention/builder.ts:138-329; called from
 * packages/core/src/dispatch/handlers/composite.ts:312-316). */
int kh_flash_attention(const void* q, const void* k, const void* v, void* o,
                       int batch, int hq, int hkv, int64_t lq, int64_t lk, int d,
                       const int64_t* strides, float scale, int causal, int dtype);

/* kh_flash_attention for fp32 q / k / v / o in split-bf16 form: every fp32 operand value x is
 * taken as hi = bf16(x) plus lo = bf16(x - hi) and every product as three bf16 MFMAs (hi*hi +
 * hi*lo + lo*hi, fp32 accumulate), so S = Q K^T and O = P V are each within about 2^-15 relative
 * of the fp32 products (l sums the fp32 P) at a sixth of the fp32 MFMA's cycles.  Taken for
 * d == 128 (any GQA ratio), scale > 0, lq > 1, 16-byte aligned rows with strides in multiples of
 * 4 elements; any other call runs kh_flash_attention's fp32 route.  Causal and not.  The float32-activation Qwen3 prefill's attention: the reference's f32 attention
 * (packages/backend-webgpu/src/kernels/attention/builder.ts:138-329) within the error above. */
int kh_flash_attention_split(const void* q, const void* k, const void* v, void* o,
                             int batch, int hq, int hkv, int64_t lq, int64_t lk, int d,
                             const int64_t* strides, float scale, int causal);

/* Scaled dot-product attention with an explicit additive mask:
 * O = softmax(scale * Q K^T + mask) V, GQA as kh_flash_attention, no causal masking.  This is the
 * reference's attnMask route (packages/core/src/dispatch/handlers/composite.ts:279-300: matmul with
 * alpha = scale, add_Tensor(mask), softmax(-1), matmul), fused into one kernel; the reference has
 * no kernel for it.  Its softmax (packages/backend-webgpu/src/kernels/normalize/shaderBuilder.ts:
 * 143-213) starts the row max at f32(-1e38), so a row whose every score is far below -1e38
 * (e.g. all -inf) is 0 / 0: that row's output is NaN.  The mask (dtype KH_F32 or KH_BF16) is
 * read as mask[b * mask_strides[0] + h * mask_strides[1] + i * mask_strides[2] + j * mask_strides[3]]
 * for batch b, query head h, query i, key j: element strides, 0 broadcasts an axis.  q/k/v/o
 * layouts and `strides` as kh_flash_attention.  bf16 with d == 64 or 128 runs the MFMA kernel (a mask
 * without unit key stride and 16-byte aligned 8-key runs is first packed into a scratch copy);
 * otherwise the fp32-math kernel (d <= 256). */
int kh_flash_attention_masked(const void* q, const void* k, const void* v, void* o,
                              int batch, int hq, int hkv, int64_t lq, int64_t lk, int d,
                              const int64_t* strides, float scale, const void* mask,
                              const int64_t* mask_strides, int mask_dtype, int dtype);

/* Decode attention for one query token per sequence against a KV cache with per-sequence
 * lengths seq_lens[b] (device int32, each in [1, max_len]); no mask (the caller turns causal off
 * for 1-token decode, reference packages/model-utils/src/attention/gqa.ts:333-336).
 * q [batch, hq, d], o [batch, hq, d] (strides: batch, head), caches [batch, hkv, max_len, d]
 * (strides: batch, head, seq).  `strides` holds 10 values: q (b, h), k (b, h, s), v (b, h, s),
 * o (b, h).  Split-K over the sequence with a log-sum-exp merge; bf16 or f32; d == 64 or 128;
 * any GQA ratio; q and the caches 16-byte aligned with strides in 16-byte units.
 * Varlen extension of flash_attention for StaticKVCache views
 * (reference: packages/model-utils/src/kv-cache.ts:197-211; register.ts:102-109). */
int kh_decode_attention(const void* q, const void* k_cache, const void* v_cache, void* o,
                        const int32_t* seq_lens, int batch, int hq, int hkv, int d, int64_t max_len,
                        const int64_t* strides, float scale, int dtype);

/* kh_decode_attention without any device allocation: the same arguments, kernels and results,
 * with the split-K partials in a file-scope device array of 16 MiB (one per GPU, held until the
 * process ends, its address taken once at kh_init) instead of the caching allocator.  No
 * counterpart in the reference: it is for callers that cannot allocate device memory during the
 * call (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Limit: batch * hq * ceil(max_len / C) * (d + 2) * 4 bytes, C = 256 keys (bf16, d == 128), 128
 * (f32, 128), 512 (bf16, 64) or 256 (f32, 64), must not exceed 16 MiB (e.g. 8 sequences x 16
 * heads up to max_len 32768 in bf16 at d == 128), else KH_ERR_INVALID.  All calls
 * on one GPU share the array: calls that overlap on one GPU (from another stream) race. */
int kh_decode_attention_noalloc(const void* q, const void* k_cache, const void* v_cache, void* o,
                                const int32_t* seq_lens, int batch, int hq, int hkv, int d, int64_t max_len,
                                const int64_t* strides, float scale, int dtype);

/* C[m, n] = alpha * sum_k A[m, k] * B'[k, n] + beta * Cin[m, n] (+ bias[n]), fp32 accumulate,
 * where B' = B^T with B stored [n, k] (trans_b = 1, the nn.Linear weight layout) or B' = B stored
 * [k, n] (trans_b = 0).  A and B have `dtype`; C, Cin and bias have `out_dtype` (bf16 inputs may
 * produce fp32 output, e.g. logits; fp32 inputs produce fp32).  Row strides lda/ldb/ldc/ldcin in
 * elements; cin/bias may be NULL and cin may alias c (in-place residual add).  Replaces the
 * `matmul` kernel's mm path with its alpha/beta/C epilogue
 * (reference: packages/core/src/dispatch/matmulOps.ts:32-125, :408-496, :649-814;
 * packages/core/src/dispatch/handlers/composite.ts:55-77; packages/backend-webgpu/src/kernels/matrix/executor.ts:438-598). */
int kh_gemm(const void* a, int64_t lda, const void* b, int64_t ldb, void* c, int64_t ldc,
            const void* cin, int64_t ldcin, const void* bias,
            int64_t m, int64_t n, int64_t k, float alpha, float beta, int trans_b, int dtype, int out_dtype);

/* kh_gemm with A and B of their own dtypes.  Beyond kh_gemm's pairs it takes a float32 A with a
 * bfloat16 B (float32 C, Cin, bias): the reference's float32 matmul of float32 activations by
 * bfloat16 checkpoint weights, which the reference widens to float32 on load
 * (packages/core/src/io/safetensor/dtypes.ts:17-31), without widening them.  With trans_b = 1 and
 * m > 8 the MFMA tiles split each A value into bfloat16 hi = bf16(a) and lo = bf16(a - hi) and
 * accumulate W hi + W lo in fp32 (relative error of each product 2^-17 or less); one-row and
 * skinny products multiply in fp32.  A bfloat16 A with a float32 B is refused.  Same matmul
 * contract as kh_gemm (reference: packages/core/src/dispatch/matmulOps.ts:32-125, :408-496). */
int kh_gemm_ex(const void* a, int64_t lda, int a_dtype, const void* b, int64_t ldb, int b_dtype, void* c,
               int64_t ldc, const void* cin, int64_t ldcin, const void* bias, int64_t m, int64_t n, int64_t k,
               float alpha, float beta, int trans_b, int out_dtype);

/* h[m, f] = silu(g[m, f]) * u[m, f], g = x W_gate^T and u = x W_up^T (x_dtype KH_BF16: bf16 x,
 * fp32 accumulate, g and u rounded to bf16 before the product and h rounded to bf16 -- the values
 * the separate GEMM and silu*mul produce; KH_F32: fp32 x split as kh_gemm_ex does, g, u and h kept
 * in fp32, h fp32), for m rows and n_half = intermediate features, from ONE weight w_gu
 * [2 n_half, k] whose rows interleave gate and up in blocks of 8: rows 16i .. 16i+7 are gate rows
 * 8i .. 8i+7 and rows 16i+8 .. 16i+15 the matching up rows.  x [m, k] and h [m, n_half] with row
 * strides ldx / ldh (elements); n_half, k, ldx, ldw multiples of 8; x and w_gu 16-byte aligned.
 * The [m, 2 n_half] gate/up intermediate is never written.  Fuses SwiGLUMLP's gate and up
 * projections with silu and mul (reference: packages/model-utils/src/mlp/swiglu.ts:119-134;
 * packages/backend-webgpu/src/kernels/pointwise/ops.ts:299 silu, :329 mul). */
int kh_gemm_swiglu(const void* x, int64_t ldx, const void* w_gu, int64_t ldw, void* h, int64_t ldh, int64_t m,
                   int64_t n_half, int64_t k, int x_dtype);

/* The QKV projection of a prefill fused with qk-norm, RoPE and the KV-cache write:
 *   qkv[t, :] = x[t, :] W^T      (bf16 x [M, k] with row stride ldx, M = n_batch * seq_len tokens;
 *                                 w_qkv [(hq + 2 hkv) * 128, k] with row stride ldw: the q heads'
 *                                 rows, then the k heads', then the v heads'; fp32 accumulate,
 *                                 each value rounded to bf16 as kh_gemm stores it)
 * then, per token t (batch b = t / seq_len, index s = t % seq_len, position p = positions[t]) and
 * head row, exactly as kh_qk_norm_rope on that bf16 output: q rows normed with wq and rotated,
 * written at q_out + b*st[0] + s*st[1] + h*st[2]; k rows normed with wk and rotated, written at
 * k_out + b*st[3] + row*st[4] + h*st[5]; v rows unchanged at v_out + b*st[6] + row*st[7] + h*st[8],
 * where row = p when kv_cache_len > 0 (positions outside [0, kv_cache_len) write no K/V row) and
 * row = s otherwise (`strides` holds these 9 element strides, 16-byte multiples).  `dtype` is that
 * of x, q_out and the caches: KH_BF16 as described, or KH_F32 (x split as kh_gemm_ex does, the
 * projection kept in fp32 -- not rounded -- before qk-norm and RoPE, fp32 rows written).  head_dim
 * must be 128; operands 16-byte aligned; k, ldx, ldw multiples of 8.  The [M, (hq + 2 hkv) * 128]
 * projection output is never written.  Each output sums over all of k: the values kh_gemm followed
 * by kh_qk_norm_rope produce whenever kh_gemm runs its MFMA tiles unsplit (M > 8 and
 * kh_gemm_split_count() == 1).  Fuses GroupedQueryAttention's q/k/v projections with
 * q_norm / k_norm, RoPE and the cache update (reference: packages/model-utils/src/attention/
 * gqa.ts:269-309; rope.ts:546-644; kv-cache.ts:164-212); no single reference kernel. */
int kh_gemm_qk_norm_rope(const void* x, int64_t ldx, const void* w_qkv, int64_t ldw, int64_t n_batch,
                         int64_t seq_len, int64_t k, int n_q_heads, int n_kv_heads, int head_dim, const void* wq,
                         const void* wk, const float* inv_freq, const int32_t* positions, void* q_out, void* k_out,
                         void* v_out, const int64_t* strides, float eps, int64_t kv_cache_len, int dtype);

/* kh_gemm_qk_norm_rope with the RoPE angles read from rope_table (kh_rope_table's layout, rows
 * indexed by the projection's row m = batch * seq_len + index, 16-byte aligned) instead of
 * evaluated per head tile; rope_table == NULL is kh_gemm_qk_norm_rope.  The table holds the same
 * values the tile would compute, so the outputs are identical.  No reference counterpart (the
 * reference builds its cos / sin tables per forward in rope.ts:193-255). */
int kh_gemm_qk_norm_rope_table(const void* x, int64_t ldx, const void* w_qkv, int64_t ldw, int64_t n_batch,
                               int64_t seq_len, int64_t k, int n_q_heads, int n_kv_heads, int head_dim,
                               const void* wq, const void* wk, const float* inv_freq, const int32_t* positions,
                               void* q_out, void* k_out, void* v_out, const int64_t* strides, float eps,
                               int64_t kv_cache_len, int dtype, const float* rope_table);

/* RoPE angle table for n tokens: out[2 (t half + i)] = cos(float(positions[t]) * inv_freq[i]) and
 * out[2 (t half + i) + 1] = sin(...), i < half, fp32 -- the reference's f32 angle product and
 * cos / sin (packages/model-utils/src/rope.ts:193-255), once per forward for every layer's fused
 * QKV projection (kh_gemm_qk_norm_rope_table). */
int kh_rope_table(const int32_t* positions, int64_t n, const float* inv_freq, int half, float* out);

/* The split count kh_gemm uses for a [m, k] x [n, k]^T product with bf16 weights and contiguous,
 * 16-byte aligned operands, whether A is bf16 or fp32 (1: not split).  A caller that splits the same product with
 * kh_gemm_splitk_partials and adds the partials in split order reproduces kh_gemm bit for bit. */
int kh_gemm_split_count(int64_t m, int64_t n, int64_t k, int* splits);

/* The split-K stage of kh_gemm alone: part[s][i][j] (fp32, s < splits, row-major [m, n], split s
 * at part + s*m*n) = the sum over split s's k range of a[i, :] * b[j, :] (bf16 a [m, k] with row
 * stride lda -- or fp32 a with a_dtype KH_F32, split as kh_gemm_ex does -- and b [n, k] with row
 * stride ldb), k ranges of ceil(k / splits) rounded up to 128.
 * splits must equal kh_gemm_split_count's count for this shape (and the operands meet the MFMA
 * path's alignment: 16-byte aligned, k, lda, ldb multiples of 8).  The producer half of the
 * projection + residual + RMSNorm fusion below (no reference counterpart as a separate step:
 * it is the matmul of packages/core/src/dispatch/matmulOps.ts:32-125 before its epilogue). */
int kh_gemm_splitk_partials(const void* a, int64_t lda, const void* b, int64_t ldb, float* part,
                            int64_t m, int64_t n, int64_t k, int splits, int a_dtype);

/* Residual add of split-K partials followed by RMSNorm, one launch:
 *   x[r, :] = (part[0][r, :] + ... + part[splits-1][r, :]) + x[r, :]    (fp32, summed in split
 *             order from 0 -- what kh_gemm's split reduction with cin = x, beta = 1 stores)
 *   y[r, :] = rms_norm(x[r, :]) * w                                       (as kh_rms_norm)
 * part[s] starts s * split_stride elements after part; x (fp32) and y (out_dtype, bf16 or fp32,
 * like w) are contiguous [rows, n]; n % 8 == 0, n <= 2048, splits <= 8, 16-byte aligned pointers.
 * Fuses the residual add after o_proj / down_proj with the RMSNorm that follows it
 * (reference: packages/model-utils/src/qwen3/decoder_layer.ts:224-238 residual adds;
 * packages/backend-webgpu/src/kernels/normalize/shaderBuilder.ts:394-411 RMSNorm). */
int kh_add_rms_norm(const float* part, int splits, int64_t split_stride, float* x, const void* w, void* y,
                    int64_t rows, int64_t n, float eps, int out_dtype);

/* One-row projection (decode) with the producing op fused in front of it:
 *   c[j] = alpha * sum_i x'[i] * w[j, i] + beta * cin[j] (+ bias[j]),  j < n, i < k,
 * w bf16 [n, k] with row stride ldw (the nn.Linear weight), c/cin/bias of out_dtype, where x' is
 * the activation row exactly as the unfused producer would have stored it: with x_dtype KH_BF16
 * rounded to bf16 (and x, x2 below bf16), with x_dtype KH_F32 kept in fp32 (x, x2 fp32):
 *   prologue 0: x' = x (bf16 [k]) — plain linear (reference: packages/core/src/nn/modules/linear/Linear.ts:135-137);
 *   prologue 1: x' = rms_norm(x, norm_w, eps) with x the fp32 residual row [k] and norm_w bf16 [k]
 *               — RMSNorm then linear (reference: packages/core/src/nn/modules/normalization/RMSNorm.ts:92-99;
 *               packages/model-utils/src/qwen3/decoder_layer.ts:191-241);
 *   prologue 2: x' = silu(x) * x2 with x, x2 bf16 [k] (gate and up) — the SwiGLU product then
 *               down_proj (reference: packages/model-utils/src/mlp/swiglu.ts:119-134);
 *   prologue 3: x'[i] = silu(x[16(i/8) + i%8]) * x[16(i/8) + 8 + i%8] with x bf16 [2k] — the same
 *               product read from the output of a gate/up projection whose weight interleaves gate
 *               and up rows in blocks of 8 (kh_gemm_swiglu's layout; k % 8 == 0).
 * Needs k % 8 == 0, ldw % 8 == 0, a 16-byte aligned w and k <= 32768.  cin may alias c. */
int kh_gemv_fused(int prologue, const void* x, const void* x2, const void* norm_w, float eps,
                  const void* w, int64_t ldw, void* c, const void* cin, const void* bias,
                  int64_t n, int64_t k, float alpha, float beta, int out_dtype, int x_dtype);

/* One-row SwiGLU projection (decode): h[f] = silu(g_f) * u_f, f < n_half, bf16 out, where g and u
 * are the gate and up projections of the activation row x' (prologue 0: x' = x, bf16 [k];
 * prologue 1: x' = rms_norm(x, norm_w, eps) of the fp32 residual row, as kh_gemv_fused) by the
 * interleaved gate/up weight w_gu [2 n_half, k] of kh_gemm_swiglu (blocks of 8 rows; row stride
 * ldw).  x_dtype KH_BF16: x bf16 (prologue 0), g and u rounded to bf16 before the product and h
 * stored as bf16 -- the values that kh_gemv_fused's gate/up projection followed by its silu * mul
 * prologue produce, without the [2 n_half] gate/up row; KH_F32: x fp32 (prologue 0), x', g, u
 * and h kept in fp32, h fp32.  Fuses SwiGLUMLP's gate and up projections with silu and mul for one
 * token (reference: packages/model-utils/src/mlp/swiglu.ts:119-134; RMSNorm before it:
 * packages/core/src/nn/modules/normalization/RMSNorm.ts:92-99).  Needs n_half % 8 == 0,
 * k % 8 == 0, ldw % 8 == 0, a 16-byte aligned w_gu and k <= 32768. */
int kh_gemv_swiglu(int prologue, const void* x, const void* norm_w, float eps, const void* w_gu, int64_t ldw,
                   void* h, int64_t n_half, int64_t k, int x_dtype);

#ifdef __cplusplus
}
#endif

#endif /* KANDLE_HIP_H */
