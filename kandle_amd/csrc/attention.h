// Internal interface between the attention entry points (attention.hip) and the bf16 MFMA
// prefill kernel (flash_prefill.hip).
#pragma once

#include "common.h"

namespace kh {

// Element strides (batch, head, seq) of q, k, v, o; the head_dim axis is contiguous.
struct AttnStrides {
  int64_t qb, qh, qs, kb, kh, ks, vb, vh, vs, ob, oh, os;
};

// Explicit additive attention mask (the reference's attnMask route, composite.ts:279-300).
struct MaskArgs {
  int64_t sb, sh, sq, sk;  // element strides over (batch, query head, query, key); 0 broadcasts
  uint32_t bytes;          // byte extent of the mask: buffer loads past it read 0
  float inv_scale;         // 1 / scale: the mask joins raw q.k scores as mask / scale
  float floor_raw;         // the reference softmax's f32(-1e38) max floor in raw q.k units
};

// True when the bf16 MFMA prefill kernel takes this call (d = 64 or 128, any GQA ratio, 16-byte
// aligned rows, strides below 2^31, per-head byte ranges addressable with 32-bit buffer offsets).
bool flash_prefill_supported(const void* q, const void* k, const void* v, const void* o, int hq, int hkv,
                             int64_t lq, int64_t lk, int d, const AttnStrides& st);

// Launches the prefill kernel on the library stream; returns KH_OK or an error code.
int launch_flash_prefill_bf16(const void* q, const void* k, const void* v, void* o, int batch, int hq, int hkv,
                              int lq, int lk, int d, const AttnStrides& st, float scale, bool causal);

// The prefill kernel with an additive mask (f32 or bf16, KH_F32 / KH_BF16) instead of causal
// masking; 64-key stages.  Requires flash_prefill_supported(), ma.sk == 1, every 8-key run of the
// mask 16-byte aligned (base and sb, sh, sq multiples of 8 elements) and ma.bytes < 2^31.
int launch_flash_prefill_bf16_masked(const void* q, const void* k, const void* v, void* o, int batch, int hq,
                                     int hkv, int lq, int lk, int d, const AttnStrides& st, float scale,
                                     const void* mask, const MaskArgs& ma, int mask_dtype);

// True when the fp32 flash kernel (flash_f32.hip) takes this fp32 call: d in {32, 64, 96, 128},
// 16-byte aligned q / k / o with strides in multiples of 4 elements, 4-byte aligned v, per-head
// byte ranges below 2^31.
bool flash_f32_supported(const void* q, const void* k, const void* v, const void* o, int64_t lq, int64_t lk, int d,
                         const AttnStrides& st);

// fp32 attention with fp32 MFMA (causal or not, any lq / lk, GQA) on the library stream.
int launch_flash_f32(const void* q, const void* k, const void* v, void* o, int batch, int hq, int hkv, int lq, int lk,
                     int d, const AttnStrides& st, float scale, bool causal);

// True when the split-bf16 fp32 kernel takes this fp32 call: head_dim 128 (any GQA ratio), scale >
// 0, 16-byte aligned rows with strides in multiples of 4 elements below 2^31, per-head byte ranges
// below 2^31.
bool flash_split_supported(const void* q, const void* k, const void* v, const void* o, int hq, int hkv, int64_t lq,
                           int64_t lk, int d, const AttnStrides& st, float scale);

// fp32 attention with each fp32 operand split into bf16 hi + lo and every product as three bf16
// MFMAs (about 2^-15 relative of the fp32 products), causal or not, on the library stream.
int launch_flash_split_f32(const void* q, const void* k, const void* v, void* o, int batch, int hq, int hkv, int lq,
                           int lk, const AttnStrides& st, float scale, bool causal);

}  // namespace kh
