// Internal interface between the attention entry points (attention.hip) and the bf16 MFMA
// prefill kernel (flash_prefill.hip).
#pragma once

#include "common.h"

namespace kh {

// Element strides (batch, head, seq) of q, k, v, o; the head_dim axis is contiguous.
struct AttnStrides {
  int64_t qb, qh, qs, kb, kh, ks, vb, vh, vs, ob, oh, os;
};

// True when the bf16 MFMA prefill kernel takes this call (d = 128, G in {1,2,4,8}, 16-byte
// aligned rows, per-head byte ranges addressable with 32-bit buffer offsets).
bool flash_prefill_supported(const void* q, const void* k, const void* v, const void* o, int hq, int hkv,
                             int64_t lq, int64_t lk, int d, const AttnStrides& st);

// Launches the prefill kernel on the library stream; returns KH_OK or an error code.
int launch_flash_prefill_bf16(const void* q, const void* k, const void* v, void* o, int batch, int hq, int hkv,
                              int lq, int lk, const AttnStrides& st, float scale, bool causal);

}  // namespace kh
