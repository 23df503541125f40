// qk-norm followed by RoPE of one head row, the arithmetic shared by qk_norm_rope_kernel (norm.hip)
// and the epilogue of the fused QKV projection (gemm.hip), so that both round identically.
// Header-only device code.
#pragma once

#include "common.h"

namespace kh {

// Head row of head_dim D held by the LPR = D / 16 lanes of an aligned lane group: lane t of the
// group holds a = columns 8t .. 8t+7 and c = columns D/2 + 8t .. 8t+7 (every lane of the group must
// execute this: the sum of squares is a DPP group sum); wa / wb are the norm weight at those
// columns, cs / sn the cosine and sine of float(position) * inv_freq at them.
//   y = x * (1 / sqrt(mean(x^2) + eps)) * w                 (gqa.ts:279-286 q_norm / k_norm)
//   out = y * cos + rotate_half(y) * sin, rotate_half(y) = cat(-y2, y1)   (rope.ts:590-630)
template <int D>
__device__ __forceinline__ void qk_norm_rope_row(const float (&a)[8], const float (&c)[8], const float (&wa)[8],
                                                 const float (&wb)[8], const float (&cs)[8], const float (&sn)[8],
                                                 float eps, float (&oa)[8], float (&oc)[8]) {
  constexpr int LPR = D / 16;
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) ss += a[j] * a[j] + c[j] * c[j];
  ss = group_sum<LPR>(ss);
  const float inv = 1.0f / sqrtf(ss / (float)D + eps);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float na = (a[j] * inv) * wa[j];
    const float nc = (c[j] * inv) * wb[j];
    oa[j] = na * cs[j] + (-nc) * sn[j];
    oc[j] = nc * cs[j] + na * sn[j];
  }
}

}  // namespace kh
