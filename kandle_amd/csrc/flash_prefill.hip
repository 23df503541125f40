// bf16 causal / non-causal GQA flash-attention prefill for gfx950, head_dim 128.
//
// Semantics follow the reference kernel (packages/backend-webgpu/src/kernels/attention/builder.ts:138-329):
// score = (q . k) * scale, key j > query i masked when causal (top-left), query head h reads kv head
// h / (hq / hkv), online softmax in fp32, O = P V / l.
//
// Workgroup = 8 waves sharing one kv head: wave w serves query head g = w / (8/G) of the G query
// heads that read this kv head (G = hq / hkv in {1, 2, 4, 8}) and 32 query rows of a BMQ = 256/G
// row block.  K/V tiles of BN keys are staged in LDS (double buffered) and shared by all 8 waves, so
// every K/V byte fetched from L2 serves 256 query rows.
//
// Per wave and tile, with v_mfma_f32_32x32x16_bf16:
//   S^T (keys x queries) = K Q^T : A = K rows from LDS, B = Q held in registers for the whole loop.
//   O^T (d x queries)   += V^T P^T: A = V^T rows from LDS (V is transposed when staged), B = P.
// Each lane owns one query column: the row max / sum of the softmax are in-lane over BN/2 scores
// plus one exchange with lane ^ 32.  K rows enter the A operand in the order "swap bits 2 and 3 of
// the row index", which makes S^T accumulator registers j = 0..7 of lane group g hold keys 8g + j
// (j = 8..15: keys 16 + 8g + j - 8) -- exactly the B-operand layout of the PV product, so P never
// leaves registers.
//
// Global loads are raw buffer loads (out-of-range rows read as zero without a branch); V^T rows are
// stored with the 8-key block index XOR-swizzled by (d / 16) % 8 so that both the transposing
// 4-byte writes and the 16-byte operand reads spread over all LDS banks.
#include <cstdlib>

#include "attention.h"

using namespace kh;

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int FA_D = 128;
constexpr int FA_WAVES = 8;
constexpr int FA_THREADS = FA_WAVES * 64;
constexpr int FA_KSTR = FA_D + 8;  // K row stride in LDS (elements): 272 B keeps 16-lane reads conflict-free

template <int BN>
struct Tile {
  static constexpr int VSTR = BN + 8;                // V^T row stride (elements)
  static constexpr int KTILE = BN * FA_KSTR;         // elements
  static constexpr int VTILE = FA_D * VSTR;          // elements
  static constexpr int STAGE = KTILE + VTILE;        // elements per LDS stage
  static constexpr int NK = BN * 16 / FA_THREADS;    // 16-byte K chunks per thread per tile
  static constexpr int NVG = BN / 64;                // 64-key V groups per thread per tile
  static constexpr int NSUB = BN / 32;               // 32-key S^T subtiles
};

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

template <int BN, bool CAUSAL>
__global__ __launch_bounds__(FA_THREADS, 1) void flash_fwd_kernel(
    const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K, const uint16_t* __restrict__ V,
    uint16_t* __restrict__ O, int batch, int hq, int hkv, int lq, int lk, AttnStrides st, float scale,
    int n_qblocks) {
  using TL = Tile<BN>;
  __shared__ __attribute__((aligned(16))) uint16_t smem[2 * TL::STAGE];

  const int G = hq / hkv;
  const int wpg = FA_WAVES / G;   // waves per query head
  const int BMQ = 32 * wpg;       // query rows per head in this workgroup
  const int tid = threadIdx.x;
  // Wave-uniform by construction; readfirstlane lets the compiler keep it (and the Q buffer
  // resource built from it) in scalar registers instead of emitting waterfall loops.
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int r = lane & 31;        // query column owned by this lane
  const int g = lane >> 5;        // lane group

  // Heaviest (last) query blocks first for causal load balance; (b, kv head) fastest-varying.
  const int bh = blockIdx.x % (batch * hkv);
  const int qblk = n_qblocks - 1 - blockIdx.x / (batch * hkv);
  const int b = bh / hkv;
  const int hk = bh % hkv;
  const int hqi = hk * G + wave / wpg;
  const int q0 = qblk * BMQ;
  const int qw0 = q0 + (wave % wpg) * 32;
  const int qi = qw0 + r;

  // ---- Q operand (B of S^T = K Q^T): lane holds query qi, d = 16c + 8g + [0, 8) ----
  bf16x8 qreg[8];
  {
    const uint16_t* qh = Q + b * st.qb + hqi * st.qh;
    const auto rq = make_rsrc(qh, (uint32_t)(((int64_t)(lq - 1) * st.qs + FA_D) * 2));
    const uint32_t qoff = (uint32_t)(((int64_t)qi * st.qs + 8 * g) * 2);
#pragma unroll
    for (int c = 0; c < 8; ++c) qreg[c] = as_bf16x8(buf_load16(rq, qoff + 32 * c));
  }

  const int kv_end = CAUSAL ? min(lk, q0 + BMQ) : lk;
  const int ntiles = (kv_end + BN - 1) / BN;
  const int wave_last_q = min(qw0 + 31, lq - 1);

  const auto rk = make_rsrc(K + b * st.kb + hk * st.kh, (uint32_t)(((int64_t)(lk - 1) * st.ks + FA_D) * 2));
  const auto rv = make_rsrc(V + b * st.vb + hk * st.vh, (uint32_t)(((int64_t)(lk - 1) * st.vs + FA_D) * 2));

  // ---- staging: global -> registers -> LDS ----
  // K: chunk id = tid + 512 i -> key id / 16, d 8 * (id % 16).
  // V: thread owns key pair p = tid / 16 + 32 vg (keys 2p, 2p + 1) and d 8 * (tid % 16) .. + 8.
  uint4 kst[TL::NK], vst[TL::NVG][2];
  const int dcol = 8 * (tid & 15);
  auto load_tile = [&](int t) {
    const int kt = t * BN;
#pragma unroll
    for (int i = 0; i < TL::NK; ++i) {
      const int key = kt + ((tid + FA_THREADS * i) >> 4);
      kst[i] = buf_load16(rk, (uint32_t)(((int64_t)key * st.ks + dcol) * 2));
    }
#pragma unroll
    for (int vg = 0; vg < TL::NVG; ++vg)
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int key = kt + 2 * ((tid >> 4) + 32 * vg) + i;
        vst[vg][i] = buf_load16(rv, (uint32_t)(((int64_t)key * st.vs + dcol) * 2));
      }
  };
  auto store_tile = [&](int buf) {
    uint16_t* ks = smem + buf * TL::STAGE;
    uint16_t* vts = ks + TL::KTILE;
#pragma unroll
    for (int i = 0; i < TL::NK; ++i)
      *reinterpret_cast<uint4*>(ks + ((tid + FA_THREADS * i) >> 4) * FA_KSTR + dcol) = kst[i];
    const int swz = (dcol >> 4) & 7;  // rows dcol .. dcol + 7 share (d / 16) % 8
#pragma unroll
    for (int vg = 0; vg < TL::NVG; ++vg) {
      const int p = (tid >> 4) + 32 * vg;
      const int word = ((((p >> 2) ^ swz)) << 2) | (p & 3);  // swizzled 8-key block, pair inside it
      const uint32_t a[4] = {vst[vg][0].x, vst[vg][0].y, vst[vg][0].z, vst[vg][0].w};
      const uint32_t c[4] = {vst[vg][1].x, vst[vg][1].y, vst[vg][1].z, vst[vg][1].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        // row d = dcol + 2e holds (V[2p][d], V[2p+1][d]); row d + 1 likewise
        const uint32_t lo = (a[e] & 0xffffu) | (c[e] << 16);
        const uint32_t hi = (a[e] >> 16) | (c[e] & 0xffff0000u);
        *reinterpret_cast<uint32_t*>(vts + (dcol + 2 * e) * TL::VSTR + 2 * word) = lo;
        *reinterpret_cast<uint32_t*>(vts + (dcol + 2 * e + 1) * TL::VSTR + 2 * word) = hi;
      }
    }
  };

  f32x16 oacc[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int j = 0; j < 16; ++j) oacc[dt][j] = 0.f;
  float m_run = -INFINITY;  // running max of raw scores (q . k) for this lane's query
  float l_run = 0.f;        // this lane's partial softmax denominator
  const float c2 = scale * kLog2e;
  const int krow = (r & ~12) | ((r & 4) << 1) | ((r & 8) >> 1);  // r with bits 2 and 3 swapped

  if (ntiles > 0) {
    load_tile(0);
    store_tile(0);
  }
  // Retire every outstanding load (Q included) before the loop, so the compiler's wait counting
  // inside the loop only ever covers the next tile's prefetch and never stalls QK^T on it.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  for (int t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    const bool has_next = t + 1 < ntiles;
    if (has_next) load_tile(t + 1);

    const int kt = t * BN;
    const uint16_t* ks = smem + buf * TL::STAGE;
    const uint16_t* vts = ks + TL::KTILE;

    const bool wave_active = qw0 < lq && (!CAUSAL || kt <= wave_last_q);
    if (wave_active) {
      // ---- S^T = K Q^T over NSUB 32-key subtiles ----
      f32x16 sacc[TL::NSUB];
#pragma unroll
      for (int s = 0; s < TL::NSUB; ++s) {
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
      const bool need_mask = (kt + BN > lk) || (CAUSAL && kt + BN - 1 > qw0);
      if (need_mask) {
        const int lim = (CAUSAL ? min(lk, qi + 1) : lk) - kt - 8 * g;
#pragma unroll
        for (int s = 0; s < TL::NSUB; ++s)
#pragma unroll
          for (int j = 0; j < 16; ++j)
            if (32 * s + 16 * (j >> 3) + (j & 7) >= lim) sacc[s][j] = -INFINITY;
      }
      // ---- online softmax (fp32) ----
      float mx = m_run;
#pragma unroll
      for (int s = 0; s < TL::NSUB; ++s)
#pragma unroll
        for (int j = 0; j < 16; ++j) mx = fmaxf(mx, sacc[s][j]);
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float m_use = (mx == -INFINITY) ? 0.f : mx;
      const float alpha = fast_exp2((m_run - m_use) * c2);
      const bool moved = mx != m_run;
      m_run = mx;
      const float mb = m_use * c2;
      float psum = 0.f;
      bf16x8 pk[2 * TL::NSUB];
#pragma unroll
      for (int s = 0; s < TL::NSUB; ++s)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          bf16x8 pv;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float p = fast_exp2(sacc[s][8 * h + e] * c2 - mb);
            psum += p;
            pv[e] = (__bf16)p;
          }
          pk[2 * s + h] = pv;
        }
      l_run = l_run * alpha + psum;
      // Rescale O only when some lane's running max moved (alpha == 1 for every other lane).
      if (__any(moved)) {
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
          for (int j = 0; j < 16; ++j) oacc[dt][j] *= alpha;
      }
      // ---- O^T += V^T P^T ----
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        const int d = 32 * dt + r;
        const int swz = (d >> 4) & 7;
        const uint16_t* vrow = vts + d * TL::VSTR;
#pragma unroll
        for (int kc = 0; kc < 2 * TL::NSUB; ++kc) {
          const int blk = (2 * kc + g) ^ swz;
          const bf16x8 vv = as_bf16x8(*reinterpret_cast<const uint4*>(vrow + 8 * blk));
          oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vv, pk[kc], oacc[dt], 0, 0, 0);
        }
      }
    }

    if (has_next) store_tile(buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue: O[qi][d] = oacc / l; lane holds d = 32dt + 8(j/4) + 4g + j%4 ----
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

int flash_bn() {
  // Keys per LDS tile: 64 (measured fastest: 128 needs more than the 256 VGPRs two waves per SIMD
  // allow and spills); KANDLE_FLASH_BN=128 selects the other variant for tile sweeps.
  static int bn = [] {
    const char* e = getenv("KANDLE_FLASH_BN");
    return (e && atoi(e) == 128) ? 128 : 64;
  }();
  return bn;
}

template <int BN, bool CAUSAL>
void launch(const void* q, const void* k, const void* v, void* o, int batch, int hq, int hkv, int lq, int lk,
            const AttnStrides& st, float scale, int nqb, int nblk) {
  flash_fwd_kernel<BN, CAUSAL><<<nblk, FA_THREADS, 0, stream()>>>(
      (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v, (uint16_t*)o, batch, hq, hkv, lq, lk, st, scale,
      nqb);
}

}  // namespace

namespace kh {

bool flash_prefill_supported(const void* q, const void* k, const void* v, const void* o, int hq, int hkv,
                             int64_t lq, int64_t lk, int d, const AttnStrides& st) {
  const int G = hq / hkv;
  if (d != FA_D || !(G == 1 || G == 2 || G == 4 || G == 8)) return false;
  if (!(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(o))) return false;
  const int64_t s16[] = {st.qb, st.qh, st.qs, st.kb, st.kh, st.ks, st.vb, st.vh, st.vs};
  for (int64_t s : s16)
    if (s % 8 != 0) return false;
  if (st.ob % 4 || st.oh % 4 || st.os % 4) return false;
  // Per-head byte offsets (including the zero-filled rows past the end) must fit 31 bits.
  const int64_t lim = int64_t(1) << 31;
  if ((lq + 256) * st.qs * 2 >= lim || (lk + 256) * st.ks * 2 >= lim || (lk + 256) * st.vs * 2 >= lim) return false;
  return true;
}

int launch_flash_prefill_bf16(const void* q, const void* k, const void* v, void* o, int batch, int hq, int hkv,
                              int lq, int lk, const AttnStrides& st, float scale, bool causal) {
  const int G = hq / hkv;
  const int BMQ = 32 * (FA_WAVES / G);
  const int nqb = (lq + BMQ - 1) / BMQ;
  const int64_t nblk = (int64_t)nqb * batch * hkv;
  KH_REQUIRE(nblk <= INT32_MAX, "kh_flash_attention: grid too large");
  const int bn = flash_bn();
  if (bn == 64) {
    if (causal) launch<64, true>(q, k, v, o, batch, hq, hkv, lq, lk, st, scale, nqb, (int)nblk);
    else launch<64, false>(q, k, v, o, batch, hq, hkv, lq, lk, st, scale, nqb, (int)nblk);
  } else {
    if (causal) launch<128, true>(q, k, v, o, batch, hq, hkv, lq, lk, st, scale, nqb, (int)nblk);
    else launch<128, false>(q, k, v, o, batch, hq, hkv, lq, lk, st, scale, nqb, (int)nblk);
  }
  KH_CHECK_LAUNCH();
  return KH_OK;
}

}  // namespace kh
