// GEMM for the projections: C = alpha * A * B' + beta * Cin (+ bias), fp32 accumulate.
//
//  * bf16 inputs, trans_b = 1 (nn.Linear weight [n, k]), m > 8: MFMA tile kernel
//    (v_mfma_f32_32x32x16_bf16).
//  * m <= 8, trans_b = 1: weight-streaming kernel that reads each weight row once (decode, lm_head).
//  * anything else: LDS-tiled fp32-math kernel.
// The output (and Cin / bias) may be bf16 or fp32 independently of bf16 inputs, e.g. fp32 logits.
//
// Reference semantics: out = alpha * op(A) op(B) + beta * C (packages/core/src/dispatch/matmulOps.ts:32-125;
// epilogue packages/backend-webgpu/src/kernels/matrix/builder.ts:152-218); linear = x W^T + b
// (packages/core/src/dispatch/handlers/composite.ts:55-77).
#include <type_traits>

#include "common.h"
#include "gemv.h"
#include "qk_rope.h"

using namespace kh;
using namespace kh::gemv;

namespace {

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

// Four consecutive outputs of one row, vectorised when the row start allows it.
template <typename TO>
__device__ __forceinline__ void store4(TO* C, int64_t off, const float (&v)[4], bool vec, int valid) {
  if (vec && valid == 4) {
    if constexpr (sizeof(TO) == 2) {
      uint2 w;
      w.x = pack_bf16x2(v[0], v[1]);
      w.y = pack_bf16x2(v[2], v[3]);
      *reinterpret_cast<uint2*>(C + off) = w;
    } else {
      *reinterpret_cast<float4*>(C + off) = make_float4(v[0], v[1], v[2], v[3]);
    }
  } else {
    for (int e = 0; e < valid; ++e) Elem<TO>::store(C, off + e, v[e]);
  }
}

// =============================================================================================
// MFMA tile kernel.  Workgroup tile (64 WTM) x (64 WTN), k-step KS, 4 waves in a 2 x 2 layout, each
// wave (32 WTM) x (32 WTN) = WTM x WTN tiles of 32 x 32 (64 x 128 tiles: 8 waves in 2 x 4, each
// 32 x 32; gemm_waves): 128 x 128 for large problems, smaller
// tiles when 128-tiles would leave CUs idle.  The tile shape does not change any result: every
// output element is summed over k in the same 16-wide MFMA steps, in the same order, whatever the
// tile that holds it.  The product is formed as C^T = B A^T
// so that each lane owns one m row and 4 consecutive n per register group: A-operand = B rows (n),
// B-operand = A rows (m), both k-contiguous 16-byte LDS reads.  LDS double buffered; global loads are
// raw buffer loads (rows past M / N and columns past the k range read as zero without a branch).
//
// SPLIT: S workgroups share one output tile, each summing its K range (kchunk columns, a multiple
// of 128) of the products into fp32 partials part[split][m][n] (row-major, leading dimension N);
// gemm_splitk_reduce_kernel -- or a consumer such as kh_add_rms_norm -- then adds the S partials
// in split order (deterministic whichever workgroup finished last) and applies the epilogue.
// =============================================================================================
constexpr int kGemmPrefetch = 3;        // k-steps of global loads in flight per workgroup
// Split launches (short k ranges, 128 x 64 tiles): 2 steps in flight (C5 prefill, two runs: o_proj
// 14.56 -> 14.12 us, down 15.25 -> 14.93 us; the unsplit qkv product is 0.5 us slower at 2).
constexpr int kGemmSplitPrefetch = 2;
constexpr int kGemmT128Min = 256;       // 128-tiles from this many tiles up
constexpr int kGemmSplitTarget = 512;   // split K until about this many 64-tile workgroups
// Tiles (64 WTM) x (64 WTN) of split launches and of products too small for 128 x 128 tiles.
// C5 prefill, M = 512 (bench.py --only gemm, three runs): split launches with 128 x 64 tiles (one
// workgroup per CU) against 64 x 64 (two per CU): o_proj 15.25 -> 14.56 us, down 16.83 -> 15.25 us;
// the unsplit qkv and gate/up products are 0.5-1.5 us slower with 128 x 64 or 64 x 128 tiles, and
// a k-step of 128 on the rectangular tiles needs 256 VGPRs + 90 AGPRs and is slower everywhere.
constexpr int kGemmSplitWTM = 2, kGemmSplitWTN = 1;
// Split launches with fp32 activations (two MFMAs per k-step) take 64 x 128 tiles: C5 o_proj
// 17.9 -> 16.3 us, down 22.0 -> 19.4 us (64 x 64: 16.7 / 20.4; 128 x 128: 21.1 / 26.2).
constexpr int kGemmSplitF32WTM = 1, kGemmSplitF32WTN = 2;
constexpr int kGemmSmallWTM = 1, kGemmSmallWTN = 1;
constexpr int kGemmRectKS = 64;         // k-step of 128 x 64 and 64 x 128 tiles
constexpr int kMaxSplits = 8;
// Waves per workgroup on 64 x 128 tiles: 2 x 4 waves of 32 x 32, two per SIMD, so that one wave's
// LDS traffic (and with fp32 activations its hi / lo split of A) overlaps the other's MFMAs.  C5
// prefill, alternating builds on one box: float32 activations 2.87-2.90 -> 2.75-2.77 ms (GEMMs
// 77.3-78.0 -> 75.2-75.8 us per layer), bf16 2.363-2.367 -> 2.316-2.332 ms.  Other tiles keep four
// waves of (32 WTM) x (32 WTN).  Each output's k-steps and their order are unchanged.
constexpr int kGemmWaves64x128 = 8;
template <int WTM, int WTN>
constexpr int gemm_waves() { return WTM == 1 && WTN == 2 ? kGemmWaves64x128 : 4; }
constexpr int g_tile(int wt) { return 64 * wt; }

// PF: k-steps of prefetch in flight (register ring of PF stages; the loop is unrolled by PF so the
// stage indices are compile-time).  Tiles are numbered column-major (all m tiles of one n tile in a
// row) and, when the workgroup count is a multiple of 8, dealt to the 8 XCDs in contiguous ranges
// (the hardware hands workgroup i to XCD i mod 8): each XCD then reads its own columns of B (the
// weights) into its L2, and only A (the activations) is read by every XCD.
// SWIGLU (bf16 output, no split): B's rows interleave the gate and up projections in blocks of 8
// (rows 16i .. 16i + 7: gate rows 8i .. 8i + 7; rows 16i + 8 .. 16i + 15: the matching up rows), so
// every lane holds each gate accumulator and its up partner, and the epilogue stores
// C[m, f] = bf16(silu(bf16(gate)) * bf16(up)) over N / 2 features f -- the values the separate
// GEMM (bf16 store) and silu*mul kernel produce, without the [M, N] intermediate.
// QKNR (bf16, 64 x 128 tiles, no split): the QKV projection of a prefill, whose output columns are
// head rows of 128 (the q heads, then the k heads, then the v heads).  The epilogue stages the
// tile, rounded to bf16 as the plain GEMM stores it, in LDS and reads it back one head row per
// group of 8 lanes -- qk_norm_rope_kernel's layout -- to apply qk-norm + RoPE to q and k rows with
// the same arithmetic (qk_norm_rope_row) and write q rows to q_out and k / v rows into the KV cache,
// so the [M, N] projection output is never written.
struct QknrArgs {
  const uint16_t* wq = nullptr;       // q_norm / k_norm weights [128], bf16
  const uint16_t* wk = nullptr;
  const float* inv_freq = nullptr;    // [64]
  const int32_t* positions = nullptr; // [M]: RoPE position (and, with kv_cache_len > 0, cache row)
  void* q_out = nullptr;              // the activations' type: bf16, or fp32 with fp32 activations
  void* k_out = nullptr;
  void* v_out = nullptr;
  int64_t s[9] = {0, 0, 0, 0, 0, 0, 0, 0, 0};  // (batch, seq, head) element strides of q_out, k_out, v_out
  int hq = 0, hkv = 0;
  uint32_t seq_len = 1;               // token m is (batch m / seq_len, index m % seq_len)
  float eps = 0.f;
  int64_t kv_cache_len = 0;           // > 0: K/V rows at positions[m] (outside [0, len): not written)
  // Optional [M][64][2] (cos, sin) of float(positions[m]) * inv_freq[i] (rope_table_kernel, the same
  // expression): read instead of evaluating sincosf in every head tile.
  const float* rope_cs = nullptr;
};

// TA = float (fp32 activations, the reference's float32 arithmetic): A is read as fp32 and each
// value a is split into bf16 hi = bf16(a) and lo = bf16(a - hi) (a - hi is exact in fp32) when the
// tile is copied to LDS, as two planes; every k-step then runs two MFMAs into the same accumulator,
// W * hi and W * lo.  The weights are exactly bf16, so each product is W * a up to the 2^-17
// relative error of hi + lo, fp32 accumulate; the epilogues keep their fp32 values (no bf16
// rounding of the SwiGLU operands or of the qk-norm + RoPE input) and store fp32.
// LDS bytes of the k loop (two stages of the A planes and the B tile): two workgroups per CU when
// they fit the CU's 160 KiB, else one.
template <typename TA, int WTM, int WTN, int KS>
constexpr int gemm_lds_bytes() {
  return 2 * ((sizeof(TA) == 4 ? 2 : 1) * g_tile(WTM) + g_tile(WTN)) * (KS + 8) * 2;
}
template <typename TA, int WTM, int WTN, int KS>
constexpr int gemm_min_blocks() {
  return 2 * gemm_lds_bytes<TA, WTM, WTN, KS>() <= 160 * 1024 ? 2 : 1;
}

template <typename TO, int WTM, int WTN, int KS, bool SPLIT, int PF = 1, bool SWIGLU = false, bool QKNR = false,
          typename TA = uint16_t, int NW = 4>
__global__ __launch_bounds__(NW * 64, (gemm_min_blocks<TA, WTM, WTN, KS>())) void gemm_bf16_nt_kernel(
    const TA* __restrict__ A, int64_t lda, const uint16_t* __restrict__ B, int64_t ldb, TO* C, int64_t ldc,
    const TO* cin, int64_t ldcin, const TO* __restrict__ bias, int M, int N, int K, float alpha, float beta,
    int tiles_n, int splits, int kchunk, float* __restrict__ part, QknrArgs qa) {
  constexpr bool AF = std::is_same<TA, float>::value;
  constexpr int GM = g_tile(WTM), GN = g_tile(WTN);
  // NW waves in a 2 x NW/2 layout, each (32 WTM) x (32 AN): AN = WTN with four waves, WTN / 2 with
  // eight (two per SIMD).
  constexpr int NT = NW * 64, NWN = NW / 2, AN = 4 * WTN / NW;
  static_assert(NW == 4 || (NW == 8 && WTN % 2 == 0), "four waves, or eight on tiles of even WTN");
  constexpr int STR = KS + 8;  // LDS row stride (elements): 16-byte aligned, breaks bank aliasing
  constexpr int APL = AF ? 2 : 1;                  // A planes in LDS: bf16, or hi and lo
  constexpr int ATILE = GM * STR, BTILE = GN * STR, ASTG = APL * ATILE;
  constexpr int AE = 16 / (int)sizeof(TA);         // A elements per 16-byte chunk
  constexpr int CPR = KS / 8;                      // 16-byte chunks per B row per k-step
  constexpr int CPRA = KS / AE;                    // 16-byte chunks per A row per k-step
  constexpr int CPTA = GM * CPRA / NT;             // chunks per thread per A tile
  constexpr int CPTB = GN * CPR / NT;              // chunks per thread per B tile
  constexpr int CPTM = CPTA > CPTB ? CPTA : CPTB;
  __shared__ __attribute__((aligned(16))) uint16_t smem[2 * (ASTG + BTILE)];
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int r = lane & 31, g = lane >> 5;
  int bid = blockIdx.x;
  if (PF > 1 && (gridDim.x & 7) == 0) bid = (bid & 7) * (gridDim.x >> 3) + (bid >> 3);
  const int tile = SPLIT ? bid / splits : bid;
  const int split = SPLIT ? bid % splits : 0;
  const int tiles_m = (M + GM - 1) / GM;
  const int tm = PF > 1 ? tile % tiles_m : tile / tiles_n, tn = PF > 1 ? tile / tiles_m : tile % tiles_n;
  const int m0 = tm * GM, n0 = tn * GN;
  const int wm = (wave / NWN) * 32 * WTM, wn = (wave % NWN) * 32 * AN;
  const int kbeg = split * kchunk, kend = min(K, kbeg + kchunk);

  // Byte ranges of this tile's rows; a row past the matrix or a column past the range reads zero.
  const int mrows = min(GM, M - m0), nrows = min(GN, N - n0);
  const auto ra = make_rsrc(A + (int64_t)m0 * lda, (uint32_t)(((int64_t)(mrows - 1) * lda + K) * sizeof(TA)));
  const auto rb = make_rsrc(B + (int64_t)n0 * ldb, (uint32_t)(((int64_t)(nrows - 1) * ldb + K) * 2));

  // Staging: the A (B) tile is GM (GN) rows x KS k = GM * CPR chunks of 16 B, CPTA (CPTB) per
  // thread, in PF register stages.
  uint4 ast[PF][CPTA], bst[PF][CPTB];
  // Byte offsets fit 32 bits (the launcher checks 128 rows of lda / ldb); columns past kend map to
  // 0xffffffff, past the range, and read zero (K % 8 == 0, so a chunk is all in or all out).  The
  // loads are branch-free, so the compiler's load counting stays exact across the prefetch ring.
  auto load_tile = [&](int stg, int kt) {
#pragma unroll
    for (int i = 0; i < CPTM; ++i) {
      const int id = tid + NT * i;
      if (i < CPTA) {
        const int row = id / CPRA, kc = kt + AE * (id % CPRA);
        const uint32_t ao =
            kc < kend ? ((uint32_t)row * (uint32_t)lda + (uint32_t)kc) * (uint32_t)sizeof(TA) : 0xffffffffu;
        ast[stg][i < CPTA ? i : 0] = buf_load16(ra, ao);
      }
      if (i < CPTB) {
        const int row = id / CPR, kc = kt + 8 * (id % CPR);
        const bool in = kc < kend;
        const uint32_t bo = in ? ((uint32_t)row * (uint32_t)ldb + (uint32_t)kc) * 2u : 0xffffffffu;
        // B (the weights) with the non-temporal hint: C5 prefill 2.413-2.428 -> 2.396-2.402 ms
        bst[stg][i < CPTB ? i : 0] = buf_load16_nt(rb, bo);
      }
    }
  };
  auto store_tile = [&](int stg, int buf) {
    uint16_t* as = smem + buf * (ASTG + BTILE);
    uint16_t* bs = as + ASTG;
#pragma unroll
    for (int i = 0; i < CPTM; ++i) {
      const int id = tid + NT * i;
      if (i < CPTA) {
        const int row = id / CPRA, kc = AE * (id % CPRA);
        const uint4 v = ast[stg][i < CPTA ? i : 0];
        if constexpr (AF) {
          // four fp32 values -> bf16 hi (plane 0) and lo = bf16(a - hi) (plane 1)
          const float f[4] = {__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w)};
          const uint32_t h01 = pack_bf16x2(f[0], f[1]), h23 = pack_bf16x2(f[2], f[3]);
          const uint32_t l01 = pack_bf16x2(f[0] - lo_bf16(h01), f[1] - hi_bf16(h01));
          const uint32_t l23 = pack_bf16x2(f[2] - lo_bf16(h23), f[3] - hi_bf16(h23));
          *reinterpret_cast<uint2*>(as + row * STR + kc) = make_uint2(h01, h23);
          *reinterpret_cast<uint2*>(as + ATILE + row * STR + kc) = make_uint2(l01, l23);
        } else {
          *reinterpret_cast<uint4*>(as + row * STR + kc) = v;
        }
      }
      if (i < CPTB) {
        const int row = id / CPR, kc = 8 * (id % CPR);
        *reinterpret_cast<uint4*>(bs + row * STR + kc) = bst[stg][i < CPTB ? i : 0];
      }
    }
  };

  f32x16 acc[AN][WTM];  // [n tile][m tile]
#pragma unroll
  for (int a = 0; a < AN; ++a)
#pragma unroll
    for (int b = 0; b < WTM; ++b)
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[a][b][j] = 0.f;

  const int nk = kend > kbeg ? (kend - kbeg + KS - 1) / KS : 0;
  // Step t is in LDS buffer t & 1 and, before that, in register stage t % PF.  Iteration t loads
  // step t + PF into the stage step t has left, computes step t, then moves step t + 1 (loaded PF - 1
  // iterations earlier) into the other LDS buffer.  Steps past the end load zeros and are stored
  // into the idle buffer, so the main loop has no branches between a load and its use.
  auto step = [&](int t, int u) {
    load_tile(u, kbeg + (t + PF) * KS);
    const uint16_t* as = smem + (t & 1) * (ASTG + BTILE);
    const uint16_t* bs = as + ASTG;
#pragma unroll
    for (int kc = 0; kc < KS / 16; ++kc) {
      bf16x8 av[APL][WTM], bv[AN];
#pragma unroll
      for (int pl = 0; pl < APL; ++pl)
#pragma unroll
        for (int i = 0; i < WTM; ++i)
          av[pl][i] = as_bf16x8(
              *reinterpret_cast<const uint4*>(as + pl * ATILE + (wm + 32 * i + r) * STR + 16 * kc + 8 * g));
#pragma unroll
      for (int i = 0; i < AN; ++i)
        bv[i] = as_bf16x8(*reinterpret_cast<const uint4*>(bs + (wn + 32 * i + r) * STR + 16 * kc + 8 * g));
#pragma unroll
      for (int a = 0; a < AN; ++a)
#pragma unroll
        for (int b = 0; b < WTM; ++b)
#pragma unroll
          for (int pl = 0; pl < APL; ++pl)
            acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bv[a], av[pl][b], acc[a][b], 0, 0, 0);
    }
    store_tile((u + 1) % PF, (t + 1) & 1);
    __syncthreads();
  };
  if (nk > 0) {
#pragma unroll
    for (int s2 = 0; s2 < PF; ++s2) load_tile(s2, kbeg + s2 * KS);
    store_tile(0, 0);
    __syncthreads();
    int t = 0;
    for (; t + PF <= nk; t += PF) {
#pragma unroll
      for (int u = 0; u < PF; ++u) step(t + u, u);
    }
#pragma unroll
    for (int u = 0; u + 1 < PF; ++u)
      if (t + u < nk) step(t + u, u);
  }

  if constexpr (SPLIT) {
    // Raw fp32 partial of this split: part[split][m][n] (N % 4 == 0, so four consecutive n of a
    // register group are all in range or all out).
    float* mine = part + (int64_t)split * M * N;
#pragma unroll
    for (int b = 0; b < WTM; ++b) {
      const int m = m0 + wm + 32 * b + r;
      if (m >= M) continue;
#pragma unroll
      for (int a = 0; a < AN; ++a)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int n = n0 + wn + 32 * a + 8 * q + 4 * g;
          if (n >= N) continue;
          *reinterpret_cast<float4*>(mine + (int64_t)m * N + n) =
              make_float4(acc[a][b][4 * q], acc[a][b][4 * q + 1], acc[a][b][4 * q + 2], acc[a][b][4 * q + 3]);
        }
    }
    return;
  }

  // Epilogue: acc[a][b] lane holds m = m0 + wm + 32b + r, n = n0 + wn + 32a + 8(j/4) + 4g + j%4.
  if constexpr (QKNR) {
    static_assert(sizeof(TO) == sizeof(TA) && WTM == 1 && WTN == 2 && !SPLIT && !SWIGLU,
                  "QKNR: 64 x 128 tiles, output of the activations' type");
    // Staged row stride (elements of TA): 272 B (bf16) or 528 B (fp32), 16-byte aligned rows.
    constexpr int TSTR = 128 + 16 / (int)sizeof(TA);
    static_assert(GM * TSTR * (int)sizeof(TA) <= 2 * (ASTG + BTILE) * 2, "the staged tile fits the k loop's LDS");
    // Every wave has passed the k loop's last barrier: its LDS is free.  The tile is staged as the
    // plain GEMM would store it: rounded to bf16, or fp32 with fp32 activations.
    TA* tile = reinterpret_cast<TA*>(smem);
#pragma unroll
    for (int a = 0; a < AN; ++a)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        TA* dst = tile + (wm + r) * TSTR + wn + 32 * a + 8 * q + 4 * g;
        if constexpr (AF) {
          *reinterpret_cast<float4*>(dst) =
              make_float4(acc[a][0][4 * q], acc[a][0][4 * q + 1], acc[a][0][4 * q + 2], acc[a][0][4 * q + 3]);
        } else {
          uint2 w;
          w.x = pack_bf16x2(acc[a][0][4 * q], acc[a][0][4 * q + 1]);
          w.y = pack_bf16x2(acc[a][0][4 * q + 2], acc[a][0][4 * q + 3]);
          *reinterpret_cast<uint2*>(dst) = w;
        }
      }
    __syncthreads();
    // 8 elements of TA at p (16 or 32 bytes) <-> 8 floats
    auto ld8 = [](const TA* p, float (&v)[8]) {
      if constexpr (AF) {
        const float4 x0 = reinterpret_cast<const float4*>(p)[0], x1 = reinterpret_cast<const float4*>(p)[1];
        v[0] = x0.x; v[1] = x0.y; v[2] = x0.z; v[3] = x0.w; v[4] = x1.x; v[5] = x1.y; v[6] = x1.z; v[7] = x1.w;
      } else {
        unpack_bf16x8(*reinterpret_cast<const uint4*>(p), v);
      }
    };
    auto st8 = [](TA* p, const float (&v)[8]) {
      if constexpr (AF) {
        reinterpret_cast<float4*>(p)[0] = make_float4(v[0], v[1], v[2], v[3]);
        reinterpret_cast<float4*>(p)[1] = make_float4(v[4], v[5], v[6], v[7]);
      } else {
        *reinterpret_cast<uint4*>(p) = pack_bf16x8(v);
      }
    };
    const int hd = n0 / 128;                      // q heads, then k heads, then v heads
    const int t8 = lane & 7, rs = lane >> 3;      // 8 lanes per head row, 8 rows per wave step
    const bool is_q = hd < qa.hq, is_k = !is_q && hd < qa.hq + qa.hkv;
    float wa[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, wb[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    float f[8];
    if (is_q || is_k) {
      const uint16_t* wn8 = is_q ? qa.wq : qa.wk;
      unpack_bf16x8(*reinterpret_cast<const uint4*>(wn8 + 8 * t8), wa);
      unpack_bf16x8(*reinterpret_cast<const uint4*>(wn8 + 64 + 8 * t8), wb);
#pragma unroll
      for (int j = 0; j < 8; ++j) f[j] = qa.inv_freq[8 * t8 + j];
    }
    const bool cache_mode = qa.kv_cache_len > 0;
#pragma unroll
    for (int st = 0; st < GM / (8 * NW); ++st) {
      const int row = wave * (GM / NW) + st * 8 + rs;
      const int m = m0 + row;
      const bool live = m < M;
      float a8[8], c8[8];
      ld8(tile + row * TSTR + 8 * t8, a8);
      ld8(tile + row * TSTR + 64 + 8 * t8, c8);
      const int32_t ipos = live ? qa.positions[m] : 0;
      const uint32_t bi = live ? (uint32_t)m / qa.seq_len : 0u, si = live ? (uint32_t)m - bi * qa.seq_len : 0u;
      const int64_t kv_row = cache_mode ? (int64_t)ipos : (int64_t)si;
      const bool kv_ok = !cache_mode || (ipos >= 0 && (int64_t)ipos < qa.kv_cache_len);
      if (is_q || is_k) {
        float cs[8], sn[8], oa[8], oc[8];
        if (qa.rope_cs != nullptr) {
          const float4* t4 = reinterpret_cast<const float4*>(qa.rope_cs + ((int64_t)(live ? m : 0) * 64 + 8 * t8) * 2);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float4 v = t4[j];
            cs[2 * j] = v.x;
            sn[2 * j] = v.y;
            cs[2 * j + 1] = v.z;
            sn[2 * j + 1] = v.w;
          }
        } else {
          const float pos = (float)ipos;
#pragma unroll
          for (int j = 0; j < 8; ++j) sincosf(pos * f[j], &sn[j], &cs[j]);
        }
        qk_norm_rope_row<128>(a8, c8, wa, wb, cs, sn, qa.eps, oa, oc);
        if (live && (is_q || kv_ok)) {
          TA* dst = is_q ? (TA*)qa.q_out + bi * qa.s[0] + si * qa.s[1] + (int64_t)hd * qa.s[2]
                         : (TA*)qa.k_out + bi * qa.s[3] + kv_row * qa.s[4] + (int64_t)(hd - qa.hq) * qa.s[5];
          st8(dst + 8 * t8, oa);
          st8(dst + 64 + 8 * t8, oc);
        }
      } else if (live && kv_ok) {
        TA* dst = (TA*)qa.v_out + bi * qa.s[6] + kv_row * qa.s[7] + (int64_t)(hd - qa.hq - qa.hkv) * qa.s[8];
        st8(dst + 8 * t8, a8);
        st8(dst + 64 + 8 * t8, c8);
      }
    }
    return;
  }
  const bool vec = ((reinterpret_cast<uintptr_t>(C) & (4 * sizeof(TO) - 1)) == 0) && ((ldc & 3) == 0);
  if constexpr (SWIGLU) {
    // Register groups q = 0, 2 hold gate rows n0 + wn + 32a + 8q + 4g + e, q + 1 the up rows 8 later:
    // feature f = (n0 + wn + 32a) / 2 + 4q + 4g + e (q = 0, 2).  N / 2 is a multiple of 8.
    const int NH = N / 2;
#pragma unroll
    for (int b = 0; b < WTM; ++b) {
      const int m = m0 + wm + 32 * b + r;
      if (m >= M) continue;
#pragma unroll
      for (int a = 0; a < AN; ++a)
#pragma unroll
        for (int q = 0; q < 4; q += 2) {
          const int f = (n0 + wn + 32 * a) / 2 + 4 * q + 4 * g;
          if (f >= NH) continue;
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if constexpr (AF)
              v[e] = silu_ref(acc[a][b][4 * q + e]) * acc[a][b][4 * q + 4 + e];
            else
              v[e] = silu_ref(round_bf16(acc[a][b][4 * q + e])) * round_bf16(acc[a][b][4 * q + 4 + e]);
          }
          store4<TO>(C, (int64_t)m * ldc + f, v, vec, 4);
        }
    }
    return;
  }
#pragma unroll
  for (int b = 0; b < WTM; ++b) {
    const int m = m0 + wm + 32 * b + r;
    if (m >= M) continue;
#pragma unroll
    for (int a = 0; a < AN; ++a)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int n = n0 + wn + 32 * a + 8 * q + 4 * g;
        if (n >= N) continue;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          v[e] = (n + e < N) ? epilogue<TO>(acc[a][b][4 * q + e], alpha, beta, cin, ldcin, bias, m, n + e) : 0.f;
        store4<TO>(C, (int64_t)m * ldc + n, v, vec, min(4, N - n));
      }
  }
}

// Split-K reduction: one thread per four consecutive outputs (N % 4 == 0), so every partial of the
// whole output is in flight at once; the splits are added in split order from 0, then the epilogue.
template <typename TO>
__global__ __launch_bounds__(256) void gemm_splitk_reduce_kernel(const float* __restrict__ part, int splits,
                                                                  TO* C, int64_t ldc, const TO* cin, int64_t ldcin,
                                                                  const TO* __restrict__ bias, int M, int N,
                                                                  float alpha, float beta) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t mn = (int64_t)M * N;
  if (gid * 4 >= mn) return;
  const int m = (int)(gid * 4 / N), n = (int)(gid * 4 % N);
  const float* tp = part + gid * 4;
  float4 pv[kMaxSplits];
#pragma unroll
  for (int s2 = 0; s2 < kMaxSplits; ++s2)
    pv[s2] = s2 < splits ? *reinterpret_cast<const float4*>(tp + s2 * mn) : make_float4(0.f, 0.f, 0.f, 0.f);
  float v[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s2 = 0; s2 < kMaxSplits; ++s2) {
    v[0] += pv[s2].x;
    v[1] += pv[s2].y;
    v[2] += pv[s2].z;
    v[3] += pv[s2].w;
  }
  const bool vec = ((reinterpret_cast<uintptr_t>(C) & (4 * sizeof(TO) - 1)) == 0) && ((ldc & 3) == 0);
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = epilogue<TO>(v[e], alpha, beta, cin, ldcin, bias, m, n + e);
  store4<TO>(C, (int64_t)m * ldc + n, v, vec, 4);
}

// =============================================================================================
// Skinny kernel for m <= 8 (trans_b = 1): each wave owns output columns n and streams weight row n
// once with 16-byte loads; the m rows of A are kept in LDS as fp32.
// =============================================================================================
constexpr int SK_MAXM = 8;
constexpr int SK_ROWS_PER_WAVE = 4;  // weight rows in flight per wave step

template <typename TA, typename T, typename TO>
__global__ __launch_bounds__(256) void gemv_nt_kernel(const TA* __restrict__ A, int64_t lda, const T* __restrict__ B,
                                                      int64_t ldb, TO* C, int64_t ldc, const TO* cin, int64_t ldcin,
                                                      const TO* __restrict__ bias, int M, int N, int K, float alpha,
                                                      float beta) {
  extern __shared__ float xs[];  // [M][K] fp32
  for (int i = threadIdx.x; i < M * K; i += blockDim.x) {
    const int mm = i / K, kk = i % K;
    xs[i] = Elem<TA>::load(A, (int64_t)mm * lda + kk);
  }
  __syncthreads();
  constexpr int EPL = 16 / sizeof(T);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int waves_total = gridDim.x * (blockDim.x >> 6);
  const int wid = blockIdx.x * (blockDim.x >> 6) + w;
  const bool vec = (K % EPL == 0) && (ldb % EPL == 0);
  for (int n0 = wid * SK_ROWS_PER_WAVE; n0 < N; n0 += waves_total * SK_ROWS_PER_WAVE) {
    float acc[SK_ROWS_PER_WAVE][SK_MAXM];
#pragma unroll
    for (int rr = 0; rr < SK_ROWS_PER_WAVE; ++rr)
#pragma unroll
      for (int mm = 0; mm < SK_MAXM; ++mm) acc[rr][mm] = 0.f;
    if (vec) {
      for (int k0 = lane * EPL; k0 < K; k0 += 64 * EPL) {
        uint4 wv[SK_ROWS_PER_WAVE];
#pragma unroll
        for (int rr = 0; rr < SK_ROWS_PER_WAVE; ++rr) {
          const int n = n0 + rr;
          wv[rr] = n < N ? *reinterpret_cast<const uint4*>(B + (int64_t)n * ldb + k0) : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int rr = 0; rr < SK_ROWS_PER_WAVE; ++rr) {
          float wf[EPL];
          if constexpr (sizeof(T) == 2) {
            const uint32_t u[4] = {wv[rr].x, wv[rr].y, wv[rr].z, wv[rr].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              wf[2 * e] = lo_bf16(u[e]);
              wf[2 * e + 1] = hi_bf16(u[e]);
            }
          } else {
            wf[0] = __uint_as_float(wv[rr].x); wf[1] = __uint_as_float(wv[rr].y);
            wf[2] = __uint_as_float(wv[rr].z); wf[3] = __uint_as_float(wv[rr].w);
          }
#pragma unroll
          for (int mm = 0; mm < SK_MAXM; ++mm) {
            if (mm < M) {
              float s = 0.f;
#pragma unroll
              for (int e = 0; e < EPL; ++e) s += wf[e] * xs[mm * K + k0 + e];
              acc[rr][mm] += s;
            }
          }
        }
      }
    } else {
      for (int kk = lane; kk < K; kk += 64)
#pragma unroll
        for (int rr = 0; rr < SK_ROWS_PER_WAVE; ++rr) {
          const int n = n0 + rr;
          const float wf = n < N ? Elem<T>::load(B, (int64_t)n * ldb + kk) : 0.f;
#pragma unroll
          for (int mm = 0; mm < SK_MAXM; ++mm)
            if (mm < M) acc[rr][mm] += wf * xs[mm * K + kk];
        }
    }
#pragma unroll
    for (int rr = 0; rr < SK_ROWS_PER_WAVE; ++rr)
#pragma unroll
      for (int mm = 0; mm < SK_MAXM; ++mm) {
        if (mm < M) {
          const float s = wave_sum(acc[rr][mm]);
          const int n = n0 + rr;
          if (lane == 0 && n < N)
            Elem<TO>::store(C, (int64_t)mm * ldc + n, epilogue<TO>(s, alpha, beta, cin, ldcin, bias, mm, n));
        }
      }
  }
}

// =============================================================================================
// One-row GEMV (decode: m = 1, bf16 weight [n, k], trans_b = 1) with an optional fused prologue
// that forms the activation row the way the unfused ops would have stored it (bf16):
//   PRO_NONE      x' = x                               (x bf16)
//   PRO_RMSNORM   x' = bf16(rms_norm(x, norm_w, eps))  (x fp32 residual row, norm_w bf16)
//   PRO_SILU_MUL  x' = bf16(silu(x) * x2)              (x, x2 bf16: gate and up halves)
//   PRO_SILU_MUL_IL x'[i] = bf16(silu(x[16(i/8) + i%8]) * x[16(i/8) + 8 + i%8])  (x bf16 [2k]: the
//                 gate/up row of a projection whose weight interleaves gate and up rows in blocks of 8)
//   PRO_ATTN_MERGE x' = bf16(split-K decode attention merged)  (x: the fp32 partials of one sequence,
//                 o[h][chunk][128] then (m, l)[h][chunk]; see AttnMerge)
// Each workgroup forms x' once in LDS (fp32, zero past k); each wave then owns U weight rows and
// streams them with raw 16-byte buffer loads, CB chunks of 512 columns per row in flight (rows past
// n read as zero), and reduces each row across the wave.  Every weight byte is read once.
// =============================================================================================
template <int U, int PRO, typename TO, bool PAIR8 = false, bool EX = false>
__global__ __launch_bounds__(256) void gemv1_kernel(const void* __restrict__ x, const void* __restrict__ x2,
                                                    const uint16_t* __restrict__ nw, float eps,
                                                    const uint16_t* __restrict__ W, int64_t ldw, uint32_t w_bytes,
                                                    TO* C, const TO* cin, const TO* __restrict__ bias, int N, int K,
                                                    int nch, float alpha, float beta, AttnMerge am) {
  extern __shared__ float xs[];
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  GemvRows<U, PAIR8, EX> g;
  g.init(W, ldw, w_bytes, N, K, nch, (int64_t)blockIdx.x * (blockDim.x >> 6) + w,
         (int64_t)gridDim.x * (blockDim.x >> 6));
  // The first batch is in flight while the workgroup forms x'.
  g.issue_first();
  gemv_prologue<PRO, EX>(xs, x, x2, nw, eps, K, nch * GV_CHUNK, am);
  g.template run<TO>(xs, C, cin, bias, alpha, beta);
}

// x' is staged in LDS as fp32: k <= 32768 (128 KiB of the CU's 160 KiB; above 64 KiB one
// workgroup per CU, the size of the down projections of 14B- and 32B-class models).
constexpr size_t kGemvMaxLds = 128 * 1024;

// Launches gemv1_kernel; returns false (nothing launched) when the operands do not fit its
// assumptions (16-byte aligned weight rows, 32-bit byte offsets, x' within kGemvMaxLds of LDS) or
// the runtime refuses the workgroup's LDS size.
template <int U, int PRO, typename TO, bool PAIR8 = false, bool EX = false>
bool gemv1_go(const void* x, const void* x2, const void* nw, float eps, const uint16_t* W, int64_t ldw,
              uint32_t w_bytes, TO* C, const TO* cin, const TO* bias, int N, int K, int nch, float alpha, float beta,
              const AttnMerge& am) {
  const int64_t waves = (N + U - 1) / U;
  int64_t grid = (waves + 3) / 4;
  // Waves stride over the rows past the first grid: lm_head (151936 rows, 8 per wave) at most 2048
  // workgroups: 69.5 -> 59.9 us graph-replayed with 4 rows per wave and 8192 workgroups before.
  if (grid > 2048) grid = 2048;
  const size_t shm = (size_t)nch * GV_CHUNK * sizeof(float);
  if (shm > 64 * 1024) {
    // dynamic LDS above 64 KiB is opted into once per kernel instantiation
    static const bool raised = hipFuncSetAttribute(reinterpret_cast<const void*>(&gemv1_kernel<U, PRO, TO, PAIR8, EX>),
                                                   hipFuncAttributeMaxDynamicSharedMemorySize,
                                                   (int)kGemvMaxLds) == hipSuccess;
    if (!raised) return false;
  }
  gemv1_kernel<U, PRO, TO, PAIR8, EX><<<(int)grid, 256, shm, stream()>>>(x, x2, (const uint16_t*)nw, eps, W, ldw,
                                                                         w_bytes, C, cin, bias, N, K, nch, alpha,
                                                                         beta, am);
  return true;
}

// The weight rows a one-row projection may address fit 32-bit byte offsets: row groups start below
// N and hold U rows, so the largest row index formed is N - 1 + U - 1 (rows at or past N are never
// stored, and the buffer range reads them as zero).
inline bool gemv_offsets_fit(int N, int U, int64_t ldw) {
  return ((int64_t)(N + U) * ldw) * 2 < (int64_t(1) << 32);
}

// SwiGLU one-row projection: h[f] = bf16(silu(bf16(gate_f)) * bf16(up_f)) (EX: silu(gate_f) * up_f in
// fp32, TO float) from the interleaved gate/up weight (2 * n_half rows, blocks of 8), one wave per
// (gate, up) row pair.  False when the operands do not fit (as launch_gemv1).
template <int PRO, bool EX = false, typename TO = uint16_t>
bool launch_gemv_swiglu(const void* x, const void* nw, float eps, const uint16_t* W, int64_t ldw, TO* H,
                        int n_half, int K) {
  const int N = 2 * n_half;
  if (n_half <= 0 || n_half % 8 != 0 || K <= 0) return false;
  const int nch = (K + GV_CHUNK - 1) / GV_CHUNK;
  const int64_t w_bytes = ((int64_t)(N - 1) * ldw + K) * 2;
  // a pair of row group q addresses rows up to 16 (q / 8) + q % 8 + 8 < N + 8
  if (K % 8 != 0 || ldw % 8 != 0 || !aligned16(W) || !gemv_offsets_fit(N, 8, ldw) ||
      (size_t)nch * GV_CHUNK * sizeof(float) > kGemvMaxLds)
    return false;
  return gemv1_go<2, PRO, TO, true, EX>(x, nullptr, nw, eps, W, ldw, (uint32_t)w_bytes, H, nullptr, nullptr, N, K, nch,
                                        1.f, 0.f, AttnMerge{});
}

template <int PRO, typename TO, bool EX = false>
bool launch_gemv1(const void* x, const void* x2, const void* nw, float eps, const uint16_t* W, int64_t ldw, TO* C,
                  const TO* cin, const TO* bias, int N, int K, float alpha, float beta, const AttnMerge& am = {}) {
  if (N <= 0 || K <= 0) return false;
  const int nch = (K + GV_CHUNK - 1) / GV_CHUNK;
  const int64_t w_bytes = ((int64_t)(N - 1) * ldw + K) * 2;
  const int U = N >= 16384 ? 8 : (N >= 2048 ? 2 : 1);
  if (K % 8 != 0 || ldw % 8 != 0 || !aligned16(W) || !gemv_offsets_fit(N, U, ldw) ||
      (size_t)nch * GV_CHUNK * sizeof(float) > kGemvMaxLds)
    return false;
  const uint32_t wb = (uint32_t)w_bytes;
  if (U == 8) return gemv1_go<8, PRO, TO, false, EX>(x, x2, nw, eps, W, ldw, wb, C, cin, bias, N, K, nch, alpha, beta, am);
  if (U == 2) return gemv1_go<2, PRO, TO, false, EX>(x, x2, nw, eps, W, ldw, wb, C, cin, bias, N, K, nch, alpha, beta, am);
  return gemv1_go<1, PRO, TO, false, EX>(x, x2, nw, eps, W, ldw, wb, C, cin, bias, N, K, nch, alpha, beta, am);
}

// =============================================================================================
// Generic tiled kernel (f32 or bf16 storage, trans_b 0/1): 16 x 16 threads, 64 x 64 tile, each
// thread 4 x 4 outputs, fp32 math.
// =============================================================================================
template <typename TA, typename T, typename TO>
__global__ __launch_bounds__(256) void gemm_generic_kernel(const TA* __restrict__ A, int64_t lda,
                                                           const T* __restrict__ B, int64_t ldb, TO* C, int64_t ldc,
                                                           const TO* cin, int64_t ldcin, const TO* __restrict__ bias,
                                                           int M, int N, int K, float alpha, float beta, int trans_b) {
  __shared__ float As[16][64 + 1];
  __shared__ float Bs[16][64 + 1];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
  float acc[4][4] = {};
  for (int k0 = 0; k0 < K; k0 += 16) {
    for (int i = threadIdx.x; i < 16 * 64; i += 256) {
      const int kk = i / 64, mm = i % 64;
      const int gm = m0 + mm, gk = k0 + kk;
      As[kk][mm] = (gm < M && gk < K) ? Elem<TA>::load(A, (int64_t)gm * lda + gk) : 0.f;
      const int gn = n0 + mm;
      float bv = 0.f;
      if (gn < N && gk < K)
        bv = trans_b ? Elem<T>::load(B, (int64_t)gn * ldb + gk) : Elem<T>::load(B, (int64_t)gk * ldb + gn);
      Bs[kk][mm] = bv;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 16; ++kk)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] += As[kk][ty * 4 + i] * Bs[kk][tx * 4 + j];
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int m = m0 + ty * 4 + i, n = n0 + tx * 4 + j;
      if (m < M && n < N)
        Elem<TO>::store(C, (int64_t)m * ldc + n, epilogue<TO>(acc[i][j], alpha, beta, cin, ldcin, bias, m, n));
    }
}

// Launch plan of the MFMA tile kernel for a bf16 [M, K] x [N, K]^T product.
struct GemmPlan {
  bool mfma = false;  // the MFMA tile kernel applies (else the skinny or generic kernel)
  int wtm = 1, wtn = 1, tiles_m = 0, tiles_n = 0, splits = 1, kchunk = 0;
  int64_t tiles = 0;
};

// Tile (64 wtm) x (64 wtn) of a product that does not split K.
inline void plain_tile(int M, int N, int& wtm, int& wtn) {
  const int64_t t128 = (int64_t)((M + 127) / 128) * ((N + 127) / 128);
  if (t128 >= kGemmT128Min) {
    wtm = wtn = 2;
  } else {
    wtm = kGemmSmallWTM;
    wtn = kGemmSmallWTN;
  }
}

// aligned: both operands start on 16 bytes.  bf16: bf16 weights B with bf16 (a_bytes 2) or fp32
// (a_bytes 4, split into hi + lo) activations A.
GemmPlan gemm_plan(bool aligned, int64_t lda, int64_t ldb, int M, int N, int K, bool bf16, int trans_b,
                   int a_bytes = 2) {
  GemmPlan p;
  const int64_t lim = int64_t(1) << 31;
  if (!(bf16 && trans_b && M > SK_MAXM && K % 8 == 0 && lda % 8 == 0 && ldb % 8 == 0 && aligned &&
        (int64_t)g_tile(2) * lda * a_bytes < lim && (int64_t)g_tile(2) * ldb * 2 < lim))
    return p;
  p.mfma = true;
  // The K split is decided on the 64-tile count, whatever tile then runs it, so a shape's k ranges
  // -- and with them its sums, bit for bit -- do not depend on the tile: split when 64-tiles would
  // leave CUs idle and K is long, over up to 8 workgroups per tile.
  const int64_t t64 = (int64_t)((M + 63) / 64) * ((N + 63) / 64);
  const int64_t t128 = (int64_t)((M + 127) / 128) * ((N + 127) / 128);
  p.kchunk = K;
  if (t64 < 256 && K >= 1024 && N % 4 == 0) {
    const int64_t want = kGemmSplitTarget / t64;
    const int splits = want < 1 ? 1 : (want > kMaxSplits ? kMaxSplits : (int)want);
    if (splits > 1) {
      p.kchunk = ((K + splits - 1) / splits + 127) / 128 * 128;   // whole k-steps of 64 and 128
      p.splits = (K + p.kchunk - 1) / p.kchunk;
    }
  }
  // 128-tiles when they fill the chip (256 CUs), else smaller tiles for more workgroups.
  if (p.splits > 1) {
    p.wtm = a_bytes == 4 ? kGemmSplitF32WTM : kGemmSplitWTM;
    p.wtn = a_bytes == 4 ? kGemmSplitF32WTN : kGemmSplitWTN;
  } else {
    plain_tile(M, N, p.wtm, p.wtn);
  }
  (void)t128;
  p.tiles_m = (M + g_tile(p.wtm) - 1) / g_tile(p.wtm);
  p.tiles_n = (N + g_tile(p.wtn) - 1) / g_tile(p.wtn);
  p.tiles = (int64_t)p.tiles_m * p.tiles_n;
  return p;
}

// One launch of the tile kernel with tile (64 WTM) x (64 WTN) and k-step KS.
template <typename TO, int WTM, int WTN, int KS, bool SWIGLU = false, typename TA = uint16_t>
void go_tiles(int nblk, int splits, const TA* A, int64_t lda, const uint16_t* B, int64_t ldb, TO* C,
              int64_t ldc, const TO* CI, int64_t ldcin, const TO* BI, int M, int N, int K, float alpha, float beta,
              int tiles_n, int kchunk, float* part) {
  // fp32 activations hold twice the A chunks per stage: two stages in flight keep the ring in registers
  constexpr int PF = std::is_same<TA, float>::value ? 2 : kGemmPrefetch;
  constexpr int NW = gemm_waves<WTM, WTN>();
  if (!SWIGLU && splits > 1)
    gemm_bf16_nt_kernel<TO, WTM, WTN, KS, true, kGemmSplitPrefetch, false, false, TA, NW><<<nblk, NW * 64, 0,
                                                                                            stream()>>>(
        A, lda, B, ldb, C, ldc, CI, ldcin, BI, M, N, K, alpha, beta, tiles_n, splits, kchunk, part, QknrArgs{});
  else
    gemm_bf16_nt_kernel<TO, WTM, WTN, KS, false, PF, SWIGLU, false, TA, NW><<<nblk, NW * 64, 0, stream()>>>(
        A, lda, B, ldb, C, ldc, CI, ldcin, BI, M, N, K, alpha, beta, tiles_n, 1, K, nullptr, QknrArgs{});
}

// Dispatch on the plan's tile: 128 x 128 with k-step 64; 64 x 64 with k-step 128 when split or
// with at most one tile per CU, else k-step 64 (C5 prefill qkv, 512 tiles: 11.75 -> 10.9 us with
// k-step 64; gate/up, 768 tiles: 14.0 -> 16.1 us with k-step 128); 128 x 64 and 64 x 128 with
// kGemmRectKS.  fp32 activations (TA float: two LDS planes of A) keep a k-step of 64 on 64 x 64
// tiles, so that two workgroups still fit a CU's LDS.
template <typename TO, bool SWIGLU = false, typename TA = uint16_t>
void launch_tile_shape(int wtm, int wtn, int64_t tiles, int splits, const TA* A, int64_t lda,
                       const uint16_t* B, int64_t ldb, TO* C, int64_t ldc, const TO* CI, int64_t ldcin, const TO* BI,
                       int M, int N, int K, float alpha, float beta, int tiles_n, int kchunk, float* part) {
  constexpr bool AF = std::is_same<TA, float>::value;
  const int nblk = (int)(tiles * splits);
  if (wtm == 2 && wtn == 2)
    go_tiles<TO, 2, 2, 64, SWIGLU, TA>(nblk, splits, A, lda, B, ldb, C, ldc, CI, ldcin, BI, M, N, K, alpha, beta,
                                       tiles_n, kchunk, part);
  else if (wtm == 2)
    go_tiles<TO, 2, 1, kGemmRectKS, SWIGLU, TA>(nblk, splits, A, lda, B, ldb, C, ldc, CI, ldcin, BI, M, N, K, alpha,
                                                beta, tiles_n, kchunk, part);
  else if (wtn == 2)
    go_tiles<TO, 1, 2, kGemmRectKS, SWIGLU, TA>(nblk, splits, A, lda, B, ldb, C, ldc, CI, ldcin, BI, M, N, K, alpha,
                                                beta, tiles_n, kchunk, part);
  else if (!AF && (splits > 1 || tiles <= 256))
    go_tiles<TO, 1, 1, AF ? 64 : 128, SWIGLU, TA>(nblk, splits, A, lda, B, ldb, C, ldc, CI, ldcin, BI, M, N, K, alpha,
                                                  beta, tiles_n, kchunk, part);
  else
    go_tiles<TO, 1, 1, 64, SWIGLU, TA>(nblk, splits, A, lda, B, ldb, C, ldc, CI, ldcin, BI, M, N, K, alpha, beta,
                                       tiles_n, kchunk, part);
}

// The MFMA tile kernel for plan p: C (or, with part != nullptr and p.splits > 1, only the fp32
// partials part[split][m][n]).
template <typename TO, typename TA = uint16_t>
void launch_gemm_tiles(const GemmPlan& p, const TA* A, int64_t lda, const uint16_t* B, int64_t ldb, TO* C,
                       int64_t ldc, const TO* CI, int64_t ldcin, const TO* BI, int M, int N, int K, float alpha,
                       float beta, float* part) {
  const int splits = part ? p.splits : 1;
  launch_tile_shape<TO, false, TA>(p.wtm, p.wtn, p.tiles, splits, A, lda, B, ldb, C, ldc, CI, ldcin, BI, M, N, K,
                                   alpha, beta, p.tiles_n, p.kchunk, part);
}

// A has element type TA, B has T (bf16 weights may meet fp32 activations: TA float, T uint16_t).
template <typename TA, typename T, typename TO>
int launch_gemm(const void* a, int64_t lda, const void* b, int64_t ldb, void* c, int64_t ldc, const void* cin,
                int64_t ldcin, const void* bias, int M, int N, int K, float alpha, float beta, int trans_b) {
  const TA* A = (const TA*)a;
  const T* B = (const T*)b;
  TO* C = (TO*)c;
  const TO* CI = (const TO*)cin;
  const TO* BI = (const TO*)bias;
  constexpr bool w_bf16 = sizeof(T) == 2;
  const GemmPlan p = gemm_plan(aligned16(a) && aligned16(b), lda, ldb, M, N, K, w_bf16, trans_b, (int)sizeof(TA));
  if constexpr (w_bf16) {
    if (p.mfma) {
      KH_REQUIRE(p.tiles <= INT32_MAX / 8, "kh_gemm: grid too large");
      float* part = nullptr;
      if (p.splits > 1) part = (float*)scratch_alloc((size_t)p.splits * M * N * sizeof(float));
      launch_gemm_tiles<TO, TA>(p, A, lda, (const uint16_t*)B, ldb, C, ldc, CI, ldcin, BI, M, N, K, alpha, beta, part);
      if (part) {
        gemm_splitk_reduce_kernel<TO><<<(int)(((int64_t)M * N / 4 + 255) / 256), 256, 0, stream()>>>(
            part, p.splits, C, ldc, CI, ldcin, BI, M, N, alpha, beta);
        scratch_free(part);  // stream-ordered reuse only
      }
      KH_CHECK_LAUNCH();
      return KH_OK;
    }
    if (trans_b && M == 1) {
      constexpr bool EX = std::is_same<TA, float>::value;
      if (launch_gemv1<PRO_NONE, TO, EX>(a, nullptr, nullptr, 0.f, (const uint16_t*)B, ldb, C, CI, BI, N, K, alpha,
                                         beta)) {
        KH_CHECK_LAUNCH();
        return KH_OK;
      }
    }
  }
  if (trans_b && M <= SK_MAXM && (size_t)M * K * sizeof(float) <= 64 * 1024 && aligned16(b)) {
    const int waves_needed = (N + SK_ROWS_PER_WAVE - 1) / SK_ROWS_PER_WAVE;
    int grid = (waves_needed + 3) / 4;
    if (grid > 4096) grid = 4096;
    const size_t shm = (size_t)M * K * sizeof(float);
    gemv_nt_kernel<TA, T, TO><<<grid, 256, shm, stream()>>>(A, lda, B, ldb, C, ldc, CI, ldcin, BI, M, N, K, alpha,
                                                            beta);
    KH_CHECK_LAUNCH();
    return KH_OK;
  }
  dim3 grid((N + 63) / 64, (M + 63) / 64);
  KH_REQUIRE(grid.y <= 65535, "kh_gemm: m too large for the generic kernel");
  gemm_generic_kernel<TA, T, TO><<<grid, 256, 0, stream()>>>(A, lda, B, ldb, C, ldc, CI, ldcin, BI, M, N, K, alpha,
                                                             beta, trans_b);
  KH_CHECK_LAUNCH();
  return KH_OK;
}

// The fused SwiGLU projection: the MFMA tile kernel with the SWIGLU epilogue, tiles chosen as in
// launch_gemm, never split over K (the epilogue needs whole sums).  TA = TO: bf16, or fp32
// activations in and out.
template <typename TA>
int launch_gemm_swiglu(const TA* X, int64_t ldx, const uint16_t* W, int64_t ldw, TA* H, int64_t ldh, int M, int N,
                       int K) {
  int wtm = 1, wtn = 1;
  // fp32 activations (two MFMAs per k-step) take 64 x 128 tiles: C5 gate/up 27.0-27.3 -> 23.7-23.8 us
  // (128 x 64: 36.2 us); bf16 keeps the plain choice.  The tile never changes a sum.
  if constexpr (std::is_same<TA, float>::value)
    wtn = 2;
  else
    plain_tile(M, N, wtm, wtn);
  const int tiles_m = (M + g_tile(wtm) - 1) / g_tile(wtm), tiles_n = (N + g_tile(wtn) - 1) / g_tile(wtn);
  const int64_t tiles = (int64_t)tiles_m * tiles_n;
  KH_REQUIRE(tiles <= INT32_MAX, "kh_gemm_swiglu: grid too large");
  launch_tile_shape<TA, true, TA>(wtm, wtn, tiles, 1, X, ldx, W, ldw, H, ldh, nullptr, 0, nullptr, M, N, K, 1.f, 0.f,
                                  tiles_n, K, nullptr);
  KH_CHECK_LAUNCH();
  return KH_OK;
}

// The fused QKV projection: 64 x 128 tiles (one head row of 128 per tile column), never split.
template <typename TA>
int launch_gemm_qk_norm_rope(const TA* X, int64_t ldx, const uint16_t* W, int64_t ldw, int M, int N, int K,
                             const QknrArgs& qa) {
  const int tiles_m = (M + 63) / 64, tiles_n = N / 128;
  const int64_t tiles = (int64_t)tiles_m * tiles_n;
  KH_REQUIRE(tiles <= INT32_MAX, "kh_gemm_qk_norm_rope: grid too large");
  constexpr int PF = std::is_same<TA, float>::value ? 2 : kGemmPrefetch;
  constexpr int NW = gemm_waves<1, 2>();
  gemm_bf16_nt_kernel<TA, 1, 2, kGemmRectKS, false, PF, false, true, TA, NW><<<(int)tiles, NW * 64, 0, stream()>>>(
      X, ldx, W, ldw, nullptr, 0, nullptr, 0, nullptr, M, N, K, 1.f, 0.f, tiles_n, 1, K, nullptr, qa);
  KH_CHECK_LAUNCH();
  return KH_OK;
}

}  // namespace

namespace kh {
// o_proj of the decode attention block: C = alpha * merge(part) W^T + beta * cin (fp32 out), with
// the split-K partials merged in every workgroup's prologue (exact: the merged row kept in fp32,
// else rounded to bf16 as the unfused path stores it).  False when the shapes do not fit.
bool launch_gemv_attn_merge(const float* part, const AttnMerge& am, const uint16_t* W, int64_t ldw, float* C,
                            const float* cin, int N, int K, float alpha, float beta, bool exact) {
  if (am.max_chunks > kAttnMergeMaxChunks || K != am.hq * 128) return false;
  if (exact)
    return launch_gemv1<PRO_ATTN_MERGE, float, true>(part, nullptr, nullptr, 0.f, W, ldw, C, cin, nullptr, N, K,
                                                     alpha, beta, am);
  return launch_gemv1<PRO_ATTN_MERGE, float>(part, nullptr, nullptr, 0.f, W, ldw, C, cin, nullptr, N, K, alpha, beta,
                                             am);
}
}  // namespace kh

extern "C" {

int kh_gemm_ex(const void* a, int64_t lda, int a_dtype, const void* b, int64_t ldb, int b_dtype, void* c,
               int64_t ldc, const void* cin, int64_t ldcin, const void* bias, int64_t m, int64_t n, int64_t k,
               float alpha, float beta, int trans_b, int out_dtype) {
  KH_REQUIRE_INIT();
  KH_REQUIRE(m >= 0 && n >= 0 && k >= 0, "kh_gemm: negative extent");
  KH_REQUIRE(m <= INT32_MAX && n <= INT32_MAX && k <= INT32_MAX, "kh_gemm: extent too large");
  KH_REQUIRE(a_dtype == KH_BF16 || a_dtype == KH_F32, "kh_gemm: unsupported dtype %d", a_dtype);
  KH_REQUIRE(b_dtype == KH_BF16 || b_dtype == KH_F32, "kh_gemm: unsupported dtype %d", b_dtype);
  KH_REQUIRE(!(a_dtype == KH_BF16 && b_dtype == KH_F32),
             "kh_gemm: a bfloat16 A with a float32 B is not supported (float32 A with bfloat16 B is)");
  KH_REQUIRE(out_dtype == KH_BF16 || out_dtype == KH_F32, "kh_gemm: unsupported output dtype %d", out_dtype);
  KH_REQUIRE(!(a_dtype == KH_F32 && out_dtype == KH_BF16),
             "kh_gemm: fp32 inputs with a bf16 output are not supported");
  if (m == 0 || n == 0) return KH_OK;
  KH_REQUIRE(a && b && c, "kh_gemm: null pointer");
  KH_REQUIRE(lda >= k && ldc >= n && (trans_b ? ldb >= k : ldb >= n), "kh_gemm: leading dimension too small");
  KH_REQUIRE(cin == nullptr || ldcin >= n, "kh_gemm: ldcin too small");
  const int M = (int)m, N = (int)n, K = (int)k;
  if (a_dtype == KH_BF16 && out_dtype == KH_BF16)
    return launch_gemm<uint16_t, uint16_t, uint16_t>(a, lda, b, ldb, c, ldc, cin, ldcin, bias, M, N, K, alpha, beta,
                                                     trans_b);
  if (a_dtype == KH_BF16)
    return launch_gemm<uint16_t, uint16_t, float>(a, lda, b, ldb, c, ldc, cin, ldcin, bias, M, N, K, alpha, beta,
                                                  trans_b);
  if (b_dtype == KH_BF16)
    return launch_gemm<float, uint16_t, float>(a, lda, b, ldb, c, ldc, cin, ldcin, bias, M, N, K, alpha, beta,
                                               trans_b);
  return launch_gemm<float, float, float>(a, lda, b, ldb, c, ldc, cin, ldcin, bias, M, N, K, alpha, beta, trans_b);
}

int kh_gemm(const void* a, int64_t lda, const void* b, int64_t ldb, void* c, int64_t ldc, const void* cin,
            int64_t ldcin, const void* bias, int64_t m, int64_t n, int64_t k, float alpha, float beta, int trans_b,
            int dtype, int out_dtype) {
  return kh_gemm_ex(a, lda, dtype, b, ldb, dtype, c, ldc, cin, ldcin, bias, m, n, k, alpha, beta, trans_b, out_dtype);
}

int kh_gemm_split_count(int64_t m, int64_t n, int64_t k, int* splits) {
  KH_REQUIRE(splits != nullptr, "kh_gemm_split_count: null pointer");
  KH_REQUIRE(m >= 0 && n >= 0 && k >= 0 && m <= INT32_MAX && n <= INT32_MAX && k <= INT32_MAX,
             "kh_gemm_split_count: bad extents");
  // bf16 weights, contiguous and 16-byte aligned operands (the split does not depend on A's type)
  const GemmPlan p = gemm_plan(true, k, k, (int)m, (int)n, (int)k, true, 1);
  *splits = p.mfma ? p.splits : 1;
  return KH_OK;
}

int kh_gemm_splitk_partials(const void* a, int64_t lda, const void* b, int64_t ldb, float* part, int64_t m,
                            int64_t n, int64_t k, int splits, int a_dtype) {
  KH_REQUIRE_INIT();
  KH_REQUIRE(m > 0 && n > 0 && k > 0 && m <= INT32_MAX && n <= INT32_MAX && k <= INT32_MAX,
             "kh_gemm_splitk_partials: bad extents");
  KH_REQUIRE(a && b && part, "kh_gemm_splitk_partials: null pointer");
  KH_REQUIRE(lda >= k && ldb >= k, "kh_gemm_splitk_partials: leading dimension too small");
  KH_REQUIRE(a_dtype == KH_BF16 || a_dtype == KH_F32, "kh_gemm_splitk_partials: unsupported dtype %d", a_dtype);
  const int ab = a_dtype == KH_F32 ? 4 : 2;
  const GemmPlan p = gemm_plan(aligned16(a) && aligned16(b), lda, ldb, (int)m, (int)n, (int)k, true, 1, ab);
  KH_REQUIRE(p.mfma && p.splits > 1 && p.splits == splits,
             "kh_gemm_splitk_partials: this product is not split %d ways (kh_gemm_split_count gives the count; "
             "operands must be 16-byte aligned with k and the leading dimensions multiples of 8)", splits);
  KH_REQUIRE(p.tiles <= INT32_MAX / 8, "kh_gemm_splitk_partials: grid too large");
  if (a_dtype == KH_F32)
    launch_gemm_tiles<float, float>(p, (const float*)a, lda, (const uint16_t*)b, ldb, nullptr, n, nullptr, 0, nullptr,
                                    (int)m, (int)n, (int)k, 1.f, 0.f, part);
  else
    launch_gemm_tiles<float>(p, (const uint16_t*)a, lda, (const uint16_t*)b, ldb, nullptr, n, nullptr, 0, nullptr,
                             (int)m, (int)n, (int)k, 1.f, 0.f, part);
  KH_CHECK_LAUNCH();
  return KH_OK;
}

int kh_gemm_swiglu(const void* x, int64_t ldx, const void* w_gu, int64_t ldw, void* h, int64_t ldh, int64_t m,
                   int64_t n_half, int64_t k, int x_dtype) {
  KH_REQUIRE_INIT();
  KH_REQUIRE(m >= 0 && n_half >= 0 && k > 0 && m <= INT32_MAX && 2 * n_half <= INT32_MAX && k <= INT32_MAX,
             "kh_gemm_swiglu: bad extents");
  KH_REQUIRE(x_dtype == KH_BF16 || x_dtype == KH_F32, "kh_gemm_swiglu: unsupported dtype %d", x_dtype);
  if (m == 0 || n_half == 0) return KH_OK;
  KH_REQUIRE(x && w_gu && h, "kh_gemm_swiglu: null pointer");
  KH_REQUIRE(n_half % 8 == 0, "kh_gemm_swiglu: the intermediate size %lld is not a multiple of 8", (long long)n_half);
  KH_REQUIRE(k % 8 == 0 && ldx % 8 == 0 && ldw % 8 == 0 && ldx >= k && ldw >= k && ldh >= n_half,
             "kh_gemm_swiglu: k and the row strides must be multiples of 8 elements (ldx, ldw >= k, ldh >= n_half)");
  KH_REQUIRE(aligned16(x) && aligned16(w_gu), "kh_gemm_swiglu: x and w_gu must be 16-byte aligned");
  const int64_t lim = int64_t(1) << 31;
  const int xb = x_dtype == KH_F32 ? 4 : 2;
  KH_REQUIRE((int64_t)g_tile(2) * ldx * xb < lim && (int64_t)g_tile(2) * ldw * 2 < lim,
             "kh_gemm_swiglu: row stride too large");
  if (x_dtype == KH_F32)
    return launch_gemm_swiglu<float>((const float*)x, ldx, (const uint16_t*)w_gu, ldw, (float*)h, ldh, (int)m,
                                     (int)(2 * n_half), (int)k);
  return launch_gemm_swiglu<uint16_t>((const uint16_t*)x, ldx, (const uint16_t*)w_gu, ldw, (uint16_t*)h, ldh, (int)m,
                                      (int)(2 * n_half), (int)k);
}

// cos / sin of float(positions[t]) * inv_freq[i] for n tokens and `half` frequencies, interleaved
// (cos, sin) per (t, i): the angles of every qk-norm + RoPE head tile of a prefill, evaluated once.
__global__ __launch_bounds__(256) void rope_table_kernel(const int32_t* __restrict__ positions, int64_t n,
                                                         const float* __restrict__ inv_freq, int half,
                                                         float* __restrict__ out) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n * half; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = i / half;
    const float pos = (float)positions[t];
    float sn, cs;
    sincosf(pos * inv_freq[i - t * half], &sn, &cs);
    out[2 * i] = cs;
    out[2 * i + 1] = sn;
  }
}

int kh_rope_table(const int32_t* positions, int64_t n, const float* inv_freq, int half, float* out) {
  KH_REQUIRE_INIT();
  KH_REQUIRE(n >= 0 && half > 0 && half <= 4096, "kh_rope_table: bad extents");
  if (n == 0) return KH_OK;
  KH_REQUIRE(positions && inv_freq && out, "kh_rope_table: null pointer");
  const int64_t total = n * half;
  const int64_t want = (total + 255) / 256;
  const int grid = (int)(want < 4096 ? want : 4096);
  rope_table_kernel<<<grid, 256, 0, stream()>>>(positions, n, inv_freq, half, out);
  KH_CHECK_LAUNCH();
  return KH_OK;
}

int kh_gemm_qk_norm_rope(const void* x, int64_t ldx, const void* w_qkv, int64_t ldw, int64_t n_batch,
                         int64_t seq_len, int64_t k, int n_q_heads, int n_kv_heads, int head_dim, const void* wq,
                         const void* wk, const float* inv_freq, const int32_t* positions, void* q_out, void* k_out,
                         void* v_out, const int64_t* strides, float eps, int64_t kv_cache_len, int dtype) {
  return kh_gemm_qk_norm_rope_table(x, ldx, w_qkv, ldw, n_batch, seq_len, k, n_q_heads, n_kv_heads, head_dim, wq, wk,
                                    inv_freq, positions, q_out, k_out, v_out, strides, eps, kv_cache_len, dtype,
                                    nullptr);
}

int kh_gemm_qk_norm_rope_table(const void* x, int64_t ldx, const void* w_qkv, int64_t ldw, int64_t n_batch,
                               int64_t seq_len, int64_t k, int n_q_heads, int n_kv_heads, int head_dim, const void* wq,
                               const void* wk, const float* inv_freq, const int32_t* positions, void* q_out,
                               void* k_out, void* v_out, const int64_t* strides, float eps, int64_t kv_cache_len,
                               int dtype, const float* rope_table) {
  KH_REQUIRE_INIT();
  KH_REQUIRE(n_batch >= 0 && seq_len >= 0 && k > 0 && k <= INT32_MAX && kv_cache_len >= 0,
             "kh_gemm_qk_norm_rope: bad extents");
  KH_REQUIRE(head_dim == 128, "kh_gemm_qk_norm_rope: head_dim %d (the fused projection takes 128)", head_dim);
  KH_REQUIRE(n_q_heads > 0 && n_kv_heads > 0, "kh_gemm_qk_norm_rope: head counts must be positive");
  KH_REQUIRE(dtype == KH_BF16 || dtype == KH_F32, "kh_gemm_qk_norm_rope: unsupported dtype %d", dtype);
  const int64_t M = n_batch * seq_len, N = (int64_t)(n_q_heads + 2 * n_kv_heads) * 128;
  KH_REQUIRE(M <= INT32_MAX && N <= INT32_MAX && seq_len <= (int64_t)UINT32_MAX, "kh_gemm_qk_norm_rope: too large");
  if (M == 0) return KH_OK;
  KH_REQUIRE(x && w_qkv && wq && wk && inv_freq && positions && q_out && k_out && v_out && strides,
             "kh_gemm_qk_norm_rope: null pointer");
  KH_REQUIRE(k % 8 == 0 && ldx % 8 == 0 && ldw % 8 == 0 && ldx >= k && ldw >= k,
             "kh_gemm_qk_norm_rope: k and the row strides must be multiples of 8 elements (ldx, ldw >= k)");
  const void* al[] = {x, w_qkv, wq, wk, q_out, k_out, v_out};
  for (const void* p : al) KH_REQUIRE(aligned16(p), "kh_gemm_qk_norm_rope: operands must be 16-byte aligned");
  const int64_t lim = int64_t(1) << 31;
  const int xb = dtype == KH_F32 ? 4 : 2;
  KH_REQUIRE((int64_t)g_tile(2) * ldx * xb < lim && (int64_t)g_tile(2) * ldw * 2 < lim,
             "kh_gemm_qk_norm_rope: row stride too large");
  QknrArgs qa;
  const int64_t vec = 16 / xb;
  for (int i = 0; i < 9; ++i) {
    KH_REQUIRE(strides[i] % vec == 0, "kh_gemm_qk_norm_rope: stride %d (%lld) breaks 16-byte alignment", i,
               (long long)strides[i]);
    qa.s[i] = strides[i];
  }
  qa.wq = (const uint16_t*)wq;
  qa.wk = (const uint16_t*)wk;
  qa.inv_freq = inv_freq;
  qa.positions = positions;
  qa.q_out = q_out;
  qa.k_out = k_out;
  qa.v_out = v_out;
  qa.hq = n_q_heads;
  qa.hkv = n_kv_heads;
  qa.seq_len = (uint32_t)(seq_len > 0 ? seq_len : 1);
  qa.eps = eps;
  qa.kv_cache_len = kv_cache_len;
  KH_REQUIRE(rope_table == nullptr || aligned16(rope_table), "kh_gemm_qk_norm_rope: rope_table must be 16-byte aligned");
  qa.rope_cs = rope_table;
  if (dtype == KH_F32)
    return launch_gemm_qk_norm_rope<float>((const float*)x, ldx, (const uint16_t*)w_qkv, ldw, (int)M, (int)N, (int)k,
                                           qa);
  return launch_gemm_qk_norm_rope<uint16_t>((const uint16_t*)x, ldx, (const uint16_t*)w_qkv, ldw, (int)M, (int)N,
                                            (int)k, qa);
}

int kh_gemv_swiglu(int prologue, const void* x, const void* norm_w, float eps, const void* w_gu, int64_t ldw,
                   void* h, int64_t n_half, int64_t k, int x_dtype) {
  KH_REQUIRE_INIT();
  KH_REQUIRE(prologue == PRO_NONE || prologue == PRO_RMSNORM, "kh_gemv_swiglu: prologue must be 0 (none) or 1 (RMSNorm)");
  KH_REQUIRE(x_dtype == KH_BF16 || x_dtype == KH_F32, "kh_gemv_swiglu: unsupported dtype %d", x_dtype);
  KH_REQUIRE(n_half > 0 && k > 0 && 2 * n_half <= INT32_MAX && k <= INT32_MAX, "kh_gemv_swiglu: bad extents");
  KH_REQUIRE(n_half % 8 == 0, "kh_gemv_swiglu: the intermediate size %lld is not a multiple of 8", (long long)n_half);
  KH_REQUIRE(x && w_gu && h, "kh_gemv_swiglu: null pointer");
  KH_REQUIRE(prologue != PRO_RMSNORM || norm_w != nullptr, "kh_gemv_swiglu: the RMSNorm prologue needs norm_w");
  KH_REQUIRE(ldw >= k, "kh_gemv_swiglu: ldw < k");
  const uint16_t* W = (const uint16_t*)w_gu;
  const int NH = (int)n_half, K = (int)k;
  bool ok;
  if (x_dtype == KH_F32)
    ok = prologue == PRO_RMSNORM ? launch_gemv_swiglu<PRO_RMSNORM, true, float>(x, norm_w, eps, W, ldw, (float*)h, NH, K)
                                 : launch_gemv_swiglu<PRO_NONE, true, float>(x, norm_w, eps, W, ldw, (float*)h, NH, K);
  else
    ok = prologue == PRO_RMSNORM ? launch_gemv_swiglu<PRO_RMSNORM>(x, norm_w, eps, W, ldw, (uint16_t*)h, NH, K)
                                 : launch_gemv_swiglu<PRO_NONE>(x, norm_w, eps, W, ldw, (uint16_t*)h, NH, K);
  KH_REQUIRE(ok, "kh_gemv_swiglu: unsupported operands (need k %% 8 == 0, ldw %% 8 == 0, a 16-byte aligned weight, "
                 "k <= 32768 and byte offsets below 4 GiB)");
  KH_CHECK_LAUNCH();
  return KH_OK;
}

int kh_gemv_fused(int prologue, const void* x, const void* x2, const void* norm_w, float eps, const void* w,
                  int64_t ldw, void* c, const void* cin, const void* bias, int64_t n, int64_t k, float alpha,
                  float beta, int out_dtype, int x_dtype) {
  KH_REQUIRE_INIT();
  KH_REQUIRE(prologue >= PRO_NONE && prologue <= PRO_SILU_MUL_IL, "kh_gemv_fused: unknown prologue %d", prologue);
  KH_REQUIRE(prologue != PRO_SILU_MUL_IL || k % 8 == 0, "kh_gemv_fused: the interleaved silu*mul prologue needs k %% 8 == 0");
  KH_REQUIRE(n >= 0 && k > 0 && n <= INT32_MAX && k <= INT32_MAX, "kh_gemv_fused: bad extents");
  KH_REQUIRE(out_dtype == KH_BF16 || out_dtype == KH_F32, "kh_gemv_fused: unsupported output dtype %d", out_dtype);
  KH_REQUIRE(x_dtype == KH_BF16 || x_dtype == KH_F32, "kh_gemv_fused: unsupported activation dtype %d", x_dtype);
  if (n == 0) return KH_OK;
  KH_REQUIRE(x && w && c, "kh_gemv_fused: null pointer");
  KH_REQUIRE(prologue != PRO_RMSNORM || norm_w != nullptr, "kh_gemv_fused: the RMSNorm prologue needs norm_w");
  KH_REQUIRE(prologue != PRO_SILU_MUL || x2 != nullptr, "kh_gemv_fused: the silu*mul prologue needs x2");
  KH_REQUIRE(ldw >= k, "kh_gemv_fused: ldw < k");
  const int N = (int)n, K = (int)k;
  const uint16_t* W = (const uint16_t*)w;
  bool ok = false;
  auto run = [&](auto* C, auto* CI, auto* BI, auto ex) {
    using TO = std::remove_const_t<std::remove_pointer_t<decltype(CI)>>;
    constexpr bool EX = decltype(ex)::value;
    if (prologue == PRO_RMSNORM)
      ok = launch_gemv1<PRO_RMSNORM, TO, EX>(x, x2, norm_w, eps, W, ldw, C, CI, BI, N, K, alpha, beta);
    else if (prologue == PRO_SILU_MUL)
      ok = launch_gemv1<PRO_SILU_MUL, TO, EX>(x, x2, norm_w, eps, W, ldw, C, CI, BI, N, K, alpha, beta);
    else if (prologue == PRO_SILU_MUL_IL)
      ok = launch_gemv1<PRO_SILU_MUL_IL, TO, EX>(x, x2, norm_w, eps, W, ldw, C, CI, BI, N, K, alpha, beta);
    else
      ok = launch_gemv1<PRO_NONE, TO, EX>(x, x2, norm_w, eps, W, ldw, C, CI, BI, N, K, alpha, beta);
  };
  const bool exact = x_dtype == KH_F32;
  if (out_dtype == KH_F32 && exact)
    run((float*)c, (const float*)cin, (const float*)bias, std::true_type{});
  else if (out_dtype == KH_F32)
    run((float*)c, (const float*)cin, (const float*)bias, std::false_type{});
  else if (exact)
    run((uint16_t*)c, (const uint16_t*)cin, (const uint16_t*)bias, std::true_type{});
  else
    run((uint16_t*)c, (const uint16_t*)cin, (const uint16_t*)bias, std::false_type{});
  KH_REQUIRE(ok, "kh_gemv_fused: unsupported operands (need k %% 8 == 0, ldw %% 8 == 0, a 16-byte aligned weight, "
                 "k <= 32768 and byte offsets below 4 GiB)");
  KH_CHECK_LAUNCH();
  return KH_OK;
}

}  // extern "C"
