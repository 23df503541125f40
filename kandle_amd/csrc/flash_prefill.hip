// bf16 causal / non-causal GQA flash-attention prefill for gfx950, head_dim 64 or 128, and the
// split-bf16 fp32 attention of the float32-activation model.
//
// Launch forms of the bf16 kernel (launch_prefill_d): the tile kernel (one workgroup per query
// block, 8 waves, or 2-4 waves on small grids); the persistent form for causal inputs with at least
// two 128-row items per CU (C3); its key-split form for one or two long sequences (too few items to
// pair); GQA ratios other than 1, 2, 4, 8 as groups of query heads on all of them.
//
// Semantics follow the reference kernel (packages/backend-webgpu/src/kernels/attention/builder.ts:138-329):
// score = (q . k) * scale, key j > query i masked when causal (top-left), query head h reads kv head
// h / (hq / hkv), online softmax in fp32, O = P V / l.
//
// A workgroup of WAVES waves shares one kv head: wave w serves query head g = w / (WAVES/G) of the
// G query heads that read this kv head (G = hq / hkv <= WAVES) and 32 query rows of a
// BMQ = 32 * WAVES / G row block.  K/V tiles of BN keys (128) are staged in LDS (double buffered, one
// barrier per tile) and shared by all waves, which compute them in chunks of 64 keys.
//
// Per wave and chunk, with v_mfma_f32_32x32x16_bf16:
//   S^T (keys x queries) = K Q^T : A = K rows from LDS, B = Q held in registers for the whole loop.
//   O^T (d x queries)   += V^T P^T: A = V^T fragments, B = P.
// Each lane owns one query column: the row statistics of the softmax are in-lane over 32 scores
// plus one exchange with lane ^ 32.  K rows are stored in LDS in the order "swap bits 2 and 3 of
// the key index", which makes S^T accumulator registers j = 0..7 of lane group g hold keys 8g + j
// (j = 8..15: keys 16 + 8g + j - 8) -- exactly the B-operand layout of the PV product, so P never
// leaves registers.  V is staged row-major like K and its V^T operand fragments are read with the
// gfx950 transposing LDS read (ds_read_b64_tr_b16) at a per-lane base plus compile-time offsets.
// Global loads are raw buffer loads (out-of-range rows read as zero without a branch).
//
// Softmax of the causal / unmasked route (SoftmaxLog2): the QK^T accumulators start at -m (m: the
// row's reference maximum, raw q.k units) instead of 0, so the MFMA itself delivers s - m and
// P = 2^((s - m) scale log2 e) is one multiply and one v_exp_f32 per score.  The reference maximum
// is the exact row maximum of the first chunk and is raised only when a lane's sum of P over its
// 32 scores exceeds kSumMax (which bounds every P, all being >= 0): the common path has no row
// maximum and no lane exchange.  O and l are rescaled together on a raise (O / l does not depend
// on the reference chosen), and l sums the bf16 P the PV product applies.
// The explicit-mask route keeps a thresholded maximum (SoftmaxRaw), which reproduces the reference
// softmax's f32(-1e38) floor and its 0 / 0 rows.
#include <type_traits>

#include "attention.h"

using namespace kh;

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kXcds = 8;  // MI355X: accelerator complex dies, one L2 each
constexpr int kPersistWaves = 8;  // waves per workgroup of the persistent causal kernel
constexpr int kPersistMinItems = 2;  // persistent from this many query blocks per CU up (0: never)
constexpr bool kPersistXcdLocal = true;  // XCD-local item order where the shape allows it
constexpr bool kMirrorSlots = true;      // mirrored row slots for the SIMD's second wave

// D: head dimension, 64 or 128.
template <int BN, int WAVES, int D = 128>
struct Cfg {
  static_assert(D == 64 || D == 128, "head_dim 64 or 128");
  static constexpr int THREADS = WAVES * 64;
  // K row stride in LDS (elements): 272 B (D 128) or 144 B (D 64) puts the 16-byte reads of 16
  // consecutive rows on 64 distinct banks.
  static constexpr int KSTR = D + 8;
  // V row stride (elements).  320 B = 80 dwords = 16 banks (mod 64) apart per row.  The LDS has 64
  // banks and serves a transposing read 32 lanes per clock: the two 16-lane groups of a clock read
  // the same 4 rows at column offsets 8 banks apart, so rows must be 16 banks apart for the 64
  // dwords to fall on 64 distinct banks (a 288-byte stride gave 2-way conflicts on 28 % of the
  // LDS-active cycles).  D 64: 192 B = 48 dwords, rows 16 banks apart the other way round.
  static constexpr int VSTR = D + 32;
  static constexpr int KTILE = BN * KSTR;            // elements
  static constexpr int VTILE = BN * VSTR;            // elements
  static constexpr int CPR = D / 8;                  // 16-byte chunks per K or V row
  static constexpr int CPR_LOG = D == 128 ? 4 : 3;
  static constexpr int NK = BN * CPR / THREADS;      // 16-byte K (and V) chunks per thread per tile
  static constexpr int NQ = D / 16;                  // 16-column MFMA k-steps of q.k (Q registers)
  static constexpr int ND = D / 32;                  // 32-column output tiles of P V
  // Compute works on 64-key chunks; a staged tile holds NCH of them.
  static constexpr int BNC = 64;
  static constexpr int NCH = BN / BNC;
  static constexpr int NSUB = BNC / 32;              // 32-key S^T subtiles per chunk
  static_assert(BN % BNC == 0, "tiles are whole 64-key chunks");
  static_assert(NK >= 1, "tile too small for the workgroup");
};

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef short v8i16 __attribute__((ext_vector_type(8)));

// gfx950 ds_read_b64_tr_b16: within each 16-lane group, element k of lane j is element (j & 3)
// of the four bf16 at the address of lane 4k + (j >> 2).
__device__ __forceinline__ v4i16 lds_read_tr16(const uint16_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4i16*)(p));
}

// Operand reads of a block of NM MFMAs (RPM LDS reads each): the reads of the first kReadsAhead
// MFMAs are issued first and each MFMA is followed by the reads of the one kReadsAhead places later,
// so several operands are in flight while the matrix core works (the default schedule keeps one or
// two).  Placed after the block's code; it orders the DS reads and MFMAs of the basic block.
constexpr int kReadsAhead = 4;
template <int NM, int RPM>
__device__ __forceinline__ void sched_reads_ahead() {
  constexpr int AHEAD = kReadsAhead < NM ? kReadsAhead : NM;
  __builtin_amdgcn_sched_group_barrier(0x100, AHEAD * RPM, 0);  // DS reads
#pragma unroll
  for (int i = 0; i < NM - AHEAD; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);          // one MFMA
    __builtin_amdgcn_sched_group_barrier(0x100, RPM, 0);        // the reads of a later one
  }
  __builtin_amdgcn_sched_group_barrier(0x008, AHEAD, 0);
}

// The two waves of a SIMD alternate between MFMA blocks (QK^T, PV) and softmax VALU work; a wave
// raises its issue priority for its MFMA blocks, so the arbiter keeps the matrix core fed while the
// other wave's VALU work fills the issue slots in between (C3: +0.5-1 %; priority on the QK^T
// block alone -0.4 %, on PV alone -3 %).
__device__ __forceinline__ void mfma_block_begin() { __builtin_amdgcn_s_setprio(1); }
__device__ __forceinline__ void mfma_block_end() { __builtin_amdgcn_s_setprio(0); }

// Shared per-workgroup setup and staging helpers.
// KSPLIT = 2 (the persistent kernel's key-split form): waves w and w + WAVES / 2 own the same rows
// and take the even and the odd 64-key chunk of every tile (key half khalf = w / SW), so an item
// holds SW / G row slots per query head, half the rows of the KSPLIT = 1 form.
template <int BN, int WAVES, int D = 128, int KSPLIT = 1>
struct Flash {
  using C = Cfg<BN, WAVES, D>;
  static_assert(KSPLIT == 1 || (KSPLIT == 2 && WAVES == 8 && C::NCH == 2), "key halves: 8 waves, 2 chunks per tile");
  static constexpr int SW = WAVES / KSPLIT;  // waves holding an item's row slots
  int G, BMQ, tid, wave, lane, r, g, b, hk, hqi, q0, qw0, qi, ntiles, wave_last_q, wave_tiles, dcol;
  int khalf = 0, half_last = -1;  // KSPLIT = 2: this wave's key half and its last chunk (-1: none)
  __amdgpu_buffer_rsrc_t rk, rv;
  // Element strides as 32-bit values (the entry checks they fit): half the scalar registers of
  // the 64-bit AttnStrides, which the persistent kernel needs for its item bookkeeping.
  struct Strides32 {
    int32_t qb, qh, qs, kb, kh, ks, vb, vh, vs, ob, oh, os;
  } st;

  // Per-workgroup fields: lane roles, GQA grouping, strides.
  __device__ __forceinline__ void setup(int hq, int hkv, const AttnStrides& s) {
    st = Strides32{(int32_t)s.qb, (int32_t)s.qh, (int32_t)s.qs, (int32_t)s.kb, (int32_t)s.kh, (int32_t)s.ks,
                   (int32_t)s.vb, (int32_t)s.vh, (int32_t)s.vs, (int32_t)s.ob, (int32_t)s.oh, (int32_t)s.os};
    G = hq / hkv;
    BMQ = 32 * (SW / G);
    tid = threadIdx.x;
    wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: keeps derived values scalar
    lane = tid & 63;
    r = lane & 31;
    g = lane >> 5;
    dcol = 8 * (tid & (C::CPR - 1));
    if constexpr (KSPLIT == 2) khalf = wave / SW;
  }
  // The wave's row-slot index among the SW waves that hold an item's rows.
  __device__ __forceinline__ int swave() const {
    if constexpr (KSPLIT == 1)
      return wave;
    else
      return wave % SW;
  }
  // 32-row slot of this wave inside its head's query block.  Waves w and w + 4 of an 8-wave
  // workgroup share a SIMD; the second four take their slots mirrored, so that on the causal
  // diagonal (where a wave's chunk count grows with its slot) each SIMD pairs a short row block
  // with a long one.  Only the rows a wave owns change, not any row's arithmetic.
  __device__ __forceinline__ int row_slot(int wpg) const {
    const int i = swave() % wpg;
    // (KSPLIT = 2: the SIMD's second wave is the other key half of the same slot)
    if (!kMirrorSlots || WAVES != 8 || KSPLIT != 1 || wave < 4 || wpg == 1) return i;
    return wpg == 8 ? 11 - i : wpg - 1 - i;
  }
  // Per-item fields: query block qblk of (batch, kv head) pair bh.  With kvsub > 1 the "kv heads"
  // are groups of G query heads, kvsub of them reading each real kv head (hk / kvsub).
  __device__ __forceinline__ void set_item(int bh, int qblk, int hkv, int lq, int lk, bool causal, const uint16_t* K,
                                           const uint16_t* V, int kvsub = 1) {
    const int wpg = SW / G;
    b = bh / hkv;
    hk = bh % hkv;
    hqi = hk * G + swave() / wpg;
    q0 = qblk * BMQ;
    qw0 = q0 + row_slot(wpg) * 32;
    qi = qw0 + r;
    const int kv_end = causal ? min(lk, q0 + BMQ) : lk;
    ntiles = (kv_end + BN - 1) / BN;
    // wave_tiles counts 64-key compute chunks (C::BNC)
    const int nchunks = (kv_end + C::BNC - 1) / C::BNC;
    wave_last_q = min(qw0 + 31, lq - 1);
    wave_tiles = qw0 >= lq ? 0 : (causal ? min(nchunks, wave_last_q / C::BNC + 1) : nchunks);
    if constexpr (KSPLIT == 2) half_last = wave_tiles > khalf ? khalf + 2 * ((wave_tiles - 1 - khalf) / 2) : -1;
    const int hkr = hk / kvsub;
    rk = make_rsrc(K + (int64_t)b * st.kb + (int64_t)hkr * st.kh, (uint32_t)(((int64_t)(lk - 1) * st.ks + D) * 2));
    rv = make_rsrc(V + (int64_t)b * st.vb + (int64_t)hkr * st.vh, (uint32_t)(((int64_t)(lk - 1) * st.vs + D) * 2));
  }
  __device__ __forceinline__ void init(int batch, int hq, int hkv, int lq, int lk, const AttnStrides& s, bool causal,
                                       int n_qblocks, const uint16_t* K, const uint16_t* V, int kvsub = 1) {
    setup(hq, hkv, s);
    // Workgroups are dispatched to the 8 XCDs round-robin (workgroup i on XCD i % 8), each XCD
    // with its own L2.  Renumber so that XCD x runs a contiguous range of logical blocks, ordered
    // (b, kv head)-major and, inside a head, heaviest (last) query block first: at any time an
    // XCD's CUs work on one or two heads, whose K/V stay resident in its L2.
    const int nblk = batch * hkv * n_qblocks;
    const int xcd = blockIdx.x % kXcds, j = blockIdx.x / kXcds;
    const int base = nblk / kXcds, extra = nblk % kXcds;  // XCD x runs base + (x < extra) blocks
    const int logical = xcd * base + min(xcd, extra) + j;
    set_item(logical / n_qblocks, n_qblocks - 1 - logical % n_qblocks, hkv, lq, lk, causal, K, V, kvsub);
  }
  // LDS row of tile key k: bits 2 and 3 of k swapped (an involution), so that lane r of the S^T
  // A operand, which reads LDS row r, holds key swap23(r) -- the order the PV B operand needs --
  // while the 32 lanes read 32 consecutive rows (no bank conflicts).
  static __device__ __forceinline__ int swap23(int k) { return (k & ~12) | ((k & 4) << 1) | ((k & 8) >> 1); }

  // Q row of this lane in item (bh, qblk) of another item than the current one (the persistent
  // kernel's prefetch), from the per-workgroup fields alone.
  __device__ __forceinline__ void load_q_of(int bh, int qblk, int hkv, const uint16_t* Q, int lq,
                                            bf16x8 (&qreg)[C::NQ]) const {
    const int wpg = SW / G;
    const int bb = bh / hkv, hqn = (bh % hkv) * G + swave() / wpg, qin = qblk * BMQ + row_slot(wpg) * 32 + r;
    const auto rq = make_rsrc(Q + (int64_t)bb * st.qb + (int64_t)hqn * st.qh,
                              (uint32_t)(((int64_t)(lq - 1) * st.qs + D) * 2));
    const uint32_t qoff = (uint32_t)(((int64_t)qin * st.qs + 8 * g) * 2);
#pragma unroll
    for (int c = 0; c < C::NQ; ++c) qreg[c] = as_bf16x8(buf_load16(rq, qoff + 32 * c));
  }
  // K and V byte ranges of pair bh (kvsub as set_item).
  __device__ __forceinline__ void kv_rsrc_of(int bh, int hkv, int lk, const uint16_t* K, const uint16_t* V,
                                             __amdgpu_buffer_rsrc_t& rkn, __amdgpu_buffer_rsrc_t& rvn,
                                             int kvsub = 1) const {
    const int bb = bh / hkv, hh = (bh % hkv) / kvsub;
    rkn = make_rsrc(K + (int64_t)bb * st.kb + (int64_t)hh * st.kh, (uint32_t)(((int64_t)(lk - 1) * st.ks + D) * 2));
    rvn = make_rsrc(V + (int64_t)bb * st.vb + (int64_t)hh * st.vh, (uint32_t)(((int64_t)(lk - 1) * st.vs + D) * 2));
  }
  // This lane's Q row: query qi, columns 8 g + 16 c .. + 7 (c = 0..7).
  __device__ __forceinline__ void load_q(const uint16_t* Q, int lq, bf16x8 (&qreg)[C::NQ]) const {
    const uint16_t* qh = Q + (int64_t)b * st.qb + (int64_t)hqi * st.qh;
    const auto rq = make_rsrc(qh, (uint32_t)(((int64_t)(lq - 1) * st.qs + D) * 2));
    const uint32_t qoff = (uint32_t)(((int64_t)qi * st.qs + 8 * g) * 2);
#pragma unroll
    for (int c = 0; c < C::NQ; ++c) qreg[c] = as_bf16x8(buf_load16(rq, qoff + 32 * c));
  }
  // K and V rows: chunk id = tid + THREADS i -> key id / 16, d 8 * (id % 16).
  __device__ __forceinline__ void load_rows(__amdgpu_buffer_rsrc_t rsrc, int64_t rstride, int t,
                                            uint4 (&stg)[C::NK]) const {
#pragma unroll
    for (int i = 0; i < C::NK; ++i) {
      const int key = t * BN + ((tid + C::THREADS * i) >> C::CPR_LOG);
      stg[i] = buf_load16(rsrc, (uint32_t)(((int64_t)key * rstride + dcol) * 2));
    }
  }
  __device__ __forceinline__ void store_k(uint16_t* ks, const uint4 (&kst)[C::NK]) const {
#pragma unroll
    for (int i = 0; i < C::NK; ++i)
      *reinterpret_cast<uint4*>(ks + swap23((tid + C::THREADS * i) >> C::CPR_LOG) * C::KSTR + dcol) = kst[i];
  }
  __device__ __forceinline__ void store_v(uint16_t* vs, const uint4 (&vst)[C::NK]) const {
#pragma unroll
    for (int i = 0; i < C::NK; ++i)
      *reinterpret_cast<uint4*>(vs + ((tid + C::THREADS * i) >> C::CPR_LOG) * C::VSTR + dcol) = vst[i];
  }
  // O^T += V^T P^T with V row-major in LDS.  The A operand of chunk kc (lane: d = 32 dt + r, keys
  // 16 kc + 8 g + e) is two transposing reads: lane l = 16 G + L supplies row 16 kc + 8 g + L / 4
  // (+ 4 for the second read), columns 32 dt + 16 (G & 1) + 4 (L & 3) .. + 3 -- a per-lane base
  // plus compile-time offsets.
  __device__ __forceinline__ void pv(const uint16_t* vs, const bf16x8 (&pk)[2 * C::NSUB], f32x16 (&oacc)[C::ND]) const {
    mfma_block_begin();
    const int L = lane & 15, Gq = lane >> 4;
    const uint16_t* vbase = vs + (8 * (Gq >> 1) + (L >> 2)) * C::VSTR + 16 * (Gq & 1) + 4 * (L & 3);
    constexpr int KC = 2 * C::NSUB;
    v8i16 af[C::ND * KC];
#pragma unroll
    for (int dt = 0; dt < C::ND; ++dt)
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) {
        const uint16_t* p0 = vbase + 16 * kc * C::VSTR + 32 * dt;
        const v4i16 lo = lds_read_tr16(p0);
        const v4i16 hi = lds_read_tr16(p0 + 4 * C::VSTR);
        af[dt * KC + kc] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      }
#pragma unroll
    for (int dt = 0; dt < C::ND; ++dt)
#pragma unroll
      for (int kc = 0; kc < KC; ++kc)
        oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, af[dt * KC + kc]), pk[kc],
                                                           oacc[dt], 0, 0, 0);
    sched_reads_ahead<C::ND * KC, 2>();
    mfma_block_end();
  }
  // S^T subtiles of one 64-key chunk in LDS; the accumulators start at cinit (INIT) or 0.
  template <bool INIT>
  __device__ __forceinline__ void qk(const uint16_t* ks, const bf16x8 (&qreg)[C::NQ], const f32x16& cinit,
                                     f32x16 (&sacc)[C::NSUB]) const {
    mfma_block_begin();
    bf16x8 kf[C::NSUB * C::NQ];
#pragma unroll
    for (int s = 0; s < C::NSUB; ++s) {
      const uint16_t* krp = ks + (32 * s + r) * C::KSTR + 8 * g;
#pragma unroll
      for (int c = 0; c < C::NQ; ++c) kf[s * C::NQ + c] = as_bf16x8(*reinterpret_cast<const uint4*>(krp + 16 * c));
    }
#pragma unroll
    for (int s = 0; s < C::NSUB; ++s) {
      if constexpr (INIT) {
        sacc[s] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[s * C::NQ], qreg[0], cinit, 0, 0, 0);
      } else {
#pragma unroll
        for (int j = 0; j < 16; ++j) sacc[s][j] = 0.f;
        sacc[s] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[s * C::NQ], qreg[0], sacc[s], 0, 0, 0);
      }
#pragma unroll
      for (int c = 1; c < C::NQ; ++c)
        sacc[s] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[s * C::NQ + c], qreg[c], sacc[s], 0, 0, 0);
    }
    sched_reads_ahead<C::NSUB * C::NQ, 1>();
    mfma_block_end();
  }
  // Causal / length mask of chunk t (only chunks crossing the diagonal or the sequence end).
  template <bool CAUSAL>
  __device__ __forceinline__ void mask(int t, int lk, f32x16 (&sc)[C::NSUB]) const {
    const int kt = t * C::BNC;  // t counts 64-key compute chunks
    if ((kt + C::BNC > lk) || (CAUSAL && kt + C::BNC - 1 > qw0)) {
      const int lim = (CAUSAL ? min(lk, qi + 1) : lk) - kt - 8 * g;
#pragma unroll
      for (int s = 0; s < C::NSUB; ++s)
#pragma unroll
        for (int j = 0; j < 16; ++j)
          if (32 * s + 16 * (j >> 3) + (j & 7) >= lim) sc[s][j] = -INFINITY;
    }
  }
  // Additive mask of a 64-key tile t for this lane's query row (MASKT 1: f32, 2: bf16), held as
  // four runs of eight keys: run (s, h) = keys 64 t + 32 s + 16 h + 8 g .. + 7, which are the S^T
  // registers sc[s][8 h .. 8 h + 7].  The mask has a unit key stride and 16-byte aligned 8-key runs
  // (the entry point packs other masks first).  Rows past lq read row lq - 1 (their output is not
  // stored); reads past the mask's byte extent return 0 (buffer range check), and keys >= lk are
  // masked to -inf by apply_mask whatever was read.
  template <int MASKT>
  struct MaskRegs {
    uint4 v[MASKT == 1 ? 8 : 4];
  };
  template <int MASKT>
  __device__ __forceinline__ void load_mask(int t, int lq, __amdgpu_buffer_rsrc_t rm, const MaskArgs& ma,
                                            MaskRegs<MASKT>& mr) const {
    constexpr int ES = MASKT == 1 ? 4 : 2;
    const int64_t rowoff = b * ma.sb + hqi * ma.sh + (int64_t)min(qi, lq - 1) * ma.sq;
#pragma unroll
    for (int run = 0; run < 4; ++run) {  // run = 2 s + h
      const uint32_t off = (uint32_t)((rowoff + t * 64 + 16 * run + 8 * g) * ES);
      if constexpr (MASKT == 1) {
        mr.v[2 * run] = buf_load16(rm, off);
        mr.v[2 * run + 1] = buf_load16(rm, off + 16);
      } else {
        mr.v[run] = buf_load16(rm, off);
      }
    }
  }
  static __device__ __forceinline__ uint32_t comp(const uint4& u, int i) {
    return i == 0 ? u.x : (i == 1 ? u.y : (i == 2 ? u.z : u.w));
  }
  // Scores of tile t become q.k + mask / scale (raw units; the exponent multiplies by scale
  // log2 e), keys >= lk become -inf.
  template <int MASKT>
  __device__ __forceinline__ void apply_mask(int t, int lk, const MaskRegs<MASKT>& mr, float inv_scale,
                                             f32x16 (&sc)[C::NSUB]) const {
#pragma unroll
    for (int s = 0; s < C::NSUB; ++s)
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int run = 2 * s + (j >> 3), e = j & 7;
        uint32_t bits;
        if constexpr (MASKT == 1)
          bits = comp(mr.v[2 * run + (e >> 2)], e & 3);
        else
          bits = (e & 1) ? (comp(mr.v[run], e >> 1) & 0xffff0000u) : (comp(mr.v[run], e >> 1) << 16);
        const float mv = __builtin_bit_cast(float, bits);
        const int key = t * 64 + 32 * s + 16 * (j >> 3) + 8 * g + e;
        sc[s][j] = key < lk ? __builtin_fmaf(mv, inv_scale, sc[s][j]) : -INFINITY;
      }
  }
  // O[qi][d] = oacc / l; lane holds d = 32dt + 8(j/4) + 4g + j%4.  A row whose sum l is 0 stores
  // zeros, or NaN with NAN_EMPTY (the reference softmax's 0 / 0 on the explicit-mask route).
  template <bool NAN_EMPTY = false>
  __device__ __forceinline__ void store_o(uint16_t* O, int lq, float l_run, const f32x16 (&oacc)[C::ND]) const {
    const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
    if (qi < lq) {
      const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
      const bool nan_row = NAN_EMPTY && !(l_tot > 0.f);
      uint16_t* orow = O + (int64_t)b * st.ob + (int64_t)hqi * st.oh + (int64_t)qi * st.os;
#pragma unroll
      for (int dt = 0; dt < C::ND; ++dt)
#pragma unroll
        for (int a = 0; a < 4; ++a) {
          const int d = 32 * dt + 8 * a + 4 * g;
          uint2 w;
          w.x = pack_bf16x2(oacc[dt][4 * a + 0] * inv, oacc[dt][4 * a + 1] * inv);
          w.y = pack_bf16x2(oacc[dt][4 * a + 2] * inv, oacc[dt][4 * a + 3] * inv);
          if (nan_row) w = make_uint2(0x7fc07fc0u, 0x7fc07fc0u);
          *reinterpret_cast<uint2*>(orow + d) = w;
        }
    }
  }
};

// Row maximum of a chunk's scores: this lane's 32, then the partner lane (lane ^ 32) that holds
// the other 32 keys of the same query row.
template <int NSUB>
__device__ __forceinline__ float chunk_row_max(const f32x16 (&sc)[NSUB]) {
  float m4[NSUB * 4];
#pragma unroll
  for (int s = 0; s < NSUB; ++s)
#pragma unroll
    for (int j = 0; j < 16; j += 4)
      m4[s * 4 + j / 4] = fmaxf(fmaxf(sc[s][j], sc[s][j + 1]), fmaxf(sc[s][j + 2], sc[s][j + 3]));
  float mx = m4[0];
#pragma unroll
  for (int i = 1; i < NSUB * 4; ++i) mx = fmaxf(mx, m4[i]);
  return fmaxf(mx, __shfl_xor(mx, 32, 64));
}

// Online softmax of the causal / unmasked route: raw q.k scores relative to the reference maximum m
// (the QK^T accumulators start at mneg = -m, 0 before the first raise); P = 2^(c (s - m)) with
// c = scale log2 e.
constexpr float kSumMax = 4096.f;  // a lane's chunk sum of P above this raises the reference

struct SoftmaxLog2 {
  float m = -INFINITY;  // reference maximum of this row (raw q.k units); -inf before the first raise
  float l = 0.f;        // partial denominator of this lane's keys, relative to m
  f32x16 mneg;          // -m in every register (0 while m = -inf)

  __device__ __forceinline__ SoftmaxLog2() {
#pragma unroll
    for (int j = 0; j < 16; ++j) mneg[j] = 0.f;
  }
  // P = 2^(c sc) as bf16 operands; returns this lane's sum of those bf16 values (two per
  // v_dot2c_f32_bf16 against (1, 1)): l then sums exactly the weights the PV product applies.
  template <int NSUB>
  static __device__ __forceinline__ float exponentiate(const f32x16 (&sc)[NSUB], float c, bf16x8 (&pk)[2 * NSUB]) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
    float ps[2 * NSUB];
#pragma unroll
    for (int s = 0; s < NSUB; ++s)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        bf16x8 pv;
#pragma unroll
        for (int e = 0; e < 8; ++e) pv[e] = (__bf16)fast_exp2(sc[s][8 * h + e] * c);
        pk[2 * s + h] = pv;
        const bf16x2 p01 = __builtin_shufflevector(pv, pv, 0, 1), p23 = __builtin_shufflevector(pv, pv, 2, 3);
        const bf16x2 p45 = __builtin_shufflevector(pv, pv, 4, 5), p67 = __builtin_shufflevector(pv, pv, 6, 7);
        float sum = __builtin_amdgcn_fdot2_f32_bf16(p01, one, 0.f, false);
        sum = __builtin_amdgcn_fdot2_f32_bf16(p23, one, sum, false);
        sum = __builtin_amdgcn_fdot2_f32_bf16(p45, one, sum, false);
        ps[2 * s + h] = __builtin_amdgcn_fdot2_f32_bf16(p67, one, sum, false);
      }
    float t = ps[0];
#pragma unroll
    for (int i = 1; i < 2 * NSUB; ++i) t += ps[i];
    return t;
  }
  // True (wave-uniform) if some row of the wave must raise its reference: the first chunk, or a
  // lane sum above kSumMax (inf included).
  __device__ __forceinline__ bool need_raise(float ps) const {
    return __any(m == -INFINITY || !(ps <= kSumMax));
  }
  // Raises every row's reference to its exact maximum over the chunk (when higher), shifts the
  // chunk's scores to the new reference and rescales O and l.  A row with nothing unmasked so far
  // keeps m = -inf (and P = 0).
  template <int NSUB, int ND>
  __device__ __forceinline__ void raise(f32x16 (&sc)[NSUB], float c, f32x16 (&oacc)[ND]) {
    const float mx = chunk_row_max(sc);  // relative to m (absolute while m = -inf)
    float d, alpha;
    if (m == -INFINITY) {
      d = mx == -INFINITY ? 0.f : mx;
      alpha = 0.f;  // O and l are still empty
      m = mx;
    } else {
      d = fmaxf(mx, 0.f);
      alpha = fast_exp2(-d * c);
      m += d;
    }
#pragma unroll
    for (int s = 0; s < NSUB; ++s)
#pragma unroll
      for (int j = 0; j < 16; ++j) sc[s][j] -= d;
    l *= alpha;
#pragma unroll
    for (int dt = 0; dt < ND; ++dt)
#pragma unroll
      for (int j = 0; j < 16; ++j) oacc[dt][j] *= alpha;
    const float mn = m == -INFINITY ? 0.f : -m;
#pragma unroll
    for (int j = 0; j < 16; ++j) mneg[j] = mn;
  }
};

// Online softmax of the explicit-mask route, raw q.k units.
//
// The exponentials use a reference max m_ref that is raised only when some row's tile max exceeds
// it by more than kRescaleLog2 (log2 units).  P = 2^((s - m_ref) c2) then stays <= 2^kRescaleLog2,
// O and l are rescaled together only on those rare raises, and the final O / l does not depend on
// the reference chosen.
constexpr float kRescaleLog2 = 8.0f;

struct SoftmaxRaw {
  float m_ref = -INFINITY;  // reference max of raw scores (q . k) for this row
  float l_run = 0.f;        // partial denominator of this lane's keys, relative to m_ref

  // Raises the reference max when this tile needs it (rescaling O and l); true (wave-uniform) if
  // any lane did, in which case P must be recomputed.  floor: the lowest row max (raw units): the
  // reference softmax starts its max at f32(-1e38).
  template <int NSUB, int ND>
  __device__ __forceinline__ bool update(const f32x16 (&sc)[NSUB], float c2, f32x16 (&oacc)[ND], float floor) {
    const float mx = fmaxf(chunk_row_max(sc), floor);
    // NaN-free by construction (this file is compiled assuming no NaNs, so that fmaxf needs no
    // canonicalisation): a row with nothing unmasked (mx = -inf) never asks for a raise, and
    // m_ref = -inf only before the first raise, where alpha = 2^-inf = 0 clears the empty O and l.
    const bool need = mx != -INFINITY && (m_ref == -INFINITY || (mx - m_ref) * c2 > kRescaleLog2);
    if (__any(need)) {
      const float m_new = need ? fmaxf(m_ref, mx) : m_ref;
      const float alpha = m_ref == -INFINITY ? 0.f : fast_exp2((m_ref - m_new) * c2);
      m_ref = m_new;
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < ND; ++dt)
#pragma unroll
        for (int j = 0; j < 16; ++j) oacc[dt][j] *= alpha;
      return true;
    }
    return false;
  }
  // P = 2^(s c2 - m_ref c2) as bf16 operands; returns this lane's sum of the fp32 values.
  template <int NSUB>
  __device__ __forceinline__ float exponentiate(const f32x16 (&sc)[NSUB], float c2, bf16x8 (&pk)[2 * NSUB]) const {
    const float mb = (m_ref == -INFINITY ? 0.f : m_ref) * c2;
    float ps[2] = {0.f, 0.f};
#pragma unroll
    for (int s = 0; s < NSUB; ++s)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        bf16x8 pv;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          // one v_fma_f32 per score (written out: contraction would fuse m_ref * c2 instead)
          const float p = fast_exp2(__builtin_fmaf(sc[s][8 * h + e], c2, -mb));
          ps[h] += p;
          pv[e] = (__bf16)p;
        }
        pk[2 * s + h] = pv;
      }
    return ps[0] + ps[1];
  }
};

// =============================================================================================
// Tile-synchronous kernel.
// =============================================================================================
// MASKT: 0 = causal / none as CAUSAL says; 1, 2 = additive f32 / bf16 mask M (64-key tiles, no
// causal mask, the reference's explicit-mask route).
template <int BN, int WAVES, int MINB, bool CAUSAL, int MASKT = 0, int D = 128>
__global__ __launch_bounds__(WAVES * 64, MINB) void flash_fwd_kernel(
    const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K, const uint16_t* __restrict__ V,
    uint16_t* __restrict__ O, int batch, int hq, int hkv, int lq, int lk, AttnStrides st, float scale,
    int n_qblocks, const void* __restrict__ M, MaskArgs ma, int kvsub) {
  using C = Cfg<BN, WAVES, D>;
  using FL = Flash<BN, WAVES, D>;
  static_assert(MASKT == 0 || (BN == 64 && !CAUSAL), "masked tiles are 64 keys, not causal");
  constexpr int STAGE = C::KTILE + C::VTILE;
  __shared__ __attribute__((aligned(16))) uint16_t smem[2 * STAGE];
  FL F;
  F.init(batch, hq, hkv, lq, lk, st, CAUSAL, n_qblocks, K, V, kvsub);
  const float c2 = scale * kLog2e;
  bf16x8 qreg[C::NQ];
  F.load_q(Q, lq, qreg);

  uint4 kst[C::NK], vst[C::NK];
  f32x16 oacc[C::ND];
#pragma unroll
  for (int dt = 0; dt < C::ND; ++dt)
#pragma unroll
    for (int j = 0; j < 16; ++j) oacc[dt][j] = 0.f;
  SoftmaxLog2 sl;
  SoftmaxRaw sr;
  const int ntiles = F.ntiles;

  if (ntiles > 0) {
    F.load_rows(F.rk, F.st.ks, 0, kst);
    F.load_rows(F.rv, F.st.vs, 0, vst);
    F.store_k(smem, kst);
    F.store_v(smem + C::KTILE, vst);
  }
  // Retire every outstanding load (Q included) before the loop, so the compiler's wait counting
  // inside the loop only ever covers the next tile's prefetch and never stalls QK^T on it.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  using MR = typename FL::template MaskRegs<MASKT == 0 ? 2 : MASKT>;
  const __amdgpu_buffer_rsrc_t rm = make_rsrc(M, MASKT == 0 ? 0u : ma.bytes);
  for (int t = 0; t < ntiles; ++t) {
    const bool has_next = t + 1 < ntiles;
    // The mask loads go out before the next tile's K/V prefetch, so that waiting for them never
    // waits for the prefetch (the vector-memory counter retires in issue order).
    MR mreg;
    if constexpr (MASKT != 0) F.template load_mask<MASKT>(t, lq, rm, ma, mreg);
    if (has_next) {
      F.load_rows(F.rk, F.st.ks, t + 1, kst);
      F.load_rows(F.rv, F.st.vs, t + 1, vst);
    }
    const uint16_t* ks = smem + (t & 1) * STAGE;
#pragma unroll
    for (int c = 0; c < C::NCH; ++c) {
      const int tc = t * C::NCH + c;  // 64-key compute chunk
      if (tc < F.wave_tiles) {
        f32x16 sacc[C::NSUB];
        bf16x8 pk[2 * C::NSUB];
        if constexpr (MASKT == 0) {
          F.template qk<true>(ks + c * C::BNC * C::KSTR, qreg, sl.mneg, sacc);
          F.template mask<CAUSAL>(tc, lk, sacc);
          float ps = SoftmaxLog2::exponentiate(sacc, c2, pk);
          if (sl.need_raise(ps)) {
            sl.raise(sacc, c2, oacc);
            ps = SoftmaxLog2::exponentiate(sacc, c2, pk);
          }
          sl.l += ps;
        } else {
          F.template qk<false>(ks + c * C::BNC * C::KSTR, qreg, sl.mneg, sacc);
          F.template apply_mask<MASKT>(tc, lk, mreg, ma.inv_scale, sacc);
          // Written as P computed with the current reference max, then recomputed after a raise
          // (rare after the first tile); the compiler folds the two into one exponentiation
          // after the max check.
          float ps = sr.exponentiate(sacc, c2, pk);
          if (sr.update(sacc, c2, oacc, ma.floor_raw)) ps = sr.exponentiate(sacc, c2, pk);
          sr.l_run += ps;
        }
        F.pv(ks + C::KTILE + c * C::BNC * C::VSTR, pk, oacc);
      }
    }
    if (has_next) {
      uint16_t* nxt = smem + ((t + 1) & 1) * STAGE;
      F.store_k(nxt, kst);
      F.store_v(nxt + C::KTILE, vst);
    }
    __syncthreads();
  }
  F.template store_o<MASKT != 0>(O, lq, MASKT == 0 ? sl.l : sr.l_run, oacc);
}

// Persistent form of the causal / unmasked route: one workgroup per CU walks a fixed list of
// (query block, (batch, kv head)) items, so a CU never waits for a new workgroup to start and load
// its Q and first K/V tile: the next item's Q and first tile are requested during the current
// item's last tile.  Items are ranked heaviest first (query block descending) and dealt in a snake
// (ranks w, 2P - 1 - w, 2P + w, ... to workgroup w of P), which gives every workgroup the same
// number of tiles when the query blocks of all pairs are uniform (C3: 32 + 17 + 16 + 1 = 66 tiles
// each).  When P is a multiple of the pair count, the odd passes are mirrored so that a workgroup
// keeps one (batch, kv head) pair for all its items (its K/V stay in its XCD's L2).  The per-item
// arithmetic is the tile kernel's, so outputs are identical to it.
// KSPLIT = 2 (one sequence of a few thousand tokens: too few 128-row items to pair): items of half
// the rows, each row slot held by two waves that take the even and the odd 64-key chunk of every
// tile; at the end of an item the two halves' (m, l, O) merge through the staging buffer the loop
// left free, and the first half stores the rows.  Its sums are grouped differently from the
// KSPLIT = 1 form, so its outputs differ from it within the rounding of the split.
// GROUPS: hkv counts groups of G query heads, kvsub of them per real kv head (a GQA ratio other than
// 1, 2, 4, 8, as the tile kernel's kvsub); without it kvsub is ignored.
template <bool CAUSAL, int D = 128, int KSPLIT = 1, bool GROUPS = false>
__global__ __launch_bounds__(kPersistWaves * 64, 1) void flash_fwd_persistent_kernel(
    const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K, const uint16_t* __restrict__ V,
    uint16_t* __restrict__ O, int batch, int hq, int hkv, int lq, int lk, AttnStrides st, float scale, int n_qblocks,
    int kvsub) {
  constexpr int BN = 128, WAVES = kPersistWaves;
  using C = Cfg<BN, WAVES, D>;
  using FL = Flash<BN, WAVES, D, KSPLIT>;
  constexpr int STAGE = C::KTILE + C::VTILE;
  __shared__ __attribute__((aligned(16))) uint16_t smem[2 * STAGE];
  const int P = gridDim.x, w = blockIdx.x;
  const int npairs = batch * hkv;
  const int nitems = npairs * n_qblocks;  // < 2^31 (the launcher checks)
  const bool mirror = P % npairs == 0;
  // XCD-local order, when the shape allows it: the P / 8 workgroups of XCD x (w % 8 = x, local
  // index j = w / 8) take its npairs / 8 pairs one after another, query block n_qblocks - 1 - j of
  // the even ones and j of the odd ones (n_qblocks + 1 tiles per two items for every j), so an
  // XCD's L2 holds about two pairs' K/V at a time.
  const int ppx = npairs / kXcds;
  const bool xcd_local = kPersistXcdLocal && P % kXcds == 0 && npairs % kXcds == 0 && ppx % 2 == 0 &&
                         P / kXcds == n_qblocks;
  auto item = [&](int k, int& bh, int& qblk) -> bool {
    if (xcd_local) {
      if (k >= ppx) return false;
      const int x = w % kXcds, j = w / kXcds;
      bh = ppx * x + k;
      qblk = (k & 1) ? j : n_qblocks - 1 - j;
      return true;
    }
    const int v = P * k + ((k & 1) ? P - 1 - w : w);
    if (v >= nitems) return false;
    const int cls = v / npairs, slot = v - cls * npairs;
    bh = (mirror && (k & 1)) ? npairs - 1 - slot : slot;
    qblk = n_qblocks - 1 - cls;
    return true;
  };
  int k = 0, bh = 0, qblk = 0;
  if (!item(0, bh, qblk)) return;
  FL F;
  F.setup(hq, hkv, st);
  F.set_item(bh, qblk, hkv, lq, lk, CAUSAL, K, V, GROUPS ? kvsub : 1);
  const float c2 = scale * kLog2e;
  bf16x8 qreg[C::NQ];
  F.load_q(Q, lq, qreg);
  uint4 kst[C::NK], vst[C::NK];
  f32x16 oacc[C::ND];
#pragma unroll
  for (int dt = 0; dt < C::ND; ++dt)
#pragma unroll
    for (int j = 0; j < 16; ++j) oacc[dt][j] = 0.f;
  SoftmaxLog2 sl;
  F.load_rows(F.rk, F.st.ks, 0, kst);
  F.load_rows(F.rv, F.st.vs, 0, vst);
  F.store_k(smem, kst);
  F.store_v(smem + C::KTILE, vst);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  int buf = 0;
  while (true) {
    int bhn = 0, qbn = 0;
    const bool more = item(k + 1, bhn, qbn);
    // A wave's Q registers are free once it has formed its last chunk's scores: the next item's Q
    // is loaded into them there (at the start for a wave with no rows in this item).
    if (more && (KSPLIT == 1 ? F.wave_tiles == 0 : F.half_last < 0)) F.load_q_of(bhn, qbn, hkv, Q, lq, qreg);
    const int ntiles = F.ntiles;
    for (int t = 0; t < ntiles; ++t) {
      const bool next_same = t + 1 < ntiles;
      if (next_same) {
        F.load_rows(F.rk, F.st.ks, t + 1, kst);
        F.load_rows(F.rv, F.st.vs, t + 1, vst);
      } else if (more) {
        __amdgpu_buffer_rsrc_t rkn, rvn;
        F.kv_rsrc_of(bhn, hkv, lk, K, V, rkn, rvn, GROUPS ? kvsub : 1);
        F.load_rows(rkn, F.st.ks, 0, kst);
        F.load_rows(rvn, F.st.vs, 0, vst);
      }
      const uint16_t* ks = smem + buf * STAGE;
#pragma unroll
      for (int c = 0; c < C::NCH; ++c) {
        const int tc = t * C::NCH + c;  // 64-key compute chunk
        if (tc < F.wave_tiles && (KSPLIT == 1 || c == F.khalf)) {
          f32x16 sacc[C::NSUB];
          bf16x8 pk[2 * C::NSUB];
          F.template qk<true>(ks + c * C::BNC * C::KSTR, qreg, sl.mneg, sacc);
          if (more && tc == (KSPLIT == 1 ? F.wave_tiles - 1 : F.half_last)) F.load_q_of(bhn, qbn, hkv, Q, lq, qreg);
          F.template mask<CAUSAL>(tc, lk, sacc);
          float ps = SoftmaxLog2::exponentiate(sacc, c2, pk);
          if (sl.need_raise(ps)) {
            sl.raise(sacc, c2, oacc);
            ps = SoftmaxLog2::exponentiate(sacc, c2, pk);
          }
          sl.l += ps;
          F.pv(ks + C::KTILE + c * C::BNC * C::VSTR, pk, oacc);
        }
      }
      if (next_same || more) {
        uint16_t* nxt = smem + (buf ^ 1) * STAGE;
        F.store_k(nxt, kst);
        F.store_v(nxt + C::KTILE, vst);
      }
      __syncthreads();
      buf ^= 1;
    }
    if constexpr (KSPLIT == 1) {
      F.template store_o<false>(O, lq, sl.l, oacc);
    } else {
      // Merge the two key halves of each row slot: the second writes (m, l, O) per lane into the
      // free staging buffer (the other holds the next item's first tile), the first combines them
      // with the log-sum-exp rule and stores the rows.  The last barrier keeps the buffer until
      // every read is done: the next item's second tile is staged there.
      constexpr int MS = 2 + 16 * C::ND;  // floats per lane
      static_assert(WAVES / 2 * MS * 64 * 4 <= STAGE * 2, "the merge fits a staging buffer");
      float* mp = reinterpret_cast<float*>(smem + (buf ^ 1) * STAGE) + F.swave() * MS * 64 + F.lane;
      if (F.khalf == 1) {
        mp[0] = sl.m;
        mp[64] = sl.l;
#pragma unroll
        for (int dt = 0; dt < C::ND; ++dt)
#pragma unroll
          for (int j = 0; j < 16; ++j) mp[(2 + 16 * dt + j) * 64] = oacc[dt][j];
      }
      __syncthreads();
      if (F.khalf == 0) {
        const float m1 = mp[0], l1 = mp[64];
        const float mt = fmaxf(sl.m, m1);
        // a half with no unmasked key has m = -inf and adds nothing (its l and O are 0)
        const float a0 = sl.m == -INFINITY ? 0.f : fast_exp2((sl.m - mt) * c2);
        const float a1 = m1 == -INFINITY ? 0.f : fast_exp2((m1 - mt) * c2);
#pragma unroll
        for (int dt = 0; dt < C::ND; ++dt)
#pragma unroll
          for (int j = 0; j < 16; ++j) oacc[dt][j] = oacc[dt][j] * a0 + mp[(2 + 16 * dt + j) * 64] * a1;
        F.template store_o<false>(O, lq, sl.l * a0 + l1 * a1, oacc);
      }
      __syncthreads();
    }
    if (!more) break;
    F.set_item(bhn, qbn, hkv, lq, lk, CAUSAL, K, V, GROUPS ? kvsub : 1);
#pragma unroll
    for (int dt = 0; dt < C::ND; ++dt)
#pragma unroll
      for (int j = 0; j < 16; ++j) oacc[dt][j] = 0.f;
    sl = SoftmaxLog2();
    ++k;
  }
}

constexpr int kWaves = 8;  // waves per workgroup: query rows of 32 * 8 / G, one kv head
// Short prompts: a grid of fewer than kSmallGrid 8-wave workgroups leaves most CUs idle and its time
// is the key loop of the last query block.  Such launches use workgroups of max(G, 2) waves (G <= 4)
// over kSmallBN-key tiles instead: one 32-row slot per query head, so there are 8 / waves times as
// many workgroups, and each wave has a SIMD to itself.  C5 prefill (S = 512, G = 2): 2-wave
// workgroups (128 of them) 2.392 -> 2.355 ms over 28 layers against 4-wave (64); 64-key tiles
// measured the same as 128-key ones.
constexpr int kSmallGrid = 256;
constexpr int kSmallBN = 128;

// hkv here counts groups of hq / hkv query heads sharing K/V tiles; with kvsub > 1 they are
// sub-groups, kvsub of them per real kv head (see prefill_groups).
template <int BN, int WAVES, bool CAUSAL, int D>
void launch_fwd(const void* q, const void* k, const void* v, void* o, int batch, int hq, int hkv, int lq, int lk,
                const AttnStrides& st, float scale, int kvsub) {
  const int BMQ = 32 * (WAVES / (hq / hkv));
  const int nqb = (lq + BMQ - 1) / BMQ;
  const int nblk = nqb * batch * hkv;
  flash_fwd_kernel<BN, WAVES, 1, CAUSAL, 0, D><<<nblk, WAVES * 64, 0, stream()>>>(
      (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v, (uint16_t*)o, batch, hq, hkv, lq, lk, st, scale,
      nqb, nullptr, MaskArgs{}, kvsub);
}

// The tile kernels serve G = 1, 2, 4 or 8 query heads per kv head.  Another ratio R is served in
// groups of G = the largest of 8, 4, 2, 1 dividing R: kvsub = R / G groups per kv head, each a
// "kv head" of the launch (hkv * kvsub of them) that reads real kv head group / kvsub.
struct PrefillGroups {
  int G, kvsub, hkv;
};
inline PrefillGroups prefill_groups(int hq, int hkv) {
  const int R = hq / hkv;
  const int G = R % 8 == 0 ? 8 : (R % 4 == 0 ? 4 : (R % 2 == 0 ? 2 : 1));
  return PrefillGroups{G, R / G, hkv * (R / G)};
}

template <int D>
int launch_prefill_d(const void* q, const void* k, const void* v, void* o, int batch, int hq, int hkv_real, int lq,
                     int lk, const AttnStrides& st, float scale, bool causal) {
  const PrefillGroups pg = prefill_groups(hq, hkv_real);
  const int G = pg.G, kvsub = pg.kvsub, hkv = pg.hkv;
  const int BMQ = 32 * (kWaves / G);
  const int nqb = (lq + BMQ - 1) / BMQ;
  const int64_t nblk64 = (int64_t)nqb * batch * hkv;
  KH_REQUIRE(nblk64 <= INT32_MAX, "kh_flash_attention: grid too large");
  // The persistent forms (one resident workgroup per CU); GROUPS instantiations serve kvsub > 1.
  auto persist = [&](auto ksplit, int n_qb) {
    constexpr int KSP = decltype(ksplit)::value;
    if (kvsub > 1)
      flash_fwd_persistent_kernel<true, D, KSP, true><<<cu_count(), kPersistWaves * 64, 0, stream()>>>(
          (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v, (uint16_t*)o, batch, hq, hkv, (int)lq, (int)lk,
          st, scale, n_qb, kvsub);
    else
      flash_fwd_persistent_kernel<true, D, KSP, false><<<cu_count(), kPersistWaves * 64, 0, stream()>>>(
          (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v, (uint16_t*)o, batch, hq, hkv, (int)lq, (int)lk,
          st, scale, n_qb, 1);
  };
  if (causal && G <= 4 && kPersistMinItems > 0 && nblk64 < (int64_t)kPersistMinItems * cu_count()) {
    // Too few 128-row items to pair heavy with light ones (one sequence of a few thousand tokens:
    // 256 items of very unequal length on 256 CUs): the key-split persistent form, whose items
    // hold half the rows, when that gives at least half the CUs one (B = 1, 16 / 8 heads: S = 4096
    // 117.6 -> 103.0 us, 2048 63.4 -> 42.1, 1024 30.1 -> 24.6; shorter prompts keep the small
    // workgroups below).
    const int BMQ2 = 32 * (kPersistWaves / 2 / G);
    const int nqb2 = (lq + BMQ2 - 1) / BMQ2;
    if ((int64_t)nqb2 * batch * hkv >= cu_count() / 2) {
      persist(std::integral_constant<int, 2>{}, nqb2);
      KH_CHECK_LAUNCH();
      return KH_OK;
    }
  }
  if (nblk64 < kSmallGrid && G <= 2) {
    if (causal)
      launch_fwd<kSmallBN, 2, true, D>(q, k, v, o, batch, hq, hkv, lq, lk, st, scale, kvsub);
    else
      launch_fwd<kSmallBN, 2, false, D>(q, k, v, o, batch, hq, hkv, lq, lk, st, scale, kvsub);
  } else if (nblk64 < kSmallGrid && G == 4) {
    if (causal)
      launch_fwd<kSmallBN, 4, true, D>(q, k, v, o, batch, hq, hkv, lq, lk, st, scale, kvsub);
    else
      launch_fwd<kSmallBN, 4, false, D>(q, k, v, o, batch, hq, hkv, lq, lk, st, scale, kvsub);
  } else if (causal && kPersistMinItems > 0 && nblk64 >= (int64_t)kPersistMinItems * cu_count()) {
    // Enough causal query blocks for every CU to take several: one resident workgroup per CU.
    static_assert(kPersistWaves == kWaves, "the persistent kernel's query blocks are the tile kernel's");
    persist(std::integral_constant<int, 1>{}, nqb);
  } else if (causal) {
    launch_fwd<128, kWaves, true, D>(q, k, v, o, batch, hq, hkv, lq, lk, st, scale, kvsub);
  } else {
    launch_fwd<128, kWaves, false, D>(q, k, v, o, batch, hq, hkv, lq, lk, st, scale, kvsub);
  }
  KH_CHECK_LAUNCH();
  return KH_OK;
}

// =============================================================================================
// fp32 attention in split-bf16 form (the float32-activation prefill).
// =============================================================================================
// Q, K, V and O are fp32, head_dim 128, any GQA ratio.  Every operand value x is carried as two
// bf16 values, hi = bf16(x) and lo = bf16(x - hi) (x - hi is exact in fp32, and |x - hi - lo| <=
// 2^-16 |x|), and every product as three v_mfma_f32_32x32x16_bf16 into one fp32 accumulator,
// hi * hi + hi * lo + lo * hi (lo * lo, below 2^-16 of the product, is dropped): S^T = K Q^T and
// O^T += V^T P^T each within about 2^-15 of the fp32 products, in 96 MFMA cycles per 16-wide
// k-step where the fp32 MFMA takes 512.  P is split the same way after the exponential; l sums
// the fp32 P.
//
// A workgroup is (batch, query head, 32-row query block) with four waves, one per SIMD; wave w
// takes the block's 32-key chunks w, w + 4, w + 8, ... (causal: up to the block's last row), so
// the longest block's chain is a quarter of its keys.  A chunk is used by one wave only, so a wave
// loads its operands straight from memory into registers in the MFMA layouts and splits them
// there -- the next chunk's K once QK^T has consumed the current one, the next V once PV has --
// with no LDS staging and no barrier:
//  - K (the A operand of S^T): lane (r, g) reads key row swap23(r) of the chunk, columns
//    16 c + 8 g .. + 7 -- 64 contiguous bytes of a row per lane pair and k-step.  swap23 (bits 2
//    and 3 of the key index exchanged) makes accumulator registers j = 0..7 of lane group g hold
//    keys 8 g + j and j = 8..15 keys 16 + 8 g + j - 8, the B-operand layout of the PV product.
//  - V^T (the A operand of O^T): row m of output tile dt is column d = 4 m + dt (a permutation
//    of the rows, which changes no sum), so lane (r, g) needs V[16 kc + 8 g + e][4 r + dt] for
//    dt = 0..3 -- one 16-byte load per key e = 0..7, the 32 lanes of a group reading 512
//    contiguous bytes of one key row -- and the four tiles' accumulator registers j form 16
//    contiguous output bytes.  (4-byte loads along 32 dt + r took four times the load
//    instructions, and with 80 loads per chunk the wave stalled at issue on the 63 loads the
//    counter tracks: C5's attention 19.3 -> 18.2 us per layer, outputs bit-identical.)
// The four waves' (m, l, O) are merged through LDS at the end by wave 0, in wave order.  Softmax
// as SoftmaxLog2 (the QK^T accumulators start at -m; the reference is raised when a lane's sum of
// P exceeds kSumMax).
// Measured and not kept: converting K and V once per call into bf16 hi / lo planes (V transposed)
// in a separate launch, so that the attention loop only loads ready operands -- C1 13.3 -> 20.2 us
// and C5's prefill 3.23 -> 3.42 ms: the extra dependent launch costs more than the conversion.
constexpr int kSplitWaves = 4;
using FL128 = Flash<128, 8, 128>;  // for its swap23 and 32-bit strides
using SplitStrides = FL128::Strides32;

// Four floats -> their bf16 hi parts and the bf16 of the remainders, as two 8-byte rows.
__device__ __forceinline__ void split4(const uint4& x, uint2& hi, uint2& lo) {
  const float a = __uint_as_float(x.x), b = __uint_as_float(x.y), c = __uint_as_float(x.z), d = __uint_as_float(x.w);
  hi.x = pack_bf16x2(a, b);
  hi.y = pack_bf16x2(c, d);
  lo.x = pack_bf16x2(a - __uint_as_float(hi.x << 16), b - __uint_as_float(hi.x & 0xffff0000u));
  lo.y = pack_bf16x2(c - __uint_as_float(hi.y << 16), d - __uint_as_float(hi.y & 0xffff0000u));
}
// Eight floats (as two loads) -> hi and lo bf16x8 operands.
__device__ __forceinline__ void split8(const uint4& x0, const uint4& x1, bf16x8& hi, bf16x8& lo) {
  uint2 h0, l0, h1, l1;
  split4(x0, h0, l0);
  split4(x1, h1, l1);
  hi = __builtin_bit_cast(bf16x8, make_uint4(h0.x, h0.y, h1.x, h1.y));
  lo = __builtin_bit_cast(bf16x8, make_uint4(l0.x, l0.y, l1.x, l1.y));
}

// One 32-key chunk's operands of one wave, as loaded: K rows (8 k-steps of two 16-byte loads) and
// V rows (2 key steps x 8 keys, columns 4 r .. 4 r + 3 of each).
struct SplitK {
  uint4 k[16];
};
struct SplitV {
  uint4 v[16];
};
// Word i (compile-time) of a 16-byte load.
template <int I>
__device__ __forceinline__ uint32_t word(const uint4& u) {
  if constexpr (I == 0) return u.x;
  else if constexpr (I == 1) return u.y;
  else if constexpr (I == 2) return u.z;
  else return u.w;
}

template <bool CAUSAL>
__global__ __launch_bounds__(kSplitWaves * 64, 1) void flash_split_kernel(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V, float* __restrict__ O,
    int hq, int ratio, int lq, int lk, SplitStrides st, float scale, int n_qblocks) {
  constexpr int D = 128, NQ = D / 16, ND = D / 32;
  __shared__ __attribute__((aligned(16))) float part[(kSplitWaves - 1) * 66 * 64];  // [wave - 1][66][lane]
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63, r = lane & 31, g = lane >> 5;
  // Workgroups go to the 8 XCDs round-robin (workgroup i on XCD i % 8), each with its own L2.
  // When the grid divides by 8, XCD x runs a contiguous range of logical blocks -- whole query
  // heads, so a kv head's K / V are read into one L2 and reused there -- heaviest (last) query
  // block of a head first.
  int logical = blockIdx.x;
  if (gridDim.x % kXcds == 0) logical = (blockIdx.x % kXcds) * (gridDim.x / kXcds) + blockIdx.x / kXcds;
  const int qblk = n_qblocks - 1 - logical % n_qblocks, bh = logical / n_qblocks;
  const int b = bh / hq, h = bh % hq, hk = h / ratio;
  const int q0 = qblk * 32, qi = q0 + r;
  const int kv_end = CAUSAL ? min(lk, q0 + 32) : lk;
  const int nchunks = (kv_end + 31) / 32;
  const float c2 = scale * kLog2e;

  // This lane's Q row (query qi, columns 16 c + 8 g .. + 7) as hi and lo operands.
  bf16x8 qh[NQ], ql[NQ];
  {
    const auto rq = make_rsrc(Q + (int64_t)b * st.qb + (int64_t)h * st.qh, (uint32_t)(((int64_t)(lq - 1) * st.qs + D) * 4));
    const uint32_t qoff = (uint32_t)(((int64_t)qi * st.qs + 8 * g) * 4);
#pragma unroll
    for (int c = 0; c < NQ; ++c) split8(buf_load16(rq, qoff + 64 * c), buf_load16(rq, qoff + 64 * c + 16), qh[c], ql[c]);
  }
  const auto rk = make_rsrc(K + (int64_t)b * st.kb + (int64_t)hk * st.kh, (uint32_t)(((int64_t)(lk - 1) * st.ks + D) * 4));
  const auto rv = make_rsrc(V + (int64_t)b * st.vb + (int64_t)hk * st.vh, (uint32_t)(((int64_t)(lk - 1) * st.vs + D) * 4));
  const int krow = FL128::swap23(r);
  auto load_k = [&](int tc, SplitK& ch) {
    const uint32_t ko = (uint32_t)(((int64_t)(32 * tc + krow) * st.ks + 8 * g) * 4);
#pragma unroll
    for (int c = 0; c < NQ; ++c) {
      ch.k[2 * c] = buf_load16(rk, ko + 64 * c);
      ch.k[2 * c + 1] = buf_load16(rk, ko + 64 * c + 16);
    }
  };
  auto load_v = [&](int tc, SplitV& ch) {
#pragma unroll
    for (int kc = 0; kc < 2; ++kc)
#pragma unroll
      for (int e = 0; e < 8; ++e)
        ch.v[8 * kc + e] = buf_load16(rv, (uint32_t)(((int64_t)(32 * tc + 16 * kc + 8 * g + e) * st.vs + 4 * r) * 4));
  };

  f32x16 oacc[ND];
#pragma unroll
  for (int dt = 0; dt < ND; ++dt)
#pragma unroll
    for (int j = 0; j < 16; ++j) oacc[dt][j] = 0.f;
  SoftmaxLog2 sl;
  // QK^T, mask and softmax of chunk tc; P (hi, lo) out
  auto scores = [&](int tc, const SplitK& ch, bf16x8 (&ph)[2], bf16x8 (&pl)[2]) {
    f32x16 sacc[1];
    {
      f32x16 acc = sl.mneg;
#pragma unroll
      for (int c = 0; c < NQ; ++c) {
        bf16x8 kh8, kl8;
        split8(ch.k[2 * c], ch.k[2 * c + 1], kh8, kl8);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kh8, qh[c], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kh8, ql[c], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kl8, qh[c], acc, 0, 0, 0);
      }
      sacc[0] = acc;
    }
    // causal / length mask (keys 32 tc + 8 g + (j & 7) + 16 (j >> 3) of this lane)
    const int kb = 32 * tc;
    if (kb + 32 > lk || (CAUSAL && kb + 31 > q0)) {
      const int lim = (CAUSAL ? min(lk, qi + 1) : lk) - kb - 8 * g;
#pragma unroll
      for (int j = 0; j < 16; ++j)
        if (16 * (j >> 3) + (j & 7) >= lim) sacc[0][j] = -INFINITY;
    }
    // P = 2^(c2 (s - m)) in fp32, split into bf16 hi and lo operands; returns this lane's fp32 sum
    auto exponentiate = [&]() -> float {
      float sum = 0.f;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        float pv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          pv[e] = fast_exp2(sacc[0][8 * hh + e] * c2);
          sum += pv[e];
        }
        split8(make_uint4(__float_as_uint(pv[0]), __float_as_uint(pv[1]), __float_as_uint(pv[2]), __float_as_uint(pv[3])),
               make_uint4(__float_as_uint(pv[4]), __float_as_uint(pv[5]), __float_as_uint(pv[6]), __float_as_uint(pv[7])),
               ph[hh], pl[hh]);
      }
      return sum;
    };
    float ps = exponentiate();
    if (sl.need_raise(ps)) {
      sl.raise(sacc, c2, oacc);
      ps = exponentiate();
    }
    sl.l += ps;
  };
  // O^T += V^T P^T over the chunk's two 16-key steps; tile dt's A row m is column d = 4 m + dt
  auto pv_tile = [&](auto dt_c, const SplitV& ch, const bf16x8 (&ph)[2], const bf16x8 (&pl)[2]) {
    constexpr int DT = decltype(dt_c)::value;
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) {
      const uint4* vv = ch.v + 8 * kc;
      bf16x8 vh8, vl8;
      split8(make_uint4(word<DT>(vv[0]), word<DT>(vv[1]), word<DT>(vv[2]), word<DT>(vv[3])),
             make_uint4(word<DT>(vv[4]), word<DT>(vv[5]), word<DT>(vv[6]), word<DT>(vv[7])), vh8, vl8);
      oacc[DT] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vh8, ph[kc], oacc[DT], 0, 0, 0);
      oacc[DT] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vh8, pl[kc], oacc[DT], 0, 0, 0);
      oacc[DT] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vl8, ph[kc], oacc[DT], 0, 0, 0);
    }
  };
  auto pv = [&](const SplitV& ch, const bf16x8 (&ph)[2], const bf16x8 (&pl)[2]) {
    static_assert(ND == 4, "four output tiles");
    pv_tile(std::integral_constant<int, 0>{}, ch, ph, pl);
    pv_tile(std::integral_constant<int, 1>{}, ch, ph, pl);
    pv_tile(std::integral_constant<int, 2>{}, ch, ph, pl);
    pv_tile(std::integral_constant<int, 3>{}, ch, ph, pl);
  };
  // This wave's chunks wave, wave + 4, ...: one register set each for K and V.  The next chunk's K
  // loads once QK^T has consumed the current one (and lands during the softmax and PV), the next
  // V once PV has (landing during the next QK^T and softmax).  One loop body, not unrolled: a
  // wave's first pass through each copy of unrolled code waits on instruction fetches.  (K in two
  // register sets, the next chunk's K loading during the whole current chunk, needs the body twice:
  // C5-shape call 17.6 -> 18.2 us, 32-key call 7.4 -> 8.1 us.)
  {
    SplitK ka;
    SplitV vv;
    int tc = wave;
    if (tc < nchunks) {
      load_k(tc, ka);
      load_v(tc, vv);
    }
#pragma unroll 1
    while (tc < nchunks) {
      const int nx = tc + kSplitWaves;
      bf16x8 ph[2], pl[2];
      scores(tc, ka, ph, pl);
      if (nx < nchunks) load_k(nx, ka);
      pv(vv, ph, pl);
      if (nx < nchunks) load_v(nx, vv);
      tc = nx;
    }
  }
  // Merge: waves 1..3 write (m, l, O) to LDS; wave 0 combines them in wave order.
  float l = sl.l;
  if (wave > 0) {
    float* p = part + (wave - 1) * 66 * 64 + lane;
    p[0] = sl.m;
    p[64] = l;
#pragma unroll
    for (int dt = 0; dt < ND; ++dt)
#pragma unroll
      for (int j = 0; j < 16; ++j) p[(2 + 16 * dt + j) * 64] = oacc[dt][j];
  }
  __syncthreads();
  if (wave > 0) return;
  float mo[kSplitWaves];
  mo[0] = sl.m;
#pragma unroll
  for (int w2 = 1; w2 < kSplitWaves; ++w2) mo[w2] = part[(w2 - 1) * 66 * 64 + lane];
  float mt = mo[0];
#pragma unroll
  for (int w2 = 1; w2 < kSplitWaves; ++w2) mt = fmaxf(mt, mo[w2]);
  // a wave with no unmasked key has m = -inf and adds nothing (its l and O are 0)
  const float a0 = mo[0] == -INFINITY ? 0.f : fast_exp2((mo[0] - mt) * c2);
  l *= a0;
#pragma unroll
  for (int dt = 0; dt < ND; ++dt)
#pragma unroll
    for (int j = 0; j < 16; ++j) oacc[dt][j] *= a0;
#pragma unroll
  for (int w2 = 1; w2 < kSplitWaves; ++w2) {
    const float* p = part + (w2 - 1) * 66 * 64 + lane;
    const float a = mo[w2] == -INFINITY ? 0.f : fast_exp2((mo[w2] - mt) * c2);
    l += a * p[64];
#pragma unroll
    for (int dt = 0; dt < ND; ++dt)
#pragma unroll
      for (int j = 0; j < 16; ++j) oacc[dt][j] += a * p[(2 + 16 * dt + j) * 64];
  }
  // O[qi][d] = O / l (l: this lane's keys plus lane ^ 32's).  Register j = 4 a + i of tile dt holds
  // A row m = 8 a + 4 g + i, i.e. d = 4 m + dt: the four tiles' registers j form 16 contiguous bytes.
  const float l_tot = l + __shfl_xor(l, 32, 64);
  if (qi < lq) {
    const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
    float* orow = O + (int64_t)b * st.ob + (int64_t)h * st.oh + (int64_t)qi * st.os;
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        *reinterpret_cast<float4*>(orow + 4 * (8 * a + 4 * g + i)) =
            make_float4(oacc[0][4 * a + i] * inv, oacc[1][4 * a + i] * inv, oacc[2][4 * a + i] * inv,
                        oacc[3][4 * a + i] * inv);
  }
}

}  // namespace

namespace kh {

bool flash_prefill_supported(const void* q, const void* k, const void* v, const void* o, int hq, int hkv,
                             int64_t lq, int64_t lk, int d, const AttnStrides& st) {
  (void)hq;
  (void)hkv;
  if (!(d == 64 || d == 128)) return false;  // any GQA ratio (prefill_groups)
  if (!(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(o))) return false;
  const int64_t all[] = {st.qb, st.qh, st.qs, st.kb, st.kh, st.ks, st.vb, st.vh, st.vs, st.ob, st.oh, st.os};
  for (int64_t s : all)
    if (s < 0 || s > INT32_MAX) return false;  // the kernels hold strides as 32-bit values
  const int64_t s16[] = {st.qb, st.qh, st.qs, st.kb, st.kh, st.ks, st.vb, st.vh, st.vs};
  for (int64_t s : s16)
    if (s % 8 != 0) return false;
  if (st.ob % 4 || st.oh % 4 || st.os % 4) return false;
  // Per-head byte offsets (including the zero-filled rows past the end) must fit 31 bits.
  const int64_t lim = int64_t(1) << 31;
  // (Tiles are prefetched up to two ahead: keys up to lk + 383 are addressed and read as zero.)
  if ((lq + 512) * st.qs * 2 >= lim || (lk + 512) * st.ks * 2 >= lim || (lk + 512) * st.vs * 2 >= lim) return false;
  return true;
}

bool flash_split_supported(const void* q, const void* k, const void* v, const void* o, int hq, int hkv, int64_t lq,
                           int64_t lk, int d, const AttnStrides& st, float scale) {
  (void)hq;
  (void)hkv;
  if (d != 128 || !(scale > 0.f)) return false;
  if (!(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(o))) return false;
  const int64_t all[] = {st.qb, st.qh, st.qs, st.kb, st.kh, st.ks, st.vb, st.vh, st.vs, st.ob, st.oh, st.os};
  for (int64_t s : all)
    if (s < 0 || s > INT32_MAX || s % 4 != 0) return false;  // 16-byte rows, 32-bit strides
  const int64_t lim = int64_t(1) << 31;
  return (lq * st.qs + d) * 4 < lim && (lk * st.ks + d) * 4 < lim && (lk * st.vs + d) * 4 < lim;
}

int launch_flash_split_f32(const void* q, const void* k, const void* v, void* o, int batch, int hq, int hkv, int lq,
                           int lk, const AttnStrides& st, float scale, bool causal) {
  const int nqb = (lq + 31) / 32;
  const int64_t grid = (int64_t)nqb * batch * hq;
  KH_REQUIRE(grid <= INT32_MAX, "kh_flash_attention_split: grid too large");
  const SplitStrides s32{(int32_t)st.qb, (int32_t)st.qh, (int32_t)st.qs, (int32_t)st.kb, (int32_t)st.kh, (int32_t)st.ks,
                         (int32_t)st.vb, (int32_t)st.vh, (int32_t)st.vs, (int32_t)st.ob, (int32_t)st.oh, (int32_t)st.os};
  const float *Q = (const float*)q, *K = (const float*)k, *V = (const float*)v;
  float* O = (float*)o;
  if (causal)
    flash_split_kernel<true><<<(int)grid, kSplitWaves * 64, 0, stream()>>>(Q, K, V, O, hq, hq / hkv, lq, lk, s32, scale,
                                                                          nqb);
  else
    flash_split_kernel<false><<<(int)grid, kSplitWaves * 64, 0, stream()>>>(Q, K, V, O, hq, hq / hkv, lq, lk, s32,
                                                                           scale, nqb);
  KH_CHECK_LAUNCH();
  return KH_OK;
}

int launch_flash_prefill_bf16(const void* q, const void* k, const void* v, void* o, int batch, int hq, int hkv,
                              int lq, int lk, int d, const AttnStrides& st, float scale, bool causal) {
  if (d == 64) return launch_prefill_d<64>(q, k, v, o, batch, hq, hkv, lq, lk, st, scale, causal);
  return launch_prefill_d<128>(q, k, v, o, batch, hq, hkv, lq, lk, st, scale, causal);
}

int launch_flash_prefill_bf16_masked(const void* q, const void* k, const void* v, void* o, int batch, int hq,
                                     int hkv_real, int lq, int lk, int d, const AttnStrides& st, float scale,
                                     const void* mask, const MaskArgs& ma, int mask_dtype) {
  const PrefillGroups pg = prefill_groups(hq, hkv_real);
  const int G = pg.G, kvsub = pg.kvsub, hkv = pg.hkv;
  const int BMQ = 32 * (kWaves / G);
  const int nqb = (lq + BMQ - 1) / BMQ;
  const int64_t nblk64 = (int64_t)nqb * batch * hkv;
  KH_REQUIRE(nblk64 <= INT32_MAX, "kh_flash_attention_masked: grid too large");
  const int nblk = (int)nblk64;
  const uint16_t *Q = (const uint16_t*)q, *K = (const uint16_t*)k, *V = (const uint16_t*)v;
  uint16_t* O = (uint16_t*)o;
#define KH_MASKED_LAUNCH(MT, DD)                                                                               \
  flash_fwd_kernel<64, kWaves, 1, false, MT, DD><<<nblk, kWaves * 64, 0, stream()>>>(Q, K, V, O, batch, hq, hkv, lq, \
                                                                                     lk, st, scale, nqb, mask, ma, kvsub)
  if (d == 64) {
    if (mask_dtype == KH_F32)
      KH_MASKED_LAUNCH(1, 64);
    else
      KH_MASKED_LAUNCH(2, 64);
  } else {
    if (mask_dtype == KH_F32)
      KH_MASKED_LAUNCH(1, 128);
    else
      KH_MASKED_LAUNCH(2, 128);
  }
#undef KH_MASKED_LAUNCH
  KH_CHECK_LAUNCH();
  return KH_OK;
}

}  // namespace kh
