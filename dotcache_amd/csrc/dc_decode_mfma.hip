// MFMA fast path of the fused paged decode (gfx950, v_mfma_f32_16x16x32_f16).
//
// One wavefront -- one workgroup -- runs one work item: it walks the item's
// pages in order, scores each 32-token chunk for the GQA query heads of its
// KV head, folds the logits into a running (max, sum) per head and mixes the
// value codes, all from the compressed page bytes.  At the end it writes the
// normalised output (an item that covers its whole sequence) or a split-K
// partial (m, l, o) for the merge kernel.  Accepted pages: keys M3 fp16 or
// M0 4- or 8-bit (group 32, affine or symmetric; one width per launch);
// values M0 4- or 8-bit (group 32 or 64, affine or symmetric) or M3 fp16;
// up to 16 query heads per KV head.  Other formats take the generic kernel
// (dc_decode.hip).
//
// Prologue: the item, then its pages' table entries, then their
// descriptors -- or, with page records (dc_gather_page_records), the item
// and its pages' descriptors in one round, indexed by the workgroup id.
// Pipelined instances with DMA keys then issue the item's first chunk
// straight from page 0's descriptors, before the batch layout.
//
// Pipeline (one wave per SIMD, head_dim <= 128, one key format, no M3
// values): while chunk j is mixed, chunk j + 1 is staged and scored and
// chunk j + 2 is being loaded, so the score's MFMA chain, the mix's
// unpacking and the loads of one wavefront overlap.  Other pools keep one
// chunk in flight (instances built for two waves per SIMD overlap across
// waves instead).  M3 key and value rows reach LDS by DMA
// (buffer_load ... lds).
//
// Exactness.  Every MFMA operand is exact: escape rows are fp16 already,
// codes minus zero point are small integers, and each fp32 operand (scaled
// query, softmax weight x value scale) is carried as two fp16 operands, its
// high part and its residual, each multiplied by the same exact other
// operand and accumulated in fp32.  Per-(token, group) key scales and biases
// are applied in fp32 after the MFMA, in the reference's streaming form
// s * (codes . q_g) + b * sum(q_g) (reference
// dotcache/attention_reference.py:101-126, :168-192).
//
// Lane maps (lane l, r = l % 16, kb = l / 16; a 16x16x32 MFMA gives lane l
// row r of A, column r of B, k-slots 8 kb .. 8 kb + 7, and the D values of
// rows 4 kb + i, column r):
//   score  D[token, q] = K[token, :] . Q[q, :]  (A = key rows, B = queries,
//          one MFMA per 32 channels).  In tile hh, A row m is chunk token
//          8 (m / 4) + 4 hh + m % 4, so lane (r, kb) ends up with the logits
//          of chunk tokens 8 kb + e, e < 8, for head r.
//   mix    D[q, d] = A[q, token] x B[token, d]  (A = weights, k = tokens).
//          Lane (r, kb) feeds A row r = head r at k-slots = chunk tokens
//          8 kb + e: exactly the logits it holds, so weights never cross
//          lanes.  Column r of tile h of value group g is channel
//          VGS g + 8 (r / L) + r % L + L h with L = 128 / VGS, which lets
//          every lane unpack its codes with one byte permute per pair of
//          tokens.
//
// Group blocks.  With n_q <= 4 (or <= 8) most of the 16 columns / rows above
// would be dead heads.  Instead they hold GB = 4 (or 2) copies of the NQB = 4
// (8) heads, copy c = r / NQB working on group c of every block of GB
// consecutive key / value groups:
//   score  group g's query fragment is zero outside copy g % GB's columns, so
//          the GB groups of a block accumulate into one tile pair, each
//          copy's column holding its own group's dot product; one scale /
//          bias step per block then serves GB groups, and rotate-adds within
//          each 16-lane row sum the copies, which leaves every copy with the
//          whole logit of its head.
//   mix    row (c, q) is weight_q x the scale of group GB b + c: one weight x
//          scale operand per block instead of one per group, and tile h of
//          group g keeps only copy g % GB's rows.
// The products are the same; only the lanes that form them change.
#include <type_traits>

#include "dc_common.h"
#include "dc_decode.h"

namespace dc {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

union Frag {
  half8 h;
  uint32_t u[4];
};

__device__ __forceinline__ f32x4 mfma(const Frag& a, const Frag& b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a.h, b.h, c, 0, 0, 0);
}

__device__ __forceinline__ uint32_t bits_of(h2 v) { return __builtin_bit_cast(uint32_t, v); }
__device__ __forceinline__ h2 h2_of(uint32_t v) { return __builtin_bit_cast(h2, v); }

// The value of lane (l - N) mod 16 of the lane's row of 16 (DPP row rotate).
template <int N>
__device__ __forceinline__ float row_ror(float x) {
  static_assert(N > 0 && N < 16, "row rotate by 1 .. 15");
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x120 + N, 0xf, 0xf, false));
}

// fp16 pair (lo, hi) from two floats, round to nearest even.
__device__ __forceinline__ uint32_t pack_h2(float lo, float hi) { return bits_of(h2{(_Float16)lo, (_Float16)hi}); }

// The products a0 * b0 and a1 * b1 (fp32 times fp16-exact values) as fp16
// pairs: high parts hi = rne16(a b) and residuals rne16(a b - hi), each one
// mixed-precision fma that writes an fp16 half (v_fma_mix_lo/hi_f16, a
// single rounding of the exact a b or a b - hi).  The pair carries a b to
// about 2^-22 relative while hi and the residual stay in fp16's normal range.
struct Split2 {
  uint32_t hi, res;
};
__device__ __forceinline__ Split2 split_products(float a0, float b0, float a1, float b1) {
  const _Float16 h0 = (_Float16)__builtin_fmaf(a0, b0, 0.f), h1 = (_Float16)__builtin_fmaf(a1, b1, 0.f);
  const _Float16 l0 = (_Float16)__builtin_fmaf(a0, b0, -float(h0)), l1 = (_Float16)__builtin_fmaf(a1, b1, -float(h1));
  return {bits_of(h2{h0, h1}), bits_of(h2{l0, l1})};
}

// Weights are exp2(logit - m_ref), with m_ref the head's running max when it
// last moved; it moves only when a chunk's max exceeds it by more than this
// (log2 units), so weights stay <= 2^kLazy and the accumulators are rescaled
// rarely.
constexpr float kLazy = 2.f;

// Key-page mix of a pool: only M3 rows, only M0 codes (4- or 8-bit, one
// width per pool), or both.
enum KeyMode { KEYS_M3 = 0, KEYS_M0 = 1, KEYS_MIXED = 2 };

template <int HD, int VGS, int VBITS>
struct MfmaCfg {
  static constexpr int KG = HD / 32;          // key groups of 32 channels (= contraction steps of the score)
  static constexpr int VG = HD / VGS;         // value groups
  static constexpr int H = VGS / 16;          // mix column tiles per value group
  static constexpr int LPW4 = 128 / VGS;      // lanes sharing one code word
  static constexpr int NACC = HD / 16;        // mix accumulator tiles
  static constexpr int W = VBITS * VGS / 32;  // code words per (token, value group)
  // LDS staging of a chunk's value codes: per group 32 tokens of W words with
  // W pad words after every 8 tokens, so the words that the lanes of one read
  // touch fall in distinct banks
  static constexpr int PAD = W;
  static constexpr int GSTRIDE = 32 * W + 4 * PAD;
  static constexpr int NVP = VG * 8 * W / 64;  // 16-byte code pieces per lane per chunk
  static constexpr int VSW = 16 * VG;          // value scale words per chunk ([32][VG] fp16)
  static constexpr int KSW = 16 * KG;          // key scale words per chunk ([32][KG] fp16)
  static constexpr int NVS = (VSW + 63) / 64;
  static constexpr int NKS = (KSW + 63) / 64;
  // scales / biases are staged as loaded ([32][G] fp16) or, where a lane
  // needs one group of 8 consecutive tokens (group blocks), transposed:
  // [G][SP] fp16, row pitch SP = 40 halves (16-byte aligned rows, and the
  // transposing 16-bit stores of one instruction spread over the banks)
  static constexpr int SP = 40;
  static constexpr int VSR = VSW > VG * SP / 2 ? VSW : VG * SP / 2;  // words of one value scale region
  static constexpr int KSR = KSW > KG * SP / 2 ? KSW : KG * SP / 2;
  static constexpr int VPAY = 0, VSC = VG * GSTRIDE, VBS = VSC + VSR, KSC = VBS + VSR, KBS = KSC + KSR;
  static constexpr int STAGE = KBS + KSR;  // words of one staged chunk
  static_assert(VG * 8 * W % 64 == 0, "value pieces must spread evenly over the wave");
  static_assert(W % 4 == 0, "value code rows are staged in 16-byte pieces");
};

// Waves per SIMD an instance is built for.  Pools with M0 keys at
// head_dim 128 and up to 8 heads per block are bound by instruction issue:
// two unpipelined waves per SIMD (at most 256 registers each) hide each
// other's waits, where one pipelined wave cannot (C4: 42.1 against 49.3 us
// per launch).  Pools of M3 keys (C3) stream bytes and keep one pipelined
// wave (two waves: 32.9 against 32.7 us).  At head_dim 256 (M0 keys and
// values, 4-bit, blocks of 4 heads) the same holds once the key codes
// come by DMA: 133.1 against 156.1 us per launch on C5's pages without the
// fp16 window (the M0 pool, paired replays).
template <int HD, int KMODE, int KBITS, int VBITS, int NQB>
constexpr int waves_per_simd() {
  // (8-bit keys and values with 8 heads per block, and head_dim 256 with 8,
  // spill at 256 registers)
  return (HD == 128 && KMODE != KEYS_M3 && NQB <= 8 && !(KBITS == 8 && VBITS == 8 && NQB == 8)) ||
                 (HD == 256 && KMODE == KEYS_M0 && KBITS == 4 && VBITS == 4 && NQB == 4)
             ? 2
             : 1;
}

// Two staged chunks in flight where the registers allow it: one wave per
// SIMD, head_dim <= 128, no M3 values, one key format.
template <int HD, int KMODE, int KBITS, int VBITS, bool VM3, int NQB>
constexpr bool pipelined() {
  return HD <= 128 && !VM3 && KMODE != KEYS_MIXED && waves_per_simd<HD, KMODE, KBITS, VBITS, NQB>() == 1;
}

// Registers one chunk needs from HBM: this lane's KW words of each M0 key
// code block (KWREG: pipelined instances; the others take M0 codes and M3
// key rows straight to LDS), the value code pieces and the scale / bias
// words.
template <int HD, int VGS, int VBITS, int KMODE, int KBITS, bool KWREG = true>
struct ChunkRegs {
  using Cfg = MfmaCfg<HD, VGS, VBITS>;
  static constexpr bool kKeyWords = KMODE != KEYS_M3 && KWREG;
  static constexpr int KW = KBITS / 4;  // code words of one lane's 8 channels
  uint32_t kw[kKeyWords ? 2 : 1][kKeyWords ? Cfg::KG * KW : 1];
  u32x4 vr[Cfg::NVP];  // value code pieces, blob byte order
  uint32_t ks[Cfg::NKS], kbw[Cfg::NKS], vs[Cfg::NVS], vb[Cfg::NVS];  // scale / bias words
};

// Slot swizzle of the key rows staged in LDS: row t of PPR 16-byte pieces
// keeps piece p at slot p ^ key_swz(t).  Bits {0, 1, 3, 4} of t (PPR >= 16)
// or {1, 3, 4} (PPR = 8): the 16 rows one score read touches, 8 (r / 4) +
// 4 hh + r % 4 for r < 16, get 16 (8) distinct values, which puts their
// pieces in distinct 16-byte bank groups.  A bit selection, so it splits
// over rows whose set bits are disjoint: key_swz(a | b) = key_swz(a) ^
// key_swz(b).
template <int PPR>
__device__ __forceinline__ constexpr uint32_t key_swz(uint32_t t) {
  return PPR >= 16 ? (t & 3u) | (((t >> 3) & 3u) << 2) : ((t >> 1) & 1u) | (((t >> 3) & 3u) << 1);
}

// One chunk: the page it belongs to (wave-uniform, in SGPRs) and its first token.
struct PageMeta {
  __amdgpu_buffer_rsrc_t krs, vrs;  // buffer resources of the key / value blobs
  const uint8_t* vp;                // value blob (M3 value rows are loaded from it)
  int T;                            // tokens of the page
  int kfmt, vfmt;
  uint32_t ksc, kbs, vsc, vbs;  // byte offsets of scales / biases in the blobs (0 where absent)
  int c0;                       // first token of the chunk
};

// KBITS: code width of the pool's M0 keys (4 or 8).  KAFF / VAFF: the key /
// value pool may hold affine M0 pages (bias terms); false drops that code
// entirely.
//
// NQB: query heads per block of the MFMA's 16 columns (score) / rows (mix),
// 4, 8 or 16.  Below 16 the 16 slots hold GB = 16 / NQB copies of the NQB
// heads, and copy c works on group c of each block of GB consecutive
// groups (see "Group blocks" above).
template <int HD, int VGS, int KMODE, int KBITS, int VBITS, bool VM3, bool KAFF, bool VAFF, int NQB>
__global__ void __launch_bounds__(64, (waves_per_simd<HD, KMODE, KBITS, VBITS, NQB>()))
    decode_mfma_kernel(DecodeArgs a) {
  static_assert(KBITS == 4 || KBITS == 8, "M0 keys are 4- or 8-bit");
  using Cfg = MfmaCfg<HD, VGS, VBITS>;
  constexpr bool kPipe = pipelined<HD, KMODE, KBITS, VBITS, VM3, NQB>();
  constexpr int KBLK = 4 * KBITS;  // bytes of one (token, group) key code block
  constexpr int KG = Cfg::KG, VG = Cfg::VG, H = Cfg::H, LPW4 = Cfg::LPW4, W = Cfg::W, NACC = Cfg::NACC;
  static_assert(NQB == 4 || NQB == 8 || NQB == 16, "4, 8 or 16 heads per block");
  constexpr int GB = 16 / NQB;                // groups per block
  constexpr int KNB = KG / GB, VNB = VG / GB;  // key / value group blocks
  static_assert(KG % GB == 0 && VG % GB == 0, "key and value groups come in whole blocks");
  // two staged chunks in flight where the registers allow it
  __shared__ uint32_t lds_all[(kPipe ? 2 : 1) * Cfg::STAGE];
  // M3 keys (pools that may hold them): each chunk's 32 key rows go straight
  // from HBM into an LDS buffer (buffer_load ... lds), 1 KiB-contiguous per
  // instruction, and the score reads them back in the MFMA's A layout, with
  // the slot swizzle key_swz.  One buffer per chunk in flight, as separate
  // objects, so a read of one waits only for its own loads.
  constexpr bool kDmaK = KMODE != KEYS_M0;
  // pools with 4-bit M0 keys order each lane's 8 channels as pairs (i, i + 4)
  constexpr bool kPairedQ = KMODE != KEYS_M3 && KBITS == 4;
  __shared__ __attribute__((aligned(16))) uint32_t kbuf0[kDmaK ? 32 * HD / 2 : 1];
  __shared__ __attribute__((aligned(16))) uint32_t kbuf1[kDmaK && kPipe ? 32 * HD / 2 : 1];
  // M3 value rows of the chunk being mixed, by DMA in the same slot layout
  // (pools that may hold M3 values; these are never pipelined)
  static_assert(!(VM3 && kPipe), "pools with M3 values run one chunk in flight");
  __shared__ __attribute__((aligned(16))) uint32_t vbuf[VM3 ? 32 * HD / 2 : 1];
  // key buffer 0 or 1, chosen at compile time (std::integral_constant), so
  // every LDS address the loads and reads use is a constant of one object
  auto kbuf = [&](auto bi) -> uint32_t* {
    if constexpr (decltype(bi)::value == 0)
      return kbuf0;
    else
      return kbuf1;
  };
  using KB0 = std::integral_constant<int, 0>;
  using KB1 = std::integral_constant<int, 1>;
  // M0 key codes of the unpipelined instances go to LDS by DMA too: 16-byte
  // loads, each instruction 1 KiB of two (4-bit) or one (8-bit) groups'
  // code blocks, contiguous in HBM.  In registers (a 4-byte load per group
  // and tile: four 64-byte pieces of two cache lines per instruction) the
  // same bytes cost the memory system far more: the C5 kernel with its
  // arithmetic left out took 139 us per launch with those loads and 117 us
  // with 16-byte ones.  Layout [group][slot][KBLK bytes]: chunk token t at
  // slot 16 hh + m, its row m of tile hh (t = 8 (m / 4) + 4 hh + m % 4), so
  // the 64 words one score read takes (16 rows x 4 lanes) are contiguous.
  // Slot 0 shares kbuf0 with the M3 key rows (a chunk holds one or the
  // other); the one-wave M0 walk double-buffers into slot 1 (vbuf, which M0
  // chunks leave unused, or a buffer of its own).
  constexpr bool kDmaM0 = KMODE != KEYS_M3 && !kPipe;
  constexpr bool kM0Two = kDmaM0 && waves_per_simd<HD, KMODE, KBITS, VBITS, NQB>() == 1;
  constexpr int KCW = 8 * Cfg::KG * KBLK;  // words of one chunk's key codes
  static_assert(KCW <= 16 * HD, "a chunk's M0 codes fit the M3 row buffers");
  __shared__ __attribute__((aligned(16))) uint32_t kcb0[kDmaM0 && !kDmaK ? KCW : 1];
  __shared__ __attribute__((aligned(16))) uint32_t kcb1[kM0Two && !VM3 ? KCW : 1];
  auto kcode = [&](auto bi) -> uint32_t* {
    if constexpr (decltype(bi)::value == 0) {
      if constexpr (kDmaK) return kbuf0; else return kcb0;
    } else {
      if constexpr (VM3) return vbuf; else return kcb1;
    }
  };

  // The kernel arguments the prologue uses, read in one round of scalar
  // loads at entry.  Read where each is first used, they were waited for one
  // at a time along the dependent chain item -> page table -> descriptors
  // (C3: 32.65 -> 32.35 us per launch).
  asm volatile("" ::"s"(a.items), "s"(a.k_table), "s"(a.v_table), "s"(a.kpool.descs), "s"(a.vpool.descs),
               "s"(a.kpool.arena), "s"(a.vpool.arena), "s"(a.queries), "s"(a.table_stride), "s"(a.n_seqs),
               "s"(a.n_kv_heads), "s"(a.n_q), "s"(a.kpool.n_descs), "s"(a.vpool.n_descs),
               "s"(a.kpool.geometry.page_capacity), "s"(a.queries_dtype), "s"(a.q_scale), "s"(a.kpool.arena_bytes),
               "s"(a.vpool.arena_bytes), "s"(a.recs), "s"(a.rec_stride));
  // With page records, lane i's record (the descriptors of the item's page
  // i) is loaded together with the item: no dependence on it.
  u32x4 rec = {0u, 0u, 0u, 0u};
  if (a.recs != nullptr) {
    const int slot = int(threadIdx.x) < a.rec_stride ? int(threadIdx.x) : a.rec_stride - 1;
    rec = reinterpret_cast<const u32x4*>(a.recs)[int64_t(blockIdx.x) * a.rec_stride + slot];
  }
  const dc_work_item it = a.items[blockIdx.x];
  if (!item_in_bounds(it, a)) return;
  const int lane = threadIdx.x;
  const int r = lane & 15, kb = lane >> 4;
  const int nq = a.n_q;
  const int CAP = a.kpool.geometry.page_capacity;
  // this lane's score column / mix row: head qh of group copy gsel
  const int qh = r % NQB, gsel = r / NQB;
  const bool head_live = qh < nq;

  // The prologue's loads go out in two rounds: the queries and the first
  // page batch's table entries together, then the descriptors those name.
  // Every load is unconditional (clamped index or a bounds-checked buffer
  // resource), so no load waits on a branch.
  // ---- queries, raw: lane (r, kb) holds channels 32 g + 8 kb + i of head r ----
  const int64_t qbase = (int64_t(it.seq) * a.n_kv_heads + it.kv_head) * nq * HD;
  const int64_t qrow = qbase + int64_t(head_live ? qh : 0) * HD + 8 * kb;
  const bool q_f32 = a.queries_dtype == DC_F32;
  u32x4 qraw[2 * KG];  // fp32: two 16-byte pieces per group; fp16 / bf16: one
  if (q_f32) {
    const u32x4* q = reinterpret_cast<const u32x4*>(reinterpret_cast<const float*>(a.queries) + qrow);
#pragma unroll
    for (int g = 0; g < KG; ++g) {
      qraw[2 * g] = q[8 * g];
      qraw[2 * g + 1] = q[8 * g + 1];
    }
  } else {
    const u32x4* q = reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(a.queries) + qrow);
#pragma unroll
    for (int g = 0; g < KG; ++g) qraw[g] = q[4 * g];
  }

  // ---- page metadata: lane i holds the ids / descriptors of page begin + base + i ----
  const int64_t trow = (int64_t(it.seq) * a.n_kv_heads + it.kv_head) * a.table_stride;
  const int np = it.page_end - it.page_begin;
  const int kn = a.kpool.n_descs, vn = a.vpool.n_descs;
  // descriptor arrays as buffer resources: an id past the end reads zeros
  const __amdgpu_buffer_rsrc_t kdr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<void*>(static_cast<const void*>(a.kpool.descs)), 0, kn < (1 << 28) ? kn * 8 : (1 << 31) - 8, 0x00020000);
  const __amdgpu_buffer_rsrc_t vdr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<void*>(static_cast<const void*>(a.vpool.descs)), 0, vn < (1 << 28) ? vn * 8 : (1 << 31) - 8, 0x00020000);
  uint32_t k0 = 0, k1 = 0, v0 = 0, v1 = 0;
  int ok = 0, kid = 0, vid = 0;
  auto load_ids = [&](int base) {  // lanes past the batch re-read its last entry
    const int nb = np - base < 64 ? np - base : 64;
    const int p = it.page_begin + base + (lane < nb ? lane : nb - 1);
    kid = a.k_table[trow + p];
    vid = a.v_table[trow + p];
    ok = lane < nb;
  };
  auto load_descs = [&]() {
    ok = ok && kid >= 0 && kid < kn && vid >= 0 && vid < vn;
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    const u32x2 kd = __builtin_amdgcn_raw_buffer_load_b64(kdr, ok ? int(uint32_t(kid) * 8u) : -16, 0, 0);
    const u32x2 vd = __builtin_amdgcn_raw_buffer_load_b64(vdr, ok ? int(uint32_t(vid) * 8u) : -16, 0, 0);
    k0 = kd.x; k1 = kd.y; v0 = vd.x; v1 = vd.y;
  };
  if (a.recs != nullptr && np <= a.rec_stride) {  // (rec_stride <= 64: one batch)
    ok = lane < np;
    k0 = ok ? rec.x : 0u;
    k1 = ok ? rec.y : 0u;
    v0 = ok ? rec.z : 0u;
    v1 = ok ? rec.w : 0u;
  } else {
    if (np > 0) load_ids(0);
    load_descs();  // unconditional: an empty item's lanes are not ok and read zeros
  }

  // ---- queries scaled by query_scale * log2(e): B fragments hi / residual ----
  // converted once, after the item's first chunk loads are issued, so the
  // conversion overlaps them
  const float qmul = a.q_scale * kLog2e;
  // B fragments of group g are zero in the columns of the other group
  // copies (g % GB != gsel); qsum[b]: sum of head qh's channels of group
  // GB b + gsel, the group this lane's column carries in block b
  Frag qhi[KG], qlo[KG];
  float qsum[KNB];
  bool q_ready = false;
  // (the per-chunk lambdas are always inlined: at head_dim 256 the compiler
  // otherwise calls some of them, passing the register sets through scratch)
  auto prep_queries = [&]() __attribute__((always_inline)) {
    if (q_ready) return;
    q_ready = true;
    // Pipelined instances: the raw queries pass through an empty asm here,
    // so their conversion stays where it is called.  Without it the
    // compiler hoists the conversion (loop-invariant) above the page walk,
    // and the layout then waits for the query loads before the first
    // chunk's loads can issue (C3: 32.65 -> 32.15 us per launch).  The
    // unpipelined instances measured 0.4-1 us slower with it.
    if constexpr (kPipe) {
#pragma unroll
      for (int i = 0; i < 2 * KG; ++i) asm volatile("" : "+v"(qraw[i]));
    }
    float qv[KG][8];
    if (q_f32) {
#pragma unroll
      for (int g = 0; g < KG; ++g)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          qv[g][i] = __uint_as_float(qraw[2 * g][i]);
          qv[g][4 + i] = __uint_as_float(qraw[2 * g + 1][i]);
        }
    } else if (a.queries_dtype == DC_BF16) {
#pragma unroll
      for (int g = 0; g < KG; ++g)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          qv[g][2 * i] = __uint_as_float(qraw[g][i] << 16);
          qv[g][2 * i + 1] = __uint_as_float(qraw[g][i] & 0xffff0000u);
        }
    } else {
#pragma unroll
      for (int g = 0; g < KG; ++g)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          qv[g][2 * i] = float(h2_of(qraw[g][i])[0]);
          qv[g][2 * i + 1] = float(h2_of(qraw[g][i])[1]);
        }
    }
#pragma unroll
    for (int g = 0; g < KG; ++g) {
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        // k-slot pair i: channels (2i, 2i + 1) of the lane's 8, or (i, i + 4)
        // where 4-bit M0 keys occur (the order their nibble unpack produces)
        const int c0 = kPairedQ ? i : 2 * i, c1 = kPairedQ ? i + 4 : 2 * i + 1;
        const float x0 = head_live ? qv[g][c0] * qmul : 0.f, x1 = head_live ? qv[g][c1] * qmul : 0.f;
        const bool mine = GB == 1 || g % GB == gsel;
        const uint32_t hi = pack_h2(x0, x1);
        const h2 hv = h2_of(hi);
        qhi[g].u[i] = mine ? hi : 0u;
        qlo[g].u[i] = mine ? pack_h2(x0 - float(hv[0]), x1 - float(hv[1])) : 0u;
        s += x0 + x1;
      }
      s += __shfl_xor(s, 16, 64);
      s += __shfl_xor(s, 32, 64);  // sum of group g of head qh
      if (g % GB == 0 || g % GB == gsel) qsum[g / GB] = s;  // ends as group GB b + gsel
    }
  };

  // mix column of this lane in tile h of value group g: d = VGS g + dcol + LPW4 h
  const int jj = r % LPW4, w4 = r / LPW4;
  const int dcol = 8 * w4 + jj;
  // byte-permute selectors of this lane's code in tile h: the byte of token
  // 2p into byte 0, of token 2p + 1 into byte 2 (4-bit: the byte of word w4
  // holding nibble jj + LPW4 h; 8-bit: byte (jj + LPW4 h) % 4 of word
  // 2 w4 + (jj + LPW4 h) / 4)
  uint32_t vsel[H];
  int vword[H];
#pragma unroll
  for (int h = 0; h < H; ++h) {
    const int e = jj + LPW4 * h;
    const uint32_t b = VBITS == 4 ? uint32_t(e >> 1) : uint32_t(e & 3);
    vsel[h] = 0x0c000c00u | b | ((4u + b) << 16);
    vword[h] = VBITS == 4 ? w4 : 2 * w4 + (e >> 2);
  }
  const uint32_t nib_mask = (jj & 1) ? 0x00f000f0u : 0x000f000fu;  // low or high nibble of the byte
  const h2 nib_mul = (jj & 1) ? h2{(_Float16)0.0625f, (_Float16)0.0625f} : h2{(_Float16)1.f, (_Float16)1.f};
  // LDS word of (token 8 kb + e, word w) of group g: g GSTRIDE + vrow + e W + w
  const int vrow = 8 * kb * W + kb * Cfg::PAD;

  f32x4 acc[NACC];
#pragma unroll
  for (int t = 0; t < NACC; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  float bsum[VNB];  // value bias sums of head qh, group GB b + gsel
#pragma unroll
  for (int b = 0; b < VNB; ++b) bsum[b] = 0.f;
  float m_ref = -INFINITY, l_part = 0.f;
  // the fp16 magic 0x6400 pair, held in a VGPR the compiler cannot see
  // through: (w & mask) | magic with a scalar mask is then one v_and_or_b32
  // (a VOP3 here takes no literal and at most one scalar operand)
  uint32_t fp16_magic = 0x64006400u;
  asm volatile("" : "+v"(fp16_magic));


  auto key_is_m3 = [&](const PageMeta& m) -> bool {
    if constexpr (KMODE == KEYS_M3) return true;
    if constexpr (KMODE == KEYS_M0) return false;
    return m.kfmt == DC_FMT_M3_F16;
  };
  // The per-chunk steps take a compile-time flag (GEN / M0P): M0P compiles
  // them for chunks known to hold M0 keys and values only, without the M3
  // paths and their wave-uniform branches (the M0 chunks of pools that also
  // hold M3 pages).
  using GEN = std::false_type;
  using M0P = std::true_type;

  // ---- loads of one chunk into registers ----
  // Buffer loads against a per-page resource (base = the blob, size = the
  // blob's bytes, so an access past the page reads zeros instead of another
  // page): a per-lane offset fixed for the whole item, a wave-uniform chunk
  // offset and a constant, with no per-chunk address arithmetic in VGPRs.
  // this lane's KW words (channels 8 kb .. 8 kb + 7) of the (token, group 0)
  // code block of A-row token 8 (r / 4) + 4 hh + r % 4 in tile hh
  uint32_t koff_m0[2];
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) koff_m0[hh] = (8 * (r >> 2) + 4 * hh + (r & 3)) * KBLK + KBITS * kb;
  // M0 code DMA: lane l of instruction i fetches 16-byte piece pc of the
  // code block of group GPI i + gl, chunk token t of slot s (gl = l / (32
  // NPC), s = (l % (32 NPC)) / NPC, pc = l % NPC): the lane's part of the
  // source offset is fixed for the item, the instruction's part (GPI i
  // groups) wave-uniform.  kcrd: this lane's score read, slot r of tile 0,
  // word kb KBITS / 4.
  constexpr int NPC = KBLK / 16, GPI = 2 / NPC, NKD = KG / GPI;
  uint32_t kcsrc = 0, kcrd = 0;
  if constexpr (kDmaM0) {
    const uint32_t l = uint32_t(lane), gl = l / (32 * NPC), sl = (l % (32 * NPC)) / NPC, pc = l % NPC;
    const uint32_t t = 8 * ((sl & 15) >> 2) + 4 * (sl >> 4) + (sl & 3);
    kcsrc = gl * uint32_t(CAP * KBLK) + t * KBLK + 16 * pc;
    kcrd = uint32_t(r * (KBLK / 4) + kb * (KBITS / 4));
  }
  // key DMA: rows of PPR pieces, RPI rows per instruction, NDMA instructions
  // per chunk; instruction i writes rows RPI i .. RPI i + RPI - 1, lane l slot
  // l % PPR of row RPI i + l / PPR, from source piece (l % PPR) ^ key_swz(row).
  // The row's bits split into RPI i and l / PPR, so the lane's offset is
  // kdma0 ^ 16 key_swz(RPI i): one register per distinct swizzle constant.
  constexpr int PPR = HD / 8, RPI = 64 / PPR, NDMA = 32 / RPI;
  static_assert(NDMA <= 16, "at most 16 DMA instructions per chunk");
  auto dma_off = [](uint32_t l, int i) -> uint32_t {
    const uint32_t base = (l / PPR) * PPR * 16 + 16u * ((l % PPR) ^ key_swz<PPR>(l / PPR));
    return base ^ (16u * key_swz<PPR>(uint32_t(RPI * i)));
  };
  // score read of tile hh, group g: row ta = 8 (r / 4) + 4 hh + r % 4, piece
  // 4 g + kb at slot (4 g + kb) ^ key_swz(ta); key_swz(ta) < 16, so group g
  // reads krd_off(hh, g % 4) + 64 (g / 4) words
  auto krd_off = [](uint32_t l, int hh, int j) -> uint32_t {
    const uint32_t rr = l & 15u, ta = 8 * (rr >> 2) + 4 * hh + (rr & 3);
    return ta * (HD / 2) + 4u * ((uint32_t(4 * j) + (l >> 4)) ^ key_swz<PPR>(ta));  // in words
  };
  // M3-only key pools read LDS keys every chunk: their offsets are computed
  // once (equal swizzle constants give equal values, which share a
  // register; literal bounds: hipcc's host pass drops the kernel stubs when
  // such an array's size is a dependent constant).  Other pools meet M3
  // chunks rarely and derive the offsets where they are used, from a lane
  // index the compiler cannot hoist, so none of them stays live across the
  // chunk loop.
  uint32_t kdma[16], krd[2][4];
  if constexpr (KMODE == KEYS_M3) {
#pragma unroll
    for (int i = 0; i < NDMA; ++i) kdma[i] = dma_off(uint32_t(lane), i);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int j = 0; j < (KG < 4 ? KG : 4); ++j) krd[hh][j] = krd_off(uint32_t(lane), hh, j);
  }
  auto fresh_lane = []() __attribute__((always_inline)) -> uint32_t {
    uint32_t l = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
    asm volatile("" : "+v"(l));
    return l;
  };
  uint32_t voff[Cfg::NVP];
#pragma unroll
  for (int k = 0; k < Cfg::NVP; ++k) {
    const int e = lane + 64 * k;
    const int g = e / (8 * W), piece = e - g * (8 * W);
    voff[k] = uint32_t(g * CAP * W * 4 + piece * 16);
  }
  const uint32_t vsoff = uint32_t(lane % Cfg::VSW) * 4, ksoff = uint32_t(lane % Cfg::KSW) * 4;
  constexpr int kNT = 2;  // cache policy: nontemporal (page bytes are read once per launch)
  // part 0: the whole chunk; 1: value pieces and all scales / biases;
  // 2: key codes or rows; 3: M0 key codes only; 4: M3 key rows only
  auto load_part = [&](const PageMeta& m, auto& R, auto kbi, auto part, auto m0) __attribute__((always_inline)) {
    constexpr int P = decltype(part)::value;
    constexpr bool kM0 = decltype(m0)::value;
    const int c0 = m.c0;
    auto dma_keys = [&](__amdgpu_buffer_rsrc_t rs) __attribute__((always_inline)) {
      const uint32_t l = KMODE == KEYS_M3 ? 0u : fresh_lane();
#pragma unroll
      for (int i = 0; i < NDMA; ++i) {
        // (the offset goes to the builtin as a plain variable: hipcc's host
        // pass drops the kernel stubs when this argument is an expression
        // with a call or an array element of a dependent size)
        const uint32_t off = KMODE == KEYS_M3 ? kdma[i] : dma_off(l, i);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)(kbuf(kbi) + 256 * i),
                                                 16, off, c0 * HD * 2 + 1024 * i, 0, kNT);
      }
    };
    auto word_keys = [&](__amdgpu_buffer_rsrc_t rs) __attribute__((always_inline)) {
      if constexpr ((P == 0 || P == 2 || P == 3) && kDmaM0) {
#pragma unroll
        for (int i = 0; i < NKD; ++i) {
          // (plain variables for the offsets, as in dma_keys)
          const int soff = c0 * KBLK + i * GPI * CAP * KBLK;
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)(kcode(kbi) + 256 * i),
                                                   16, kcsrc, soff, 0, kNT);
        }
      } else if constexpr (P == 0 || P == 2 || P == 3)
#pragma unroll
      for (int g = 0; g < KG; ++g)
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const int co = c0 * KBLK + g * CAP * KBLK;
          if constexpr (KBITS == 4) {
            R.kw[hh][g] = __builtin_amdgcn_raw_buffer_load_b32(rs, int(koff_m0[hh]), co, kNT);
          } else {
            typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
            const u32x2 x = __builtin_amdgcn_raw_buffer_load_b64(rs, int(koff_m0[hh]), co, kNT);
            R.kw[hh][2 * g] = x.x;
            R.kw[hh][2 * g + 1] = x.y;
          }
        }
      // the scale / bias offsets are wave-uniform; readfirstlane says so, or
      // the compiler wraps each of these loads in a per-value loop
      const int ksc = __builtin_amdgcn_readfirstlane(int(m.ksc)), kbs = __builtin_amdgcn_readfirstlane(int(m.kbs));
      if constexpr (P == 0 || P == 1)
#pragma unroll
      for (int k = 0; k < Cfg::NKS; ++k) {
        R.ks[k] = __builtin_amdgcn_raw_buffer_load_b32(rs, int(ksoff), ksc + c0 * KG * 2 + 256 * k, kNT);
        if constexpr (KAFF)
          R.kbw[k] = __builtin_amdgcn_raw_buffer_load_b32(rs, int(ksoff), kbs + c0 * KG * 2 + 256 * k, kNT);
      }
    };
    if constexpr (KMODE == KEYS_M3) {
      if constexpr (P == 0 || P == 2 || P == 4) dma_keys(m.krs);
    } else if constexpr (KMODE == KEYS_M0) {
      if constexpr (P != 4) word_keys(m.krs);
    } else if (!kM0 && key_is_m3(m)) {  // one chunk in flight: a wave-uniform branch
      if constexpr (P == 0 || P == 2 || P == 4) dma_keys(m.krs);
    } else {
      if constexpr (P != 4) word_keys(m.krs);
    }
    if constexpr (P >= 2) return;
#pragma unroll
    for (int k = 0; k < Cfg::NVP; ++k)
      R.vr[k] = __builtin_amdgcn_raw_buffer_load_b128(m.vrs, int(voff[k]), c0 * W * 4, kNT);
    const int vsc = __builtin_amdgcn_readfirstlane(int(m.vsc)), vbs = __builtin_amdgcn_readfirstlane(int(m.vbs));
#pragma unroll
    for (int k = 0; k < Cfg::NVS; ++k) {
      R.vs[k] = __builtin_amdgcn_raw_buffer_load_b32(m.vrs, int(vsoff), vsc + c0 * VG * 2 + 256 * k, kNT);
      if constexpr (VAFF)
        R.vb[k] = __builtin_amdgcn_raw_buffer_load_b32(m.vrs, int(vsoff), vbs + c0 * VG * 2 + 256 * k, kNT);
    }
  };
  constexpr bool kSplitReload = !kPipe && waves_per_simd<HD, KMODE, KBITS, VBITS, NQB>() == 1;
  using LP0 = std::integral_constant<int, 0>;
  using LP1 = std::integral_constant<int, 1>;
  using LP2 = std::integral_constant<int, 2>;
  using LP3 = std::integral_constant<int, 3>;
  using LP4 = std::integral_constant<int, 4>;
  auto load_chunk = [&](const PageMeta& m, auto& R, auto kbi, auto m0) __attribute__((always_inline)) {
    load_part(m, R, kbi, LP0{}, m0);
  };

  // ---- registers -> an LDS stage buffer: value codes in padded rows, scales as loaded ([32][G] fp16) ----
  auto stage_chunk = [&](const auto& R, uint32_t* lds) __attribute__((always_inline)) {
#pragma unroll
    for (int k = 0; k < Cfg::NVP; ++k) {
      const int e = lane + 64 * k;
      const int g = e / (8 * W), piece = e - g * (8 * W);
      const int t = piece / (W / 4), wc = piece - t * (W / 4);
      *reinterpret_cast<u32x4*>(lds + Cfg::VPAY + g * Cfg::GSTRIDE + t * W + (t >> 3) * Cfg::PAD + 4 * wc) = R.vr[k];
    }
    // word e of a [32][G] fp16 scale array holds (token e / (G / 2), groups
    // 2 j, 2 j + 1), j = e % (G / 2); with group blocks its halves go to the
    // transposed rows 2 j and 2 j + 1
    auto put = [&](uint32_t* dst, uint32_t w, int e, int G) __attribute__((always_inline)) {
      if constexpr (GB == 1) {
        dst[e] = w;
      } else {
        const int t = e / (G / 2), j = e - t * (G / 2);
        uint16_t* d16 = reinterpret_cast<uint16_t*>(dst);
        d16[(2 * j) * Cfg::SP + t] = uint16_t(w);
        d16[(2 * j + 1) * Cfg::SP + t] = uint16_t(w >> 16);
      }
    };
#pragma unroll
    for (int k = 0; k < Cfg::NVS; ++k) {
      const int e = lane + 64 * k;
      if (Cfg::VSW % 64 == 0 || e < Cfg::VSW) {
        put(lds + Cfg::VSC, R.vs[k], e, VG);
        if constexpr (VAFF) put(lds + Cfg::VBS, R.vb[k], e, VG);
      }
    }
    if constexpr (KMODE != KEYS_M3) {
#pragma unroll
      for (int k = 0; k < Cfg::NKS; ++k) {
        const int e = lane + 64 * k;
        if (Cfg::KSW % 64 == 0 || e < Cfg::KSW) {
          put(lds + Cfg::KSC, R.ks[k], e, KG);
          if constexpr (KAFF) put(lds + Cfg::KBS, R.kbw[k], e, KG);
        }
      }
    }
  };

  // ---- score of one chunk: logits of chunk tokens 8 kb + e for head r ----
  auto score_chunk = [&](const PageMeta& m, const auto& R, const uint32_t* lds, auto kbi, float* Ls,
                         auto m0) __attribute__((always_inline)) {
    constexpr bool kM0 = decltype(m0)::value;
    const uint32_t* kl = kbuf(kbi);
    // MFMA results are read a few instructions after issue only at the very
    // end: the M3 paths keep four independent accumulation chains (token
    // tile hh x high / residual query part), the M0 path scales group g - 1
    // while the MFMAs of group g run
    if (!kM0 && key_is_m3(m)) {
      if constexpr (kDmaK) {
        const uint32_t l3 = KMODE == KEYS_M3 ? 0u : fresh_lane();
        f32x4 dh[2], dl[2];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) dh[hh] = dl[hh] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int g = 0; g < KG; ++g) {
          Frag ka[2];
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {
            // channels (0, 1), (2, 3), (4, 5), (6, 7) of the lane's 8
            u32x4 x;
            if constexpr (KMODE == KEYS_M3)
              x = *reinterpret_cast<const u32x4*>(kl + krd[hh][g % 4] + 64 * (g / 4));
            else
              x = *reinterpret_cast<const u32x4*>(kl + krd_off(l3, hh, g % 4) + 64 * (g / 4));
            if constexpr (kPairedQ) {  // -> (0, 4), (1, 5), (2, 6), (3, 7)
              ka[hh].u[0] = __builtin_amdgcn_perm(x.z, x.x, 0x05040100u);
              ka[hh].u[1] = __builtin_amdgcn_perm(x.z, x.x, 0x07060302u);
              ka[hh].u[2] = __builtin_amdgcn_perm(x.w, x.y, 0x05040100u);
              ka[hh].u[3] = __builtin_amdgcn_perm(x.w, x.y, 0x07060302u);
            } else {
              ka[hh].u[0] = x.x; ka[hh].u[1] = x.y; ka[hh].u[2] = x.z; ka[hh].u[3] = x.w;
            }
          }
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) dh[hh] = mfma(ka[hh], qhi[g], dh[hh]);
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) dl[hh] = mfma(ka[hh], qlo[g], dl[hh]);
        }
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
          for (int i = 0; i < 4; ++i) Ls[4 * hh + i] = dh[hh][i] + dl[hh][i];
      }
    } else if constexpr (KMODE != KEYS_M3) {  // M0 4- or 8-bit, group 32: scale and bias per group in fp32
      // affine: codes n, bias b; symmetric: codes n - (2^(KBITS-1) - 1), no
      // bias (bf = 0 zeroes the bias words, which then alias the scales)
      const bool k_affine = KAFF && m.kfmt == DC_FMT_M0_AFFINE;
      const float zp = k_affine ? 0.f : float((1 << (KBITS - 1)) - 1);
      const float bf = k_affine ? 1.f : 0.f;
      float qb[KNB];  // bias weight of the column's group in block b: its query sum (affine pages only)
#pragma unroll
      for (int b = 0; b < KNB; ++b) qb[b] = bf * qsum[b];
      // (1024 + n, 1024 + n') -> (n - zp, n' - zp); (1024 + 16 n, ..) / 16 - 64 - zp likewise
      const h2 kadd0 = {(_Float16)(-1024.f - zp), (_Float16)(-1024.f - zp)};
      const h2 kadd1 = {(_Float16)(-64.f - zp), (_Float16)(-64.f - zp)};
      const h2 k16 = {(_Float16)0.0625f, (_Float16)0.0625f};
      // scales / biases of the D-row tokens 8 kb + 4 hh + i: with one group
      // per block all groups, [4][KG] fp16 per tile, read up front; with
      // group blocks the column's group GB b + gsel, read per block
      uint32_t sw[2][GB == 1 ? 2 * KG : 1], bw[2][GB == 1 ? 2 * KG : 1];
      if constexpr (GB == 1) {
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
          for (int k = 0; k < 2 * KG; k += 4) {
            const u32x4 s4 = *reinterpret_cast<const u32x4*>(lds + Cfg::KSC + (8 * kb + 4 * hh) * KG / 2 + k);
            sw[hh][k] = s4.x; sw[hh][k + 1] = s4.y; sw[hh][k + 2] = s4.z; sw[hh][k + 3] = s4.w;
            if constexpr (KAFF) {
              const u32x4 b4 = *reinterpret_cast<const u32x4*>(lds + Cfg::KBS + (8 * kb + 4 * hh) * KG / 2 + k);
              bw[hh][k] = b4.x; bw[hh][k + 1] = b4.y; bw[hh][k + 2] = b4.z; bw[hh][k + 3] = b4.w;
            }
          }
      }
      // group blocks: tokens 8 kb .. 8 kb + 7 of the column's group in block
      // b, one 16-byte read of the transposed rows each
      uint32_t sq[GB == 1 ? 1 : KNB][4], bq[GB == 1 ? 1 : KNB][4];
      if constexpr (GB > 1) {
#pragma unroll
        for (int b = 0; b < KNB; ++b) {
          const int o = ((GB * b + gsel) * Cfg::SP + 8 * kb) / 2;
          const u32x4 s4 = *reinterpret_cast<const u32x4*>(lds + Cfg::KSC + o);
          sq[b][0] = s4.x; sq[b][1] = s4.y; sq[b][2] = s4.z; sq[b][3] = s4.w;
          if constexpr (KAFF) {
            const u32x4 b4 = *reinterpret_cast<const u32x4*>(lds + Cfg::KBS + o);
            bq[b][0] = b4.x; bq[b][1] = b4.y; bq[b][2] = b4.z; bq[b][3] = b4.w;
          }
        }
      }
      float Lh[2][4];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int i = 0; i < 4; ++i) Lh[hh][i] = 0.f;
      // D row 4 kb + i of tile hh is chunk token 8 kb + 4 hh + i; fp16 scale /
      // bias times an fp32 value: one v_fma_mix_f32 each
      auto post = [&](const f32x4* d, int b) __attribute__((always_inline)) {
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            float sc, bs;
            if constexpr (GB == 1) {
              const int e = i * KG + b;  // (token, g) entry: half e % 2 of word e / 2
              sc = float(h2_of(sw[hh][e >> 1])[e & 1]);
              bs = KAFF ? float(h2_of(bw[hh][e >> 1])[e & 1]) : 0.f;
            } else {
              const int t = 4 * hh + i;  // token 8 kb + t: half t % 2 of word t / 2
              sc = float(h2_of(sq[b][t >> 1])[t & 1]);
              bs = KAFF ? float(h2_of(bq[b][t >> 1])[t & 1]) : 0.f;
            }
            Lh[hh][i] = __builtin_fmaf(sc, d[hh][i], Lh[hh][i]);
            if constexpr (KAFF) Lh[hh][i] = __builtin_fmaf(bs, qb[b], Lh[hh][i]);
          }
      };
      // block b: the MFMAs of its GB groups accumulate into one tile pair
      // (the other copies' query columns are zero), then block b - 1 is
      // scaled while they run
      f32x4 dprev[2];
#pragma unroll
      for (int b = 0; b < KNB; ++b) {
        f32x4 d[2];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) d[hh] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int gi = 0; gi < GB; ++gi) {
          const int g = GB * b + gi;
          Frag ka[2];
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {
            if constexpr (KBITS == 4) {
              uint32_t w;
              if constexpr (kDmaM0)
                w = kcode(kbi)[kcrd + g * 8 * KBLK + hh * 4 * KBLK];
              else
                w = R.kw[hh][g];
              // nibble i of the word is channel i; channels i and i + 4 sit 16
              // bits apart, so one mask and the fp16 magic 0x6400 give the pair
              // (1024 + n_i, 1024 + n_{i+4}) (nibbles 0, 2) or 16 x that offset
              // (nibbles 1, 3), and one packed add / fma makes it n - zp exactly
              const uint32_t w8 = w >> 8;
              ka[hh].u[0] = bits_of(h2_of((w & 0x000f000fu) | fp16_magic) + kadd0);
              ka[hh].u[1] = bits_of(h2_of((w & 0x00f000f0u) | fp16_magic) * k16 + kadd1);
              ka[hh].u[2] = bits_of(h2_of((w8 & 0x000f000fu) | fp16_magic) + kadd0);
              ka[hh].u[3] = bits_of(h2_of((w8 & 0x00f000f0u) | fp16_magic) * k16 + kadd1);
            } else {
              // byte i of the two words is channel i: one byte permute puts
              // bytes (2j, 2j + 1) under the magic's 0x64 bytes, giving the
              // pair (1024 + n_2j, 1024 + n_2j+1), and one packed add makes
              // it n - zp exactly (|n - zp| <= 255 is exact in fp16)
              uint32_t wa, wb;
              if constexpr (kDmaM0) {
                const uint32_t* kc = kcode(kbi) + kcrd + g * 8 * KBLK + hh * 4 * KBLK;
                wa = kc[0];
                wb = kc[1];
              } else {
                wa = R.kw[hh][2 * g];
                wb = R.kw[hh][2 * g + 1];
              }
              ka[hh].u[0] = bits_of(h2_of(__builtin_amdgcn_perm(fp16_magic, wa, 0x05010500u)) + kadd0);
              ka[hh].u[1] = bits_of(h2_of(__builtin_amdgcn_perm(fp16_magic, wa, 0x05030502u)) + kadd0);
              ka[hh].u[2] = bits_of(h2_of(__builtin_amdgcn_perm(fp16_magic, wb, 0x05010500u)) + kadd0);
              ka[hh].u[3] = bits_of(h2_of(__builtin_amdgcn_perm(fp16_magic, wb, 0x05030502u)) + kadd0);
            }
          }
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) d[hh] = mfma(ka[hh], qhi[g], d[hh]);
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) d[hh] = mfma(ka[hh], qlo[g], d[hh]);
        }
        if (b > 0) post(dprev, b - 1);
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) dprev[hh] = d[hh];
      }
      post(dprev, KNB - 1);
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int i = 0; i < 4; ++i) Ls[4 * hh + i] = Lh[hh][i];
    }
    // group blocks: the column of copy c holds the part of the logit from
    // the groups c carries; two (GB = 4) or one (GB = 2) rotate-adds within
    // each row of 16 lanes give every copy the whole logit
    if constexpr (GB > 1) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        Ls[e] += row_ror<NQB>(Ls[e]);
        if constexpr (GB == 4) Ls[e] += row_ror<2 * NQB>(Ls[e]);
      }
    }
  };

  // ---- online softmax of one scored chunk: weights pa of head r on tokens 8 kb + e ----
  auto softmax_chunk = [&](const PageMeta& m, float* Ls, float* pa) __attribute__((always_inline)) {
    if (m.c0 + 32 > m.T) {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (m.c0 + 8 * kb + e >= m.T) Ls[e] = -INFINITY;
    }
    float mx = Ls[0];
#pragma unroll
    for (int e = 1; e < 8; ++e) mx = fmaxf(mx, Ls[e]);
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));  // chunk max of head r
    const bool move = mx > m_ref + kLazy;
    if (__any(move)) {
      const float m_new = move ? mx : m_ref;
      const float alpha = m_ref == -INFINITY ? 0.f : exp2f(m_ref - m_new);
      m_ref = m_new;
      l_part *= alpha;
#pragma unroll
      for (int b = 0; b < VNB; ++b) bsum[b] *= alpha;
      // D row 4 kb + i of the accumulators is head (4 kb + i) % NQB, as is
      // lane 4 kb + i: its alpha lives there
      float arow[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) arow[i] = __shfl(alpha, 4 * kb + i, 64);
#pragma unroll
      for (int t = 0; t < NACC; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[t][i] *= arow[i];
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float w = __builtin_amdgcn_exp2f(Ls[e] - m_ref);
      pa[e] = head_live ? w : 0.f;
      l_part += pa[e];
    }
  };

  // ---- mix of one staged chunk with its weights ----
  // The A operand is weight x scale (x 1 for M3 values) times kVS, split
  // into fp16 high and residual parts.  An 8-bit scale is 17 times finer
  // than a 4-bit one over the same value range, which puts weight x scale
  // 2^4 lower in fp16's range, where small products lose bits to
  // subnormals; kVS = 16 puts it back where 4-bit codes have it (with the
  // same overflow margin: weight x scale x 16 reaches fp16's maximum only
  // for 8-bit scales above 1023).  The epilogue divides by kVS.
  constexpr float kVS = VBITS == 8 ? 16.f : 1.f;
  auto mix_chunk = [&](const PageMeta& m, const uint32_t* lds, const float* pa, auto m0) __attribute__((always_inline)) {
    constexpr bool kM0 = decltype(m0)::value;
    bool v_m0 = true;
    if constexpr (VM3 && !kM0) v_m0 = is_m0(m.vfmt);
    if (v_m0) {
      const bool v_affine = VAFF && m.vfmt == DC_FMT_M0_AFFINE;
      const float zp = v_affine ? 0.f : float((1 << (VBITS - 1)) - 1);
      const float bf = v_affine ? 1.f : 0.f;
      float pb[8], pw[8];  // weights of the bias sums (0 on symmetric pages), of the codes
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        pb[e] = bf * pa[e];
        pw[e] = kVS * pa[e];
      }
      // codes become fp16 (1024 + c), or (1024 + 16 c) for a code in the high
      // nibble of its byte; one packed fma maps either to c - zp exactly
      const h2 vadd = VBITS == 4 && (jj & 1) ? h2{(_Float16)(-64.f - zp), (_Float16)(-64.f - zp)}
                                              : h2{(_Float16)(-1024.f - zp), (_Float16)(-1024.f - zp)};
      // scales (and biases) of tokens 8 kb + e: with one group per block all
      // groups, [8][VG] fp16 = 4 VG words read up front; with group blocks
      // the row's group GB b + gsel, read per block
      uint32_t sw[GB == 1 ? 4 * VG : 1], bw[GB == 1 ? 4 * VG : 1];
      if constexpr (GB == 1) {
#pragma unroll
        for (int k = 0; k < 4 * VG; k += 4) {
          const u32x4 s4 = *reinterpret_cast<const u32x4*>(lds + Cfg::VSC + 4 * VG * kb + k);
          sw[k] = s4.x; sw[k + 1] = s4.y; sw[k + 2] = s4.z; sw[k + 3] = s4.w;
          if constexpr (VAFF) {
            const u32x4 b4 = *reinterpret_cast<const u32x4*>(lds + Cfg::VBS + 4 * VG * kb + k);
            bw[k] = b4.x; bw[k + 1] = b4.y; bw[k + 2] = b4.z; bw[k + 3] = b4.w;
          }
        }
      }
      uint32_t sq[GB == 1 ? 1 : VNB][4], bq[GB == 1 ? 1 : VNB][4];
      if constexpr (GB > 1) {
#pragma unroll
        for (int b = 0; b < VNB; ++b) {
          const int o = ((GB * b + gsel) * Cfg::SP + 8 * kb) / 2;
          const u32x4 s4 = *reinterpret_cast<const u32x4*>(lds + Cfg::VSC + o);
          sq[b][0] = s4.x; sq[b][1] = s4.y; sq[b][2] = s4.z; sq[b][3] = s4.w;
          if constexpr (VAFF) {
            const u32x4 b4 = *reinterpret_cast<const u32x4*>(lds + Cfg::VBS + o);
            bq[b][0] = b4.x; bq[b][1] = b4.y; bq[b][2] = b4.z; bq[b][3] = b4.w;
          }
        }
      }
      auto vscale = [&](int e, int b) __attribute__((always_inline)) -> float {  // token 8 kb + e
        if constexpr (GB == 1) {
          const int x = e * VG + b;
          return float(h2_of(sw[x >> 1])[x & 1]);
        } else {
          return float(h2_of(sq[b][e >> 1])[e & 1]);
        }
      };
      auto vbias = [&](int e, int b) __attribute__((always_inline)) -> float {
        if constexpr (GB == 1) {
          const int x = e * VG + b;
          return float(h2_of(bw[x >> 1])[x & 1]);
        } else {
          return float(h2_of(bq[b][e >> 1])[e & 1]);
        }
      };
      // block b: one weight x scale operand serves its GB groups (row copy c
      // carries group GB b + c; the other copies' rows of a group's tiles
      // are never stored)
#pragma unroll
      for (int b = 0; b < VNB; ++b) {
        Frag fa_hi, fa_res;
#pragma unroll
        for (int pp = 0; pp < 4; ++pp) {
          // weight x fp16 scale straight to fp16 high and residual parts
          const Split2 sp = split_products(pw[2 * pp], vscale(2 * pp, b), pw[2 * pp + 1], vscale(2 * pp + 1, b));
          fa_hi.u[pp] = sp.hi;
          fa_res.u[pp] = sp.res;
          if constexpr (VAFF) {  // fp16 bias times weight: one v_fma_mix_f32 each
            bsum[b] = __builtin_fmaf(vbias(2 * pp, b), pb[2 * pp], bsum[b]);
            bsum[b] = __builtin_fmaf(vbias(2 * pp + 1, b), pb[2 * pp + 1], bsum[b]);
          }
        }
#pragma unroll
        for (int gi = 0; gi < GB; ++gi) {
          const int g = GB * b + gi;
          const uint32_t* P = lds + Cfg::VPAY + g * Cfg::GSTRIDE + vrow;  // token 8 kb + e at P[e W]
#pragma unroll
          for (int h = 0; h < H; ++h) {
            Frag fb;
#pragma unroll
            for (int pp = 0; pp < 4; ++pp) {
              const uint32_t x =
                  __builtin_amdgcn_perm(P[(2 * pp + 1) * W + vword[h]], P[(2 * pp) * W + vword[h]], vsel[h]);
              if constexpr (VBITS == 4)
                fb.u[pp] = bits_of(h2_of((x & nib_mask) | 0x64006400u) * nib_mul + vadd);
              else
                fb.u[pp] = bits_of(h2_of(x | 0x64006400u) + vadd);
            }
            acc[g * H + h] = mfma(fa_hi, fb, acc[g * H + h]);
            acc[g * H + h] = mfma(fa_res, fb, acc[g * H + h]);
          }
        }
      }
    } else if constexpr (VM3) {  // M3 fp16 values (the exact recent window): rows staged in vbuf
      Frag fa_hi, fa_res;
#pragma unroll
      for (int pp = 0; pp < 4; ++pp) {
        const Split2 sp = split_products(pa[2 * pp], kVS, pa[2 * pp + 1], kVS);
        fa_hi.u[pp] = sp.hi;
        fa_res.u[pp] = sp.res;
      }
      // B fragment of tile h of group g: column d = VGS g + dcol + LPW4 h of
      // chunk tokens 8 kb + e; row t keeps piece d / 8 at slot (d / 8) ^
      // key_swz(t).  A token at or past the page's count reads 0 (its
      // weight is 0, and the row's bytes need not be finite).
      const uint16_t* V = reinterpret_cast<const uint16_t*>(vbuf);
      const uint32_t l = fresh_lane(), kbv = l >> 4, rv = l & 15u;
      const uint32_t dcolv = 8 * (rv / LPW4) + rv % LPW4;
      const int tvalid = m.T - m.c0 - 8 * int(kbv);  // tokens 8 kb + e with e < tvalid are valid
#pragma unroll
      for (int g = 0; g < VG; ++g)
#pragma unroll
        for (int h = 0; h < H; ++h) {
          const uint32_t d = uint32_t(VGS * g + LPW4 * h) + dcolv;
          Frag fb;
#pragma unroll
          for (int pp = 0; pp < 4; ++pp) {
            const uint32_t t0 = 8 * kbv + uint32_t(2 * pp), t1 = t0 + 1;
            uint32_t lo = V[t0 * HD + 8 * ((d >> 3) ^ key_swz<PPR>(t0)) + (d & 7)];
            uint32_t hi = V[t1 * HD + 8 * ((d >> 3) ^ key_swz<PPR>(t1)) + (d & 7)];
            if (2 * pp >= tvalid) lo = 0;
            if (2 * pp + 1 >= tvalid) hi = 0;
            fb.u[pp] = lo | (hi << 16);
          }
          acc[g * H + h] = mfma(fa_hi, fb, acc[g * H + h]);
          acc[g * H + h] = mfma(fa_res, fb, acc[g * H + h]);
        }
    }
  };
  // the M3 value rows of a chunk into vbuf, against a resource that ends at
  // the page's last valid row
  auto load_value_rows = [&](const PageMeta& m) __attribute__((always_inline)) {
    const __amdgpu_buffer_rsrc_t rows =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(m.vp), 0, m.T * HD * 2, 0x00020000);
    const uint32_t l = fresh_lane();
#pragma unroll
    for (int i = 0; i < NDMA; ++i) {
      const uint32_t off = dma_off(l, i);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rows, (__attribute__((address_space(3))) void*)(vbuf + 256 * i), 16,
                                               off, m.c0 * HD * 2 + 1024 * i, 0, kNT);
    }
  };

  // head_dim 256 converts up front: holding its raw queries across the first
  // loads costs registers (converted after them, the C5 instance took 439
  // registers instead of 311 and ran 164.5 -> 170.1 us per launch)
  if constexpr (HD > 128) prep_queries();

  // Lane i: everything about page base + i of a batch whose descriptors
  // are in (k0, k1, v0, v1), vector work instead of per-page scalar work:
  // token count, formats, blob sizes, scale / bias offsets.  Blob layout
  // (dc_common.h blob_layout) of the formats this kernel accepts, from its
  // fixed geometry: keys M3 fp16 or M0 KBITS-bit group 32, values M3 fp16
  // or M0 VBITS-bit group VGS, capacity CAP.  (The early first chunk below
  // uses these helpers; the batch walk computes the same fields inline,
  // which the unpipelined instances compile to faster code.)
  struct PageFields {
    uint32_t ktot, vtot, info, koffs, voffs;
    int T;
  };
  auto page_fields = [&](int nb) __attribute__((always_inline)) -> PageFields {
    const int kf = int(k1 >> 16) & 0xff, vf = int(v1 >> 16) & 0xff;
    const uint32_t cap = uint32_t(CAP), m3_bytes = cap * HD * 2;
    const uint32_t kpay = uint32_t(KG) * cap * KBLK, ksb = (cap * KG * 2 + 15) & ~15u;
    const uint32_t vpay = uint32_t(VG) * cap * W * 4, vsb = (cap * VG * 2 + 15) & ~15u;
    const bool km0 = is_m0(kf), vm0 = is_m0(vf), kaff = kf == DC_FMT_M0_AFFINE, vaff = vf == DC_FMT_M0_AFFINE;
    const uint32_t ksc = km0 ? kpay : 0u, kbs = kaff ? kpay + ksb : ksc;
    const uint32_t vsc = vm0 ? vpay : 0u, vbs = vaff ? vpay + vsb : vsc;
    PageFields f;
    f.ktot = km0 ? kpay + ksb + (kaff ? ksb : 0u) : m3_bytes;
    f.vtot = vm0 ? vpay + vsb + (vaff ? vsb : 0u) : m3_bytes;
    int T = min(int(k1 & 0xffff), int(v1 & 0xffff));
    T = min(T, CAP);
    // (bitwise, not short-circuit: no branch)
    const bool bad = !ok | (lane >= nb) | ((uint64_t(k0) << 8) + f.ktot > uint64_t(a.kpool.arena_bytes)) |
                     ((uint64_t(v0) << 8) + f.vtot > uint64_t(a.vpool.arena_bytes));
    f.T = bad ? 0 : T;
    f.info = uint32_t(f.T) | (uint32_t(kf) << 16) | (uint32_t(vf) << 24);
    // offsets in 16-byte units (blob offsets are 16-byte aligned): an M0
    // page at head_dim 256 and capacity 256 puts its 8-bit codes' scales at
    // 64 KiB, past a 16-bit byte offset
    f.koffs = (ksc >> 4) | ((kbs >> 4) << 16);
    f.voffs = (vsc >> 4) | ((vbs >> 4) << 16);
    return f;
  };
  // the chunk of lane i's page that starts at token c0
  auto lane_meta = [&](const PageFields& f, int i, int c0) __attribute__((always_inline)) -> PageMeta {
    PageMeta m;
    // blob pointers stay derived from the arena arguments (global memory)
    const uint8_t* kp =
        reinterpret_cast<const uint8_t*>(a.kpool.arena) + (uint64_t(__builtin_amdgcn_readlane(k0, i)) << 8);
    m.vp = reinterpret_cast<const uint8_t*>(a.vpool.arena) + (uint64_t(__builtin_amdgcn_readlane(v0, i)) << 8);
    m.krs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(kp), 0, int(__builtin_amdgcn_readlane(f.ktot, i)),
                                              0x00020000);
    m.vrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(m.vp), 0,
                                              int(__builtin_amdgcn_readlane(f.vtot, i)), 0x00020000);
    const uint32_t inf = __builtin_amdgcn_readlane(f.info, i);
    m.T = int(inf & 0xffff);
    m.kfmt = int(inf >> 16) & 0xff;
    m.vfmt = int(inf >> 24);
    const uint32_t ko = __builtin_amdgcn_readlane(f.koffs, i), vo = __builtin_amdgcn_readlane(f.voffs, i);
    m.ksc = (ko & 0xffff) << 4;
    m.kbs = (ko >> 16) << 4;
    m.vsc = (vo & 0xffff) << 4;
    m.vbs = (vo >> 16) << 4;
    m.c0 = c0;
    return m;
  };
  using R_t = ChunkRegs<HD, VGS, VBITS, KMODE, KBITS, !kDmaM0>;
  R_t RA, RB;  // the pipeline's register sets
  // Pipelined instances with DMA keys issue the item's first chunk straight
  // from page 0's descriptors, before the batch layout (its prefix sum, the
  // chunk count and the loop set-up), when page 0 holds that chunk.  The
  // layout then runs while the loads fly (C3: 32.36 -> 31.87 us per
  // launch; C2, M0 keys at head_dim 64 and two chunks per item, measured
  // 0.08 us slower with it).
  bool early = false;
  if constexpr (kPipe && kDmaK) {
    if (np > 0) {
      // (the item's chunks: from chunk cb of its first page to, with ce > 0,
      // chunk ce - 1 of its last page)
      const int cpp = CAP >> 5;
      const int cb = min(it.chunk_begin, cpp - 1), ce = min(it.chunk_end, cpp);
      const PageFields f = page_fields(np < 64 ? np : 64);
      const int nch0 = (__builtin_amdgcn_readlane(f.T, 0) + 31) >> 5;
      early = cb < (np == 1 && ce > 0 ? min(nch0, ce) : nch0);
      if (early) load_chunk(lane_meta(f, 0, cb * 32), RA, KB0{}, GEN{});
    }
  }

  // ---- walk the pages: metadata 64 pages at a time, chunks pipelined ----
  for (int base = 0; base < np; base += 64) {
    const int nb = np - base < 64 ? np - base : 64;
    if (base > 0) {
      load_ids(base);
      load_descs();
    }
    const int kf = int(k1 >> 16) & 0xff, vf = int(v1 >> 16) & 0xff;
    const uint32_t cap = uint32_t(CAP), m3_bytes = cap * HD * 2;
    const uint32_t kpay = uint32_t(KG) * cap * KBLK, ksb = (cap * KG * 2 + 15) & ~15u;
    const uint32_t vpay = uint32_t(VG) * cap * W * 4, vsb = (cap * VG * 2 + 15) & ~15u;
    const bool km0 = is_m0(kf), vm0 = is_m0(vf), kaff = kf == DC_FMT_M0_AFFINE, vaff = vf == DC_FMT_M0_AFFINE;
    const uint32_t ksc = km0 ? kpay : 0u, kbs = kaff ? kpay + ksb : ksc;
    const uint32_t vsc = vm0 ? vpay : 0u, vbs = vaff ? vpay + vsb : vsc;
    const uint32_t ktot = km0 ? kpay + ksb + (kaff ? ksb : 0u) : m3_bytes;
    const uint32_t vtot = vm0 ? vpay + vsb + (vaff ? vsb : 0u) : m3_bytes;
    int T = min(int(k1 & 0xffff), int(v1 & 0xffff));
    T = min(T, CAP);
    // (bitwise, not short-circuit: no branch)
    const bool bad = !ok | (lane >= nb) | ((uint64_t(k0) << 8) + ktot > uint64_t(a.kpool.arena_bytes)) |
                     ((uint64_t(v0) << 8) + vtot > uint64_t(a.vpool.arena_bytes));
    if (bad) T = 0;
    const uint32_t info = uint32_t(T) | (uint32_t(kf) << 16) | (uint32_t(vf) << 24);
    // (16-byte units, as in page_fields)
    const uint32_t koffs = (ksc >> 4) | ((kbs >> 4) << 16), voffs = (vsc >> 4) | ((vbs >> 4) << 16);
    const int nch = (T + 31) >> 5;  // <= 8 (capacity <= 256)
    // The item's chunks of page lane: [lo, hi).  It starts at chunk cb of
    // its first page (lane 0 of the first batch: `off` chunks skipped) and,
    // with ce > 0, ends after chunk ce - 1 of its last page.
    const int cpp = CAP >> 5, cps = __builtin_ctz(uint32_t(cpp));
    const int cb = min(it.chunk_begin, cpp - 1), ce = min(it.chunk_end, cpp);
    const int off = base == 0 ? cb : 0;
    const bool last_batch = base + nb == np;
    const int lo = lane == 0 ? off : 0;
    const int hi = last_batch && ce > 0 && lane == nb - 1 ? min(nch, ce) : nch;
    const int cnt = max(hi - lo, 0);
    // Every page of the batch full, with a power-of-two count of chunks per
    // page (2^cps): the batch's chunk j is chunk g = j + off of the pages
    // laid end to end, in page g >> cps.  Otherwise an inclusive prefix sum
    // of cnt over the lanes, bit by bit (ballot of the bit, count of set
    // lanes at or below this one): page lane holds chunks [cend - cnt, cend).
    const bool fast = __ballot(lane < nb && T != CAP) == 0 && (cpp & (cpp - 1)) == 0;
    int cend = 0;
    if (!fast) {
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int bit = (cnt >> b) & 1;
        const uint64_t bal = __ballot(bit);
        const int below = __builtin_amdgcn_mbcnt_hi(uint32_t(bal >> 32), __builtin_amdgcn_mbcnt_lo(uint32_t(bal), 0u));
        cend += (below + bit) << b;
      }
    }
    const int cbeg = cend - cnt;
    const int total = fast ? max((nb << cps) - off - (last_batch && ce > 0 ? cpp - ce : 0), 0)
                           : __builtin_amdgcn_readlane(cend, 63);
    if (total == 0) continue;
    // chunk j lies in the first page whose end chunk exceeds j
    // a chunk past the end: the same loads against empty buffer resources,
    // which return zeros without touching memory
    auto no_chunk = [&](PageMeta m) __attribute__((always_inline)) -> PageMeta {
      m.krs = __builtin_amdgcn_make_buffer_rsrc(nullptr, 0, 0, 0x00020000);
      m.vrs = m.krs;
      return m;
    };
    auto chunk_meta = [&](int j) __attribute__((always_inline)) -> PageMeta {
      const int i = fast ? (j + off) >> cps : __builtin_amdgcn_readfirstlane(int(__popcll(__ballot(cend <= j))));
      PageMeta m;
      // blob pointers stay derived from the arena arguments (global memory)
      const uint8_t* kp =
          reinterpret_cast<const uint8_t*>(a.kpool.arena) + (uint64_t(__builtin_amdgcn_readlane(k0, i)) << 8);
      m.vp = reinterpret_cast<const uint8_t*>(a.vpool.arena) + (uint64_t(__builtin_amdgcn_readlane(v0, i)) << 8);
      m.krs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(kp), 0, int(__builtin_amdgcn_readlane(ktot, i)),
                                                0x00020000);
      m.vrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(m.vp), 0,
                                                int(__builtin_amdgcn_readlane(vtot, i)), 0x00020000);
      const uint32_t inf = __builtin_amdgcn_readlane(info, i);
      m.T = int(inf & 0xffff);
      m.kfmt = int(inf >> 16) & 0xff;
      m.vfmt = int(inf >> 24);
      const uint32_t ko = __builtin_amdgcn_readlane(koffs, i), vo = __builtin_amdgcn_readlane(voffs, i);
      m.ksc = (ko & 0xffff) << 4;
      m.kbs = (ko >> 16) << 4;
      m.vsc = (vo & 0xffff) << 4;
      m.vbs = (vo >> 16) << 4;
      m.c0 = fast ? ((j + off) & (cpp - 1)) * 32 : (j - __builtin_amdgcn_readlane(cbeg, i) + (i == 0 ? off : 0)) * 32;
      return m;
    };

    if constexpr (kPipe) {
      // chunk j is mixed from stage buffer j % 2 while chunk j + 1 is staged
      // into the other buffer and scored, and the loads of chunk j + 2 fly
      // into the register set chunk j + 1 came in; past the last chunk the
      // loads go to an empty resource (no memory traffic)
      uint32_t* const buf0 = lds_all;
      uint32_t* const buf1 = lds_all + Cfg::STAGE;
      PageMeta cur = chunk_meta(0);
      PageMeta nxt = total > 1 ? chunk_meta(1) : no_chunk(cur);
      if (!(early && base == 0)) load_chunk(cur, RA, KB0{}, GEN{});  // (early: the same chunk, already issued)
      load_chunk(nxt, RB, KB1{}, GEN{});
      prep_queries();
      float Ls[8], pa[8];
      stage_chunk(RA, buf0);
      // A chunk's key rows (LDS filled by DMA) are read only after its
      // stage, whose waits for the chunk's register loads also cover the
      // key DMA issued before them (vector memory loads complete in order).
      // The compiler's own wait for the DMA went missing on a path into
      // this block once the first chunk could be issued before the loop,
      // and the reads it hoisted above the stage then saw stale rows.
      if constexpr (kDmaK) asm volatile("" ::: "memory");
      score_chunk(cur, RA, buf0, KB0{}, Ls, GEN{});
      softmax_chunk(cur, Ls, pa);
      int j = 0;
      // chunk j: values in stage buffer bm (keys in km, already scored);
      // chunk j + 1: registers X, keys in ks; chunk j + 2 loads into Y, km
      auto step = [&](R_t& X, R_t& Y, uint32_t* bm, uint32_t* bs, auto km, auto ks) __attribute__((always_inline)) -> bool {
        if (j + 1 >= total) {  // last chunk: mix only
          mix_chunk(cur, bm, pa, GEN{});
          return false;
        }
        const PageMeta n2 = j + 2 < total ? chunk_meta(j + 2) : no_chunk(nxt);
        load_chunk(n2, Y, km, GEN{});
        float Ln[8];
        stage_chunk(X, bs);
        if constexpr (kDmaK) asm volatile("" ::: "memory");  // (as for the first chunk)
        score_chunk(nxt, X, bs, ks, Ln, GEN{});
        mix_chunk(cur, bm, pa, GEN{});
        softmax_chunk(nxt, Ln, pa);
        cur = nxt;
        nxt = n2;
        ++j;
        return true;
      };
      while (step(RB, RA, buf0, buf1, KB0{}, KB1{}) && step(RA, RB, buf1, buf0, KB1{}, KB0{})) {
      }
    } else {  // one register set and stage buffer: reload as soon as the chunk has consumed them
      // (M3 value rows go to vbuf once the previous chunk's mix has read it)
      // LDS DMA of M3 rows.  Vector memory loads complete in issue order, so
      // a stage's wait for its chunk's register loads covers every DMA
      // issued before them: a chunk's M3 key and value rows are always
      // issued before its value pieces and scales (LP1), and the score and
      // the mix read the rows only after the stage.
      // Chunks [j0, j1) of the batch; m0 = M0P where every one of them holds
      // M0 keys and values.
      auto walk = [&](auto m0, int j0, int j1) __attribute__((always_inline)) {
        constexpr bool kM0 = decltype(m0)::value;
        if constexpr (kM0 && kM0Two) {
          // M0 chunks at one wave per SIMD: the codes double-buffered, so
          // chunk j + 1's go out right after chunk j is staged, into the
          // other slot, before its value pieces and scales, whose wait at
          // the next stage then covers the codes too (vector memory loads
          // complete in issue order).  Two steps per pass: each slot is a
          // fixed LDS object.
          R_t R;
          PageMeta cur = chunk_meta(j0);
          load_chunk(cur, R, KB0{}, m0);
          prep_queries();
          int j = j0;
          auto step = [&](auto ks, auto kn) __attribute__((always_inline)) -> bool {
            const PageMeta nm = j + 1 < j1 ? chunk_meta(j + 1) : no_chunk(cur);
            float Ls[8], pa[8];
            stage_chunk(R, lds_all);
            asm volatile("" ::: "memory");  // (the codes of slot ks are read only after the stage)
            load_part(nm, R, kn, LP3{}, m0);
            load_part(nm, R, kn, LP1{}, m0);
            score_chunk(cur, R, lds_all, ks, Ls, m0);
            softmax_chunk(cur, Ls, pa);
            mix_chunk(cur, lds_all, pa, m0);
            cur = nm;
            return ++j < j1;
          };
          while (step(KB0{}, KB1{}) && step(KB1{}, KB0{})) {
          }
          return;
        }
        R_t R, RN;
        PageMeta cur = chunk_meta(j0);
        // The compiler does not order an LDS DMA (buffer_load ... lds) after
        // earlier reads of the same buffer: it moved a next chunk's key DMA
        // in between the score's reads of the codes it overwrote.  Asm
        // statements with a memory clobber keep every DMA below the reads of
        // its buffer, and wait for those reads (lgkmcnt) before it: here
        // (after the other walk's last reads), after the score (key buffer)
        // and after the mix (value row buffer).
        asm volatile("" ::: "memory");
        if constexpr (VM3 && !kM0)
          if (!is_m0(cur.vfmt)) load_value_rows(cur);
        load_chunk(cur, R, KB0{}, m0);  // (M3 key rows first, then the register loads)
        prep_queries();
        for (int j = j0; j < j1; ++j) {
          const PageMeta nm = j + 1 < j1 ? chunk_meta(j + 1) : no_chunk(cur);
          float Ls[8], pa[8];
          stage_chunk(R, lds_all);
          // At one wave per SIMD the value pieces, scales and M0 key codes of
          // chunk j + 1 go out as soon as this chunk is staged (the codes into
          // a second set, copied over after the mix), and M3 key rows once
          // this chunk is scored, its key buffer then being free (C5: 164.4 ->
          // 162.6 us per launch for the values and scales, -> 161.6 us with
          // the codes); with two waves per SIMD the other wave covers the
          // wait, and the early values measured slower (C4: 40.7 -> 41.4 us).
          // (a next chunk with M3 key or value rows, rare and wave-uniform,
          // takes its register loads after those rows' DMA, at the end of the
          // step; LP0 issues the key rows before the register loads)
          const bool nm_vrows = VM3 && !kM0 && j + 1 < j1 && !is_m0(nm.vfmt);
          // (with M0 codes by DMA every chunk's keys come as rows: after the
          // score, which frees slot 0, and before the register loads)
          const bool nm_rows = kDmaM0 || (!kM0 && key_is_m3(nm)) || nm_vrows;
          if constexpr (kSplitReload) {
            if (!nm_rows) load_part(nm, R, KB0{}, LP1{}, m0);
            if constexpr (KMODE != KEYS_M3 && !kDmaM0)
              load_part(nm, RN, KB0{}, LP3{}, m0);  // (an M3 key page loads none)
          }
          score_chunk(cur, R, lds_all, KB0{}, Ls, m0);
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
          if constexpr (kSplitReload && kDmaM0)
            load_part(nm, R, KB0{}, LP2{}, m0);
          else if constexpr (kSplitReload)
            load_part(nm, R, KB0{}, LP4{}, m0);
          else if (!nm_vrows)
            load_part(nm, R, KB0{}, LP0{}, m0);
          softmax_chunk(cur, Ls, pa);
          mix_chunk(cur, lds_all, pa, m0);
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
          if constexpr (VM3 && !kM0)
            if (nm_vrows) load_value_rows(nm);
          if constexpr (kSplitReload) {
            if (nm_rows) load_part(nm, R, KB0{}, LP1{}, m0);
          } else if (nm_vrows) {
            load_part(nm, R, KB0{}, LP0{}, m0);
          }
          if constexpr (kSplitReload && KMODE != KEYS_M3 && !kDmaM0)
#pragma unroll
            for (int hh = 0; hh < 2; ++hh)
#pragma unroll
              for (int i = 0; i < Cfg::KG * (KBITS / 4); ++i) R.kw[hh][i] = RN.kw[hh][i];
          cur = nm;
        }
      };
      if constexpr ((KMODE == KEYS_MIXED || VM3) && waves_per_simd<HD, KMODE, KBITS, VBITS, NQB>() == 1) {
        // Pools that may hold M3 pages (one wave per SIMD): the batch's
        // chunks before its first page with M3 keys or values take the
        // M0-only walk.  Its per-chunk code has none of the M3 branches: on
        // C5 about 150 fewer scalar and 90 fewer vector instructions per
        // chunk, and 161.6 -> 154.0 us per launch.  (Built for two waves per
        // SIMD, the instances with two walks spill.)
        const bool m3p = lane < nb && cnt > 0 && (kf == DC_FMT_M3_F16 || !is_m0(vf));
        const uint64_t m3b = __ballot(m3p);
        int jm3 = total;
        if (m3b != 0) {
          const int i0 = int(__builtin_ctzll(m3b));
          jm3 = fast ? max((i0 << cps) - off, 0) : __builtin_amdgcn_readlane(cbeg, i0);
        }
        if (jm3 > 0) walk(M0P{}, 0, jm3);
        if (jm3 < total) walk(GEN{}, jm3, total);
      } else if constexpr (KMODE == KEYS_M0 && !VM3) {
        walk(M0P{}, 0, total);
      } else {
        walk(GEN{}, 0, total);
      }
    }
  }

  // ---- end of the item: (m, l, o) of every head straight from the registers ----
  float l = l_part;
  l += __shfl_xor(l, 16, 64);
  l += __shfl_xor(l, 32, 64);  // head r
  if constexpr (VAFF) {
#pragma unroll
    for (int b = 0; b < VNB; ++b) {
      bsum[b] += __shfl_xor(bsum[b], 16, 64);
      bsum[b] += __shfl_xor(bsum[b], 32, 64);
    }
  }
  const bool final_out = it.partial < 0;
  if (!final_out && it.partial >= a.max_partials) return;
  float* dst = final_out ? a.out + qbase : a.part_o + int64_t(it.partial) * nq * HD;
  // D row 4 kb + i is head q = (4 kb + i) % NQB of group copy c = 4 kb / NQB
  // (every i: NQB is a multiple of 4); lane 4 kb + i holds the same head and
  // copy, so q's sum and copy c's bias sums live there.  Rows of copy c are
  // stored for the groups c carries (all groups when GB = 1).
  const int orow = (4 * kb) % NQB, ocopy = (4 * kb) / NQB;
  float inv[4], bq[4][VNB];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float lq = __shfl(l, 4 * kb + i, 64);
    inv[i] = final_out ? 1.f / fmaxf(lq, 1e-30f) : 1.f;
#pragma unroll
    for (int b = 0; b < VNB; ++b) bq[i][b] = VAFF ? __shfl(bsum[b], 4 * kb + i, 64) : 0.f;
  }
  // one per-lane pointer (head orow, column dcol); every store is a constant offset from it
  float* dq = dst + orow * HD + dcol;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (orow + i < nq)
#pragma unroll
      for (int g = 0; g < VG; ++g)
        if (GB == 1 || g % GB == ocopy)
#pragma unroll
          for (int h = 0; h < H; ++h)
            dq[i * HD + VGS * g + LPW4 * h] = (acc[g * H + h][i] * (1.f / kVS) + bq[i][g / GB]) * inv[i];
  if (!final_out && kb == 0 && r < nq) {  // heads r < nq (copy 0)
    a.part_ml[(int64_t(it.partial) * nq + r) * 2 + 0] = m_ref;
    a.part_ml[(int64_t(it.partial) * nq + r) * 2 + 1] = l;
  }
}

// Set while dc_decode_waves_per_simd walks the instance selection: the
// instance's launcher then reports its waves per SIMD instead of launching.
static thread_local bool g_query_waves = false;

template <int HD, int VGS, int KMODE, int KBITS, int VBITS, bool VM3, bool KAFF, bool VAFF, int NQB = 16>
static int launch_t(const DecodeArgs& a, hipStream_t stream) {
  if (g_query_waves) return waves_per_simd<HD, KMODE, KBITS, VBITS, NQB>();
  hipLaunchKernelGGL((decode_mfma_kernel<HD, VGS, KMODE, KBITS, VBITS, VM3, KAFF, VAFF, NQB>),
                     dim3(uint32_t(a.n_items)), dim3(64), 0, stream, a);
  return check_hip(hipGetLastError(), "decode_mfma_kernel launch");
}

// Smallest head block a launch may use (0 = automatic: 4, 8 or 16).
static int g_min_nqb = 0;

// The smallest head block that holds n_q, from QMIN (the smallest the
// instance's group counts allow) up.
template <int HD, int VGS, int KMODE, int KBITS, int VBITS, bool VM3, bool KAFF, bool VAFF, int QMIN>
static int launch_q(const DecodeArgs& a, hipStream_t stream) {
  const int nq = a.n_q > g_min_nqb ? a.n_q : g_min_nqb;
  if constexpr (QMIN <= 4)
    if (nq <= 4) return launch_t<HD, VGS, KMODE, KBITS, VBITS, VM3, KAFF, VAFF, 4>(a, stream);
  if constexpr (QMIN <= 8)
    if (nq <= 8) return launch_t<HD, VGS, KMODE, KBITS, VBITS, VM3, KAFF, VAFF, 8>(a, stream);
  return launch_t<HD, VGS, KMODE, KBITS, VBITS, VM3, KAFF, VAFF, 16>(a, stream);
}

static constexpr uint64_t fbit(int fmt, int bits) { return uint64_t(1) << (fmt * 9 + bits); }

int launch_decode_mfma(const DecodeArgs& a, hipStream_t stream, bool* launched) {
  *launched = false;
  const dc_page_geometry& kg = a.kpool.geometry;
  const dc_page_geometry& vg = a.vpool.geometry;
  if (a.n_q > 16 || kg.layout != 0 || vg.layout != 0 || kg.group_size != 32) return DC_OK;
  if (kg.page_capacity % 32 != 0) return DC_OK;
  // formats present in the pools (bit = format * 9 + bits, as in dc_pool)
  const uint64_t km = a.kpool.format_mask, vm = a.vpool.format_mask;
  const uint64_t m0_4 = fbit(DC_FMT_M0_AFFINE, 4) | fbit(DC_FMT_M0_SYMMETRIC, 4);
  const uint64_t m0_8 = fbit(DC_FMT_M0_AFFINE, 8) | fbit(DC_FMT_M0_SYMMETRIC, 8);
  const uint64_t k_m3 = fbit(DC_FMT_M3_F16, 0), k_m0 = m0_4 | m0_8;
  const uint64_t aff = fbit(DC_FMT_M0_AFFINE, 4) | fbit(DC_FMT_M0_AFFINE, 8);
  if (km == 0 || vm == 0 || (km & ~(k_m3 | k_m0)) || (vm & ~(k_m3 | m0_4 | m0_8))) return DC_OK;
  // one key code width and one value code width per launch
  if (((km & m0_4) && (km & m0_8)) || ((vm & m0_4) && (vm & m0_8))) return DC_OK;
  const int kmode = (km & k_m3) && (km & k_m0) ? KEYS_MIXED : (km & k_m3) ? KEYS_M3 : KEYS_M0;
  const int kbits = (km & m0_8) ? 8 : 4;
  const int vbits = (vm & m0_8) ? 8 : 4;
  const bool vm3 = (vm & k_m3) != 0;
  const bool kaff = (km & aff) != 0, vaff = (vm & aff) != 0;
  const int hd = kg.head_dim, vgs = vg.group_size;
  int rc = -1;
  // specialised instantiations for the common pools (every BASELINE
  // configuration, and 8-bit keys at head_dim 128), each with head blocks
  // from QM_ up, and a general one per shape and code widths otherwise
  // (KEYS_M3 ignores kbits)
#define DC_EXACT(HD_, VGS_, KM_, KB_, VB_, VM3_, KA_, VA_, QM_)                                            \
  if (rc < 0 && hd == HD_ && vgs == VGS_ && kmode == KM_ && (KM_ == KEYS_M3 || kbits == KB_) &&          \
      vbits == VB_ && vm3 == VM3_ && kaff == KA_ && vaff == VA_)                                         \
    rc = launch_q<HD_, VGS_, KM_, KB_, VB_, VM3_, KA_, VA_, QM_>(a, stream);
// (general instances take head blocks from the smallest their group counts
// allow: 4 heads where key and value groups come in fours, 8 in twos)
#define DC_GENERAL(HD_, VGS_, VB_)                                                                  \
  if (rc < 0 && hd == HD_ && vgs == VGS_ && vbits == VB_) {                                         \
    constexpr int kq = (HD_ / 32) % 4 == 0 && (HD_ / VGS_) % 4 == 0   ? 4                            \
                       : (HD_ / 32) % 2 == 0 && (HD_ / VGS_) % 2 == 0 ? 8                            \
                                                                      : 16;                          \
    rc = kbits == 8 ? launch_q<HD_, VGS_, KEYS_MIXED, 8, VB_, true, true, true, kq>(a, stream)      \
                    : launch_q<HD_, VGS_, KEYS_MIXED, 4, VB_, true, true, true, kq>(a, stream);     \
  }
  DC_EXACT(64, 32, KEYS_M0, 4, 4, false, false, false, 8)     // config 1
  DC_EXACT(64, 32, KEYS_M0, 4, 4, false, true, true, 8)       // config 2
  DC_EXACT(128, 32, KEYS_M3, 4, 4, false, false, false, 16)   // config 3 (blocks of 8: slower)
  DC_EXACT(128, 64, KEYS_MIXED, 4, 8, false, true, false, 8)  // config 4
  DC_EXACT(128, 64, KEYS_M0, 4, 8, false, true, false, 8)
  DC_EXACT(128, 32, KEYS_M0, 4, 4, false, true, true, 4)
  DC_EXACT(256, 32, KEYS_MIXED, 4, 4, true, true, true, 4)  // config 5 (fp16 recent window)
  DC_EXACT(256, 32, KEYS_M0, 4, 4, false, true, true, 4)
  DC_EXACT(256, 32, KEYS_M3, 4, 4, true, false, false, 4)  // config 5's window launch (fp16 keys and values)
  DC_EXACT(128, 32, KEYS_M0, 8, 4, false, true, true, 4)  // 8-bit keys, 4-bit values
  DC_EXACT(128, 32, KEYS_M0, 8, 8, false, true, true, 4)  // 8-bit keys and values
  DC_EXACT(128, 64, KEYS_M0, 8, 8, false, true, false, 8)     // config 4 with 8-bit keys
  DC_EXACT(128, 64, KEYS_MIXED, 8, 8, false, true, false, 8)
  DC_EXACT(256, 32, KEYS_M0, 8, 4, false, true, true, 4)      // config 5 with 8-bit keys (decode launch)
  DC_GENERAL(64, 32, 4)
  DC_GENERAL(64, 32, 8)
  DC_GENERAL(64, 64, 4)
  DC_GENERAL(64, 64, 8)
  DC_GENERAL(128, 32, 4)
  DC_GENERAL(128, 32, 8)
  DC_GENERAL(128, 64, 4)
  DC_GENERAL(128, 64, 8)
  DC_GENERAL(256, 32, 4)
  DC_GENERAL(256, 32, 8)
  DC_GENERAL(256, 64, 4)
  DC_GENERAL(256, 64, 8)
#undef DC_EXACT
#undef DC_GENERAL
  if (rc < 0) return DC_OK;
  *launched = true;
  return rc;
}

// Waves per SIMD of the MFMA instance a decode with these pools and n_q
// would launch (0: the MFMA kernel does not take them).
int decode_mfma_waves(const DecodeArgs& a) {
  bool launched = false;
  g_query_waves = true;
  const int w = launch_decode_mfma(a, nullptr, &launched);
  g_query_waves = false;
  return launched ? w : 0;
}

}  // namespace dc

extern "C" int dc_set_mfma_head_block(int32_t nqb) {
  if (nqb != 0 && nqb != 4 && nqb != 8 && nqb != 16)
    return dc::fail(DC_EINVAL, "MFMA head block must be 0 (automatic), 4, 8 or 16");
  dc::g_min_nqb = nqb;
  return DC_OK;
}
