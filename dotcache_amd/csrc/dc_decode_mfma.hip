// MFMA fast path of the fused paged decode (gfx950, v_mfma_f32_16x16x32_f16).
//
// One wavefront runs one work item: it walks its pages, scores the page's
// tokens for the GQA query heads of its KV head, folds them into a running
// (max, sum) per head, and mixes the value page -- all from the compressed
// page bytes.  Accepted pages: keys M3 fp16 or M0 4-bit (group 32, affine or
// symmetric); values M0 4- or 8-bit (group 32 or 64, affine or symmetric) or
// M3 fp16.  Other formats take the generic kernel (dc_decode.hip).
//
// Exactness.  Every MFMA operand is exact: escape rows are fp16 already,
// codes (c - zero point) are small integers, and the fp32 operands (scaled
// queries, softmax weight x value scale) are split into an fp16 high part
// and an fp16 residual, so each product is an exact fp16 x fp16 product
// accumulated in fp32.  Per-(token, group) scales and biases are applied in
// fp32 outside the MFMA, in the reference's streaming form
// s * (codes . q_g) + b * sum(q_g) (reference
// dotcache/attention_reference.py:101-126, :168-192).
//
// Pages are processed in chunks of 32 tokens: stage the chunk's value codes
// and scales in LDS, score it (two 16-token MFMA tiles), update the running
// max / sum, mix it.  Lane maps (lane l, r = l % 16, kb = l / 16; a
// 16x16x32 MFMA gives lane l row r of A, column r of B and the D values of
// rows 4 kb + i, column r):
//   score  D[token, q] = K[token, :] . Q[q, :]   (A = key rows, B = queries).
//          Tile hh, A row m is chunk token 8 (m / 4) + 4 hh + m % 4, so the
//          D rows a lane holds are chunk tokens 8 kb + e, e < 8 -- the same
//          tokens the lane feeds as A k-slots of the mix, so a softmax weight
//          never leaves the lane that produced it except for the row shuffle
//          to the residual rows.
//   mix    D[qrow, d] = A[qrow, token] x B[token, d]; qrow < n_q is the high
//          part of query head qrow, n_q <= qrow < 2 n_q the residual of head
//          qrow - n_q; the two rows are added once at the end.  Column r of
//          tile h of value group g is channel VGS g + 8 (r / L) + r % L + L h
//          with L = 128 / VGS, which lets every lane unpack its codes with one
//          byte permute per pair of tokens.
#include "dc_common.h"
#include "dc_decode.h"

namespace dc {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

union Frag {
  half8 h;
  uint32_t u[4];
};

__device__ __forceinline__ f32x4 mfma(const Frag& a, const Frag& b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a.h, b.h, c, 0, 0, 0);
}

// fp16 pair (lo, hi) from two floats, round to nearest even.
__device__ __forceinline__ uint32_t pack_h2(float lo, float hi) {
  const _Float16 a = (_Float16)lo, b = (_Float16)hi;
  return uint32_t(__builtin_bit_cast(uint16_t, a)) | (uint32_t(__builtin_bit_cast(uint16_t, b)) << 16);
}

// fp32 -> fp16 high part, or the fp16 residual x - f32(f16(x)).
__device__ __forceinline__ float split_part(float x, bool residual) {
  const float hi = float((_Float16)x);
  return residual ? x - hi : x;
}

// Packed fp16 pair (1024 + a, 1024 + b) -> (a - z, b - z), exact.
__device__ __forceinline__ uint32_t magic_sub(uint32_t x, uint32_t neg_bias_pair) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const h2 v = __builtin_bit_cast(h2, x) + __builtin_bit_cast(h2, neg_bias_pair);
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ uint32_t h2_const(float v) { return pack_h2(v, v); }

// fp16 bits (low 16 bits of x) -> float
__device__ __forceinline__ float h2f(uint32_t x) { return float(__builtin_bit_cast(_Float16, uint16_t(x))); }

// Two fp32 values as packed fp16: their high parts rtz(x) (res_neg = 0) or
// their residuals rtz(x - rtz(x)) (res_neg = -1).  x - rtz(x) is exact in
// fp32, so high part + residual carries x to about 2^-20 relative.
__device__ __forceinline__ uint32_t split_pair(float x0, float x1, float res_neg) {
  typedef _Float16 h2v __attribute__((ext_vector_type(2)));
  const h2v hi = __builtin_bit_cast(h2v, __builtin_amdgcn_cvt_pkrtz(x0, x1));
  const float r0 = fmaf(float(hi[0]), res_neg, x0);
  const float r1 = fmaf(float(hi[1]), res_neg, x1);
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(r0, r1));
}

constexpr int kWaves = 4;  // waves per workgroup; each walks its own pages of the work item

// Key-page mix of a pool: only M3 rows, only M0 4-bit codes, or both.
enum KeyMode { KEYS_M3 = 0, KEYS_M0 = 1, KEYS_MIXED = 2 };

template <int HD, int VGS, int VBITS>
struct MfmaCfg {
  static constexpr int KG = HD / 32;        // key groups of 32 channels (= contraction steps of the score)
  static constexpr int VG = HD / VGS;       // value groups
  static constexpr int H = VGS / 16;        // mix column tiles per value group
  static constexpr int LPW4 = 128 / VGS;    // lanes sharing one 4-bit code word
  static constexpr int NACC = VG * H;       // = HD / 16 accumulator tiles
  static constexpr int W = VBITS == 8 ? VGS / 4 : VGS / 8;  // code words per (token, value group)
  static constexpr int NVP = VG * 8 * W / 64;                // 16-byte value-code pieces per lane per chunk
  static constexpr int NKS = (16 * KG + 63) / 64;            // key scale words per lane per chunk
  static constexpr int NVS = (16 * VG + 63) / 64;            // value scale words per lane per chunk
  // per-wave LDS: chunk staging -- value codes [VG][32][W], value scales /
  // biases and key scales / biases transposed to [group][32 tokens] fp16 --
  // later reused for the end-of-item rows
  static constexpr int VPAY = VG * 32 * W;
  static constexpr int VSC = VPAY, VBS = VSC + 16 * VG, KSC = VBS + 16 * VG, KBS = KSC + 16 * KG;
  static constexpr int STAGE = KBS + 16 * KG;
  static constexpr int ROWS = 16 * HD + 16 * VG;  // D rows of the mix + bias sums
  static constexpr int WAVE_WORDS = STAGE > ROWS ? STAGE : ROWS;
  static constexpr int LDS_WORDS = kWaves * WAVE_WORDS;
  static_assert(VG * 8 * W % 64 == 0, "value pieces must spread evenly over the wave");
};

// Registers one chunk needs from HBM.  The next chunk's loads are issued
// into them as soon as the current chunk has consumed them (values and
// scales after staging, keys after the score), so they are in flight during
// its mix.  Every chunk issues the same loads whatever its page formats, so
// the compiler never has to drain the queue to merge register versions.
template <int HD, int VGS, int VBITS>
struct ChunkRegs {
  using Cfg = MfmaCfg<HD, VGS, VBITS>;
  u32x4 kr[2][Cfg::KG];  // key rows (M3: 8 fp16) or the 16-byte code block of (token, group) (M0)
  u32x4 vr[Cfg::NVP];    // value code pieces, blob byte order
  uint32_t ks[Cfg::NKS], kbw[Cfg::NKS], vs[Cfg::NVS], vb[Cfg::NVS];  // scale / bias words
};

struct PageMeta {
  const uint8_t* kp;
  const uint8_t* vp;
  int T;  // tokens to read (0: skip the page)
  int kfmt, vfmt, vbits;
  uint32_t ksc, kbs, vsc, vbs;  // byte offsets of scales / biases in the blobs (0 where absent)
};

template <int HD, int VGS, int KMODE, int VBITS, bool VM3>
__global__ void __launch_bounds__(kWaves * 64, HD >= 256 ? 1 : 2) decode_mfma_kernel(DecodeArgs a) {
  using Cfg = MfmaCfg<HD, VGS, VBITS>;
  using Regs = ChunkRegs<HD, VGS, VBITS>;
  constexpr int KG = Cfg::KG, VG = Cfg::VG, H = Cfg::H, LPW4 = Cfg::LPW4, W = Cfg::W;
  __shared__ uint32_t lds_all[Cfg::LDS_WORDS];
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));

  const dc_work_item it = a.items[blockIdx.x];
  // readfirstlane tells the compiler the wave index is uniform, so page and
  // chunk loop state, blob pointers and page metadata live in SGPRs
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int r = lane & 15, kb = lane >> 4;
  const int nq = a.n_q;
  const int CAP = a.kpool.geometry.page_capacity;
  uint32_t* lds = lds_all + wave * Cfg::WAVE_WORDS;
  uint16_t* vsc = reinterpret_cast<uint16_t*>(lds + Cfg::VSC);
  uint16_t* vbs = reinterpret_cast<uint16_t*>(lds + Cfg::VBS);
  uint16_t* ksc = reinterpret_cast<uint16_t*>(lds + Cfg::KSC);
  uint16_t* kbs = reinterpret_cast<uint16_t*>(lds + Cfg::KBS);

  // ---- queries scaled by query_scale * log2(e); B fragments hi / residual ----
  // lane (r, kb) holds channels 32 g + 8 kb + i of head r; one vector load per
  // group.
  const int64_t qbase = (int64_t(it.seq) * a.n_kv_heads + it.kv_head) * nq * HD;
  const float qmul = a.q_scale * kLog2e;
  const int64_t qrow = qbase + int64_t(r < nq ? r : 0) * HD + 8 * kb;
  Frag qhi[KG], qlo[KG];
  float qsum[KG];
  auto setup_queries = [&]() {
    float qv[KG][8];
    if (a.queries_dtype == DC_F32) {
      const float* q = reinterpret_cast<const float*>(a.queries) + qrow;
  #pragma unroll
      for (int g = 0; g < KG; ++g) {
        const float4 x0 = *reinterpret_cast<const float4*>(q + 32 * g);
        const float4 x1 = *reinterpret_cast<const float4*>(q + 32 * g + 4);
        qv[g][0] = x0.x; qv[g][1] = x0.y; qv[g][2] = x0.z; qv[g][3] = x0.w;
        qv[g][4] = x1.x; qv[g][5] = x1.y; qv[g][6] = x1.z; qv[g][7] = x1.w;
      }
    } else {
      const uint16_t* q = reinterpret_cast<const uint16_t*>(a.queries) + qrow;
      const bool bf = a.queries_dtype == DC_BF16;
  #pragma unroll
      for (int g = 0; g < KG; ++g) {
        const uint4 x = *reinterpret_cast<const uint4*>(q + 32 * g);
        const uint32_t xs[4] = {x.x, x.y, x.z, x.w};
  #pragma unroll
        for (int i = 0; i < 4; ++i) {
          qv[g][2 * i] = bf ? __uint_as_float(xs[i] << 16) : h2f(xs[i] & 0xffffu);
          qv[g][2 * i + 1] = bf ? __uint_as_float(xs[i] & 0xffff0000u) : h2f(xs[i] >> 16);
        }
      }
    }
  #pragma unroll
    for (int g = 0; g < KG; ++g) {
      float s = 0.f;
  #pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float v0 = r < nq ? qv[g][2 * i] * qmul : 0.f, v1 = r < nq ? qv[g][2 * i + 1] * qmul : 0.f;
        qhi[g].u[i] = pack_h2(v0, v1);
        qlo[g].u[i] = pack_h2(split_part(v0, true), split_part(v1, true));
        s += v0 + v1;
      }
      s += __shfl_xor(s, 16, 64);
      s += __shfl_xor(s, 32, 64);
      qsum[g] = s;  // sum over group g for head r
    }
  };

  // mix A-row role of this lane: high part (r < nq) or residual (nq <= r < 2 nq) of head qa
  const bool row_live = r < 2 * nq;
  const bool residual = r >= nq;
  const int pa_src = kb * 16 + (row_live ? (residual ? r - nq : r) : 0);
  int rowq[4];  // head of mix D rows 4 kb + i
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = 4 * kb + i;
    rowq[i] = row < nq ? row : (row < 2 * nq ? row - nq : 0);
  }
  // mix column of this lane in tile h of value group g: d = VGS g + dcol + LPW4 h
  const int jj = r % LPW4, w4 = r / LPW4;
  const int dcol = 8 * w4 + jj;
  const float res_neg = residual ? -1.f : 0.f;
  // byte-permute selectors of this lane's code in tile h: the byte of token
  // 2p into byte 0, of token 2p + 1 into byte 2 (4-bit: byte holding nibble
  // jj + LPW4 h; 8-bit: byte (jj + LPW4 h) % 4)
  uint32_t vsel[H];
#pragma unroll
  for (int h = 0; h < H; ++h) {
    const uint32_t b = VBITS == 4 ? uint32_t((jj + LPW4 * h) >> 1) : uint32_t((jj + LPW4 * h) & 3);
    vsel[h] = 0x0c000c00u | b | ((4u + b) << 16);
  }
  const uint32_t nib_mask = (jj & 1) ? 0x00f000f0u : 0x000f000fu;  // low or high nibble of the byte
  const h2 nib_mul = (jj & 1) ? h2{(_Float16)0.0625f, (_Float16)0.0625f} : h2{(_Float16)1.f, (_Float16)1.f};

  f32x4 acc[Cfg::NACC];
#pragma unroll
  for (int t = 0; t < Cfg::NACC; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  float bsum[VG];
#pragma unroll
  for (int g = 0; g < VG; ++g) bsum[g] = 0.f;
  float m_run = -INFINITY, l_part = 0.f;

  const dc_page_geometry kgeo = a.kpool.geometry, vgeo = a.vpool.geometry;
  const int64_t trow = (int64_t(it.seq) * a.n_kv_heads + it.kv_head) * a.table_stride;
  const int n_item = it.page_end - it.page_begin;
  const int np = n_item > wave ? (n_item - wave + kWaves - 1) / kWaves : 0;  // pages of this wave

  auto key_is_m3 = [&](const PageMeta& m) -> bool {
    if constexpr (KMODE == KEYS_M3) return true;
    if constexpr (KMODE == KEYS_M0) return false;
    return m.kfmt == DC_FMT_M3_F16;
  };
  auto value_is_m0 = [&](const PageMeta& m) -> bool {
    if constexpr (!VM3) return true;
    return is_m0(m.vfmt);
  };

  // ---- loads of one chunk into registers (the same loads for every format) ----
  auto load_keys = [&](const PageMeta& m, int c0, Regs& R) {
    const bool km3 = key_is_m3(m);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int ta = c0 + 8 * (r >> 2) + 4 * hh + (r & 3);
#pragma unroll
      for (int g = 0; g < KG; ++g) {
        const int off = km3 ? (ta * HD + 32 * g + 8 * kb) * 2 : (g * CAP + ta) * 16;
        R.kr[hh][g] = *reinterpret_cast<const u32x4*>(m.kp + off);
      }
    }
    if constexpr (KMODE != KEYS_M3) {
      const uint32_t* S = reinterpret_cast<const uint32_t*>(m.kp + m.ksc) + c0 * KG / 2;
      const uint32_t* B = reinterpret_cast<const uint32_t*>(m.kp + m.kbs) + c0 * KG / 2;
#pragma unroll
      for (int k = 0; k < Cfg::NKS; ++k) {
        const int e = (lane + 64 * k) % (16 * KG);
        R.ks[k] = S[e];
        R.kbw[k] = B[e];
      }
    }
  };
  auto load_values = [&](const PageMeta& m, int c0, Regs& R) {
#pragma unroll
    for (int k = 0; k < Cfg::NVP; ++k) {
      const int e = lane + 64 * k;
      const int g = e / (8 * W), piece = e - g * (8 * W);
      R.vr[k] = *reinterpret_cast<const u32x4*>(m.vp + (((g * CAP + c0) * W) / 4 + piece) * 16);
    }
    const uint32_t* S = reinterpret_cast<const uint32_t*>(m.vp + m.vsc) + c0 * VG / 2;
    const uint32_t* B = reinterpret_cast<const uint32_t*>(m.vp + m.vbs) + c0 * VG / 2;
#pragma unroll
    for (int k = 0; k < Cfg::NVS; ++k) {
      const int e = (lane + 64 * k) % (16 * VG);
      R.vs[k] = S[e];
      R.vb[k] = B[e];
    }
  };

  // ---- registers -> this wave's LDS staging area ----
  auto stage_chunk = [&](const Regs& R) {
    u32x4* dst = reinterpret_cast<u32x4*>(lds);
#pragma unroll
    for (int k = 0; k < Cfg::NVP; ++k) dst[lane + 64 * k] = R.vr[k];
    // scale word e holds (token, group) entries 2e and 2e + 1 of the chunk's [32][G] array
#pragma unroll
    for (int k = 0; k < Cfg::NVS; ++k) {
      const int e = lane + 64 * k;
      if (e < 16 * VG) {
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          const int hidx = 2 * e + s, t = hidx / VG, g = hidx - t * VG;
          vsc[g * 32 + t] = uint16_t(R.vs[k] >> (16 * s));
          vbs[g * 32 + t] = uint16_t(R.vb[k] >> (16 * s));
        }
      }
    }
    if constexpr (KMODE != KEYS_M3) {
#pragma unroll
      for (int k = 0; k < Cfg::NKS; ++k) {
        const int e = lane + 64 * k;
        if (e < 16 * KG) {
#pragma unroll
          for (int s = 0; s < 2; ++s) {
            const int hidx = 2 * e + s, t = hidx / KG, g = hidx - t * KG;
            ksc[g * 32 + t] = uint16_t(R.ks[k] >> (16 * s));
            kbs[g * 32 + t] = uint16_t(R.kbw[k] >> (16 * s));
          }
        }
      }
    }
  };

  // ---- score of one chunk: logits of this lane's chunk tokens 8 kb + e for head r ----
  auto score_chunk = [&](const PageMeta& m, const Regs& R, float* Ls) {
    if (key_is_m3(m)) {
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int g = 0; g < KG; ++g) {
          Frag ka;
          ka.u[0] = R.kr[hh][g].x; ka.u[1] = R.kr[hh][g].y; ka.u[2] = R.kr[hh][g].z; ka.u[3] = R.kr[hh][g].w;
          d = mfma(ka, qhi[g], d);
          d = mfma(ka, qlo[g], d);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) Ls[4 * hh + i] = d[i];
      }
    } else {  // M0 4-bit, group 32: scale and bias applied per group in fp32
      const bool k_affine = m.kfmt == DC_FMT_M0_AFFINE;
      const float zp = k_affine ? 0.f : 7.f;
      // (1024 + n_lo, 1024 + 16 n_hi) -> (n_lo - zp, n_hi - zp)
      const h2 kmul = {(_Float16)1.f, (_Float16)0.0625f};
      const h2 kadd = {(_Float16)(-1024.f - zp), (_Float16)(-64.f - zp)};
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        float Lh[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int g = 0; g < KG; ++g) {
          const uint32_t w = kb == 0 ? R.kr[hh][g].x : kb == 1 ? R.kr[hh][g].y : kb == 2 ? R.kr[hh][g].z : R.kr[hh][g].w;
          Frag ka;
#pragma unroll
          for (int p = 0; p < 4; ++p) {
            // byte p holds channel 2p (low nibble) and 2p + 1 (high nibble)
            const uint32_t x = __builtin_amdgcn_perm(w, w, 0x0c040c00u + 0x00010001u * p);
            const h2 v = __builtin_bit_cast(h2, (x & 0x00f0000fu) | 0x64006400u) * kmul + kadd;
            ka.u[p] = __builtin_bit_cast(uint32_t, v);
          }
          f32x4 d = {0.f, 0.f, 0.f, 0.f};
          d = mfma(ka, qhi[g], d);
          d = mfma(ka, qlo[g], d);
          // D rows 4 kb + i are chunk tokens 8 kb + 4 hh + i
          const uint2 sw = *reinterpret_cast<const uint2*>(ksc + g * 32 + 8 * kb + 4 * hh);
          const uint2 bw = *reinterpret_cast<const uint2*>(kbs + g * 32 + 8 * kb + 4 * hh);
          const uint32_t sv[4] = {sw.x & 0xffffu, sw.x >> 16, sw.y & 0xffffu, sw.y >> 16};
          const uint32_t bv[4] = {bw.x & 0xffffu, bw.x >> 16, bw.y & 0xffffu, bw.y >> 16};
#pragma unroll
          for (int i = 0; i < 4; ++i) Lh[i] += h2f(sv[i]) * d[i] + (k_affine ? h2f(bv[i]) * qsum[g] : 0.f);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) Ls[4 * hh + i] = Lh[i];
      }
    }
  };

  // ---- online softmax update and mix of one staged chunk ----
  auto mix_chunk = [&](const PageMeta& m, int c0, float* Ls) {
    // online softmax for head r (the four kb lanes hold its 32 tokens)
    float mx = -INFINITY;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if (c0 + 8 * kb + e >= m.T) Ls[e] = -INFINITY;
      mx = fmaxf(mx, Ls[e]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_run, mx);
    const float alpha = m_new == -INFINITY ? 1.f : exp2f(m_run - m_new);
    float psum = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      Ls[e] = Ls[e] == -INFINITY ? 0.f : exp2f(Ls[e] - m_new);
      psum += Ls[e];
    }
    l_part = l_part * alpha + psum;
    m_run = m_new;
    if (__any(alpha != 1.f)) {
      float arow[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) arow[i] = __shfl(alpha, rowq[i], 64);
#pragma unroll
      for (int t = 0; t < Cfg::NACC; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[t][i] *= arow[i];
#pragma unroll
      for (int g = 0; g < VG; ++g) bsum[g] *= alpha;
    }

    // weights of this lane's A-row head on its 8 tokens
    float pa[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float v = __shfl(Ls[e], pa_src, 64);
      pa[e] = row_live ? v : 0.f;
    }
    if (value_is_m0(m)) {
      const bool v_affine = m.vfmt == DC_FMT_M0_AFFINE;
      const float zp = v_affine ? 0.f : float((1 << (VBITS - 1)) - 1);
      // codes become fp16 (1024 + c), or (1024 + 16 c) for a code in the high
      // nibble of its byte; one packed fma maps either to c - zp exactly
      const h2 vadd = VBITS == 4 && (jj & 1) ? h2{(_Float16)(-64.f - zp), (_Float16)(-64.f - zp)}
                                              : h2{(_Float16)(-1024.f - zp), (_Float16)(-1024.f - zp)};
#pragma unroll
      for (int g = 0; g < VG; ++g) {
        const uint4 s8 = *reinterpret_cast<const uint4*>(vsc + g * 32 + 8 * kb);
        const uint32_t sx[4] = {s8.x, s8.y, s8.z, s8.w};
        Frag fa;
#pragma unroll
        for (int pp = 0; pp < 4; ++pp) {
          const h2 sv = __builtin_bit_cast(h2, sx[pp]);
          fa.u[pp] = split_pair(pa[2 * pp] * float(sv[0]), pa[2 * pp + 1] * float(sv[1]), res_neg);
        }
        if (v_affine) {
          const uint4 b8 = *reinterpret_cast<const uint4*>(vbs + g * 32 + 8 * kb);
          const uint32_t bx[4] = {b8.x, b8.y, b8.z, b8.w};
#pragma unroll
          for (int pp = 0; pp < 4; ++pp) {
            const h2 bv = __builtin_bit_cast(h2, bx[pp]);
            bsum[g] += Ls[2 * pp] * float(bv[0]) + Ls[2 * pp + 1] * float(bv[1]);
          }
        }
        const uint32_t* Pw = lds + (g * 32 + 8 * kb) * W;  // words of tokens 8 kb + e
#pragma unroll
        for (int h = 0; h < H; ++h) {
          Frag fb;
          if constexpr (VBITS == 4) {
#pragma unroll
            for (int pp = 0; pp < 4; ++pp) {
              const uint32_t x = __builtin_amdgcn_perm(Pw[(2 * pp + 1) * W + w4], Pw[(2 * pp) * W + w4], vsel[h]);
              const h2 c = __builtin_bit_cast(h2, (x & nib_mask) | 0x64006400u) * nib_mul + vadd;
              fb.u[pp] = __builtin_bit_cast(uint32_t, c);
            }
          } else {
            const int wsel = 2 * w4 + ((jj + LPW4 * h) >> 2);  // channel dcol + LPW4 h: word 2 w4 + e / 4, byte e % 4
#pragma unroll
            for (int pp = 0; pp < 4; ++pp) {
              const uint32_t x = __builtin_amdgcn_perm(Pw[(2 * pp + 1) * W + wsel], Pw[(2 * pp) * W + wsel], vsel[h]);
              const h2 c = __builtin_bit_cast(h2, x | 0x64006400u) + vadd;
              fb.u[pp] = __builtin_bit_cast(uint32_t, c);
            }
          }
          acc[g * H + h] = mfma(fa, fb, acc[g * H + h]);
        }
        __builtin_amdgcn_sched_barrier(0);  // keep every group's LDS reads from being hoisted at once
      }
    } else if constexpr (VM3) {  // M3 fp16 values (the exact recent window): gather columns from the rows
      const uint16_t* V = reinterpret_cast<const uint16_t*>(m.vp);
      Frag fa;
#pragma unroll
      for (int pp = 0; pp < 4; ++pp) fa.u[pp] = split_pair(pa[2 * pp], pa[2 * pp + 1], res_neg);
#pragma unroll
      for (int g = 0; g < VG; ++g)
#pragma unroll
        for (int h = 0; h < H; ++h) {
          const int d = VGS * g + dcol + LPW4 * h;
          Frag fb;
#pragma unroll
          for (int pp = 0; pp < 4; ++pp) {
            const int t0 = c0 + 8 * kb + 2 * pp;
            const uint32_t lo = t0 < m.T ? V[t0 * HD + d] : 0u;
            const uint32_t hi = t0 + 1 < m.T ? V[(t0 + 1) * HD + d] : 0u;
            fb.u[pp] = lo | (hi << 16);
          }
          acc[g * H + h] = mfma(fa, fb, acc[g * H + h]);
        }
    }
  };

  // ---- walk this wave's pages: page meta 64 pages at a time, chunks pipelined ----
  // lane i < nb holds the ids / descriptors of the wave's page base + i; the
  // first batch is fetched before the query setup so the two overlap
  uint32_t k0 = 0, k1 = 0, v0 = 0, v1 = 0;
  int ok = 0;
  auto load_meta = [&](int base) {
    const int nb = np - base < 64 ? np - base : 64;
    k0 = k1 = v0 = v1 = 0u;
    ok = 0;
    if (lane < nb) {
      const int p = it.page_begin + wave + kWaves * (base + lane);
      const int kid = a.k_table[trow + p], vid = a.v_table[trow + p];
      if (kid >= 0 && kid < a.kpool.n_descs && vid >= 0 && vid < a.vpool.n_descs) {
        const uint2 kd = *reinterpret_cast<const uint2*>(a.kpool.descs + kid);
        const uint2 vd = *reinterpret_cast<const uint2*>(a.vpool.descs + vid);
        k0 = kd.x; k1 = kd.y; v0 = vd.x; v1 = vd.y;
        ok = 1;
      }
    }
  };
  if (np > 0) load_meta(0);
  setup_queries();
  for (int base = 0; base < np; base += 64) {
    const int nb = np - base < 64 ? np - base : 64;
    if (base > 0) load_meta(base);
    auto meta_of = [&](int i) -> PageMeta {
      PageMeta m{};
      const uint32_t kw0 = __builtin_amdgcn_readlane(k0, i), kw1 = __builtin_amdgcn_readlane(k1, i);
      const uint32_t vw0 = __builtin_amdgcn_readlane(v0, i), vw1 = __builtin_amdgcn_readlane(v1, i);
      const int good = __builtin_amdgcn_readlane(ok, i);
      dc_page_desc kd, vd;
      kd.block = kw0; kd.tokens = uint16_t(kw1 & 0xffff); kd.format = uint8_t(kw1 >> 16); kd.bits = uint8_t(kw1 >> 24);
      vd.block = vw0; vd.tokens = uint16_t(vw1 & 0xffff); vd.format = uint8_t(vw1 >> 16); vd.bits = uint8_t(vw1 >> 24);
      const BlobLayout KL = blob_layout(kd.format, kd.bits, kgeo), VL = blob_layout(vd.format, vd.bits, vgeo);
      int T = kd.tokens < vd.tokens ? kd.tokens : vd.tokens;
      if (T > CAP) T = CAP;
      if (!good || (int64_t(kd.block) << 8) + KL.total > a.kpool.arena_bytes ||
          (int64_t(vd.block) << 8) + VL.total > a.vpool.arena_bytes)
        T = 0;
      m.T = T;
      m.kp = blob_ptr(a.kpool.arena, kd);
      m.vp = blob_ptr(a.vpool.arena, vd);
      m.kfmt = kd.format;
      m.vfmt = vd.format;
      m.vbits = vd.bits;
      const bool km0 = is_m0(kd.format), vm0 = is_m0(vd.format);
      m.ksc = km0 ? uint32_t(KL.scales_off) : 0u;
      m.kbs = kd.format == DC_FMT_M0_AFFINE ? uint32_t(KL.bias_off) : m.ksc;
      m.vsc = vm0 ? uint32_t(VL.scales_off) : 0u;
      m.vbs = vd.format == DC_FMT_M0_AFFINE ? uint32_t(VL.bias_off) : m.vsc;
      return m;
    };

    int i = 0;
    PageMeta cur = meta_of(0);
    while (cur.T <= 0 && i + 1 < nb) cur = meta_of(++i);
    if (cur.T <= 0) continue;
    int c0 = 0;
    Regs R;
    load_keys(cur, c0, R);
    load_values(cur, c0, R);
    while (true) {
      // next chunk of this batch; the current chunk again when there is none
      int ni = i, nc0 = c0 + 32;
      PageMeta nm = cur;
      if (nc0 >= cur.T) {
        nc0 = 0;
        ni = i + 1;
        while (ni < nb) {
          nm = meta_of(ni);
          if (nm.T > 0) break;
          ++ni;
        }
      }
      const bool more = ni < nb;
      if (!more) {
        nm = cur;
        nc0 = c0;
      }
      float Ls[8];
      if constexpr (HD <= 128) {
        Regs Rn;  // the next chunk's loads fly while this one is scored and mixed
        load_keys(nm, nc0, Rn);
        load_values(nm, nc0, Rn);
        stage_chunk(R);  // value codes and scales -> LDS
        score_chunk(cur, R, Ls);
        mix_chunk(cur, c0, Ls);
        R = Rn;
      } else {  // one register set: reload it as soon as the chunk has consumed it
        stage_chunk(R);
        score_chunk(cur, R, Ls);
        load_keys(nm, nc0, R);
        load_values(nm, nc0, R);
        mix_chunk(cur, c0, Ls);
      }
      if (!more) break;
      cur = nm;
      i = ni;
      c0 = nc0;
    }
  }

  // ---- per wave: rows q and q + n_q, bias sums -> o[q][d]; then (m, l) ----
  float l_tot = l_part;
  l_tot += __shfl_xor(l_tot, 16, 64);
  l_tot += __shfl_xor(l_tot, 32, 64);
#pragma unroll
  for (int g = 0; g < VG; ++g) {
    bsum[g] += __shfl_xor(bsum[g], 16, 64);
    bsum[g] += __shfl_xor(bsum[g], 32, 64);
  }
  float* rows = reinterpret_cast<float*>(lds);  // [16][HD] D rows, then [16][VG] bias sums
#pragma unroll
  for (int g = 0; g < VG; ++g)
#pragma unroll
    for (int h = 0; h < H; ++h) {
      const int d = VGS * g + dcol + LPW4 * h;
#pragma unroll
      for (int i = 0; i < 4; ++i) rows[(4 * kb + i) * HD + d] = acc[g * H + h][i];
    }
  if (kb == 0 && r < nq)
#pragma unroll
    for (int g = 0; g < VG; ++g) rows[16 * HD + r * VG + g] = bsum[g];
  constexpr int NO = 8 * HD / 64;  // o values per lane (n_q <= 8)
  float o[NO];
#pragma unroll
  for (int k = 0; k < NO; ++k) {
    const int idx = lane + 64 * k;
    const int q = idx / HD, d = idx - q * HD;
    o[k] = q < nq ? rows[q * HD + d] + rows[(q + nq) * HD + d] + rows[16 * HD + q * VG + d / VGS] : 0.f;
  }
#pragma unroll
  for (int k = 0; k < NO; ++k) rows[lane + 64 * k] = o[k];  // o [8][HD]
  if (kb == 0 && r < nq) {
    rows[8 * HD + 2 * r] = m_run;
    rows[8 * HD + 2 * r + 1] = l_tot;
  }
  __syncthreads();

  // ---- workgroup: merge the waves' (m, l, o) by log-sum-exp ----
  const bool final_out = it.partial < 0;
  if (!final_out && it.partial >= a.max_partials) return;
  float* dst = final_out ? a.out + qbase : a.part_o + int64_t(it.partial) * nq * HD;
  for (int idx = threadIdx.x; idx < nq * HD; idx += kWaves * 64) {
    const int q = idx / HD;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, reinterpret_cast<const float*>(lds_all + w * Cfg::WAVE_WORDS)[8 * HD + 2 * q]);
    float L = 0.f, Ov = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float* wr = reinterpret_cast<const float*>(lds_all + w * Cfg::WAVE_WORDS);
      const float mw = wr[8 * HD + 2 * q];
      const float wt = mw == -INFINITY ? 0.f : exp2f(mw - M);
      L += wr[8 * HD + 2 * q + 1] * wt;
      Ov += wr[idx] * wt;
    }
    if (final_out) {
      dst[idx] = L > 0.f ? Ov / L : 0.f;
    } else {
      dst[idx] = Ov;
      if (idx - q * HD == 0) {
        a.part_ml[(int64_t(it.partial) * nq + q) * 2 + 0] = M;
        a.part_ml[(int64_t(it.partial) * nq + q) * 2 + 1] = L;
      }
    }
  }
}

template <int HD, int VGS, int KMODE, int VBITS, bool VM3>
static int launch_t(const DecodeArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL((decode_mfma_kernel<HD, VGS, KMODE, VBITS, VM3>), dim3(uint32_t(a.n_items)), dim3(kWaves * 64),
                     0, stream, a);
  return check_hip(hipGetLastError(), "decode_mfma_kernel launch");
}

static constexpr uint64_t fbit(int fmt, int bits) { return uint64_t(1) << (fmt * 9 + bits); }

int launch_decode_mfma(const DecodeArgs& a, hipStream_t stream, bool* launched) {
  *launched = false;
  const dc_page_geometry& kg = a.kpool.geometry;
  const dc_page_geometry& vg = a.vpool.geometry;
  if (a.n_q > 8 || kg.layout != 0 || vg.layout != 0 || kg.group_size != 32) return DC_OK;
  if (kg.page_capacity % 32 != 0) return DC_OK;
  // formats present in the pools (bit = format * 9 + bits, as in dc_pool)
  const uint64_t km = a.kpool.format_mask, vm = a.vpool.format_mask;
  const uint64_t k_m3 = fbit(DC_FMT_M3_F16, 0), k_m0 = fbit(DC_FMT_M0_AFFINE, 4) | fbit(DC_FMT_M0_SYMMETRIC, 4);
  const uint64_t v4 = fbit(DC_FMT_M0_AFFINE, 4) | fbit(DC_FMT_M0_SYMMETRIC, 4);
  const uint64_t v8 = fbit(DC_FMT_M0_AFFINE, 8) | fbit(DC_FMT_M0_SYMMETRIC, 8);
  if (km == 0 || vm == 0 || (km & ~(k_m3 | k_m0)) || (vm & ~(k_m3 | v4 | v8))) return DC_OK;
  if ((vm & v4) && (vm & v8)) return DC_OK;  // one value code width per launch
  const int kmode = (km & k_m3) && (km & k_m0) ? KEYS_MIXED : (km & k_m3) ? KEYS_M3 : KEYS_M0;
  const int vbits = (vm & v8) ? 8 : 4;
  const bool vm3 = (vm & k_m3) != 0;
  const int hd = kg.head_dim, vgs = vg.group_size;
  int rc = -1;
  // specialised instantiations for common pools, a general one per shape otherwise
#define DC_EXACT(HD_, VGS_, KM_, VB_, VM3_)                                                          \
  if (rc < 0 && hd == HD_ && vgs == VGS_ && kmode == KM_ && vbits == VB_ && vm3 == VM3_) \
    rc = launch_t<HD_, VGS_, KM_, VB_, VM3_>(a, stream);
#define DC_GENERAL(HD_, VGS_, VB_) \
  if (rc < 0 && hd == HD_ && vgs == VGS_ && vbits == VB_) rc = launch_t<HD_, VGS_, KEYS_MIXED, VB_, true>(a, stream);
  DC_EXACT(64, 32, KEYS_M0, 4, false)
  DC_EXACT(128, 32, KEYS_M3, 4, false)
  DC_EXACT(128, 32, KEYS_M0, 4, false)
  DC_EXACT(128, 64, KEYS_MIXED, 8, false)
  DC_EXACT(128, 64, KEYS_M0, 8, false)
  DC_EXACT(256, 32, KEYS_M0, 4, false)
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

}  // namespace dc
