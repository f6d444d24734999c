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

constexpr int kWaves = 4;  // waves per workgroup; each walks its own pages of the work item

template <int HD, int VGS>
struct MfmaCfg {
  static constexpr int KG = HD / 32;       // key groups of 32 channels (= contraction steps of the score)
  static constexpr int VG = HD / VGS;      // value groups
  static constexpr int H = VGS / 16;       // mix column tiles per value group
  static constexpr int LPW4 = 128 / VGS;   // lanes sharing one 4-bit code word
  static constexpr int NACC = VG * H;      // = HD / 16 accumulator tiles
  static constexpr int NVR = HD / 32;      // 16-byte value-code pieces per lane per chunk (8-bit pages)
  static constexpr int NSW = (16 * (HD / 16) + 63) / 64;  // scale words per lane per chunk (<= 16 G words)
  // per-wave LDS: chunk staging -- value codes [VG][32][W] (W up to VGS / 4),
  // value scales / biases and key scales / biases transposed to
  // [group][32 tokens] fp16 -- later reused for the end-of-item rows
  static constexpr int VPAY = VG * 32 * (VGS / 4);
  static constexpr int VSC = VPAY, VBS = VSC + 16 * VG, KSC = VBS + 16 * VG, KBS = KSC + 16 * KG;
  static constexpr int STAGE = KBS + 16 * KG;
  static constexpr int ROWS = 16 * HD + 16 * VG;  // D rows of the mix + bias sums
  static constexpr int WAVE_WORDS = STAGE > ROWS ? STAGE : ROWS;
  static constexpr int LDS_WORDS = kWaves * WAVE_WORDS;
};

// Registers one chunk needs from HBM.  The next chunk's loads are issued
// into them as soon as the current chunk has consumed them (keys after its
// score, values after staging), so they are in flight during its mix.
template <int HD, int VGS>
struct ChunkRegs {
  using Cfg = MfmaCfg<HD, VGS>;
  u32x4 kr[2][Cfg::KG];     // key rows (M3: 8 fp16 per lane) or code words (M0: .x)
  u32x4 vr[Cfg::NVR];       // value code pieces, blob byte order
  uint32_t vs[Cfg::NSW], vb[Cfg::NSW], ks[Cfg::NSW], kbw[Cfg::NSW];  // scale / bias words
};

struct PageMeta {
  const uint8_t* kp;
  const uint8_t* vp;
  int T;           // tokens to read (0: skip the page)
  int kfmt, vfmt, vbits;
  int64_t kscale_off, kbias_off, vscale_off, vbias_off;
};

template <int HD, int VGS>
__global__ void __launch_bounds__(kWaves * 64, HD >= 256 ? 1 : 2) decode_mfma_kernel(DecodeArgs a) {
  using Cfg = MfmaCfg<HD, VGS>;
  using Regs = ChunkRegs<HD, VGS>;
  constexpr int KG = Cfg::KG, VG = Cfg::VG, H = Cfg::H, LPW4 = Cfg::LPW4;
  __shared__ uint32_t lds_all[Cfg::LDS_WORDS];
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));

  const dc_work_item it = a.items[blockIdx.x];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int r = lane & 15, kb = lane >> 4;
  const int nq = a.n_q;
  const int CAP = a.kpool.geometry.page_capacity;
  uint32_t* lds = lds_all + wave * Cfg::WAVE_WORDS;
  uint16_t* vsc = reinterpret_cast<uint16_t*>(lds + Cfg::VSC);
  uint16_t* vbs = reinterpret_cast<uint16_t*>(lds + Cfg::VBS);
  uint16_t* ksc = reinterpret_cast<uint16_t*>(lds + Cfg::KSC);
  uint16_t* kbs = reinterpret_cast<uint16_t*>(lds + Cfg::KBS);

  // ---- queries scaled by query_scale * log2(e); B fragments hi / residual ----
  const int64_t qbase = (int64_t(it.seq) * a.n_kv_heads + it.kv_head) * nq * HD;
  const float qmul = a.q_scale * kLog2e;
  Frag qhi[KG], qlo[KG];
  float qsum[KG];
#pragma unroll
  for (int g = 0; g < KG; ++g) {
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
      v[i] = r < nq ? load_value(a.queries, a.queries_dtype, qbase + int64_t(r) * HD + 32 * g + 8 * kb + i) * qmul : 0.f;
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      qhi[g].u[i] = pack_h2(v[2 * i], v[2 * i + 1]);
      qlo[g].u[i] = pack_h2(split_part(v[2 * i], true), split_part(v[2 * i + 1], true));
      s += v[2 * i] + v[2 * i + 1];
    }
    s += __shfl_xor(s, 16, 64);
    s += __shfl_xor(s, 32, 64);
    qsum[g] = s;  // sum over group g for head r
  }

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

  // ---- loads of one chunk into registers: keys, then values ----
  auto load_keys = [&](const PageMeta& m, int c0, Regs& R) {
    if (m.kfmt == DC_FMT_M3_F16) {
      const _Float16* K = reinterpret_cast<const _Float16*>(m.kp);
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int ta = c0 + 8 * (r >> 2) + 4 * hh + (r & 3);
#pragma unroll
        for (int g = 0; g < KG; ++g) R.kr[hh][g] = *reinterpret_cast<const u32x4*>(K + ta * HD + 32 * g + 8 * kb);
      }
    } else {
      const uint32_t* P = reinterpret_cast<const uint32_t*>(m.kp);
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int ta = c0 + 8 * (r >> 2) + 4 * hh + (r & 3);
#pragma unroll
        for (int g = 0; g < KG; ++g) R.kr[hh][g].x = P[(g * CAP + ta) * 4 + kb];
      }
      const uint32_t* S = reinterpret_cast<const uint32_t*>(m.kp + m.kscale_off) + c0 * KG / 2;
      const uint32_t* B = reinterpret_cast<const uint32_t*>(m.kp + m.kbias_off) + c0 * KG / 2;
#pragma unroll
      for (int k = 0; k < Cfg::NSW; ++k) {
        const int e = lane + 64 * k;
        if (e < 16 * KG) {
          R.ks[k] = S[e];
          if (m.kfmt == DC_FMT_M0_AFFINE) R.kbw[k] = B[e];
        }
      }
    }
  };
  auto load_values = [&](const PageMeta& m, int c0, Regs& R) {
    if (is_m0(m.vfmt)) {
      const int W = m.vbits == 8 ? VGS / 4 : VGS / 8;
      const int per_g = 8 * W;
      const u32x4* src = reinterpret_cast<const u32x4*>(m.vp);
#pragma unroll
      for (int k = 0; k < Cfg::NVR; ++k) {
        const int e = lane + 64 * k;
        if (e < VG * per_g) {
          const int g = e / per_g, piece = e - g * per_g;
          R.vr[k] = src[((g * CAP + c0) * W) / 4 + piece];
        }
      }
      const uint32_t* S = reinterpret_cast<const uint32_t*>(m.vp + m.vscale_off) + c0 * VG / 2;
      const uint32_t* B = reinterpret_cast<const uint32_t*>(m.vp + m.vbias_off) + c0 * VG / 2;
#pragma unroll
      for (int k = 0; k < Cfg::NSW; ++k) {
        const int e = lane + 64 * k;
        if (e < 16 * VG) {
          R.vs[k] = S[e];
          if (m.vfmt == DC_FMT_M0_AFFINE) R.vb[k] = B[e];
        }
      }
    }
  };

  // ---- registers -> this wave's LDS staging area ----
  auto stage_chunk = [&](const PageMeta& m, const Regs& R) {
    if (is_m0(m.vfmt)) {
      const int W = m.vbits == 8 ? VGS / 4 : VGS / 8;
      u32x4* dst = reinterpret_cast<u32x4*>(lds);
#pragma unroll
      for (int k = 0; k < Cfg::NVR; ++k) {
        const int e = lane + 64 * k;
        if (e < VG * 8 * W) dst[e] = R.vr[k];
      }
      // scale word e holds tokens / groups 2e and 2e + 1 of the [32][VG] array
#pragma unroll
      for (int k = 0; k < Cfg::NSW; ++k) {
        const int e = lane + 64 * k;
        if (e < 16 * VG) {
#pragma unroll
          for (int s = 0; s < 2; ++s) {
            const int hidx = 2 * e + s, t = hidx / VG, g = hidx - t * VG;
            vsc[g * 32 + t] = uint16_t(R.vs[k] >> (16 * s));
            if (m.vfmt == DC_FMT_M0_AFFINE) vbs[g * 32 + t] = uint16_t(R.vb[k] >> (16 * s));
          }
        }
      }
    }
    if (m.kfmt != DC_FMT_M3_F16) {
#pragma unroll
      for (int k = 0; k < Cfg::NSW; ++k) {
        const int e = lane + 64 * k;
        if (e < 16 * KG) {
#pragma unroll
          for (int s = 0; s < 2; ++s) {
            const int hidx = 2 * e + s, t = hidx / KG, g = hidx - t * KG;
            ksc[g * 32 + t] = uint16_t(R.ks[k] >> (16 * s));
            if (m.kfmt == DC_FMT_M0_AFFINE) kbs[g * 32 + t] = uint16_t(R.kbw[k] >> (16 * s));
          }
        }
      }
    }
  };

  // ---- score of one chunk: logits of this lane's chunk tokens 8 kb + e for head r ----
  auto score_chunk = [&](const PageMeta& m, const Regs& R, float* Ls) {
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      if (m.kfmt == DC_FMT_M3_F16) {
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
      } else {  // M0 4-bit, group 32: scale and bias applied per group in fp32
        const bool k_affine = m.kfmt == DC_FMT_M0_AFFINE;
        const float zp = k_affine ? 0.f : 7.f;
        // (1024 + n_lo, 1024 + 16 n_hi) -> (n_lo - zp, n_hi - zp)
        const h2 kmul = {(_Float16)1.f, (_Float16)0.0625f};
        const h2 kadd = {(_Float16)(-1024.f - zp), (_Float16)(-64.f - zp)};
        float Lh[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int g = 0; g < KG; ++g) {
          const uint32_t w = R.kr[hh][g].x;
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
          const uint2 bw = k_affine ? *reinterpret_cast<const uint2*>(kbs + g * 32 + 8 * kb + 4 * hh) : uint2{0u, 0u};
          const uint32_t sv[4] = {sw.x & 0xffffu, sw.x >> 16, sw.y & 0xffffu, sw.y >> 16};
          const uint32_t bv[4] = {bw.x & 0xffffu, bw.x >> 16, bw.y & 0xffffu, bw.y >> 16};
#pragma unroll
          for (int i = 0; i < 4; ++i) Lh[i] += h2f(sv[i]) * d[i] + h2f(bv[i]) * qsum[g];
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

    // mix: weights of this lane's A-row head on its 8 tokens
    float pa[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float v = __shfl(Ls[e], pa_src, 64);
      pa[e] = row_live ? v : 0.f;
    }
    if (is_m0(m.vfmt)) {
      const bool v_affine = m.vfmt == DC_FMT_M0_AFFINE;
      const int vbits = m.vbits;
      const int W = vbits == 8 ? VGS / 4 : VGS / 8;
      const float zp = v_affine ? 0.f : float((1 << (vbits - 1)) - 1);
      const uint32_t negb = h2_const(-1024.f - zp);
      const uint32_t nib_shift = 4u * uint32_t(jj & 1);
#pragma unroll
      for (int g = 0; g < VG; ++g) {
        const uint4 s8 = *reinterpret_cast<const uint4*>(vsc + g * 32 + 8 * kb);
        const uint32_t sx[4] = {s8.x, s8.y, s8.z, s8.w};
        Frag fa;
#pragma unroll
        for (int pp = 0; pp < 4; ++pp) {
          const float x0 = pa[2 * pp] * h2f(sx[pp] & 0xffffu);
          const float x1 = pa[2 * pp + 1] * h2f(sx[pp] >> 16);
          fa.u[pp] = pack_h2(split_part(x0, residual), split_part(x1, residual));
        }
        if (v_affine) {
          const uint4 b8 = *reinterpret_cast<const uint4*>(vbs + g * 32 + 8 * kb);
          const uint32_t bx[4] = {b8.x, b8.y, b8.z, b8.w};
#pragma unroll
          for (int pp = 0; pp < 4; ++pp)
            bsum[g] += Ls[2 * pp] * h2f(bx[pp] & 0xffffu) + Ls[2 * pp + 1] * h2f(bx[pp] >> 16);
        }
        const uint32_t* Pw = lds + (g * 32 + 8 * kb) * W;  // words of tokens 8 kb + e
#pragma unroll
        for (int h = 0; h < H; ++h) {
          Frag fb;
          if (vbits == 4) {
            const int nib = jj + LPW4 * h;  // low nibble of byte nib / 2 after the shift
            const uint32_t sel = 0x0c000c00u | uint32_t(nib >> 1) | (uint32_t(4 + (nib >> 1)) << 16);
#pragma unroll
            for (int pp = 0; pp < 4; ++pp) {
              const uint32_t w0 = Pw[(2 * pp) * W + w4] >> nib_shift;
              const uint32_t w1 = Pw[(2 * pp + 1) * W + w4] >> nib_shift;
              fb.u[pp] = magic_sub((__builtin_amdgcn_perm(w1, w0, sel) & 0x000f000fu) | 0x64006400u, negb);
            }
          } else {
            const int e8 = jj + LPW4 * h;  // channel dcol + LPW4 h = word 2 w4 + e8 / 4, byte e8 % 4
            const int wsel = 2 * w4 + (e8 >> 2);
            const uint32_t sel = 0x0c000c00u | uint32_t(e8 & 3) | (uint32_t(4 + (e8 & 3)) << 16);
#pragma unroll
            for (int pp = 0; pp < 4; ++pp) {
              const uint32_t w0 = Pw[(2 * pp) * W + wsel];
              const uint32_t w1 = Pw[(2 * pp + 1) * W + wsel];
              fb.u[pp] = magic_sub(__builtin_amdgcn_perm(w1, w0, sel) | 0x64006400u, negb);
            }
          }
          acc[g * H + h] = mfma(fa, fb, acc[g * H + h]);
        }
        // keep the scheduler from hoisting every group's LDS reads at once
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {  // M3 fp16 values (the exact recent window): gather columns from the rows
      const uint16_t* V = reinterpret_cast<const uint16_t*>(m.vp);
      Frag fa;
#pragma unroll
      for (int pp = 0; pp < 4; ++pp) fa.u[pp] = pack_h2(split_part(pa[2 * pp], residual), split_part(pa[2 * pp + 1], residual));
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
  for (int base = 0; base < np; base += 64) {
    const int nb = np - base < 64 ? np - base : 64;
    // lane i < nb holds the ids / descriptors of the wave's page base + i
    uint32_t k0 = 0, k1 = 0, v0 = 0, v1 = 0;
    int ok = 0;
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
      m.kscale_off = KL.scales_off;
      m.kbias_off = KL.bias_off;
      m.vscale_off = VL.scales_off;
      m.vbias_off = VL.bias_off;
      return m;
    };

    int i = 0;
    PageMeta cur = meta_of(0);
    while (i < nb && cur.T <= 0) {
      ++i;
      if (i < nb) cur = meta_of(i);
    }
    if (i >= nb) continue;
    int c0 = 0;
    Regs R;
    load_keys(cur, c0, R);
    load_values(cur, c0, R);
    while (true) {
      // next chunk of this batch, if any
      int ni = i, nc0 = c0 + 32;
      PageMeta nm = cur;
      if (nc0 >= cur.T) {
        nc0 = 0;
        do {
          ++ni;
          if (ni < nb) nm = meta_of(ni);
        } while (ni < nb && nm.T <= 0);
      }
      const bool more = ni < nb;
      stage_chunk(cur, R);  // value codes and scales -> LDS; frees their registers
      float Ls[8];
      score_chunk(cur, R, Ls);  // frees the key registers
      if (more) {  // the next chunk's loads fly while this one is mixed
        load_keys(nm, nc0, R);
        load_values(nm, nc0, R);
      }
      mix_chunk(cur, c0, Ls);
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

template <int HD, int VGS>
static int launch_t(const DecodeArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL((decode_mfma_kernel<HD, VGS>), dim3(uint32_t(a.n_items)), dim3(kWaves * 64), 0, stream, a);
  return check_hip(hipGetLastError(), "decode_mfma_kernel launch");
}

// Formats the fast path reads (bit = format * 9 + bits, as in dc_pool).
static constexpr uint64_t fbit(int fmt, int bits) { return uint64_t(1) << (fmt * 9 + bits); }

static bool fast_formats(uint64_t kmask, uint64_t vmask) {
  const uint64_t k_ok = fbit(DC_FMT_M3_F16, 0) | fbit(DC_FMT_M0_AFFINE, 4) | fbit(DC_FMT_M0_SYMMETRIC, 4);
  const uint64_t v_ok = k_ok | fbit(DC_FMT_M0_AFFINE, 8) | fbit(DC_FMT_M0_SYMMETRIC, 8);
  return kmask != 0 && vmask != 0 && (kmask & ~k_ok) == 0 && (vmask & ~v_ok) == 0;
}

int launch_decode_mfma(const DecodeArgs& a, hipStream_t stream, bool* launched) {
  *launched = false;
  const dc_page_geometry& kg = a.kpool.geometry;
  const dc_page_geometry& vg = a.vpool.geometry;
  if (a.n_q > 8 || kg.layout != 0 || vg.layout != 0 || kg.group_size != 32) return DC_OK;
  if (!fast_formats(a.kpool.format_mask, a.vpool.format_mask)) return DC_OK;
  const int hd = kg.head_dim, vgs = vg.group_size;
  if (kg.page_capacity % 32 != 0) return DC_OK;
  int rc = -1;
#define DC_TRY(HD_, VGS_) \
  if (hd == HD_ && vgs == VGS_) rc = launch_t<HD_, VGS_>(a, stream);
  DC_TRY(64, 32)
  DC_TRY(64, 64)
  DC_TRY(128, 32)
  DC_TRY(128, 64)
  DC_TRY(256, 32)
  DC_TRY(256, 64)
#undef DC_TRY
  if (rc < 0) return DC_OK;
  *launched = true;
  return rc;
}

}  // namespace dc
