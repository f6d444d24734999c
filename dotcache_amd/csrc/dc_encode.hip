// M0 / M3 page encode and token append (gfx950).
//
// Bit-exact with reference dotcache/modes/m0_affine.py:15-53 +
// dotcache/packing.py:14-48 + dotcache/encode.py:399-445: every step is one
// IEEE fp32 operation (subtract, correctly rounded divide, max), rintf
// rounds half to even like np.round, and scales / biases are rounded to fp16
// with RNE after the codes were computed from the fp32 scale.  This file is
// compiled with -ffp-contract=off so no step is fused.
//
// Two kernels:
//   encode_rows8_kernel (the fast path): 8 consecutive channels per lane,
//     a row on head_dim / 8 lanes and several rows per wavefront.  A lane
//     loads its channels with 16-byte loads, a group's min / max / max |x|
//     is a butterfly over the group's lanes, and a lane's 8 codes are one
//     word at 4 bits and two at 8 bits, stored as they are; 2- and 3-bit
//     words (which lanes share) are OR-ed together in LDS.  A code comes
//     from the reciprocal of its group's scale, and from the correctly
//     rounded division only where that could round differently
//     (rint_quotients8: the same bits, about 5 instead of 13 instructions
//     per code).  Taken when the
//     group size and head_dim are multiples of 8 and the padded head_dim / 8
//     and group size / 8 are powers of two (every configuration here).
//   encode_rows_kernel (the general path): one thread per (row, group),
//     for any other geometry.
#include "dc_common.h"

namespace dc {

__global__ void __launch_bounds__(256) encode_rows_kernel(const void* __restrict__ values, int32_t dtype,
                                                          int64_t n_rows, int64_t row_stride,
                                                          const int32_t* __restrict__ row_page,
                                                          const int32_t* __restrict__ row_slot, dc_pool pool,
                                                          int32_t G) {
  const int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= n_rows * G) return;
  const int64_t r = idx / G;
  const int32_t g = int32_t(idx - r * G);
  const int32_t pid = row_page[r];
  if (pid < 0 || pid >= pool.n_descs) return;
  const dc_page_desc d = pool.descs[pid];
  const dc_page_geometry geo = pool.geometry;
  const int32_t t = row_slot[r];
  if (t < 0 || t >= geo.page_capacity) return;
  const BlobLayout L = blob_layout(d.format, d.bits, geo);
  if ((int64_t(d.block) << 8) + L.total > pool.arena_bytes) return;
  uint8_t* blob = reinterpret_cast<uint8_t*>(pool.arena) + (uint64_t(d.block) << 8);
  const int64_t rb = r * row_stride;
  const int32_t gs = geo.group_size, hd = geo.head_dim, c0 = g * gs;

  if (is_m0(d.format)) {
    float lo = INFINITY, hi = -INFINITY, amax = 0.f;
    for (int32_t k = 0; k < gs; ++k) {
      const int32_t c = c0 + k;
      const float x = c < hd ? load_value(values, dtype, rb + c) : 0.f;  // zero padding joins min/max
      lo = fminf(lo, x);
      hi = fmaxf(hi, x);
      amax = fmaxf(amax, fabsf(x));
    }
    const int32_t bits = d.bits;
    const uint32_t top = (1u << bits) - 1u;
    float scale, offset;
    int32_t zero_point;
    if (d.format == DC_FMT_M0_AFFINE) {
      scale = fmaxf((hi - lo) / float(top), 1e-8f);
      offset = lo;
      zero_point = 0;
    } else {
      const int32_t qmax = (1 << (bits - 1)) - 1;
      scale = fmaxf(amax / float(qmax > 1 ? qmax : 1), 1e-8f);
      offset = 0.f;
      zero_point = qmax;
    }
    uint32_t* payload = reinterpret_cast<uint32_t*>(blob);
    const int64_t wbase =
        geo.layout == 0 ? (int64_t(g) * geo.page_capacity + t) * L.words : (int64_t(t) * G + g) * L.words;
    uint64_t acc = 0;
    int32_t nacc = 0, wi = 0;
    for (int32_t k = 0; k < gs; ++k) {
      const int32_t c = c0 + k;
      const float x = c < hd ? load_value(values, dtype, rb + c) : 0.f;
      uint32_t code;
      if (d.format == DC_FMT_M0_AFFINE) {
        const float q = rintf((x - offset) / scale);
        code = uint32_t(fminf(fmaxf(q, 0.f), float(top)));
      } else {
        const float qmaxf = float(zero_point);
        const float q = fminf(fmaxf(rintf(x / scale), -qmaxf), qmaxf);
        const int32_t sc = int32_t(q) + zero_point;
        code = uint32_t(sc < 0 ? 0 : (sc > int32_t(top) ? int32_t(top) : sc));
      }
      acc |= uint64_t(code) << nacc;
      nacc += bits;
      if (nacc >= 32) {
        payload[wbase + wi++] = uint32_t(acc);
        acc >>= 32;
        nacc -= 32;
      }
    }
    if (nacc > 0) payload[wbase + wi] = uint32_t(acc);
    reinterpret_cast<__half*>(blob + L.scales_off)[t * G + g] = __float2half_rn(scale);
    if (d.format == DC_FMT_M0_AFFINE) reinterpret_cast<__half*>(blob + L.bias_off)[t * G + g] = __float2half_rn(lo);
    return;
  }

  if (d.format == DC_FMT_M3_I8) {
    if (g != 0) return;  // the whole row shares one scale
    float amax = 0.f;
    for (int32_t c = 0; c < hd; ++c) amax = fmaxf(amax, fabsf(load_value(values, dtype, rb + c)));
    const __half s16 = __float2half_rn(fmaxf(amax / 127.0f, 1e-8f));
    const float s = __half2float(s16);
    int8_t* rows = reinterpret_cast<int8_t*>(blob);
    for (int32_t c = 0; c < hd; ++c) {
      const float q = fminf(fmaxf(rintf(load_value(values, dtype, rb + c) / s), -127.f), 127.f);
      rows[int64_t(t) * hd + c] = int8_t(q);
    }
    reinterpret_cast<__half*>(blob + L.scales_off)[t] = s16;
    return;
  }

  const int32_t c1 = c0 + gs < hd ? c0 + gs : hd;
  for (int32_t c = c0; c < c1; ++c) {
    const float x = load_value(values, dtype, rb + c);
    if (d.format == DC_FMT_M3_F16)
      reinterpret_cast<__half*>(blob)[int64_t(t) * hd + c] = __float2half_rn(x);
    else
      reinterpret_cast<float*>(blob)[int64_t(t) * hd + c] = x;
  }
}

// ---- fast path ---------------------------------------------------------

// One encode job: rows of `values` into (row_page[r], row_slot[r]) of `pool`.
struct EncodeJob {
  const void* values;
  const int32_t* row_page;
  const int32_t* row_slot;
  dc_pool pool;
};

constexpr int kEncThreads = 256;
// LDS words per wavefront for 2- / 3-bit packing
constexpr int kPackWords = 64;
typedef _Float16 enc_h2 __attribute__((ext_vector_type(2)));
// row blocks (kEncThreads / 64 wavefronts x one row per lane group) per
// workgroup of encode_rows8_kernel, their loads all in flight together
constexpr int kEncRowBlocks = 2;

// q[i] = rintf(d[i] / s) (the correctly rounded quotient, rounded half to
// even: the reference's np.round of an fp32 division) from a reciprocal.
// With rcp = v_rcp_f32(s), within 1 ulp (2^-23 relative) of 1 / s, the
// product y = d rcp (one more rounding, 2^-24) lies within |y| 2^-22 of
// fl(d / s) (whose own rounding adds the last 2^-24), so rint(y) =
// rint(fl(d / s)) unless a half-integer lies that close to y.  The nearest
// half-integer is |y - rint(y)| from 1/2 away; if any of the lane's 8
// values comes within twice that distance (|y - rint(y)| + |y| 2^-21 >=
// 1/2, one fma whose own rounding, 2^-24 relative, stays far inside the
// margin), or exact is set, all 8 take the correctly rounded division
// instead (a branch the lane rarely takes: for uniform data about |y|
// 2^-20 of the codes are that close; the empty asm keeps the compiler from
// running the divisions unconditionally).
__device__ __forceinline__ void rint_quotients8(const float (&d)[8], float s, float rcp, bool exact, float (&q)[8]) {
  float e = 0.f;  // the largest |y - rint(y)| + |y| 2^-21 of the 8
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float y = d[i] * rcp;
    q[i] = rintf(y);
    e = fmaxf(e, __builtin_fmaf(fabsf(y), 0x1p-21f, fabsf(y - q[i])));
  }
  if (exact || e >= 0.5f) {
    asm volatile("");
#pragma unroll
    for (int i = 0; i < 8; ++i) q[i] = rintf(d[i] / s);
  }
}

__device__ __forceinline__ float seg_min(float v, int lanes) {
  for (int o = 1; o < lanes; o <<= 1) v = fminf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float seg_max(float v, int lanes) {
  for (int o = 1; o < lanes; o <<= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// Eight consecutive values of row r from channel c0 (dtype DC_F32 / F16 /
// BF16); vec: the row start is 16-byte aligned for this dtype.
template <int32_t dtype, bool vec>
__device__ __forceinline__ void load8(const void* values, int64_t off, float* x) {
  if constexpr (dtype == DC_F32) {
    const float* p = reinterpret_cast<const float*>(values) + off;
    if constexpr (vec) {
      const float4 a = *reinterpret_cast<const float4*>(p), b = *reinterpret_cast<const float4*>(p + 4);
      x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
      return;
    }
  } else if constexpr (vec) {
    const uint4 u = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(values) + off);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (dtype == DC_F16) {
        x[2 * i] = __half2float(__ushort_as_half(uint16_t(w[i] & 0xffffu)));
        x[2 * i + 1] = __half2float(__ushort_as_half(uint16_t(w[i] >> 16)));
      } else {
        x[2 * i] = __uint_as_float(w[i] << 16);
        x[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
      }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = load_value(values, dtype, off + i);
}

// One row's part of encode_rows8_kernel: lane (q, rw) encodes channels
// c0 .. c0 + 7 of the row into slot t of the page d describes.
__device__ __forceinline__ void encode_row(const EncodeJob& J, const float (&x)[8], int32_t t, const dc_page_desc& d,
                                           bool live, uint32_t (*pack)[kPackWords], int32_t lds_pack, int lane,
                                           int wave, int q, int rw, int32_t c0, int32_t g, int32_t li, int lpr,
                                           int lpg) {
  const dc_page_geometry geo = J.pool.geometry;
  const int32_t hd = geo.head_dim, gs = geo.group_size, C = geo.page_capacity;
  const int32_t G = (hd + gs - 1) / gs;
  const BlobLayout L = blob_layout(d.format, d.bits, geo);
  live = live && (int64_t(d.block) << 8) + L.total <= J.pool.arena_bytes;
  uint8_t* blob = reinterpret_cast<uint8_t*>(J.pool.arena) + (uint64_t(d.block) << 8);

  const bool m0 = live && is_m0(d.format);
  uint32_t w0 = 0, w1 = 0;  // this lane's code bits (8 codes, little-endian)
  const int bits = d.bits;
  if (m0) {
    const bool affine = d.format == DC_FMT_M0_AFFINE;
    // the group's min and max (affine) or max |x| (symmetric), over its lanes
    float lo = 0.f, hi = 0.f, am = 0.f;
    if (affine) {
      lo = x[0];
      hi = x[0];
#pragma unroll
      for (int i = 1; i < 8; ++i) {
        lo = fminf(lo, x[i]);
        hi = fmaxf(hi, x[i]);
      }
      lo = seg_min(lo, lpg);
      hi = seg_max(hi, lpg);
    } else {
      am = fabsf(x[0]);
#pragma unroll
      for (int i = 1; i < 8; ++i) am = fmaxf(am, fabsf(x[i]));
      am = seg_max(am, lpg);
    }
    const uint32_t top = (1u << bits) - 1u;
    const int32_t qmax = (1 << (bits - 1)) - 1;
    const float scale = affine ? fmaxf((hi - lo) / float(top), 1e-8f) : fmaxf(am / float(qmax > 1 ? qmax : 1), 1e-8f);
    float dv[8], qq[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) dv[i] = affine ? x[i] - lo : x[i];
    // (scale >= 1e-8: normal, and so is its reciprocal)
    rint_quotients8(dv, scale, __builtin_amdgcn_rcpf(scale), false, qq);
    if (bits >= 4) {
      // 4- and 8-bit codes as bytes (v_cvt_pk_u8_f32 of exact integers),
      // then 4-bit pairs into nibbles.  The reference's clip never binds
      // here: d <= fl(hi - lo) and s >= fl(hi - lo) / top (1 - 2^-24) keep
      // y below top (1 + 2^-21) < top + 1/2, and |x| <= max|x| keeps |y|
      // below qmax + 1/2 (a floored scale only makes y smaller), so
      // rint(y) is in [0, top] (affine) or [-qmax, qmax] (symmetric).
      const float zp = affine ? 0.f : float(qmax);
      uint32_t lo4 = 0, hi4 = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        lo4 = __builtin_amdgcn_cvt_pk_u8_f32(qq[i] + zp, uint32_t(i), lo4);
        hi4 = __builtin_amdgcn_cvt_pk_u8_f32(qq[i + 4] + zp, uint32_t(i), hi4);
      }
      if (bits == 8) {
        w0 = lo4;
        w1 = hi4;
      } else {
        // byte 2j of (b | b >> 4) is code 2j | code 2j+1 << 4
        w0 = __builtin_amdgcn_perm(hi4 | (hi4 >> 4), lo4 | (lo4 >> 4), 0x06040200u);
      }
    } else {
      uint64_t acc = 0;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        uint32_t code;
        const float qv = qq[i];
        if (affine) {
          code = uint32_t(fminf(fmaxf(qv, 0.f), float(top)));
        } else {
          const float qc = fminf(fmaxf(qv, -float(qmax)), float(qmax));
          const int32_t sc = int32_t(qc) + qmax;
          code = uint32_t(sc < 0 ? 0 : (sc > int32_t(top) ? int32_t(top) : sc));
        }
        acc |= uint64_t(code) << (i * bits);
      }
      w0 = uint32_t(acc);
      w1 = uint32_t(acc >> 32);
    }
    uint32_t* payload = reinterpret_cast<uint32_t*>(blob);
    const int64_t wb = geo.layout == 0 ? (int64_t(g) * C + t) * L.words : (int64_t(t) * G + g) * L.words;
    if (bits == 4) {
      payload[wb + li] = w0;
    } else if (bits == 8) {
      *reinterpret_cast<uint2*>(payload + wb + 2 * li) = uint2{w0, w1};
    }
    if (li == 0) {
      reinterpret_cast<__half*>(blob + L.scales_off)[t * G + g] = __float2half_rn(scale);
      if (affine) reinterpret_cast<__half*>(blob + L.bias_off)[t * G + g] = __float2half_rn(lo);
    }
  } else if (live && c0 < hd) {
    const int64_t e = int64_t(t) * hd + c0;
    if (d.format == DC_FMT_M3_F16) {
      uint32_t h[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)  // (one v_cvt_pk_f16_f32 per pair, round to nearest even)
        h[i] = __builtin_bit_cast(uint32_t, enc_h2{(_Float16)x[2 * i], (_Float16)x[2 * i + 1]});
      *reinterpret_cast<uint4*>(reinterpret_cast<__half*>(blob) + e) = uint4{h[0], h[1], h[2], h[3]};
    } else if (d.format == DC_FMT_M3_F32) {
      float* o = reinterpret_cast<float*>(blob) + e;
      *reinterpret_cast<float4*>(o) = float4{x[0], x[1], x[2], x[3]};
      *reinterpret_cast<float4*>(o + 4) = float4{x[4], x[5], x[6], x[7]};
    }
  }
  if (live && d.format == DC_FMT_M3_I8) {  // one fp16 scale for the whole row
    float am = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) am = fmaxf(am, fabsf(x[i]));
    am = seg_max(am, lpr);
    const __half s16 = __float2half_rn(fmaxf(am / 127.0f, 1e-8f));
    const float sv = __half2float(s16);
    if (c0 < hd) {
      uint32_t b[2] = {0u, 0u};
      // (sv may be 0: fp16 flushes 1e-8 to zero, and x / 0 must give the
      // reference's +-inf / nan, so that row takes the division)
      float qq[8];
      rint_quotients8(x, sv, __builtin_amdgcn_rcpf(sv), !(sv > 0.f), qq);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float qv = fminf(fmaxf(qq[i], -127.f), 127.f);
        b[i >> 2] |= (uint32_t(int32_t(qv)) & 0xffu) << (8 * (i & 3));
      }
      *reinterpret_cast<uint2*>(blob + int64_t(t) * hd + c0) = uint2{b[0], b[1]};
    }
    if (q == 0) reinterpret_cast<__half*>(blob + L.scales_off)[t] = s16;
  }
  if (!lds_pack) return;  // uniform: no 2- / 3-bit pages in this launch's pools

  // 2- and 3-bit codes: a lane's 8 codes (16 or 24 bits) start at bit
  // 8 bits li of its group's words and may share words with the next lane;
  // OR them into the wavefront's LDS words, then store whole words
  const bool narrow = m0 && bits < 4;
  const int wpr = G * L.words;  // words of one row (the same for every narrow row of this job)
  for (int i = lane; i < kPackWords; i += 64) pack[wave][i] = 0u;
  __syncthreads();
  if (narrow) {
    const int bit = 8 * bits * li, wi = bit >> 5, off = bit & 31;
    uint32_t* rowp = pack[wave] + rw * wpr + g * L.words;
    atomicOr(rowp + wi, w0 << off);
    if (off + 8 * bits > 32) atomicOr(rowp + wi + 1, w0 >> (32 - off));
  }
  __syncthreads();
  if (narrow && li == 0) {
    uint32_t* payload = reinterpret_cast<uint32_t*>(blob);
    const int64_t wb = geo.layout == 0 ? (int64_t(g) * C + t) * L.words : (int64_t(t) * G + g) * L.words;
    for (int w = 0; w < L.words; ++w) payload[wb + w] = pack[wave][rw * wpr + g * L.words + w];
  }
}

// blockIdx.y selects the job (K rows, V rows).  Row r of the job is handled
// by lanes [lpr * (r % rpw), ...) of wavefront r / rpw, lpr = padded
// head_dim / 8 lanes per row, rpw = 64 / lpr rows per wavefront.
// (Measured on the bulk encode of a C3 layer, 708.8 MB per launch: walking
// several row blocks per wavefront with the next block's loads in flight
// took 202 us, and giving each XCD one contiguous slice of the rows 220 us,
// against 170 us for one row block per wavefront in launch order.)
template <int32_t dtype, bool vec>
__global__ void __launch_bounds__(kEncThreads) encode_rows8_kernel(EncodeJob j0, EncodeJob j1, int64_t n_rows,
                                                                   int64_t row_stride, int32_t lds_pack) {
  __shared__ uint32_t pack[kEncThreads / 64][kPackWords];
  const EncodeJob J = blockIdx.y == 0 ? j0 : j1;
  const dc_page_geometry geo = J.pool.geometry;
  const int32_t hd = geo.head_dim, gs = geo.group_size, C = geo.page_capacity;
  const int32_t G = (hd + gs - 1) / gs, Gp = G * gs;
  const int lpr = Gp / 8, lpg = gs / 8, rpw = 64 / lpr;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int q = lane % lpr, rw = lane / lpr;  // lane within its row, row within the wavefront
  const int32_t c0 = 8 * q, g = c0 / gs, li = (c0 - g * gs) / 8;

  // The workgroup's kEncRowBlocks row blocks: every row's page, slot and
  // values in one round of loads, from a clamped row and channel so that no
  // load waits on a branch (the values array has n_rows >= 1 rows, hd is a
  // multiple of 8), then the pages' descriptors (a clamped id:
  // J.pool.n_descs >= 1): two dependent rounds, with kEncRowBlocks rows'
  // loads in flight per lane.  Rows that do not exist or name no valid
  // destination stay idle (they still reach the block barriers).
  int32_t pid[kEncRowBlocks], ts[kEncRowBlocks];
  float xs[kEncRowBlocks][8];
  bool ok[kEncRowBlocks];
#pragma unroll
  for (int u = 0; u < kEncRowBlocks; ++u) {
    const int64_t r = ((int64_t(blockIdx.x) * kEncRowBlocks + u) * (kEncThreads / 64) + wave) * rpw + rw;
    const bool in_rows = rw < rpw && r < n_rows;
    const int64_t rr = in_rows ? r : 0;
    pid[u] = J.row_page[rr];
    ts[u] = J.row_slot[rr];
    float y[8];
    load8<dtype, vec>(J.values, rr * row_stride + (c0 < hd ? c0 : 0), y);
    const bool has = in_rows && c0 < hd;  // channels past hd: zero padding
#pragma unroll
    for (int i = 0; i < 8; ++i) xs[u][i] = has ? y[i] : 0.f;
    ok[u] = in_rows;
  }
  dc_page_desc ds[kEncRowBlocks];
#pragma unroll
  for (int u = 0; u < kEncRowBlocks; ++u) {
    ok[u] = ok[u] && pid[u] >= 0 && pid[u] < J.pool.n_descs && ts[u] >= 0 && ts[u] < C;
    ds[u] = J.pool.descs[ok[u] ? pid[u] : 0];
  }
#pragma unroll
  for (int u = 0; u < kEncRowBlocks; ++u) encode_row(J, xs[u], ts[u], ds[u], ok[u], pack, lds_pack, lane, wave, q,
                                                     rw, c0, g, li, lpr, lpg);
}

// Whether a pool's geometry fits encode_rows8_kernel: 8-channel lanes that
// tile its groups and rows within one wavefront, and (2-/3-bit pages) the
// wavefront's packed words within its LDS share.
static bool fits_rows8(const dc_page_geometry& g) {
  const int32_t G = num_groups(g), Gp = G * g.group_size;
  auto pow2 = [](int32_t v) { return v > 0 && (v & (v - 1)) == 0; };
  if (g.head_dim % 8 || g.group_size % 8 || !pow2(g.group_size / 8) || !pow2(Gp / 8) || Gp / 8 > 64) return false;
  // narrow packing: rows per wavefront x words per row <= kPackWords
  const int32_t rpw = 64 / (Gp / 8);
  return int64_t(rpw) * G * words_per_group(g.group_size, 3) <= kPackWords;
}

static bool has_narrow(const dc_pool& p) {
  const uint64_t narrow = (uint64_t(1) << (DC_FMT_M0_AFFINE * 9 + 2)) | (uint64_t(1) << (DC_FMT_M0_AFFINE * 9 + 3)) |
                          (uint64_t(1) << (DC_FMT_M0_SYMMETRIC * 9 + 2)) |
                          (uint64_t(1) << (DC_FMT_M0_SYMMETRIC * 9 + 3));
  return p.format_mask == 0 || (p.format_mask & narrow) != 0;
}

static int g_encode_path = 0;  // 0: fast kernel where it fits; 1: general kernel only

static int encode_launch(const EncodeJob* jobs, int n_jobs, int32_t dtype, int64_t n_rows, int64_t row_stride,
                         hipStream_t stream) {
  // the fast kernel for every job whose geometry fits it, in one launch
  bool fast[2] = {false, false};
  int32_t rows_per_block = 1 << 30;
  bool vec = true, narrow = false;
  const int esize = dtype == DC_F32 ? 4 : 2;
  for (int i = 0; i < n_jobs; ++i) {
    fast[i] = g_encode_path == 0 && fits_rows8(jobs[i].pool.geometry);
    if (!fast[i]) continue;
    const dc_page_geometry& g = jobs[i].pool.geometry;
    const int32_t lpr = num_groups(g) * g.group_size / 8;
    rows_per_block = rows_per_block < (kEncThreads / lpr) ? rows_per_block : kEncThreads / lpr;
    vec = vec && (reinterpret_cast<uintptr_t>(jobs[i].values) % 16 == 0) && (row_stride * esize) % 16 == 0;
    narrow = narrow || has_narrow(jobs[i].pool);
  }
  const bool all_fast = fast[0] && (n_jobs < 2 || fast[1]);
  if (fast[0] || (n_jobs > 1 && fast[1])) {
    const int64_t blocks = (n_rows + int64_t(rows_per_block) * kEncRowBlocks - 1) / (int64_t(rows_per_block) * kEncRowBlocks);
    if (blocks > 0x7fffffff) return fail(DC_EINVAL, "too many rows");
    // (one instance per input dtype and alignment: the loads carry no branch)
    const EncodeJob& a = all_fast ? jobs[0] : (fast[0] ? jobs[0] : jobs[1]);
    const EncodeJob& b = all_fast && n_jobs > 1 ? jobs[1] : a;
    const dim3 grid(uint32_t(blocks), all_fast ? uint32_t(n_jobs) : 1u);
#define DC_ENC8(DT_, VEC_)                                                                                     \
  hipLaunchKernelGGL((encode_rows8_kernel<DT_, VEC_>), grid, dim3(kEncThreads), 0, stream, a, b, n_rows, row_stride, \
                     int32_t(narrow))
    if (dtype == DC_F32 && vec)
      DC_ENC8(DC_F32, true);
    else if (dtype == DC_F32)
      DC_ENC8(DC_F32, false);
    else if (dtype == DC_F16 && vec)
      DC_ENC8(DC_F16, true);
    else if (dtype == DC_F16)
      DC_ENC8(DC_F16, false);
    else if (vec)
      DC_ENC8(DC_BF16, true);
    else
      DC_ENC8(DC_BF16, false);
#undef DC_ENC8
    if (int rc = check_hip(hipGetLastError(), "encode_rows8_kernel launch")) return rc;
  }
  for (int i = 0; i < n_jobs; ++i) {
    if (fast[i]) continue;
    const int32_t G = num_groups(jobs[i].pool.geometry);
    const int64_t blocks = (n_rows * G + 255) / 256;
    if (blocks > 0x7fffffff) return fail(DC_EINVAL, "too many rows");
    hipLaunchKernelGGL(encode_rows_kernel, dim3(uint32_t(blocks)), dim3(256), 0, stream, jobs[i].values, dtype, n_rows,
                       row_stride, jobs[i].row_page, jobs[i].row_slot, jobs[i].pool, G);
    if (int rc = check_hip(hipGetLastError(), "encode_rows_kernel launch")) return rc;
  }
  return DC_OK;
}

static int check_encode_args(const void* values, int32_t dtype, int64_t n_rows, int64_t row_stride,
                             const int32_t* row_page, const int32_t* row_slot, const dc_pool& pool, const char* who) {
  if (int rc = validate_geometry(pool.geometry)) return rc;
  if (!values || !row_page || !row_slot || !pool.arena || !pool.descs) return fail(DC_EINVAL, "%s: null pointer", who);
  if (pool.n_descs <= 0) return fail(DC_EINVAL, "%s: the pool has no pages to write rows into", who);
  if (row_stride < pool.geometry.head_dim) return fail(DC_EINVAL, "%s: row_stride is smaller than head_dim", who);
  return DC_OK;
}

}  // namespace dc

extern "C" int dc_encode_rows_kv(const void* k_values, const void* v_values, int32_t values_dtype, int64_t n_rows,
                                 int64_t row_stride, const int32_t* k_row_page, const int32_t* k_row_slot,
                                 const int32_t* v_row_page, const int32_t* v_row_slot, dc_pool k_pool, dc_pool v_pool,
                                 dc_stream_t stream) {
  if (n_rows < 0) return dc::fail(DC_EINVAL, "n_rows must be non-negative");
  if (values_dtype != DC_F32 && values_dtype != DC_F16 && values_dtype != DC_BF16)
    return dc::fail(DC_EINVAL, "values_dtype must be DC_F32, DC_F16 or DC_BF16");
  if (n_rows == 0) return DC_OK;
  if (int rc = dc::check_encode_args(k_values, values_dtype, n_rows, row_stride, k_row_page, k_row_slot, k_pool,
                                     "dc_encode_rows_kv (keys)"))
    return rc;
  if (int rc = dc::check_encode_args(v_values, values_dtype, n_rows, row_stride, v_row_page, v_row_slot, v_pool,
                                     "dc_encode_rows_kv (values)"))
    return rc;
  const dc::EncodeJob jobs[2] = {{k_values, k_row_page, k_row_slot, k_pool}, {v_values, v_row_page, v_row_slot, v_pool}};
  return dc::encode_launch(jobs, 2, values_dtype, n_rows, row_stride, hipStream_t(stream));
}

extern "C" int dc_encode_rows(const void* values, int32_t values_dtype, int64_t n_rows, int64_t row_stride,
                              const int32_t* row_page, const int32_t* row_slot, dc_pool pool,
                              dc_stream_t stream) {
  if (int rc = dc::validate_geometry(pool.geometry)) return rc;
  if (n_rows < 0) return dc::fail(DC_EINVAL, "n_rows must be non-negative");
  if (n_rows == 0) return DC_OK;
  if (values_dtype != DC_F32 && values_dtype != DC_F16 && values_dtype != DC_BF16)
    return dc::fail(DC_EINVAL, "values_dtype must be DC_F32, DC_F16 or DC_BF16");
  if (int rc = dc::check_encode_args(values, values_dtype, n_rows, row_stride, row_page, row_slot, pool,
                                     "dc_encode_rows"))
    return rc;
  const dc::EncodeJob job{values, row_page, row_slot, pool};
  return dc::encode_launch(&job, 1, values_dtype, n_rows, row_stride, hipStream_t(stream));
}

// Process-wide encode kernel choice (0: the fast kernel where it fits, 1:
// the general kernel only), for cross-checking the two.
extern "C" int dc_set_encode_path(int32_t path) {
  if (path < 0 || path > 1) return dc::fail(DC_EINVAL, "encode path must be 0 (auto) or 1 (general)");
  dc::g_encode_path = path;
  return DC_OK;
}
