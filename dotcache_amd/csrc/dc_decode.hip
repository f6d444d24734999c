// Fused paged decode: score -> single-pass online softmax -> mix, straight
// from compressed pages, plus the split-K log-sum-exp merge.
//
// This file holds the generic path, which reads every page format the pool
// can hold (M0 affine / symmetric 2/3/4/8-bit, any group size, both layouts;
// M3 fp16 / fp32 / int8) and up to kMaxQ GQA query heads per KV head.  The
// MFMA fast path for the common formats lives in dc_decode_mfma.hip and is
// chosen by dc_decode_paged when every page of the call fits it.
//
// Semantics: reference dotcache/attention_runtime.py:260-315 (concatenate
// page logits, one softmax over the whole context, mix every value page)
// computed as the online softmax of reference
// dotcache/backends/torch_mps.py:4331-4435 (running max m, running sum l,
// rescale by exp(m_old - m_new), divide at the end).  Exponentials are
// taken base 2 on logits pre-multiplied by log2(e).
#include "dc_common.h"
#include "dc_decode.h"

namespace dc {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kMaxHD = 256;
constexpr int kTokChunk = 64;
constexpr int kParts = kThreads / kTokChunk;  // channel partitions in the score phase
constexpr int kMaxGroups = 64;

__device__ __forceinline__ float score_partial_m0(const uint8_t* blob, const dc_page_desc& d, const BlobLayout& L,
                                                  const dc_page_geometry& geo, int32_t t, int32_t part,
                                                  const float* __restrict__ qs, const float* __restrict__ qsum,
                                                  int32_t phd, int32_t nq, float* acc) {
  const uint32_t* payload = reinterpret_cast<const uint32_t*>(blob);
  const __half* sc = reinterpret_cast<const __half*>(blob + L.scales_off);
  const __half* bs = reinterpret_cast<const __half*>(blob + L.bias_off);
  const int32_t G = L.groups, gs = geo.group_size;
  const float zp = float((1 << (d.bits - 1)) - 1);
  for (int32_t g = part; g < G; g += kParts) {
    float dot[kMaxQ];
#pragma unroll
    for (int j = 0; j < kMaxQ; ++j) dot[j] = 0.f;
    for (int32_t k = 0; k < gs; ++k) {
      float code = float(m0_code(payload, t, g, k, d.bits, L.words, G, geo.page_capacity, geo.layout));
      if (d.format == DC_FMT_M0_SYMMETRIC) code -= zp;
      const int32_t c = g * gs + k;
#pragma unroll
      for (int j = 0; j < kMaxQ; ++j)
        if (j < nq) dot[j] += code * qs[j * phd + c];
    }
    const float s = __half2float(sc[t * G + g]);
    const float b = d.format == DC_FMT_M0_AFFINE ? __half2float(bs[t * G + g]) : 0.f;
#pragma unroll
    for (int j = 0; j < kMaxQ; ++j)
      if (j < nq) acc[j] += s * dot[j] + b * qsum[j * G + g];
  }
  return 0.f;
}

__global__ void __launch_bounds__(kThreads) decode_generic_kernel(DecodeArgs a) {
  const dc_work_item it = a.items[blockIdx.x];
  if (!item_in_bounds(it, a)) return;
  const dc_page_geometry geo = a.kpool.geometry, vgeo = a.vpool.geometry;
  const int32_t hd = geo.head_dim, gs = geo.group_size;
  const int32_t G = (hd + gs - 1) / gs, phd = G * gs;
  const int32_t nq = a.n_q;
  const int32_t tid = threadIdx.x;

  __shared__ float qs[kMaxQ * kMaxHD];        // scaled queries, zero padded to phd
  __shared__ float qsum[kMaxQ * kMaxGroups];  // per-group query sums
  __shared__ float red[kParts][kMaxQ][kTokChunk];
  __shared__ float prob[kMaxQ][kMaxCap];
  __shared__ float m_run[kMaxQ], l_run[kMaxQ], alpha[kMaxQ];

  // queries: [seq, kv_head, q, hd]
  const int64_t qbase = (int64_t(it.seq) * a.n_kv_heads + it.kv_head) * nq * hd;
  for (int32_t i = tid; i < nq * phd; i += kThreads) {
    const int32_t j = i / phd, c = i - j * phd;
    qs[j * phd + c] = c < hd ? load_value(a.queries, a.queries_dtype, qbase + int64_t(j) * hd + c) * a.q_scale : 0.f;
  }
  __syncthreads();
  for (int32_t i = tid; i < nq * G; i += kThreads) {
    const int32_t j = i / G, g = i - j * G;
    float s = 0.f;
    for (int32_t k = 0; k < gs; ++k) s += qs[j * phd + g * gs + k];
    qsum[j * G + g] = s;
  }
  if (tid < kMaxQ) {
    m_run[tid] = -INFINITY;
    l_run[tid] = 0.f;
    alpha[tid] = 1.f;
  }
  float acc[kMaxQ];
#pragma unroll
  for (int j = 0; j < kMaxQ; ++j) acc[j] = 0.f;
  __syncthreads();

  const int64_t trow = (int64_t(it.seq) * a.n_kv_heads + it.kv_head) * a.table_stride;
  for (int32_t p = it.page_begin; p < it.page_end; ++p) {
    const int32_t kid = a.k_table[trow + p], vid = a.v_table[trow + p];
    if (kid < 0 || kid >= a.kpool.n_descs || vid < 0 || vid >= a.vpool.n_descs) continue;
    const dc_page_desc kd = a.kpool.descs[kid], vd = a.vpool.descs[vid];
    const BlobLayout KL = blob_layout(kd.format, kd.bits, geo), VL = blob_layout(vd.format, vd.bits, vgeo);
    if ((int64_t(kd.block) << 8) + KL.total > a.kpool.arena_bytes) continue;
    if ((int64_t(vd.block) << 8) + VL.total > a.vpool.arena_bytes) continue;
    int32_t T = kd.tokens < vd.tokens ? kd.tokens : vd.tokens;
    if (T > geo.page_capacity) T = geo.page_capacity;
    // the item's tokens of this page, [tl, tl + Tn): it may start and end
    // inside a page, on 32-token chunk boundaries
    const int32_t tl = p == it.page_begin ? 32 * it.chunk_begin : 0;
    const int32_t th = p == it.page_end - 1 && it.chunk_end > 0 ? min(T, 32 * it.chunk_end) : T;
    const int32_t Tn = th - tl;
    if (Tn <= 0) continue;
    const uint8_t* kb = blob_ptr(a.kpool.arena, kd);
    const uint8_t* vb = blob_ptr(a.vpool.arena, vd);

    // ---- score: thread (token, part); parts split the channels ----
    for (int32_t t0 = 0; t0 < Tn; t0 += kTokChunk) {
      const int32_t t = t0 + (tid % kTokChunk), part = tid / kTokChunk;
      float s[kMaxQ];
#pragma unroll
      for (int j = 0; j < kMaxQ; ++j) s[j] = 0.f;
      if (t < Tn) {
        if (is_m0(kd.format)) {
          score_partial_m0(kb, kd, KL, geo, t + tl, part, qs, qsum, phd, nq, s);
        } else {
          for (int32_t c = part; c < hd; c += kParts) {
            const float v = page_value(kb, kd, KL, geo, t + tl, c);
#pragma unroll
            for (int j = 0; j < kMaxQ; ++j)
              if (j < nq) s[j] += v * qs[j * phd + c];
          }
        }
      }
#pragma unroll
      for (int j = 0; j < kMaxQ; ++j) red[part][j][tid % kTokChunk] = s[j];
      __syncthreads();
      for (int32_t i = tid; i < nq * kTokChunk; i += kThreads) {
        const int32_t j = i / kTokChunk, tt = i - j * kTokChunk;
        if (t0 + tt < Tn) prob[j][t0 + tt] = (red[0][j][tt] + red[1][j][tt] + red[2][j][tt] + red[3][j][tt]) * kLog2e;
      }
      __syncthreads();
    }

    // ---- online softmax: one wave per query head ----
    const int32_t wave = tid / 64, lane = tid % 64;
    for (int32_t j = wave; j < nq; j += kThreads / 64) {
      float mx = -INFINITY;
      for (int32_t t = lane; t < Tn; t += 64) mx = fmaxf(mx, prob[j][t]);
      mx = wave_max(mx);
      const float m_old = m_run[j];
      const float m_new = fmaxf(m_old, mx);
      float sum = 0.f;
      for (int32_t t = lane; t < Tn; t += 64) {
        const float e = exp2f(prob[j][t] - m_new);
        prob[j][t] = e;
        sum += e;
      }
      sum = wave_sum(sum);
      if (lane == 0) {
        const float al = exp2f(m_old - m_new);
        alpha[j] = al;
        l_run[j] = l_run[j] * al + sum;
        m_run[j] = m_new;
      }
    }
    __syncthreads();

    // ---- mix: one thread per channel (hd <= kThreads is checked on the host) ----
    if (tid < hd) {
      const int32_t c = tid;
#pragma unroll
      for (int j = 0; j < kMaxQ; ++j) acc[j] *= alpha[j];
      for (int32_t t = 0; t < Tn; ++t) {
        const float v = page_value(vb, vd, VL, vgeo, t + tl, c);
#pragma unroll
        for (int j = 0; j < kMaxQ; ++j)
          if (j < nq) acc[j] += prob[j][t] * v;
      }
    }
    __syncthreads();
  }

  // ---- write the normalised output or a split-K partial ----
  if (it.partial >= a.max_partials) return;
  if (tid < hd) {
    if (it.partial < 0) {
      float* o = a.out + qbase + tid;
#pragma unroll
      for (int j = 0; j < kMaxQ; ++j)
        if (j < nq) o[int64_t(j) * hd] = acc[j] / fmaxf(l_run[j], 1e-30f);
    } else {
      float* o = a.part_o + int64_t(it.partial) * nq * hd + tid;
#pragma unroll
      for (int j = 0; j < kMaxQ; ++j)
        if (j < nq) o[int64_t(j) * hd] = acc[j];
    }
  }
  if (it.partial >= 0 && tid < nq) {
    a.part_ml[(int64_t(it.partial) * nq + tid) * 2 + 0] = m_run[tid];
    a.part_ml[(int64_t(it.partial) * nq + tid) * 2 + 1] = l_run[tid];
  }
}

// The raw words of eight query values q[i .. i + 7] (i a multiple of 8):
// two 16-byte pieces for fp32, one (w[0]) for fp16 / bf16.  Converted
// apart (q8_floats), so that the load does not wait on the dtype's branch.
__device__ __forceinline__ void load_q8_raw(const void* q, int32_t dtype, int64_t i, uint4* w) {
  if (dtype == DC_F32) {
    const uint4* p = reinterpret_cast<const uint4*>(reinterpret_cast<const float*>(q) + i);
    w[0] = p[0];
    w[1] = p[1];
  } else {
    w[0] = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(q) + i);
    w[1] = uint4{0u, 0u, 0u, 0u};
  }
}

__device__ __forceinline__ void q8_floats(const uint4* w, int32_t dtype, float* o) {
  if (dtype == DC_F32) {
    const uint32_t a[8] = {w[0].x, w[0].y, w[0].z, w[0].w, w[1].x, w[1].y, w[1].z, w[1].w};
#pragma unroll
    for (int k = 0; k < 8; ++k) o[k] = __builtin_bit_cast(float, a[k]);
    return;
  }
  const uint32_t ws[4] = {w[0].x, w[0].y, w[0].z, w[0].w};
  if (dtype == DC_BF16) {  // bf16 -> fp32 is exact: the bits move up
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      o[2 * k] = __builtin_bit_cast(float, ws[k] << 16);
      o[2 * k + 1] = __builtin_bit_cast(float, ws[k] & 0xffff0000u);
    }
    return;
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    o[2 * k] = float(__builtin_bit_cast(_Float16, uint16_t(ws[k] & 0xffffu)));
    o[2 * k + 1] = float(__builtin_bit_cast(_Float16, uint16_t(ws[k] >> 16)));
  }
}

__device__ __forceinline__ float half_lo(uint32_t w) { return float(__builtin_bit_cast(_Float16, uint16_t(w & 0xffffu))); }
__device__ __forceinline__ float half_hi(uint32_t w) { return float(__builtin_bit_cast(_Float16, uint16_t(w >> 16))); }

// One 256-thread block per (merge item, query head j, column slice z),
// viewed as R = 256 / cols rows of `cols` threads, each thread holding V
// channels (channels (cols z + col) V .. + V - 1).  Row r combines partials
// r, r + R, ... against its own running maximum, U per pass, loading each
// partial's (m, l) and o together, so a pass's loads are all in flight at
// once; the rows' (m_r, l_r, o_r) are then combined through LDS:
//   M = max m_r,  out = sum_r o_r exp2(m_r - M) / sum_r l_r exp2(m_r - M)
// (log2 domain).  launch_merge picks the shape: a whole head_dim row per
// block up to head_dim 128 (C3's 32 partials per stream in one pass of 8
// rows x 4), slices of 16 x V channels beyond (C5's 132 partials in two
// passes of 16 rows x 8 instead of nine passes of 4 rows x 4: 7.6 -> 5.4 us;
// the slices measured slower at head_dim 128, C3 3.3 -> 4.4 us).
//
// HD > 0 (dc_window_merge): the block also attends its stream's window, up
// to kMaxWinTokens tokens of fp16 key and value pages (windows[item]).
// Every load goes out first: each row's value pieces of its window tokens
// (tokens r, r + R, ...), then four lanes per token its key row (every
// fourth 16-byte piece each) and the query pieces those lanes need;
// the partial passes run while they fly.  The logits (q . k times
// query_scale log2 e, the decode's log2 domain) go through LDS with the
// waves' maxima, one barrier, and each row folds the window's
// (m_w, sum_t p_t, sum_t p_t v_t) of its tokens into its state as one more
// partial.
template <int V, int U, int HD>
__global__ void __launch_bounds__(256) merge_kernel(const dc_merge_item* __restrict__ merges, const float* part_o,
                                                    const float* part_ml, float* out, int32_t n_seqs, int32_t n_kv_heads,
                                                    int32_t nq, int32_t hd, int64_t max_partials, int32_t cols,
                                                    const dc_window_range* __restrict__ windows, DecodeArgs wa) {
  struct Vec {
    float v[V];
  };
  __shared__ Vec red[256];
  __shared__ float2 red_ml[256];
  const dc_merge_item mi = merges[blockIdx.x];
  const int j = blockIdx.y, t = threadIdx.x;
  if (mi.partial_begin < 0 || mi.count <= 0 || int64_t(mi.partial_begin) + mi.count > max_partials) return;
  if (mi.seq < 0 || mi.seq >= n_seqs || mi.kv_head < 0 || mi.kv_head >= n_kv_heads) return;
  const int R = 256 / cols;  // cols <= 256, so R >= 1
  const int row = t / cols, col = t - row * cols;
  const int ch = (int(blockIdx.z) * cols + col) * V;  // first channel of this thread
  const bool live = ch < hd;                          // (hd is a multiple of V)

  // ---- window: page layout and every load ----
  constexpr bool kWin = HD > 0;
  constexpr int CQ = kWin ? HD / 4 : 8, NKL = CQ / 8;            // key channels per lane, 16-byte loads per token
  constexpr int RW = !kWin ? 1 : HD > 128 ? 16 : 256 / (HD / 4);  // rows of the launch shape for HD
  constexpr int MT = kWin ? kMaxWinTokens / RW : 1;               // window tokens per row
  constexpr int NP = kWin ? kMaxWinTokens / 64 : 1;               // 64-token passes of the logits
  __shared__ float lg[kWin ? kMaxWinTokens : 1];
  __shared__ float wmax[4];
  int W = 0;
  uint2 vr[MT];
  u32x4_t kr[NP][NKL];
  uint4 qw[NKL][2];
  const int tk = t >> 2, sub = t & 3;
  if constexpr (kWin) {
    if (R != RW || hd != HD) return;  // (launch_merge keeps to these)
    const dc_window_range wr = windows[blockIdx.x];
    const int pb = wr.page_begin, npg = wr.page_end - wr.page_begin;
    const bool rng_ok = pb >= 0 && npg > 0 && npg <= kMaxWinPages && wr.page_end <= wa.table_stride;
    const int64_t trow = (int64_t(mi.seq) * n_kv_heads + mi.kv_head) * wa.table_stride + (rng_ok ? pb : 0);
    const uint8_t* kb[kMaxWinPages];
    const uint8_t* vb[kMaxWinPages];
    int start[kMaxWinPages];
#pragma unroll
    for (int p = 0; p < kMaxWinPages; ++p) {
      kb[p] = vb[p] = nullptr;
      start[p] = W;  // (a skipped or unused page holds no tokens: the next page starts at the same token)
      if (rng_ok && p < npg) {
        // the page's descriptors: from the window records (one load per
        // page, indexed by the block alone) or through the tables
        const int32_t kid = wa.recs ? 0 : wa.k_table[trow + p], vid = wa.recs ? 0 : wa.v_table[trow + p];
        if (kid >= 0 && kid < wa.kpool.n_descs && vid >= 0 && vid < wa.vpool.n_descs) {
          const dc_page_desc kd = wa.recs ? wa.recs[int64_t(blockIdx.x) * kMaxWinPages + p].key : wa.kpool.descs[kid];
          const dc_page_desc vd = wa.recs ? wa.recs[int64_t(blockIdx.x) * kMaxWinPages + p].value : wa.vpool.descs[vid];
          int T = kd.tokens < wa.kpool.geometry.page_capacity ? int(kd.tokens) : wa.kpool.geometry.page_capacity;
          T = T < kMaxWinTokens - W ? T : kMaxWinTokens - W;
          const int64_t need = int64_t(T) * HD * 2;
          if (kd.format == DC_FMT_M3_F16 && vd.format == DC_FMT_M3_F16 && kd.tokens == vd.tokens &&
              (int64_t(kd.block) << 8) + need <= wa.kpool.arena_bytes &&
              (int64_t(vd.block) << 8) + need <= wa.vpool.arena_bytes && T > 0) {
            kb[p] = blob_ptr(wa.kpool.arena, kd);
            vb[p] = blob_ptr(wa.vpool.arena, vd);
            W += T;
          }
        }
      }
    }
    // the page of window token u and its row within the page
    auto locate = [&](int u, const uint8_t* const* base) -> const uint8_t* {
      int p = 0;
#pragma unroll
      for (int q = 1; q < kMaxWinPages; ++q) p += (u >= start[q]) ? 1 : 0;
      return base[p] + int64_t(u - start[p]) * HD * 2;
    };
    // Unconditional loads (a token past the window reloads its last token,
    // masked off where used): a load under a per-lane condition made the
    // compiler wait for each one before the next.
    if (W > 0) {  // (block-uniform)
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        if (RW * i >= W) break;  // (block-uniform: no load waits on a lane's condition)
        const int u = min(row + RW * i, W - 1);
        vr[i] = *reinterpret_cast<const uint2*>(locate(u, vb) + (live ? ch : 0) * 2);
      }
#pragma unroll
      // lane `sub` of a token's four takes its row's 16-byte pieces sub,
      // sub + 4, ...: the four lanes of one load read 64 contiguous bytes
      // (a quarter row per lane read 16 bytes of each of 64 cache lines)
      for (int pi = 0; pi < NP; ++pi) {
        if (pi * 64 >= W) break;  // (block-uniform)
        const int u = min(pi * 64 + tk, W - 1);
        const u32x4_t* krow = reinterpret_cast<const u32x4_t*>(locate(u, kb)) + sub;
#pragma unroll
        for (int k = 0; k < NKL; ++k) kr[pi][k] = krow[4 * k];
      }
      const int64_t qrow = ((int64_t(mi.seq) * n_kv_heads + mi.kv_head) * nq + j) * HD + 8 * sub;
#pragma unroll
      for (int k = 0; k < NKL; ++k) load_q8_raw(wa.queries, wa.queries_dtype, qrow + 32 * k, qw[k]);
    }
  }

  const float* ml = part_ml + (int64_t(mi.partial_begin) * nq + j) * 2;                    // partial s at ml[2 nq s]
  const float* po = part_o + (int64_t(mi.partial_begin) * nq + j) * hd + (live ? ch : 0);  // partial s at po[nq hd s]
  const int64_t mstep = int64_t(nq) * 2, step = int64_t(nq) * hd;
  float m_r = -INFINITY, l_r = 0.f;
  Vec acc;
#pragma unroll
  for (int e = 0; e < V; ++e) acc.v[e] = 0.f;
  if (row < R) {
    // U partials per pass; a slot past the count loads partial s0 again
    // (always in bounds) and is masked off, so no load waits on a branch
    for (int s0 = row; s0 < mi.count; s0 += U * R) {
      float mv[U], lv[U];
      Vec xv[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int s = s0 + u * R < mi.count ? s0 + u * R : s0;
        mv[u] = ml[s * mstep];
        lv[u] = ml[s * mstep + 1];
        if constexpr (V == 4) {
          const float4 y = *reinterpret_cast<const float4*>(po + s * step);
          xv[u].v[0] = y.x;
          xv[u].v[1] = y.y;
          xv[u].v[2] = y.z;
          xv[u].v[3] = y.w;
        } else {
          xv[u].v[0] = po[s * step];
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (s0 + u * R >= mi.count) mv[u] = -INFINITY;
      float m_new = m_r;
#pragma unroll
      for (int u = 0; u < U; ++u) m_new = fmaxf(m_new, mv[u]);
      if (m_new == -INFINITY) continue;  // every partial so far is empty
      const float c_old = m_r == -INFINITY ? 0.f : exp2f(m_r - m_new);
      l_r *= c_old;
#pragma unroll
      for (int e = 0; e < V; ++e) acc.v[e] *= c_old;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const float c = mv[u] == -INFINITY ? 0.f : exp2f(mv[u] - m_new);  // an empty partial adds nothing
        l_r += lv[u] * c;
#pragma unroll
        for (int e = 0; e < V; ++e) acc.v[e] += xv[u].v[e] * c;
      }
      m_r = m_new;
    }
  }

  // ---- window: logits, their maximum, and each row's share ----
  if constexpr (kWin) {
    if (W > 0) {  // (block-uniform)
      const float qmul = wa.q_scale * kLog2e;
      float qf[CQ];
#pragma unroll
      for (int k = 0; k < NKL; ++k) q8_floats(qw[k], wa.queries_dtype, qf + 8 * k);
      float lmax = -INFINITY;
#pragma unroll
      for (int pi = 0; pi < NP; ++pi) {
        if (pi * 64 >= W) break;
        float d = 0.f;
#pragma unroll
        for (int k = 0; k < NKL; ++k) {
          const uint32_t kw[4] = {kr[pi][k][0], kr[pi][k][1], kr[pi][k][2], kr[pi][k][3]};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            d = fmaf(qf[8 * k + 2 * e], half_lo(kw[e]), d);
            d = fmaf(qf[8 * k + 2 * e + 1], half_hi(kw[e]), d);
          }
        }
        d += __shfl_xor(d, 1, 64);
        d += __shfl_xor(d, 2, 64);  // the token's whole dot product, in all four lanes
        const int u = pi * 64 + tk;
        const float lgv = u < W ? d * qmul : -INFINITY;
        if (sub == 0 && u < W) lg[u] = lgv;
        lmax = fmaxf(lmax, lgv);
      }
      lmax = wave_max(lmax);
      if ((t & 63) == 0) wmax[t >> 6] = lmax;
      __syncthreads();
      const float m_w = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
      float l_w = 0.f, aw[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        if (RW * i >= W) break;
        const int u = row + RW * i;
        if (u < W) {
          const float pw = exp2f(lg[u] - m_w);
          l_w += pw;
          aw[0] = fmaf(pw, half_lo(vr[i].x), aw[0]);
          aw[1] = fmaf(pw, half_hi(vr[i].x), aw[1]);
          aw[2] = fmaf(pw, half_lo(vr[i].y), aw[2]);
          aw[3] = fmaf(pw, half_hi(vr[i].y), aw[3]);
        }
      }
      if (row < R && l_w > 0.f) {  // fold (m_w, l_w, aw) into the row's state
        const float M = fmaxf(m_r, m_w);
        const float c_old = m_r == -INFINITY ? 0.f : exp2f(m_r - M), c_w = exp2f(m_w - M);
        l_r = l_r * c_old + l_w * c_w;
#pragma unroll
        for (int e = 0; e < V; ++e) acc.v[e] = acc.v[e] * c_old + aw[e] * c_w;
        m_r = M;
      }
    }
  }

  red[t] = acc;
  red_ml[t] = float2{m_r, l_r};
  __syncthreads();
  if (t < cols && live) {
    float M = -INFINITY;
    for (int r = 0; r < R; ++r) M = fmaxf(M, red_ml[r * cols + t].x);
    float L = 0.f;
#pragma unroll
    for (int e = 0; e < V; ++e) acc.v[e] = 0.f;
    if (M != -INFINITY)
      for (int r = 0; r < R; ++r) {
        const float2 q = red_ml[r * cols + t];
        const float w = q.x == -INFINITY ? 0.f : exp2f(q.x - M);
        L += q.y * w;
#pragma unroll
        for (int e = 0; e < V; ++e) acc.v[e] += red[r * cols + t].v[e] * w;
      }
    const float inv = 1.f / fmaxf(L, 1e-30f);
    float* o = out + ((int64_t(mi.seq) * n_kv_heads + mi.kv_head) * nq + j) * hd + ch;
    if constexpr (V == 4)
      *reinterpret_cast<float4*>(o) = float4{acc.v[0] * inv, acc.v[1] * inv, acc.v[2] * inv, acc.v[3] * inv};
    else
      o[0] = acc.v[0] * inv;
  }
}

int launch_decode_generic(const DecodeArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL(decode_generic_kernel, dim3(uint32_t(a.n_items)), dim3(kThreads), 0, stream, a);
  return check_hip(hipGetLastError(), "decode_generic_kernel launch");
}

// 0 = fastest kernel that fits, 1 = generic kernel only, 2 = MFMA kernel only
static int g_decode_path = 0;

int launch_decode(const DecodeArgs& a, hipStream_t stream) {
  bool launched = false;
  if (g_decode_path != 1)
    if (int rc = launch_decode_mfma(a, stream, &launched)) return rc;
  if (!launched && g_decode_path == 2)
    return fail(DC_EINVAL, "decode path 2: the MFMA kernel does not cover these pools");
  return launched ? DC_OK : launch_decode_generic(a, stream);
}

int launch_merge(const DecodeArgs& a, const dc_merge_item* merges, int32_t n_merges, hipStream_t stream,
                 const dc_window_range* windows) {
  if (n_merges <= 0) return DC_OK;
  const int hd = a.kpool.geometry.head_dim;
  // float4 rows when every partial row and output row starts 16-byte aligned
  const bool vec4 = (hd & 3) == 0 && ((reinterpret_cast<uintptr_t>(a.part_o) | reinterpret_cast<uintptr_t>(a.out)) & 15) == 0;
  const int V = vec4 ? 4 : 1;
  // a whole row per block up to head_dim 128, else slices of 16 x V channels
  const bool sliced = hd > 128;
  const int cols = sliced ? 16 : hd / V;
  const dim3 grid(uint32_t(n_merges), uint32_t(a.n_q), uint32_t((hd / V + cols - 1) / cols));
#define DC_MERGE(V_, U_, HD_)                                                                                    \
  hipLaunchKernelGGL((merge_kernel<V_, U_, HD_>), grid, dim3(256), 0, stream, merges, a.part_o, a.part_ml, a.out, \
                     a.n_seqs, a.n_kv_heads, a.n_q, hd, a.max_partials, cols, windows, a)
  if (windows != nullptr) {
    if (!vec4 || (hd != 64 && hd != 128 && hd != 256))
      return fail(DC_EINVAL, "window merge: head_dim must be 64, 128 or 256 and out / workspace 16-byte aligned");
    if (hd == 256)
      DC_MERGE(4, 8, 256);
    else if (hd == 128)
      DC_MERGE(4, 4, 128);
    else
      DC_MERGE(4, 4, 64);
  } else if (vec4 && sliced)
    DC_MERGE(4, 8, 0);
  else if (vec4)
    DC_MERGE(4, 4, 0);
  else if (sliced)
    DC_MERGE(1, 8, 0);
  else
    DC_MERGE(1, 4, 0);
#undef DC_MERGE
  return check_hip(hipGetLastError(), "merge_kernel launch");
}

// One thread per (item, record slot): the key and value descriptors of page
// page_begin + slot of the item, read through its tables as the decode
// kernels read them (an id outside a pool, or a slot past the item's pages,
// gives a zero record).
__global__ void __launch_bounds__(256) gather_records_kernel(DecodeArgs a, dc_page_record* recs) {
  const int64_t e = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (e >= int64_t(a.n_items) * a.rec_stride) return;
  const int32_t i = int32_t(e / a.rec_stride), slot = int32_t(e - int64_t(i) * a.rec_stride);
  const dc_work_item it = a.items[i];
  dc_page_record r{};
  if (item_in_bounds(it, a) && slot < it.page_end - it.page_begin) {
    const int64_t row = (int64_t(it.seq) * a.n_kv_heads + it.kv_head) * a.table_stride + it.page_begin + slot;
    const int32_t kid = a.k_table[row], vid = a.v_table[row];
    if (kid >= 0 && kid < a.kpool.n_descs && vid >= 0 && vid < a.vpool.n_descs) {
      r.key = a.kpool.descs[kid];
      r.value = a.vpool.descs[vid];
    }
  }
  recs[e] = r;
}

}  // namespace dc

extern "C" int dc_decode_paged(dc_pool k_pool, dc_pool v_pool, const int32_t* k_table, const int32_t* v_table, int32_t table_stride,
                               const dc_work_item* items, int32_t n_items, const dc_merge_item* merges,
                               int32_t n_merges, const void* queries, int32_t queries_dtype, float query_scale,
                               int32_t n_seqs, int32_t n_kv_heads, int32_t n_q, float* out, void* workspace,
                               int64_t workspace_bytes, dc_stream_t stream) {
  return dc_decode_paged_records(k_pool, v_pool, k_table, v_table, table_stride, items, n_items, merges, n_merges,
                                 queries, queries_dtype, query_scale, n_seqs, n_kv_heads, n_q, out, workspace,
                                 workspace_bytes, nullptr, 0, stream);
}

extern "C" int dc_gather_page_records(dc_pool k_pool, dc_pool v_pool, const int32_t* k_table, const int32_t* v_table,
                                      int32_t table_stride, const dc_work_item* items, int32_t n_items,
                                      int32_t n_seqs, int32_t n_kv_heads, dc_page_record* records, int32_t rec_stride,
                                      dc_stream_t stream) {
  if (n_items < 0 || n_seqs <= 0 || n_kv_heads <= 0 || table_stride < 0 || rec_stride <= 0 || rec_stride > 64)
    return dc::fail(DC_EINVAL, "dc_gather_page_records: bad sizes (rec_stride must be in [1, 64])");
  if (n_items == 0) return DC_OK;
  if (!k_table || !v_table || !items || !records || !k_pool.descs || !v_pool.descs)
    return dc::fail(DC_EINVAL, "dc_gather_page_records: null pointer");
  dc::DecodeArgs a{};
  a.kpool = k_pool;
  a.vpool = v_pool;
  a.k_table = k_table;
  a.v_table = v_table;
  a.table_stride = table_stride;
  a.items = items;
  a.n_items = n_items;
  a.n_seqs = n_seqs;
  a.n_kv_heads = n_kv_heads;
  a.rec_stride = rec_stride;
  const int64_t n = int64_t(n_items) * rec_stride;
  hipLaunchKernelGGL(dc::gather_records_kernel, dim3(uint32_t((n + 255) / 256)), dim3(256), 0, hipStream_t(stream), a,
                     records);
  return dc::check_hip(hipGetLastError(), "gather_records_kernel launch");
}

extern "C" int dc_decode_paged_records(dc_pool k_pool, dc_pool v_pool, const int32_t* k_table, const int32_t* v_table,
                                       int32_t table_stride, const dc_work_item* items, int32_t n_items,
                                       const dc_merge_item* merges, int32_t n_merges, const void* queries,
                                       int32_t queries_dtype, float query_scale, int32_t n_seqs, int32_t n_kv_heads,
                                       int32_t n_q, float* out, void* workspace, int64_t workspace_bytes,
                                       const dc_page_record* records, int32_t rec_stride, dc_stream_t stream) {
  if (records != nullptr && (rec_stride <= 0 || rec_stride > 64))
    return dc::fail(DC_EINVAL, "dc_decode_paged_records: rec_stride must be in [1, 64]");
  if (int rc = dc::validate_geometry(k_pool.geometry)) return rc;
  if (int rc = dc::validate_geometry(v_pool.geometry)) return rc;
  const dc_page_geometry& g = k_pool.geometry;
  if (v_pool.geometry.head_dim != g.head_dim || v_pool.geometry.page_capacity != g.page_capacity)
    return dc::fail(DC_EINVAL, "key and value pools must share head_dim and page_capacity");
  if (n_items < 0 || n_merges < 0 || n_seqs <= 0 || n_kv_heads <= 0)
    return dc::fail(DC_EINVAL, "dc_decode_paged: bad counts");
  if (n_q <= 0 || n_q > dc::kMaxQ) return dc::fail(DC_EINVAL, "n_q must be in [1, %d]", dc::kMaxQ);
  if (g.head_dim > dc::kMaxHD) return dc::fail(DC_EINVAL, "head_dim %d exceeds %d", g.head_dim, dc::kMaxHD);
  if (dc::num_groups(g) * g.group_size > dc::kMaxHD)
    return dc::fail(DC_EINVAL, "padded head_dim %d exceeds %d", dc::num_groups(g) * g.group_size, dc::kMaxHD);
  if (dc::num_groups(g) > dc::kMaxGroups || dc::num_groups(v_pool.geometry) > dc::kMaxGroups) return dc::fail(DC_EINVAL, "more than %d groups per head", dc::kMaxGroups);
  if (g.page_capacity > dc::kMaxCap)
    return dc::fail(DC_EINVAL, "page_capacity %d exceeds %d for decode", g.page_capacity, dc::kMaxCap);
  if (queries_dtype != DC_F32 && queries_dtype != DC_F16 && queries_dtype != DC_BF16)
    return dc::fail(DC_EINVAL, "queries_dtype must be DC_F32, DC_F16 or DC_BF16");
  if (n_items == 0) return DC_OK;
  if (!k_table || !v_table || !items || !queries || !out || !k_pool.arena || !k_pool.descs || !v_pool.arena ||
      !v_pool.descs)
    return dc::fail(DC_EINVAL, "dc_decode_paged: null pointer");
  if (n_merges > 0 && !merges) return dc::fail(DC_EINVAL, "dc_decode_paged: null merges");

  dc::DecodeArgs a{};
  a.kpool = k_pool;
  a.vpool = v_pool;
  a.k_table = k_table;
  a.v_table = v_table;
  a.table_stride = table_stride;
  a.items = items;
  a.n_items = n_items;
  a.queries = queries;
  a.queries_dtype = queries_dtype;
  a.q_scale = query_scale;
  a.n_seqs = n_seqs;
  a.n_kv_heads = n_kv_heads;
  a.n_q = n_q;
  a.out = out;
  // the workspace holds as many partial slots as fit; kernels skip any
  // item or merge naming a slot past that count
  const int64_t per_partial = int64_t(n_q) * (g.head_dim + 2) * 4;
  const int64_t n_partials = per_partial > 0 ? workspace_bytes / per_partial : 0;
  a.part_o = reinterpret_cast<float*>(workspace);
  a.part_ml = a.part_o + n_partials * n_q * g.head_dim;
  a.max_partials = n_partials;
  a.recs = records;
  a.rec_stride = records ? rec_stride : 0;
  if (n_merges > 0 && (!workspace || n_partials <= 0))
    return dc::fail(DC_ESPACE, "dc_decode_paged: split-K items need a workspace");

  int rc = dc::launch_decode(a, hipStream_t(stream));
  if (rc) return rc;
  return dc::launch_merge(a, merges, n_merges, hipStream_t(stream));
}

extern "C" int dc_lse_merge(const dc_merge_item* merges, int32_t n_merges, const void* workspace,
                            int64_t workspace_bytes, int32_t n_seqs, int32_t n_kv_heads, int32_t n_q, int32_t head_dim,
                            float* out, dc_stream_t stream) {
  if (n_merges < 0 || n_seqs <= 0 || n_kv_heads <= 0 || head_dim <= 0 || head_dim > dc::kMaxHD)
    return dc::fail(DC_EINVAL, "dc_lse_merge: bad sizes");
  if (n_q <= 0 || n_q > dc::kMaxQ) return dc::fail(DC_EINVAL, "n_q must be in [1, %d]", dc::kMaxQ);
  if (n_merges == 0) return DC_OK;
  if (!merges || !out) return dc::fail(DC_EINVAL, "dc_lse_merge: null pointer");
  const int64_t per_partial = int64_t(n_q) * (head_dim + 2) * 4;
  const int64_t n_partials = workspace_bytes / per_partial;
  if (!workspace || n_partials <= 0) return dc::fail(DC_ESPACE, "dc_lse_merge: no partials in the workspace");
  dc::DecodeArgs a{};
  a.n_seqs = n_seqs;
  a.n_kv_heads = n_kv_heads;
  a.n_q = n_q;
  a.out = out;
  a.kpool.geometry.head_dim = head_dim;
  a.part_o = reinterpret_cast<float*>(const_cast<void*>(workspace));
  a.part_ml = a.part_o + n_partials * n_q * head_dim;
  a.max_partials = n_partials;
  return dc::launch_merge(a, merges, n_merges, hipStream_t(stream));
}

extern "C" int dc_window_merge(dc_pool k_pool, dc_pool v_pool, const int32_t* k_table, const int32_t* v_table,
                               int32_t table_stride, const dc_merge_item* merges, const dc_window_range* windows,
                               int32_t n_merges, const void* queries, int32_t queries_dtype, float query_scale,
                               int32_t n_seqs, int32_t n_kv_heads, int32_t n_q, float* out, const void* workspace,
                               int64_t workspace_bytes, const dc_page_record* records, dc_stream_t stream) {
  if (int rc = dc::validate_geometry(k_pool.geometry)) return rc;
  const int hd = k_pool.geometry.head_dim;
  if (v_pool.geometry.head_dim != hd || v_pool.geometry.page_capacity != k_pool.geometry.page_capacity)
    return dc::fail(DC_EINVAL, "key and value pools must share head_dim and page_capacity");
  if (n_merges < 0 || n_seqs <= 0 || n_kv_heads <= 0 || table_stride <= 0)
    return dc::fail(DC_EINVAL, "dc_window_merge: bad sizes");
  if (n_q <= 0 || n_q > dc::kMaxQ) return dc::fail(DC_EINVAL, "n_q must be in [1, %d]", dc::kMaxQ);
  if (queries_dtype != DC_F32 && queries_dtype != DC_F16 && queries_dtype != DC_BF16)
    return dc::fail(DC_EINVAL, "queries_dtype must be DC_F32, DC_F16 or DC_BF16");
  if (n_merges == 0) return DC_OK;
  if (!merges || !windows || !out || !queries || !k_table || !v_table || !k_pool.arena || !k_pool.descs ||
      !v_pool.arena || !v_pool.descs)
    return dc::fail(DC_EINVAL, "dc_window_merge: null pointer");
  if ((reinterpret_cast<uintptr_t>(queries) & 15) != 0)
    return dc::fail(DC_EINVAL, "dc_window_merge: queries must be 16-byte aligned");
  const int64_t per_partial = int64_t(n_q) * (hd + 2) * 4;
  const int64_t n_partials = workspace_bytes / per_partial;
  if (!workspace || n_partials <= 0) return dc::fail(DC_ESPACE, "dc_window_merge: no partials in the workspace");
  dc::DecodeArgs a{};
  a.kpool = k_pool;
  a.vpool = v_pool;
  a.k_table = k_table;
  a.v_table = v_table;
  a.table_stride = table_stride;
  a.queries = queries;
  a.queries_dtype = queries_dtype;
  a.q_scale = query_scale;
  a.n_seqs = n_seqs;
  a.n_kv_heads = n_kv_heads;
  a.n_q = n_q;
  a.out = out;
  a.part_o = reinterpret_cast<float*>(const_cast<void*>(workspace));
  a.part_ml = a.part_o + n_partials * n_q * hd;
  a.max_partials = n_partials;
  a.recs = records;
  a.rec_stride = records ? dc::kMaxWinPages : 0;
  return dc::launch_merge(a, merges, n_merges, hipStream_t(stream), windows);
}

extern "C" int32_t dc_decode_waves_per_simd(dc_pool k_pool, dc_pool v_pool, int32_t n_q) {
  if (n_q <= 0 || n_q > dc::kMaxQ) return 1;
  dc::DecodeArgs a{};
  a.kpool = k_pool;
  a.vpool = v_pool;
  a.n_q = n_q;
  if (dc::g_decode_path == 1) return 1;
  const int w = dc::decode_mfma_waves(a);
  return w > 0 ? w : 1;
}

extern "C" int dc_set_decode_path(int32_t path) {
  if (path < 0 || path > 2) return dc::fail(DC_EINVAL, "decode path must be 0 (auto), 1 (generic) or 2 (mfma)");
  dc::g_decode_path = path;
  return DC_OK;
}
