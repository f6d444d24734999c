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

// One 256-thread block per (merge item, query head j), viewed as rows of
// C = head_dim / V threads, each thread holding V channels.  Row r combines
// partials r, r + R, ... (R = 256 / C rows) against its own running maximum,
// loading each partial's (m, l) and o together, so all of a merge's loads
// are in flight at once; the rows' (m_r, l_r, o_r) are then combined through
// LDS:  M = max m_r,  out = sum_r o_r exp2(m_r - M) / sum_r l_r exp2(m_r - M)
// (log2 domain).
template <int V>
__global__ void __launch_bounds__(256) merge_kernel(const dc_merge_item* __restrict__ merges, const float* part_o,
                                                    const float* part_ml, float* out, int32_t n_seqs, int32_t n_kv_heads,
                                                    int32_t nq, int32_t hd, int64_t max_partials) {
  struct Vec {
    float v[V];
  };
  __shared__ Vec red[256];
  __shared__ float2 red_ml[256];
  const dc_merge_item mi = merges[blockIdx.x];
  const int j = blockIdx.y, t = threadIdx.x;
  if (mi.partial_begin < 0 || mi.count <= 0 || int64_t(mi.partial_begin) + mi.count > max_partials) return;
  if (mi.seq < 0 || mi.seq >= n_seqs || mi.kv_head < 0 || mi.kv_head >= n_kv_heads) return;
  const int C = hd / V, R = 256 / C;  // hd <= 256, so R >= 1
  const int row = t / C, col = t - row * C;
  const float* ml = part_ml + (int64_t(mi.partial_begin) * nq + j) * 2;             // partial s at ml[2 nq s]
  const float* po = part_o + (int64_t(mi.partial_begin) * nq + j) * hd + col * V;  // partial s at po[nq hd s]
  const int64_t mstep = int64_t(nq) * 2, step = int64_t(nq) * hd;
  float m_r = -INFINITY, l_r = 0.f;
  Vec acc;
#pragma unroll
  for (int e = 0; e < V; ++e) acc.v[e] = 0.f;
  if (row < R) {
    // four partials per pass; a slot past the count loads partial s0 again
    // (always in bounds) and is masked off, so no load waits on a branch
    for (int s0 = row; s0 < mi.count; s0 += 4 * R) {
      float mv[4], lv[4];
      Vec xv[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
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
      for (int u = 0; u < 4; ++u)
        if (s0 + u * R >= mi.count) mv[u] = -INFINITY;
      const float m_new = fmaxf(fmaxf(m_r, fmaxf(mv[0], mv[1])), fmaxf(mv[2], mv[3]));
      if (m_new == -INFINITY) continue;  // every partial so far is empty
      const float c_old = m_r == -INFINITY ? 0.f : exp2f(m_r - m_new);
      l_r *= c_old;
#pragma unroll
      for (int e = 0; e < V; ++e) acc.v[e] *= c_old;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float c = mv[u] == -INFINITY ? 0.f : exp2f(mv[u] - m_new);  // an empty partial adds nothing
        l_r += lv[u] * c;
#pragma unroll
        for (int e = 0; e < V; ++e) acc.v[e] += xv[u].v[e] * c;
      }
      m_r = m_new;
    }
  }
  red[t] = acc;
  red_ml[t] = float2{m_r, l_r};
  __syncthreads();
  if (t < C) {
    float M = -INFINITY;
    for (int r = 0; r < R; ++r) M = fmaxf(M, red_ml[r * C + t].x);
    float L = 0.f;
#pragma unroll
    for (int e = 0; e < V; ++e) acc.v[e] = 0.f;
    if (M != -INFINITY)
      for (int r = 0; r < R; ++r) {
        const float2 q = red_ml[r * C + t];
        const float w = q.x == -INFINITY ? 0.f : exp2f(q.x - M);
        L += q.y * w;
#pragma unroll
        for (int e = 0; e < V; ++e) acc.v[e] += red[r * C + t].v[e] * w;
      }
    const float inv = 1.f / fmaxf(L, 1e-30f);
    float* o = out + ((int64_t(mi.seq) * n_kv_heads + mi.kv_head) * nq + j) * hd + t * V;
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

int launch_merge(const DecodeArgs& a, const dc_merge_item* merges, int32_t n_merges, hipStream_t stream) {
  if (n_merges <= 0) return DC_OK;
  const int hd = a.kpool.geometry.head_dim;
  // float4 rows when every partial row and output row starts 16-byte aligned
  const bool vec4 = (hd & 3) == 0 && ((reinterpret_cast<uintptr_t>(a.part_o) | reinterpret_cast<uintptr_t>(a.out)) & 15) == 0;
  const dim3 grid(uint32_t(n_merges), uint32_t(a.n_q));
  if (vec4)
    hipLaunchKernelGGL(merge_kernel<4>, grid, dim3(256), 0, stream, merges, a.part_o, a.part_ml, a.out, a.n_seqs, a.n_kv_heads,
                       a.n_q, hd, a.max_partials);
  else
    hipLaunchKernelGGL(merge_kernel<1>, grid, dim3(256), 0, stream, merges, a.part_o, a.part_ml, a.out, a.n_seqs, a.n_kv_heads,
                       a.n_q, hd, a.max_partials);
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
