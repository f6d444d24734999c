// Execution shortlist on the device: per-page summaries of key and value
// pages, page relevance against a query, and a stable top-k over candidate
// pages (reference dotcache/session_runtime.py:122-439).
//
// These are small, latency-bound kernels (a page's summary is one pass over
// its rows; relevance is a GEMV over per-page sketches), so they use plain
// VALU code with one block per page or one wave per page.
#include "dc_common.h"

namespace dc {

// One block per page, one thread per channel: mean, min and max over the
// page's dequantised rows, and the means of np.array_split(rows, R) with
// R = min(S, T) chunks (the first T % R chunks one row longer).  Sketch rows
// R .. S - 1 repeat chunk R - 1, which leaves every max over rows unchanged.
// An empty page writes zeros.
__global__ void __launch_bounds__(256) page_summaries_kernel(dc_pool pool, const int32_t* __restrict__ page_ids,
                                                             int32_t sketch_rows, float* mean, float* sketch,
                                                             float* pmin, float* pmax) {
  const dc_page_geometry geo = pool.geometry;
  const int hd = geo.head_dim, S = sketch_rows;
  const int p = blockIdx.x, c = threadIdx.x;
  if (c >= hd) return;
  const int32_t id = page_ids[p];
  float* sk = sketch + (int64_t(p) * S) * hd + c;
  if (id < 0 || id >= pool.n_descs) {
    mean[int64_t(p) * hd + c] = 0.f;
    pmin[int64_t(p) * hd + c] = 0.f;
    pmax[int64_t(p) * hd + c] = 0.f;
    for (int s = 0; s < S; ++s) sk[int64_t(s) * hd] = 0.f;
    return;
  }
  const dc_page_desc d = reinterpret_cast<const dc_page_desc*>(pool.descs)[id];
  const BlobLayout L = blob_layout(d.format, d.bits, geo);
  const uint8_t* blob = blob_ptr(pool.arena, d);
  const int T = d.tokens < geo.page_capacity ? d.tokens : geo.page_capacity;
  if (T <= 0) {
    mean[int64_t(p) * hd + c] = 0.f;
    pmin[int64_t(p) * hd + c] = 0.f;
    pmax[int64_t(p) * hd + c] = 0.f;
    for (int s = 0; s < S; ++s) sk[int64_t(s) * hd] = 0.f;
    return;
  }
  const int R = S < T ? S : T, q = T / R, rem = T % R;
  float total = 0.f, lo = INFINITY, hi = -INFINITY, csum = 0.f, last = 0.f;
  int chunk = 0, clen = rem > 0 ? q + 1 : q, cfill = 0;
  for (int t = 0; t < T; ++t) {
    const float v = page_value(blob, d, L, geo, t, c);
    total += v;
    lo = fminf(lo, v);
    hi = fmaxf(hi, v);
    csum += v;
    if (++cfill == clen) {
      last = csum / float(clen);
      sk[int64_t(chunk) * hd] = last;
      ++chunk;
      csum = 0.f;
      cfill = 0;
      clen = chunk < rem ? q + 1 : q;
    }
  }
  for (int s = R; s < S; ++s) sk[int64_t(s) * hd] = last;
  mean[int64_t(p) * hd + c] = total / float(T);
  pmin[int64_t(p) * hd + c] = lo;
  pmax[int64_t(p) * hd + c] = hi;
}

// One wave per page, the waves striding over the pages (a launch of at most
// 8192 waves, each scoring n / 8192 pages in turn): sketch mode, max over
// rows s of sketch[p, s, :] . q; envelope mode, max[p, :] . max(q, 0) +
// min[p, :] . min(q, 0).
__global__ void __launch_bounds__(256) page_relevance_kernel(const float* __restrict__ sketch, int32_t sketch_rows,
                                                             const float* __restrict__ pmin,
                                                             const float* __restrict__ pmax, int32_t mode,
                                                             const float* __restrict__ query, int32_t hd,
                                                             int32_t n_pages, float* scores) {
  const int lane = threadIdx.x & 63;
  for (int p = blockIdx.x * 4 + (threadIdx.x >> 6); p < n_pages; p += gridDim.x * 4) {
    float best = -INFINITY;
    if (mode == 0) {
      for (int s = 0; s < sketch_rows; ++s) {
        const float* row = sketch + (int64_t(p) * sketch_rows + s) * hd;
        float acc = 0.f;
        for (int c = lane; c < hd; c += 64) acc += row[c] * query[c];
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
        best = fmaxf(best, acc);
      }
    } else {
      float acc = 0.f;
      for (int c = lane; c < hd; c += 64) {
        const float qc = query[c];
        acc += pmax[int64_t(p) * hd + c] * fmaxf(qc, 0.f) + pmin[int64_t(p) * hd + c] * fminf(qc, 0.f);
      }
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
      best = acc;
    }
    if (lane == 0) scores[p] = best;
  }
}

// Stable top-k among candidates: page i is taken when fewer than k
// candidates rank before it, ranking by score descending and, among equal
// scores, by index ascending (Python's stable sort with reverse=True).  A
// block of four waves ranks 64 pages: lane l of every wave takes page
// 64 blockIdx + l and wave w counts over a quarter of each tile, the four
// partial counts meeting in LDS.  The scores go through LDS a tile of
// kTopKTile at a time, non-candidates as -inf (which never rank before a
// finite score; an equal score counts only for a candidate), read four at a
// time.
constexpr int kTopKTile = 4096;
__global__ void __launch_bounds__(256) select_top_k_kernel(const float* __restrict__ scores,
                                                           const uint8_t* __restrict__ candidate, int32_t n,
                                                           int32_t k, uint8_t* selected) {
  __shared__ __attribute__((aligned(16))) float s_sc[kTopKTile];
  __shared__ __attribute__((aligned(16))) float s_ok[kTopKTile];
  __shared__ int s_rank[4][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int i = blockIdx.x * 64 + lane;
  const bool mine = i < n && candidate[i] != 0;
  const float si = i < n ? scores[i] : 0.f;
  int rank = 0;
  for (int base = 0; base < n; base += kTopKTile) {
    const int m = n - base < kTopKTile ? n - base : kTopKTile;
    const int m16 = (m + 15) & ~15;  // <= kTopKTile, a multiple of 16: four quarters of whole float4s
    for (int u = threadIdx.x; u < m16; u += 256) {
      const bool in = u < m && candidate[base + u] != 0;
      s_sc[u] = in ? scores[base + u] : -INFINITY;
      s_ok[u] = in ? 1.f : 0.f;
    }
    __syncthreads();
    if (mine) {
      const int q = m16 / 4;
      for (int u = w * q; u < (w + 1) * q; u += 4) {
        const float4 sj = *reinterpret_cast<const float4*>(s_sc + u);
        const float4 ok = *reinterpret_cast<const float4*>(s_ok + u);
        const int j = base + u;
        rank += (sj.x > si) | ((sj.x == si) & (ok.x != 0.f) & (j < i));
        rank += (sj.y > si) | ((sj.y == si) & (ok.y != 0.f) & (j + 1 < i));
        rank += (sj.z > si) | ((sj.z == si) & (ok.z != 0.f) & (j + 2 < i));
        rank += (sj.w > si) | ((sj.w == si) & (ok.w != 0.f) & (j + 3 < i));
      }
    }
    __syncthreads();
  }
  s_rank[w][lane] = rank;
  __syncthreads();
  if (w == 0 && i < n) {
    const int total = s_rank[0][lane] + s_rank[1][lane] + s_rank[2][lane] + s_rank[3][lane];
    selected[i] = mine && total < k ? 1 : 0;
  }
}

}  // namespace dc

extern "C" int dc_page_summaries(dc_pool pool, const int32_t* page_ids, int32_t n_pages, int32_t sketch_rows,
                                 float* mean, float* sketch, float* page_min, float* page_max, dc_stream_t stream) {
  if (int rc = dc::validate_geometry(pool.geometry)) return rc;
  if (n_pages < 0 || sketch_rows <= 0) return dc::fail(DC_EINVAL, "dc_page_summaries: n_pages >= 0, sketch_rows > 0");
  if (pool.geometry.head_dim > 256) return dc::fail(DC_EINVAL, "dc_page_summaries: head_dim > 256");
  if (n_pages == 0) return DC_OK;
  if (!page_ids || !mean || !sketch || !page_min || !page_max || !pool.arena || !pool.descs)
    return dc::fail(DC_EINVAL, "dc_page_summaries: null pointer");
  hipLaunchKernelGGL(dc::page_summaries_kernel, dim3(uint32_t(n_pages)), dim3(256), 0, hipStream_t(stream), pool,
                     page_ids, sketch_rows, mean, sketch, page_min, page_max);
  return dc::check_hip(hipGetLastError(), "dc_page_summaries launch");
}

extern "C" int dc_page_relevance(const float* sketch, int32_t sketch_rows, const float* page_min, const float* page_max,
                                 int32_t mode, const float* query, int32_t head_dim, int32_t n_pages, float* scores,
                                 dc_stream_t stream) {
  if (n_pages < 0 || head_dim <= 0 || (mode != 0 && mode != 1) || (mode == 0 && sketch_rows <= 0))
    return dc::fail(DC_EINVAL, "dc_page_relevance: bad mode, head_dim, sketch_rows or n_pages");
  if (n_pages == 0) return DC_OK;
  if (!query || !scores || (mode == 0 && !sketch) || (mode == 1 && (!page_min || !page_max)))
    return dc::fail(DC_EINVAL, "dc_page_relevance: null pointer");
  const uint32_t blocks = uint32_t((n_pages + 3) / 4 < 2048 ? (n_pages + 3) / 4 : 2048);
  hipLaunchKernelGGL(dc::page_relevance_kernel, dim3(blocks), dim3(256), 0, hipStream_t(stream),
                     sketch, sketch_rows, page_min, page_max, mode, query, head_dim, n_pages, scores);
  return dc::check_hip(hipGetLastError(), "dc_page_relevance launch");
}

extern "C" int dc_select_top_k(const float* scores, const uint8_t* candidate, int32_t n, int32_t k, uint8_t* selected,
                               dc_stream_t stream) {
  if (n < 0 || k < 0) return dc::fail(DC_EINVAL, "dc_select_top_k: n and k must be non-negative");
  if (n == 0) return DC_OK;
  if (!scores || !candidate || !selected) return dc::fail(DC_EINVAL, "dc_select_top_k: null pointer");
  hipLaunchKernelGGL(dc::select_top_k_kernel, dim3(uint32_t((n + 63) / 64)), dim3(256), 0, hipStream_t(stream),
                     scores, candidate, n, k, selected);
  return dc::check_hip(hipGetLastError(), "dc_select_top_k launch");
}
