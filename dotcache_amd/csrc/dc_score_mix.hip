// Per-page score and mix entry points (the score_page / mix_page surface).
//
// These serve the reference's page-at-a-time API and its parity tests; the
// fused decode kernel (dc_decode.hip) is the throughput path.  The
// arithmetic follows the reference's streaming form
// (dotcache/attention_reference.py:97-126, :165-192): per group,
// s * (codes . q_g) + b * sum(q_g) for affine pages, s * ((codes - zp) . q_g)
// for symmetric pages, fp32 escape rows for M3 pages.
#include "dc_common.h"

namespace dc {

constexpr int kScoreQ = 8;  // queries scored per pass

// grid.x = page index, grid.y = query chunk; one thread per token.  With
// page_group, page i is scored against the queries of group page_group[i]
// (queries [n_groups][n_queries][hd]) into logits rows
// group * n_queries + q; without it every page belongs to group 0.
__global__ void __launch_bounds__(256) score_pages_kernel(dc_pool pool, const int32_t* __restrict__ page_ids,
                                                          const int32_t* __restrict__ token_offsets,
                                                          const int32_t* __restrict__ page_group, int32_t n_groups,
                                                          const float* __restrict__ queries_all, int32_t n_queries,
                                                          float* __restrict__ logits_all, int64_t logits_stride) {
  const int32_t i = blockIdx.x;
  const int32_t q0 = blockIdx.y * kScoreQ;
  const int32_t grp = page_group ? page_group[i] : 0;
  if (grp < 0 || grp >= n_groups) return;
  const float* queries = queries_all + int64_t(grp) * n_queries * pool.geometry.head_dim;
  float* logits = logits_all + int64_t(grp) * n_queries * logits_stride;
  const int32_t pid = page_ids[i];
  if (pid < 0 || pid >= pool.n_descs) return;
  const dc_page_desc d = pool.descs[pid];
  const dc_page_geometry geo = pool.geometry;
  const BlobLayout L = blob_layout(d.format, d.bits, geo);
  if ((int64_t(d.block) << 8) + L.total > pool.arena_bytes) return;
  const uint8_t* blob = blob_ptr(pool.arena, d);
  const int32_t off = token_offsets[i];
  const int32_t T = d.tokens < geo.page_capacity ? d.tokens : geo.page_capacity;
  const int32_t nq = n_queries - q0 < kScoreQ ? n_queries - q0 : kScoreQ;
  const int32_t G = L.groups, gs = geo.group_size, hd = geo.head_dim;

  for (int32_t t = threadIdx.x; t < T; t += blockDim.x) {
    float acc[kScoreQ];
#pragma unroll
    for (int j = 0; j < kScoreQ; ++j) acc[j] = 0.f;
    if (is_m0(d.format)) {
      const uint32_t* payload = reinterpret_cast<const uint32_t*>(blob);
      const __half* sc = reinterpret_cast<const __half*>(blob + L.scales_off);
      const __half* bs = reinterpret_cast<const __half*>(blob + L.bias_off);
      const float zp = float((1 << (d.bits - 1)) - 1);
      for (int32_t g = 0; g < G; ++g) {
        float dot[kScoreQ], qs[kScoreQ];
#pragma unroll
        for (int j = 0; j < kScoreQ; ++j) dot[j] = qs[j] = 0.f;
        for (int32_t k = 0; k < gs; ++k) {
          const int32_t c = g * gs + k;
          if (c >= hd) break;  // padded channels meet zero-padded queries
          float code = float(m0_code(payload, t, g, k, d.bits, L.words, G, geo.page_capacity, geo.layout));
          if (d.format == DC_FMT_M0_SYMMETRIC) code -= zp;
#pragma unroll
          for (int j = 0; j < kScoreQ; ++j) {
            if (j < nq) {
              const float qv = queries[int64_t(q0 + j) * hd + c];
              dot[j] += code * qv;
              qs[j] += qv;
            }
          }
        }
        const float s = __half2float(sc[t * G + g]);
        const float b = d.format == DC_FMT_M0_AFFINE ? __half2float(bs[t * G + g]) : 0.f;
#pragma unroll
        for (int j = 0; j < kScoreQ; ++j) acc[j] += s * dot[j] + b * qs[j];
      }
    } else {
      for (int32_t c = 0; c < hd; ++c) {
        const float v = page_value(blob, d, L, geo, t, c);
#pragma unroll
        for (int j = 0; j < kScoreQ; ++j)
          if (j < nq) acc[j] += v * queries[int64_t(q0 + j) * hd + c];
      }
    }
#pragma unroll
    for (int j = 0; j < kScoreQ; ++j)
      if (j < nq) logits[int64_t(q0 + j) * logits_stride + off + t] = acc[j];
  }
}

// grid.x = query row (group * n_queries + q), grid.y = channel block; one
// thread per channel, looping over the pages of the row's group
// [group_pages[g], group_pages[g + 1]) (every page without group_pages) and
// their tokens.
__global__ void __launch_bounds__(256) mix_pages_kernel(dc_pool pool, const int32_t* __restrict__ page_ids,
                                                        const int32_t* __restrict__ token_offsets, int32_t n_pages,
                                                        const int32_t* __restrict__ group_pages, int32_t n_queries,
                                                        const float* __restrict__ weights, int64_t weights_stride,
                                                        float* __restrict__ out, int32_t accumulate) {
  const int32_t q = blockIdx.x;
  const int32_t c = blockIdx.y * blockDim.x + threadIdx.x;
  const dc_page_geometry geo = pool.geometry;
  if (c >= geo.head_dim) return;
  const float* w = weights + int64_t(q) * weights_stride;
  int32_t i0 = 0, i1 = n_pages;
  if (group_pages) {
    const int32_t g = q / n_queries;
    i0 = group_pages[g] < 0 ? 0 : group_pages[g];
    i1 = group_pages[g + 1] > n_pages ? n_pages : group_pages[g + 1];
  }
  float acc = 0.f;
  for (int32_t i = i0; i < i1; ++i) {
    const int32_t pid = page_ids[i];
    if (pid < 0 || pid >= pool.n_descs) continue;
    const dc_page_desc d = pool.descs[pid];
    const BlobLayout L = blob_layout(d.format, d.bits, geo);
    if ((int64_t(d.block) << 8) + L.total > pool.arena_bytes) continue;
    const uint8_t* blob = blob_ptr(pool.arena, d);
    const int32_t off = token_offsets[i];
    const int32_t T = d.tokens < geo.page_capacity ? d.tokens : geo.page_capacity;
    for (int32_t t = 0; t < T; ++t) acc += w[off + t] * page_value(blob, d, L, geo, t, c);
  }
  float* o = out + int64_t(q) * geo.head_dim + c;
  *o = accumulate ? *o + acc : acc;
}

}  // namespace dc

static int score_launch(const dc_pool& pool, const int32_t* page_ids, const int32_t* token_offsets,
                        const int32_t* page_group, int32_t n_groups, int32_t n_pages, const float* queries,
                        int32_t n_queries, float* logits, int64_t logits_stride, hipStream_t stream, const char* who) {
  if (int rc = dc::validate_geometry(pool.geometry)) return rc;
  if (n_pages < 0 || n_queries < 0 || n_groups <= 0) return dc::fail(DC_EINVAL, "%s: bad counts", who);
  if (n_pages == 0 || n_queries == 0) return DC_OK;
  if (!page_ids || !token_offsets || !queries || !logits || !pool.arena || !pool.descs)
    return dc::fail(DC_EINVAL, "%s: null pointer", who);
  const uint32_t qchunks = uint32_t((n_queries + dc::kScoreQ - 1) / dc::kScoreQ);
  hipLaunchKernelGGL(dc::score_pages_kernel, dim3(uint32_t(n_pages), qchunks), dim3(128), 0, stream, pool, page_ids,
                     token_offsets, page_group, n_groups, queries, n_queries, logits, logits_stride);
  return dc::check_hip(hipGetLastError(), who);
}

static int mix_launch(const dc_pool& pool, const int32_t* page_ids, const int32_t* token_offsets, int32_t n_pages,
                      const int32_t* group_pages, int32_t n_groups, const float* weights, int32_t n_queries,
                      int64_t weights_stride, float* out, int32_t accumulate, hipStream_t stream, const char* who) {
  if (int rc = dc::validate_geometry(pool.geometry)) return rc;
  if (n_pages < 0 || n_queries < 0 || n_groups <= 0) return dc::fail(DC_EINVAL, "%s: bad counts", who);
  if (n_queries == 0) return DC_OK;
  if (!weights || !out || (n_pages > 0 && (!page_ids || !token_offsets || !pool.arena || !pool.descs)))
    return dc::fail(DC_EINVAL, "%s: null pointer", who);
  const uint32_t cblocks = uint32_t((pool.geometry.head_dim + 255) / 256);
  hipLaunchKernelGGL(dc::mix_pages_kernel, dim3(uint32_t(n_groups) * uint32_t(n_queries), cblocks), dim3(256), 0,
                     stream, pool, page_ids, token_offsets, n_pages, group_pages, n_queries, weights, weights_stride,
                     out, accumulate);
  return dc::check_hip(hipGetLastError(), who);
}

extern "C" int dc_score_pages(dc_pool pool, const int32_t* page_ids, const int32_t* token_offsets, int32_t n_pages,
                              const float* queries, int32_t n_queries, float* logits, int64_t logits_stride,
                              dc_stream_t stream) {
  return score_launch(pool, page_ids, token_offsets, nullptr, 1, n_pages, queries, n_queries, logits, logits_stride,
                      hipStream_t(stream), "dc_score_pages");
}

extern "C" int dc_mix_pages(dc_pool pool, const int32_t* page_ids, const int32_t* token_offsets, int32_t n_pages,
                            const float* weights, int32_t n_queries, int64_t weights_stride, float* out,
                            int32_t accumulate, dc_stream_t stream) {
  return mix_launch(pool, page_ids, token_offsets, n_pages, nullptr, 1, weights, n_queries, weights_stride, out,
                    accumulate, hipStream_t(stream), "dc_mix_pages");
}

extern "C" int dc_score_pages_grouped(dc_pool pool, const int32_t* page_ids, const int32_t* token_offsets,
                                      const int32_t* page_group, int32_t n_groups, int32_t n_pages,
                                      const float* queries, int32_t n_queries, float* logits, int64_t logits_stride,
                                      dc_stream_t stream) {
  if (n_pages > 0 && !page_group) return dc::fail(DC_EINVAL, "dc_score_pages_grouped: null page_group");
  return score_launch(pool, page_ids, token_offsets, page_group, n_groups, n_pages, queries, n_queries, logits,
                      logits_stride, hipStream_t(stream), "dc_score_pages_grouped");
}

extern "C" int dc_mix_pages_grouped(dc_pool pool, const int32_t* page_ids, const int32_t* token_offsets,
                                    const int32_t* group_pages, int32_t n_groups, int32_t n_pages,
                                    const float* weights, int32_t n_queries, int64_t weights_stride, float* out,
                                    int32_t accumulate, dc_stream_t stream) {
  if (!group_pages) return dc::fail(DC_EINVAL, "dc_mix_pages_grouped: null group_pages");
  return mix_launch(pool, page_ids, token_offsets, n_pages, group_pages, n_groups, weights, n_queries, weights_stride,
                    out, accumulate, hipStream_t(stream), "dc_mix_pages_grouped");
}

namespace dc {

// In-place softmax of each row (reference attention_reference.py:27-31):
// exp(x - max) / sum, fp32, one block per row.
__global__ void __launch_bounds__(256) softmax_rows_kernel(float* __restrict__ x, int32_t n_cols, int64_t stride) {
  float* row = x + int64_t(blockIdx.x) * stride;
  __shared__ float red[4];
  float mx = -INFINITY;
  for (int32_t i = threadIdx.x; i < n_cols; i += blockDim.x) mx = fmaxf(mx, row[i]);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  if (threadIdx.x % 64 == 0) red[threadIdx.x / 64] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  float sum = 0.f;
  for (int32_t i = threadIdx.x; i < n_cols; i += blockDim.x) {
    const float e = expf(row[i] - mx);
    row[i] = e;
    sum += e;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 64);
  if (threadIdx.x % 64 == 0) red[threadIdx.x / 64] = sum;
  __syncthreads();
  sum = red[0] + red[1] + red[2] + red[3];
  for (int32_t i = threadIdx.x; i < n_cols; i += blockDim.x) row[i] = row[i] / sum;
}

}  // namespace dc

extern "C" int dc_softmax_rows(float* x, int32_t n_rows, int32_t n_cols, int64_t stride, dc_stream_t stream) {
  if (n_rows < 0 || n_cols < 0 || (n_rows > 0 && stride < n_cols)) return dc::fail(DC_EINVAL, "dc_softmax_rows: bad shape");
  if (n_rows == 0 || n_cols == 0) return DC_OK;
  if (!x) return dc::fail(DC_EINVAL, "dc_softmax_rows: null pointer");
  hipLaunchKernelGGL(dc::softmax_rows_kernel, dim3(uint32_t(n_rows)), dim3(256), 0, hipStream_t(stream), x, n_cols,
                     stride);
  return dc::check_hip(hipGetLastError(), "dc_softmax_rows launch");
}
