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

// grid.x = page index, grid.y = query chunk; one thread per token.
__global__ void __launch_bounds__(256) score_pages_kernel(dc_pool pool, const int32_t* __restrict__ page_ids,
                                                          const int32_t* __restrict__ token_offsets,
                                                          const float* __restrict__ queries, int32_t n_queries,
                                                          float* __restrict__ logits, int64_t logits_stride) {
  const int32_t i = blockIdx.x;
  const int32_t q0 = blockIdx.y * kScoreQ;
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

// grid.x = query, grid.y = channel block; one thread per channel, looping
// over every page and token.
__global__ void __launch_bounds__(256) mix_pages_kernel(dc_pool pool, const int32_t* __restrict__ page_ids,
                                                        const int32_t* __restrict__ token_offsets, int32_t n_pages,
                                                        const float* __restrict__ weights, int64_t weights_stride,
                                                        float* __restrict__ out, int32_t accumulate) {
  const int32_t q = blockIdx.x;
  const int32_t c = blockIdx.y * blockDim.x + threadIdx.x;
  const dc_page_geometry geo = pool.geometry;
  if (c >= geo.head_dim) return;
  const float* w = weights + int64_t(q) * weights_stride;
  float acc = 0.f;
  for (int32_t i = 0; i < n_pages; ++i) {
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

extern "C" int dc_score_pages(dc_pool pool, const int32_t* page_ids, const int32_t* token_offsets, int32_t n_pages,
                              const float* queries, int32_t n_queries, float* logits, int64_t logits_stride,
                              dc_stream_t stream) {
  if (int rc = dc::validate_geometry(pool.geometry)) return rc;
  if (n_pages < 0 || n_queries < 0) return dc::fail(DC_EINVAL, "counts must be non-negative");
  if (n_pages == 0 || n_queries == 0) return DC_OK;
  if (!page_ids || !token_offsets || !queries || !logits || !pool.arena || !pool.descs)
    return dc::fail(DC_EINVAL, "dc_score_pages: null pointer");
  const uint32_t qchunks = uint32_t((n_queries + dc::kScoreQ - 1) / dc::kScoreQ);
  hipLaunchKernelGGL(dc::score_pages_kernel, dim3(uint32_t(n_pages), qchunks), dim3(128), 0, hipStream_t(stream),
                     pool, page_ids, token_offsets, queries, n_queries, logits, logits_stride);
  return dc::check_hip(hipGetLastError(), "dc_score_pages launch");
}

extern "C" int dc_mix_pages(dc_pool pool, const int32_t* page_ids, const int32_t* token_offsets, int32_t n_pages,
                            const float* weights, int32_t n_queries, int64_t weights_stride, float* out,
                            int32_t accumulate, dc_stream_t stream) {
  if (int rc = dc::validate_geometry(pool.geometry)) return rc;
  if (n_pages < 0 || n_queries < 0) return dc::fail(DC_EINVAL, "counts must be non-negative");
  if (n_queries == 0) return DC_OK;
  if (!weights || !out || (n_pages > 0 && (!page_ids || !token_offsets || !pool.arena || !pool.descs)))
    return dc::fail(DC_EINVAL, "dc_mix_pages: null pointer");
  const uint32_t cblocks = uint32_t((pool.geometry.head_dim + 255) / 256);
  hipLaunchKernelGGL(dc::mix_pages_kernel, dim3(uint32_t(n_queries), cblocks), dim3(256), 0, hipStream_t(stream),
                     pool, page_ids, token_offsets, n_pages, weights, weights_stride, out, accumulate);
  return dc::check_hip(hipGetLastError(), "dc_mix_pages launch");
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
