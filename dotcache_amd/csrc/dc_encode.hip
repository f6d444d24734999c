// M0 / M3 page encode and token append (gfx950).
//
// One thread per (row, group): min/max (or max |x|) over the group's
// channels, the fp32 scale, round-half-even codes, and little-endian packing
// straight into the page blob.  Bit-exact with reference
// dotcache/modes/m0_affine.py:15-53 + dotcache/packing.py:14-48 +
// dotcache/encode.py:399-445: every step is one IEEE fp32 operation
// (subtract, correctly rounded divide, max), rintf rounds half to even like
// np.round, and scales / biases are rounded to fp16 with RNE after the codes
// were computed from the fp32 scale.  This file is compiled with
// -ffp-contract=off so no step is fused.
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

}  // namespace dc

extern "C" int dc_encode_rows(const void* values, int32_t values_dtype, int64_t n_rows, int64_t row_stride,
                              const int32_t* row_page, const int32_t* row_slot, dc_pool pool,
                              dc_stream_t stream) {
  if (int rc = dc::validate_geometry(pool.geometry)) return rc;
  if (n_rows < 0) return dc::fail(DC_EINVAL, "n_rows must be non-negative");
  if (n_rows == 0) return DC_OK;
  if (!values || !row_page || !row_slot || !pool.arena || !pool.descs)
    return dc::fail(DC_EINVAL, "dc_encode_rows: null pointer");
  if (values_dtype != DC_F32 && values_dtype != DC_F16 && values_dtype != DC_BF16)
    return dc::fail(DC_EINVAL, "values_dtype must be DC_F32, DC_F16 or DC_BF16");
  if (row_stride < pool.geometry.head_dim) return dc::fail(DC_EINVAL, "row_stride is smaller than head_dim");
  const int32_t G = dc::num_groups(pool.geometry);
  const int64_t threads = n_rows * G;
  const int64_t blocks = (threads + 255) / 256;
  if (blocks > 0x7fffffff) return dc::fail(DC_EINVAL, "too many rows");
  hipLaunchKernelGGL(dc::encode_rows_kernel, dim3(uint32_t(blocks)), dim3(256), 0, hipStream_t(stream), values,
                     values_dtype, n_rows, row_stride, row_page, row_slot, pool, G);
  return dc::check_hip(hipGetLastError(), "dc_encode_rows launch");
}
