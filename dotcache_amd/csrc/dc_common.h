// Shared device/host helpers for the compressed-page kernels (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <hip/hip_bf16.h>
#include <stdint.h>

#include "../../include/dotcache_hip.h"

namespace dc {

// Blob offsets of a page; see the page-arena comment in dotcache_hip.h.
struct BlobLayout {
  int32_t groups;         // G = ceil(head_dim / group_size)
  int32_t words;          // W = ceil(group_size * bits / 32)
  int64_t payload_bytes;  // G * C * W * 4
  int64_t scales_off;
  int64_t bias_off;
  int64_t total;
};

__host__ __device__ inline int64_t align16(int64_t x) { return (x + 15) & ~int64_t(15); }

__host__ __device__ inline int32_t words_per_group(int32_t group_size, int32_t bits) {
  return (group_size * bits + 31) / 32;
}

__host__ __device__ inline int32_t num_groups(const dc_page_geometry& g) {
  return (g.head_dim + g.group_size - 1) / g.group_size;
}

__host__ __device__ inline bool is_m0(int32_t fmt) {
  return fmt == DC_FMT_M0_AFFINE || fmt == DC_FMT_M0_SYMMETRIC;
}

__host__ __device__ inline BlobLayout blob_layout(int32_t fmt, int32_t bits, const dc_page_geometry& g) {
  BlobLayout L{};
  const int64_t C = g.page_capacity;
  L.groups = num_groups(g);
  if (is_m0(fmt)) {
    L.words = words_per_group(g.group_size, bits);
    L.payload_bytes = int64_t(L.groups) * C * L.words * 4;
    L.scales_off = align16(L.payload_bytes);
    L.bias_off = L.scales_off + align16(C * L.groups * 2);
    L.total = fmt == DC_FMT_M0_AFFINE ? L.bias_off + align16(C * L.groups * 2) : L.bias_off;
  } else if (fmt == DC_FMT_M3_F16) {
    L.payload_bytes = C * g.head_dim * 2;
    L.scales_off = L.bias_off = L.total = align16(L.payload_bytes);
  } else if (fmt == DC_FMT_M3_F32) {
    L.payload_bytes = C * g.head_dim * 4;
    L.scales_off = L.bias_off = L.total = align16(L.payload_bytes);
  } else {  // DC_FMT_M3_I8
    L.payload_bytes = C * g.head_dim;
    L.scales_off = align16(L.payload_bytes);
    L.bias_off = L.scales_off + align16(C * 2);
    L.total = L.bias_off;
  }
  return L;
}

__device__ __forceinline__ const uint8_t* blob_ptr(const void* arena, const dc_page_desc& d) {
  return reinterpret_cast<const uint8_t*>(arena) + (uint64_t(d.block) << 8);
}

__device__ __forceinline__ float load_value(const void* p, int32_t dtype, int64_t i) {
  if (dtype == DC_F32) return reinterpret_cast<const float*>(p)[i];
  if (dtype == DC_F16) return __half2float(reinterpret_cast<const __half*>(p)[i]);
  return __bfloat162float(reinterpret_cast<const __hip_bfloat16*>(p)[i]);
}

// Code of channel k (0 <= k < group_size) of (token t, group g) in an M0 page.
// Symbols are packed little-endian; a symbol that crosses a word boundary
// continues in the low bits of the next word (reference packing.py:38-48).
__device__ __forceinline__ uint32_t m0_code(const uint32_t* payload, int32_t t, int32_t g, int32_t k, int32_t bits,
                                            int32_t W, int32_t G, int32_t C, int32_t layout) {
  const int64_t base = layout == 0 ? (int64_t(g) * C + t) * W : (int64_t(t) * G + g) * W;
  const int32_t bit = k * bits;
  const int32_t wi = bit >> 5, off = bit & 31;
  uint32_t v = payload[base + wi] >> off;
  if (off + bits > 32) v |= payload[base + wi + 1] << (32 - off);
  return v & ((1u << bits) - 1u);
}

// Dequantised value of (token t, channel c) for any page format; channels
// past head_dim of an M3 page read as 0.
__device__ __forceinline__ float page_value(const uint8_t* blob, const dc_page_desc& d, const BlobLayout& L,
                                            const dc_page_geometry& geo, int32_t t, int32_t c) {
  if (is_m0(d.format)) {
    const int32_t g = c / geo.group_size, k = c - g * geo.group_size;
    const uint32_t code = m0_code(reinterpret_cast<const uint32_t*>(blob), t, g, k, d.bits, L.words, L.groups,
                                  geo.page_capacity, geo.layout);
    const float s = __half2float(reinterpret_cast<const __half*>(blob + L.scales_off)[t * L.groups + g]);
    if (d.format == DC_FMT_M0_AFFINE) {
      const float b = __half2float(reinterpret_cast<const __half*>(blob + L.bias_off)[t * L.groups + g]);
      return s * float(code) + b;
    }
    return s * (float(code) - float((1 << (d.bits - 1)) - 1));
  }
  if (c >= geo.head_dim) return 0.f;
  const int64_t i = int64_t(t) * geo.head_dim + c;
  if (d.format == DC_FMT_M3_F16) return __half2float(reinterpret_cast<const __half*>(blob)[i]);
  if (d.format == DC_FMT_M3_F32) return reinterpret_cast<const float*>(blob)[i];
  const float rs = __half2float(reinterpret_cast<const __half*>(blob + L.scales_off)[t]);
  return float(reinterpret_cast<const int8_t*>(blob)[i]) * rs;
}

// Per-thread status text for dc_last_error().
int fail(int code, const char* fmt, ...);
int check_hip(hipError_t e, const char* what);
bool valid_format(int32_t fmt, int32_t bits);
int validate_geometry(const dc_page_geometry& g);

}  // namespace dc
