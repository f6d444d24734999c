// Library-level C ABI: error reporting, blob sizes and the host-side decode
// planner.  Host code only (compiled as HIP for the shared hip runtime).
#include <cstdarg>
#include <cstdio>
#include <cstring>

#include "dc_common.h"

namespace dc {

static thread_local char g_last_error[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return DC_OK;
  return fail(DC_EDEVICE, "%s: %s", what, hipGetErrorString(e));
}

bool valid_format(int32_t fmt, int32_t bits) {
  if (fmt == DC_FMT_M0_AFFINE || fmt == DC_FMT_M0_SYMMETRIC)
    return bits == 2 || bits == 3 || bits == 4 || bits == 8;
  return fmt == DC_FMT_M3_F16 || fmt == DC_FMT_M3_F32 || fmt == DC_FMT_M3_I8;
}

int validate_geometry(const dc_page_geometry& g) {
  if (g.head_dim <= 0 || g.group_size <= 0 || g.page_capacity <= 0)
    return fail(DC_EINVAL, "geometry must have positive head_dim, group_size and page_capacity");
  if (g.layout != 0 && g.layout != 1) return fail(DC_EINVAL, "layout must be 0 (group_major) or 1 (token_major)");
  if (g.page_capacity > 65535) return fail(DC_EINVAL, "page_capacity exceeds 65535");
  return DC_OK;
}

}  // namespace dc

extern "C" {

const char* dc_last_error(void) { return dc::g_last_error; }

int32_t dc_abi_version(void) { return 1; }

int64_t dc_page_blob_bytes(int32_t format, int32_t bits, dc_page_geometry geometry) {
  if (!dc::valid_format(format, bits) || dc::validate_geometry(geometry) != DC_OK) return -1;
  const int64_t t = dc::blob_layout(format, bits, geometry).total;
  return (t + 255) & ~int64_t(255);
}

int64_t dc_page_read_bytes(int32_t format, int32_t bits, int32_t tokens, dc_page_geometry geometry) {
  if (!dc::valid_format(format, bits) || dc::validate_geometry(geometry) != DC_OK) return -1;
  const int64_t G = dc::num_groups(geometry);
  const int64_t T = tokens;
  switch (format) {
    case DC_FMT_M0_AFFINE:
      return T * G * dc::words_per_group(geometry.group_size, bits) * 4 + T * G * 4;
    case DC_FMT_M0_SYMMETRIC:
      return T * G * dc::words_per_group(geometry.group_size, bits) * 4 + T * G * 2;
    case DC_FMT_M3_F16:
      return T * geometry.head_dim * 2;
    case DC_FMT_M3_F32:
      return T * geometry.head_dim * 4;
    default:
      return T * geometry.head_dim + T * 2;
  }
}

int dc_plan_decode(const int32_t* seq_pages, int32_t n_seqs, int32_t n_kv_heads, int32_t pages_per_split,
                   dc_work_item* items, int32_t max_items, int32_t* n_items, dc_merge_item* merges,
                   int32_t max_merges, int32_t* n_merges, int32_t* n_partials) {
  if (!seq_pages || n_seqs <= 0 || n_kv_heads <= 0 || !n_items || !n_merges || !n_partials)
    return dc::fail(DC_EINVAL, "dc_plan_decode: bad arguments");
  int32_t ni = 0, nm = 0, np = 0;
  for (int32_t b = 0; b < n_seqs; ++b) {
    const int32_t pages = seq_pages[b];
    if (pages <= 0) return dc::fail(DC_EINVAL, "decode requires at least one page (sequence %d has %d)", b, pages);
    const int32_t per = pages_per_split > 0 ? pages_per_split : pages;
    const int32_t splits = (pages + per - 1) / per;
    for (int32_t h = 0; h < n_kv_heads; ++h) {
      const int32_t first_partial = np;
      for (int32_t s = 0; s < splits; ++s) {
        if (items && ni < max_items) {
          // near-equal splits (sizes differ by at most one page), so no item
          // is a short remainder and none exceeds pages_per_split
          dc_work_item& it = items[ni];
          it.seq = b;
          it.kv_head = h;
          it.page_begin = int32_t(int64_t(s) * pages / splits);
          it.page_end = int32_t(int64_t(s + 1) * pages / splits);
          it.partial = splits > 1 ? np : -1;
          it.reserved[0] = it.reserved[1] = it.reserved[2] = 0;
        }
        ++ni;
        if (splits > 1) ++np;
      }
      if (splits > 1) {
        if (merges && nm < max_merges) merges[nm] = dc_merge_item{b, h, first_partial, splits};
        ++nm;
      }
    }
  }
  *n_items = ni;
  *n_merges = nm;
  *n_partials = np;
  if (ni > max_items || nm > max_merges)
    return dc::fail(DC_ESPACE, "dc_plan_decode: need %d items and %d merges", ni, nm);
  return DC_OK;
}

int64_t dc_decode_workspace_bytes(int32_t n_partials, int32_t n_q, int32_t head_dim) {
  // per partial: o [n_q][head_dim] fp32, then (m, l) [n_q][2] fp32
  return int64_t(n_partials) * n_q * (head_dim + 2) * 4;
}

}  // extern "C"
