// Library-level C ABI: error reporting, blob sizes and the host-side decode
// planner.  Host code only (compiled as HIP for the shared hip runtime).
#include <algorithm>
#include <vector>
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

int dc_plan_decode_fill(const int32_t* seq_pages, int32_t n_seqs, int32_t n_kv_heads, int32_t target_items,
                        int32_t min_pages_per_split, dc_work_item* items, int32_t max_items, int32_t* n_items,
                        dc_merge_item* merges, int32_t max_merges, int32_t* n_merges, int32_t* n_partials,
                        int32_t* largest_item) {
  if (!seq_pages || n_seqs <= 0 || n_kv_heads <= 0 || target_items <= 0 || min_pages_per_split <= 0 || !n_items ||
      !n_merges || !n_partials || !largest_item)
    return dc::fail(DC_EINVAL, "dc_plan_decode_fill: bad arguments");
  int32_t top = 1;
  for (int32_t b = 0; b < n_seqs; ++b) {
    if (seq_pages[b] <= 0)
      return dc::fail(DC_EINVAL, "decode requires at least one page (sequence %d has %d)", b, seq_pages[b]);
    top = std::max(top, seq_pages[b]);
  }
  // (1) the smallest pages-per-split (at least min_pages_per_split) whose
  // near-equal splits fit target_items
  auto count = [&](int64_t per) {
    int64_t c = 0;
    for (int32_t b = 0; b < n_seqs; ++b) c += (seq_pages[b] + per - 1) / per;
    return c * n_kv_heads;
  };
  int64_t lo = std::min<int64_t>(min_pages_per_split, top), hi = top;
  if (count(hi) <= target_items) {
    while (lo < hi) {
      const int64_t mid = (lo + hi) / 2;
      if (count(mid) <= target_items)
        hi = mid;
      else
        lo = mid + 1;
    }
  }
  std::vector<int32_t> splits(n_seqs);
  int64_t used = 0;
  for (int32_t b = 0; b < n_seqs; ++b) {
    splits[b] = int32_t((seq_pages[b] + hi - 1) / hi);
    used += int64_t(splits[b]) * n_kv_heads;
  }
  // (2) the items left in the budget go, one sequence (all its heads) at a
  // time, to the sequence with the largest items, while its items keep at
  // least min_pages_per_split pages
  for (;;) {
    if (used + n_kv_heads > target_items) break;
    // largest mean item pages[b] / splits[b] (compared exactly), ties to
    // the longer sequence
    int32_t best = -1;
    for (int32_t b = 0; b < n_seqs; ++b) {
      if (seq_pages[b] / (splits[b] + 1) < min_pages_per_split) continue;
      if (best < 0) {
        best = b;
        continue;
      }
      const int64_t lhs = int64_t(seq_pages[b]) * splits[best], rhs = int64_t(seq_pages[best]) * splits[b];
      if (lhs > rhs || (lhs == rhs && seq_pages[b] > seq_pages[best])) best = b;
    }
    if (best < 0) break;
    ++splits[best];
    used += n_kv_heads;
  }
  int32_t ni = 0, nm = 0, np = 0, largest = 0;
  for (int32_t b = 0; b < n_seqs; ++b) {
    const int32_t pages = seq_pages[b], sp = splits[b];
    for (int32_t h = 0; h < n_kv_heads; ++h) {
      const int32_t first_partial = np;
      for (int32_t s = 0; s < sp; ++s) {
        const int32_t pb = int32_t(int64_t(s) * pages / sp), pe = int32_t(int64_t(s + 1) * pages / sp);
        largest = std::max(largest, pe - pb);
        if (items && ni < max_items) {
          dc_work_item& it = items[ni];
          it.seq = b;
          it.kv_head = h;
          it.page_begin = pb;
          it.page_end = pe;
          it.partial = sp > 1 ? np : -1;
          it.reserved[0] = it.reserved[1] = it.reserved[2] = 0;
        }
        ++ni;
        if (sp > 1) ++np;
      }
      if (sp > 1) {
        if (merges && nm < max_merges) merges[nm] = dc_merge_item{b, h, first_partial, sp};
        ++nm;
      }
    }
  }
  *n_items = ni;
  *n_merges = nm;
  *n_partials = np;
  *largest_item = largest;
  if (ni > max_items || nm > max_merges)
    return dc::fail(DC_ESPACE, "dc_plan_decode_fill: need %d items and %d merges", ni, nm);
  return DC_OK;
}

int64_t dc_decode_workspace_bytes(int32_t n_partials, int32_t n_q, int32_t head_dim) {
  // per partial: o [n_q][head_dim] fp32, then (m, l) [n_q][2] fp32
  return int64_t(n_partials) * n_q * (head_dim + 2) * 4;
}

}  // extern "C"
