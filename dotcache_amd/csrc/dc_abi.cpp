// Library-level C ABI: error reporting, blob sizes and the host-side decode
// planner.  Host code only (compiled as HIP for the shared hip runtime).
#include <algorithm>
#include <cmath>
#include <cstdint>
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

int32_t dc_abi_version(void) { return 2; }

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
          it.chunk_begin = it.chunk_end = it.reserved = 0;
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

int dc_plan_decode_fill(const int32_t* seq_pages, const int32_t* last_page_tokens, int32_t n_seqs,
                        int32_t n_kv_heads, int32_t chunks_per_page, const float* page_cost, int64_t cost_stride,
                        int32_t target_items,
                        int32_t min_chunks_per_split, dc_work_item* items, int32_t max_items, int32_t* n_items,
                        dc_merge_item* merges, int32_t max_merges, int32_t* n_merges, int32_t* n_partials,
                        int32_t* largest_item) {
  if (!seq_pages || n_seqs <= 0 || n_kv_heads <= 0 || chunks_per_page <= 0 || target_items <= 0 ||
      min_chunks_per_split <= 0 || !n_items || !n_merges || !n_partials || !largest_item)
    return dc::fail(DC_EINVAL, "dc_plan_decode_fill: bad arguments");
  int32_t top = 0;
  for (int32_t b = 0; b < n_seqs; ++b) {
    if (seq_pages[b] <= 0)
      return dc::fail(DC_EINVAL, "decode requires at least one page (sequence %d has %d)", b, seq_pages[b]);
    top = std::max(top, seq_pages[b]);
    if (last_page_tokens && (last_page_tokens[b] <= 0 || last_page_tokens[b] > 32 * chunks_per_page))
      return dc::fail(DC_EINVAL, "dc_plan_decode_fill: sequence %d's last page holds %d tokens (1 .. %d allowed)", b,
                      last_page_tokens[b], 32 * chunks_per_page);
  }
  const int64_t cpp = chunks_per_page;
  // chunks that hold tokens in each sequence's last page (all of them
  // without last_page_tokens): a stream's chunks past its last token are
  // not counted, so no cut falls among them and no item is empty
  auto last_chunks = [&](int32_t b) -> int64_t {
    return last_page_tokens ? std::min<int64_t>(cpp, (last_page_tokens[b] + 31) / 32) : cpp;
  };
  if (int64_t(top) * cpp > INT32_MAX) return dc::fail(DC_EINVAL, "dc_plan_decode_fill: sequence too long");
  if (page_cost && cost_stride < top)
    return dc::fail(DC_EINVAL, "dc_plan_decode_fill: cost_stride %lld is below the longest sequence's %d pages",
                    (long long)cost_stride, top);
  const int32_t S = n_seqs * n_kv_heads;  // streams, s = b * n_kv_heads + h
  // cost of each stream; without page costs every chunk costs 1
  std::vector<double> total(S);
  for (int32_t s = 0; s < S; ++s) {
    const int32_t pages = seq_pages[s / n_kv_heads];
    double w = 0.0;
    if (page_cost) {
      const float* c = page_cost + int64_t(s) * cost_stride;
      for (int32_t p = 0; p < pages; ++p) {
        if (!(c[p] >= 0.f) || !std::isfinite(c[p]))
          return dc::fail(DC_EINVAL, "dc_plan_decode_fill: page cost %g (stream %d, page %d) is not finite and >= 0",
                          double(c[p]), s, p);
        w += c[p];
      }
    } else {
      w = double(pages - 1) * cpp + double(last_chunks(s / n_kv_heads));
    }
    total[s] = w;
  }
  // (1) splits: one item per stream, then one more split at a time for the
  // stream with the largest mean item cost total / splits (compared as
  // products, ties to the longer stream, then the lower index)
  std::vector<int32_t> splits(S, 1);
  auto chunks = [&](int32_t s) {
    const int32_t b = s / n_kv_heads;
    return int64_t(seq_pages[b] - 1) * cpp + last_chunks(b);
  };
  auto before = [&](int32_t x, int32_t y) {  // true when x's items rank below y's
    const double lx = total[x] * splits[y], ly = total[y] * splits[x];
    if (lx != ly) return lx < ly;
    if (chunks(x) != chunks(y)) return chunks(x) < chunks(y);
    return x > y;
  };
  std::vector<int32_t> heap(S);
  for (int32_t s = 0; s < S; ++s) heap[s] = s;
  std::make_heap(heap.begin(), heap.end(), before);
  int64_t used = S;
  while (used < target_items) {
    std::pop_heap(heap.begin(), heap.end(), before);
    const int32_t s = heap.back();
    if (chunks(s) / (splits[s] + 1) < min_chunks_per_split) break;
    ++splits[s];
    ++used;
    std::push_heap(heap.begin(), heap.end(), before);
  }
  // (2) cuts at whole chunks: without costs split i of n covers
  // [i len / n, (i + 1) len / n); with costs, cut i is the last chunk
  // boundary whose cost prefix stays within i / n of the stream's cost
  // (keeping every item non-empty)
  int32_t ni = 0, nm = 0, np = 0, largest = 0;
  std::vector<double> prefix;
  std::vector<int64_t> cut;
  for (int32_t s = 0; s < S; ++s) {
    const int32_t b = s / n_kv_heads, h = s % n_kv_heads, n = splits[s];
    const int64_t len = chunks(s);
    cut.assign(n + 1, 0);
    cut[n] = len;
    if (page_cost && total[s] > 0.0 && n > 1) {
      const float* c = page_cost + int64_t(s) * cost_stride;
      // a page's cost spread over its chunks (the last page's over the
      // chunks that hold tokens)
      const int64_t full = int64_t(seq_pages[b] - 1) * cpp;
      const double last_n = double(len - full);
      prefix.assign(len + 1, 0.0);
      for (int64_t u = 0; u < len; ++u)
        prefix[u + 1] = prefix[u] + double(c[u / cpp]) / (u < full ? double(cpp) : last_n);
      for (int32_t i = 1; i < n; ++i) {
        const double goal = total[s] * i / n * (1.0 + 1e-12);
        int64_t u = int64_t(std::upper_bound(prefix.begin(), prefix.end(), goal) - prefix.begin()) - 1;
        u = std::min<int64_t>(std::max<int64_t>(u, cut[i - 1] + 1), len - (n - i));
        cut[i] = u;
      }
    } else {
      for (int32_t i = 1; i < n; ++i) cut[i] = len * i / n;
    }
    const int32_t first_partial = np;
    for (int32_t i = 0; i < n; ++i) {
      const int64_t u0 = cut[i], u1 = cut[i + 1];
      largest = std::max<int32_t>(largest, int32_t(u1 - u0));
      if (items && ni < max_items) {
        dc_work_item& it = items[ni];
        it.seq = b;
        it.kv_head = h;
        it.page_begin = int32_t(u0 / cpp);
        it.chunk_begin = int32_t(u0 % cpp);
        it.page_end = int32_t((u1 + cpp - 1) / cpp);
        it.chunk_end = int32_t(u1 % cpp);
        it.partial = n > 1 ? np : -1;
        it.reserved = 0;
      }
      ++ni;
      if (n > 1) ++np;
    }
    if (n > 1) {
      if (merges && nm < max_merges) merges[nm] = dc_merge_item{b, h, first_partial, n};
      ++nm;
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
