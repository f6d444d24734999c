// Allocation-free fused decode (dc_decode_paged_noalloc): the split-K
// partials live in a static per-GPU device array instead of a caller
// workspace, for callers that cannot allocate device memory.  The kernels
// are dc_decode_paged's.
#include <mutex>

#include "dc_common.h"
#include "dc_decode.h"

// The partials live in this file-scope device array.  Each GPU holds its own copy
// (at its own address) for the life of the process.  In host code the name
// `scratch` is only a host-side stand-in for the symbol: its device address
// comes from hipGetSymbolAddress, once per device, and only that address is
// ever passed to a kernel.
namespace dc {

constexpr int64_t kScratchBytes = int64_t(32) << 20;  // 32 MiB per GPU
constexpr int kMaxDevices = 64;

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices] = {};

// Device address of the current device's scratch array (looked up on the
// first call on that device, with that device current).
static int scratch_of_current_device(void** out) {
  int dev = -1;
  if (int rc = check_hip(hipGetDevice(&dev), "hipGetDevice")) return rc;
  if (dev < 0 || dev >= kMaxDevices) return fail(DC_EDEVICE, "device %d: more than %d devices", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    if (int rc = check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)")) return rc;
    if (!p) return fail(DC_EDEVICE, "hipGetSymbolAddress(scratch) returned null on device %d", dev);
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return DC_OK;
}

}  // namespace dc

extern "C" int64_t dc_decode_noalloc_scratch_bytes(void) { return dc::kScratchBytes; }

extern "C" int dc_decode_paged_noalloc(dc_pool k_pool, dc_pool v_pool, const int32_t* k_table, const int32_t* v_table,
                                       int32_t table_stride, const dc_work_item* items, int32_t n_items,
                                       const dc_merge_item* merges, int32_t n_merges, int32_t n_partials,
                                       const void* queries, int32_t queries_dtype, float query_scale, int32_t n_seqs,
                                       int32_t n_kv_heads, int32_t n_q, float* out, dc_stream_t stream) {
  if (n_partials < 0) return dc::fail(DC_EINVAL, "dc_decode_paged_noalloc: n_partials must be non-negative");
  if (n_q <= 0 || n_q > dc::kMaxQ) return dc::fail(DC_EINVAL, "n_q must be in [1, %d]", dc::kMaxQ);
  const int64_t need = dc_decode_workspace_bytes(n_partials, n_q, k_pool.geometry.head_dim);
  if (need > dc::kScratchBytes)
    return dc::fail(DC_ESPACE,
                    "dc_decode_paged_noalloc: %d split-K partials of %d heads x head_dim %d need %lld bytes; the "
                    "static scratch holds %lld (use dc_decode_paged with a workspace, or fewer splits)",
                    n_partials, n_q, k_pool.geometry.head_dim, (long long)need, (long long)dc::kScratchBytes);
  void* ws = nullptr;
  if (n_items > 0)
    if (int rc = dc::scratch_of_current_device(&ws)) return rc;
  // exactly n_partials slots: an item naming a slot past them is skipped
  return dc_decode_paged(k_pool, v_pool, k_table, v_table, table_stride, items, n_items, merges, n_merges, queries,
                         queries_dtype, query_scale, n_seqs, n_kv_heads, n_q, out, ws, need, stream);
}
