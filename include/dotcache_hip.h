/*
 * dotcache_hip.h -- C ABI of the MI355X compressed-page decode-attention
 * backend (libdotcache_hip.so, built for gfx950).
 *
 * All pointers marked (device) are HBM addresses; all sizes are in elements
 * unless named *_bytes.  Every entry point returns 0 on success and a
 * non-zero DC_E* status otherwise; dc_last_error() then returns a message.
 * Host bindings map DC_EINVAL to ValueError and the other codes to
 * RuntimeError, the error convention of the reference's backend surface
 * (reference dotcache/attention_runtime.py:39-60).
 *
 * Work is enqueued on the given HIP stream (0 = default stream); nothing
 * synchronises unless stated.  No entry point allocates device memory: the
 * caller owns the page arena, descriptor tables, page tables, outputs and
 * workspace.
 *
 * ---- page arena and page blobs --------------------------------------
 * Pages live in one caller-owned byte arena.  A page blob starts at
 * arena + 256 * desc.block and holds, for capacity C = geometry.page_capacity
 * tokens (the token stride; desc.tokens <= C are valid):
 *
 *   M0 (affine / symmetric, b-bit codes, G groups, W = ceil(gs*b/32) words):
 *     payload  uint32 [G][C][W]   group_major   (or [C][G][W] token_major)
 *     scales   fp16   [C][G]      at align16(payload bytes)
 *     bias     fp16   [C][G]      after scales (affine only)
 *   M3 fp16 : fp16 [C][head_dim]
 *   M3 fp32 : fp32 [C][head_dim]
 *   M3 int8 : int8 [C][head_dim], then fp16 [C] row scales at align16
 *
 * which is the reference page contract: payload [G, T, W] uint32 packed
 * little-endian (reference dotcache/packing.py:14-48,
 * dotcache/page_format.py:19-23), scales / bias [T, G] fp16
 * (reference dotcache/encode.py:427-428), escape rows [T, head_dim]
 * (reference dotcache/modes/m3_escape.py:10-19).
 */
#ifndef DOTCACHE_HIP_H
#define DOTCACHE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* dc_stream_t; /* a hipStream_t */

enum dc_status {
  DC_OK = 0,
  DC_EINVAL = 1,   /* bad shape / mode / unsupported page  -> ValueError   */
  DC_EDEVICE = 2,  /* HIP runtime failure                   -> RuntimeError */
  DC_ESPACE = 3,   /* workspace or table too small          -> RuntimeError */
};

enum dc_page_format {
  DC_FMT_M3_F16 = 0,       /* exact fp16 escape rows                      */
  DC_FMT_M0_AFFINE = 1,    /* s * c + b                                   */
  DC_FMT_M0_SYMMETRIC = 2, /* s * (c - (2^(b-1) - 1))                     */
  DC_FMT_M3_F32 = 3,       /* fp32 escape rows                            */
  DC_FMT_M3_I8 = 4,        /* int8 rows * fp16 row scale                  */
};

enum dc_dtype { DC_F32 = 0, DC_F16 = 1, DC_BF16 = 2 };

/* One page: where its blob is and how to read it (8 bytes). */
typedef struct dc_page_desc {
  uint32_t block;  /* blob byte offset / 256                               */
  uint16_t tokens; /* valid tokens (<= page_capacity)                      */
  uint8_t format;  /* dc_page_format                                       */
  uint8_t bits;    /* M0 code width: 2, 3, 4 or 8 (ignored for M3)         */
} dc_page_desc;

/* The key and value descriptors of one page of a work item, gathered ahead
 * of a decode (dc_gather_page_records). */
typedef struct dc_page_record {
  dc_page_desc key;
  dc_page_desc value;
} dc_page_record;

/* Geometry shared by every page of one call (one layer's pages). */
typedef struct dc_page_geometry {
  int32_t head_dim;
  int32_t group_size;
  int32_t page_capacity; /* token stride of a blob (tokens_per_page)        */
  int32_t layout;        /* 0 = group_major, 1 = token_major                */
} dc_page_geometry;

/* A view of one page pool: the arena and its descriptor table.  Kernels
 * skip (never read) a page whose id is outside [0, n_descs) or whose blob
 * would end past arena_bytes; hosts validate tables before calling, this
 * is a fault guard only. */
typedef struct dc_pool {
  void* arena;               /* device                                  */
  int64_t arena_bytes;
  const dc_page_desc* descs; /* device [n_descs]                        */
  int32_t n_descs;
  dc_page_geometry geometry;
  /* bit (format * 9 + bits) is set for every page format the pool may
   * hold (bits = 0 for M3); decode picks its kernel from this set, so a
   * page whose format is not in the mask must not be in the pool */
  uint64_t format_mask;
} dc_pool;

/* One unit of decode work: pages [page_begin, page_end) of one
 * (sequence, kv_head).  partial < 0: the item covers the whole sequence and
 * writes the normalised output; otherwise it writes split-K partial
 * (m, l, o) slot `partial`.  An item may start and end inside a page, on
 * 32-token chunk boundaries: it skips the first chunk_begin chunks of page
 * page_begin and, when chunk_end > 0, stops after chunk chunk_end - 1 of
 * page page_end - 1 (with one page, chunks [chunk_begin, chunk_end) of it).
 * Both 0 (as dc_plan_decode writes them) cover whole pages.  Valid values:
 * 0 <= chunk_begin < ceil(page_capacity / 32), 0 <= chunk_end <=
 * ceil(page_capacity / 32). */
typedef struct dc_work_item {
  int32_t seq;
  int32_t kv_head;
  int32_t page_begin;
  int32_t page_end;
  int32_t partial;
  int32_t chunk_begin;
  int32_t chunk_end;
  int32_t reserved;
} dc_work_item;

/* Log-sum-exp merge of partials [partial_begin, partial_begin + count) into
 * the output of (seq, kv_head). */
typedef struct dc_merge_item {
  int32_t seq;
  int32_t kv_head;
  int32_t partial_begin;
  int32_t count;
} dc_merge_item;

/* Pages [page_begin, page_end) of a merge item's stream that the merge
 * itself attends (dc_window_merge): fp16 (M3) key and value pages, such as
 * an exact recent window, read by no work item. */
typedef struct dc_window_range {
  int32_t page_begin;
  int32_t page_end;
} dc_window_range;

/* ---- library ---------------------------------------------------------- */

/* Message for the last non-zero status returned on this thread. */
const char* dc_last_error(void);

/* ABI version (bumped on any signature or layout change). */
int32_t dc_abi_version(void);

/* Bytes of one page blob of the given format (host only, no GPU call).
 * Replaces the byte accounting of reference dotcache/types.py:85-106 for
 * device residency (EncodedPage.payload_nbytes + scales/bias). */
int64_t dc_page_blob_bytes(int32_t format, int32_t bits, dc_page_geometry geometry);

/* Compressed bytes a reader fetches for `tokens` valid tokens of a page
 * (codes + fp16 scales/bias, or escape rows): the roofline's
 * algorithmic-bytes figure.  Host only. */
int64_t dc_page_read_bytes(int32_t format, int32_t bits, int32_t tokens, dc_page_geometry geometry);

/* ---- write path ------------------------------------------------------- */

/* Encode rows values[r, :head_dim] (dtype DC_F32/F16/BF16, row stride
 * `row_stride` elements) into token slot row_slot[r] of page
 * row_page[r] of the arena, using that page's format.  M0 scales and
 * codes are per (token, group), so encoding a page row by row is
 * bit-identical to encoding it whole; this one entry point is both the page
 * encoder and the per-step append of a new token.  Does not change
 * desc.tokens (the caller owns page fill counts).
 * Replaces reference dotcache/encode.py:122-445 (encode_page, M0 and M3
 * branches) with dotcache/modes/m0_affine.py:15-53 and
 * dotcache/packing.py:14-48, and the tail append of
 * dotcache/model_kv_cache.py:3830-4025.  Bit-exact with them. */
int dc_encode_rows(const void* values, int32_t values_dtype, int64_t n_rows, int64_t row_stride,
                   const int32_t* row_page /* device [n_rows] */,
                   const int32_t* row_slot /* device [n_rows] */,
                   dc_pool pool, dc_stream_t stream);

/* The keys and values of the same new tokens in one launch: k_values rows
 * into (k_row_page, k_row_slot) of k_pool and v_values rows into
 * (v_row_page, v_row_slot) of v_pool, each as dc_encode_rows would (both
 * arrays have n_rows rows of one dtype and row stride).  The per-step append
 * of a decode writes both (reference dotcache/model_kv_cache.py:3830-3902,
 * append_step, encoding K and V pages at :789-830). */
int dc_encode_rows_kv(const void* k_values, const void* v_values, int32_t values_dtype, int64_t n_rows,
                      int64_t row_stride, const int32_t* k_row_page, const int32_t* k_row_slot,
                      const int32_t* v_row_page, const int32_t* v_row_slot, dc_pool k_pool, dc_pool v_pool,
                      dc_stream_t stream);

/* Process-wide encode kernel choice: 0 (default) runs the wavefront kernel
 * (8 channels per lane, several rows per wavefront) wherever the pool's
 * geometry fits it, 1 always runs the general one-thread-per-group kernel
 * (for cross-checking the two).  Host only; not thread-safe. */
int dc_set_encode_path(int32_t path);

/* ---- read path: per-page entry points (score_page / mix_page) ------- */

/* logits[q, token_offsets[i] + t] = score of query q against token t of
 * page page_ids[i], for n_queries fp32 queries [n_queries, head_dim].
 * token_offsets (device, [n_pages]) gives where each page's logits start:
 * the prefix sum of page token counts, or the starts of a subset of a
 * longer row (the pages whose logits are not cached).  Replaces reference dotcache/attention_reference.py:34-128
 * (score_page_ref) behind dotcache/backends/torch_cuda.py:53-68
 * (score_page_cuda / score_pages_cuda). */
int dc_score_pages(dc_pool pool, const int32_t* page_ids, const int32_t* token_offsets, int32_t n_pages,
                   const float* queries, int32_t n_queries, float* logits, int64_t logits_stride,
                   dc_stream_t stream);

/* out[q, :head_dim] (+)= sum_i weights[q, token_offsets[i] + t] * V(page_ids[i])[t, :].
 * accumulate != 0 adds into out (the out_acc of the reference).  Replaces
 * reference dotcache/attention_reference.py:131-194 (mix_page_ref) behind
 * dotcache/backends/torch_cuda.py:71-78 (mix_page_cuda). */
int dc_mix_pages(dc_pool pool, const int32_t* page_ids, const int32_t* token_offsets, int32_t n_pages,
                 const float* weights, int32_t n_queries, int64_t weights_stride, float* out,
                 int32_t accumulate, dc_stream_t stream);

/* Grouped forms of dc_score_pages / dc_mix_pages: one launch for G groups
 * of pages, each with its own n_queries queries, as the batched grouped
 * decode that returns logits needs (reference
 * dotcache/backends/torch_mps.py:4110-4273, behind
 * dotcache/backends/torch_cuda.py:115-145,
 * decode_grouped_multiquery_step(_prepared)_cuda_tensor).
 *   score: page i is scored against queries[page_group[i]] (device fp32
 *          [n_groups][n_queries][head_dim]) into logits rows
 *          page_group[i] * n_queries + q (row stride logits_stride) at
 *          columns token_offsets[i] + t, offsets counted within the group;
 *   mix:   out[g * n_queries + q, :] (+)= sum over pages
 *          [group_pages[g], group_pages[g + 1]) of weights row
 *          g * n_queries + q times the page's values; group_pages is device
 *          int32 [n_groups + 1]. */
int dc_score_pages_grouped(dc_pool pool, const int32_t* page_ids, const int32_t* token_offsets,
                           const int32_t* page_group, int32_t n_groups, int32_t n_pages, const float* queries,
                           int32_t n_queries, float* logits, int64_t logits_stride, dc_stream_t stream);

int dc_mix_pages_grouped(dc_pool pool, const int32_t* page_ids, const int32_t* token_offsets,
                         const int32_t* group_pages, int32_t n_groups, int32_t n_pages, const float* weights,
                         int32_t n_queries, int64_t weights_stride, float* out, int32_t accumulate,
                         dc_stream_t stream);

/* In-place row softmax exp(x - max) / sum of x[r, :n_cols] (row stride
 * `stride`), the global softmax of reference
 * dotcache/attention_reference.py:27-31 used by the decode_step entry
 * point that returns logits and weights. */
int dc_softmax_rows(float* x /* device */, int32_t n_rows, int32_t n_cols, int64_t stride, dc_stream_t stream);

/* Execution shortlist (reference dotcache/session_runtime.py:122-439).
 *
 * Per-page summaries of pages page_ids[0 .. n_pages) of a pool, from their
 * dequantised rows: mean [n][head_dim], sketch [n][sketch_rows][head_dim]
 * (means of np.array_split(rows, min(sketch_rows, tokens)); rows past that
 * repeat the last chunk mean), page_min / page_max [n][head_dim].  Replaces
 * the dense fallbacks of sketch_key_page / summarize_value_page /
 * envelope_key_page (session_runtime.py:122-162), which decode the page on
 * the host.  head_dim <= 256. */
int dc_page_summaries(dc_pool pool, const int32_t* page_ids, int32_t n_pages, int32_t sketch_rows, float* mean,
                      float* sketch, float* page_min, float* page_max, dc_stream_t stream);

/* scores[p] = max_s sketch[p, s, :] . query (mode 0, "sketch") or
 * page_max[p, :] . max(query, 0) + page_min[p, :] . min(query, 0) (mode 1,
 * "envelope").  Replaces score_page_relevance and the candidate scoring of
 * select_execution_page_indices (session_runtime.py:165-186, :268-423). */
int dc_page_relevance(const float* sketch, int32_t sketch_rows, const float* page_min, const float* page_max,
                      int32_t mode, const float* query, int32_t head_dim, int32_t n_pages, float* scores,
                      dc_stream_t stream);

/* selected[i] = 1 for the k best candidates (candidate[i] != 0) by score,
 * descending, ties to the lower index; 0 elsewhere.  Replaces the ranking
 * of select_execution_page_indices (session_runtime.py:425-436). */
int dc_select_top_k(const float* scores, const uint8_t* candidate, int32_t n, int32_t k, uint8_t* selected,
                    dc_stream_t stream);

/* ---- read path: fused paged decode ------------------------------------ */

/* Host-only planner: split each (sequence, kv_head)'s page list into
 * ceil(pages / pages_per_split) work items of near-equal size (at most
 * pages_per_split pages each; pages_per_split <= 0: one item per sequence),
 * and emit merge items for sequences that were split.
 * seq_pages: host [n_seqs].  Returns DC_ESPACE if the output arrays are too
 * small (counts are still written). */
int dc_plan_decode(const int32_t* seq_pages, int32_t n_seqs, int32_t n_kv_heads, int32_t pages_per_split,
                   dc_work_item* items, int32_t max_items, int32_t* n_items,
                   dc_merge_item* merges, int32_t max_merges, int32_t* n_merges, int32_t* n_partials);

/* Host-only planner that fills a launch with items of near-equal cost.
 * Each (sequence, kv_head) stream is a run of seq_pages[b] x chunks_per_page
 * chunks (32 tokens each; chunks_per_page = ceil(page_capacity / 32) lets
 * items split pages, 1 keeps them whole), less the chunks of its last page
 * past last_page_tokens[b] tokens (host int32 [n_seqs], each in [1, 32 x
 * chunks_per_page]; NULL: every page counts as full), so no item is cut
 * among chunks that hold no token.  A chunk costs page_cost[(b *
 * n_kv_heads + h) * cost_stride + page] / (the page's counted chunks), or 1
 * when page_cost is NULL (costs must be finite and >= 0).  Starting from one item
 * per stream, the planner adds one split at a time to the stream with the
 * largest mean item cost (ties to the longer stream, then the lower index)
 * while fewer than target_items items exist and that stream's items keep at
 * least min_chunks_per_split chunks; it stops at the first stream that
 * cannot be split further, whose items then bound the launch.  Each stream
 * is then cut at its cost quantiles (whole-chunk boundaries; without costs,
 * split s of n covers chunks [s·len/n, (s+1)·len/n)).  target_items is
 * normally one item per SIMD.  Same items, merges and DC_ESPACE convention
 * as dc_plan_decode; *largest_item receives the largest item's chunk count.
 * The chunking of the reference's grouped decode
 * (dotcache/backends/torch_mps.py:4110-4273) has no launch to fill; this
 * planner has no reference counterpart beyond it. */
int dc_plan_decode_fill(const int32_t* seq_pages, const int32_t* last_page_tokens, int32_t n_seqs,
                        int32_t n_kv_heads, int32_t chunks_per_page, const float* page_cost, int64_t cost_stride,
                        int32_t target_items,
                        int32_t min_chunks_per_split, dc_work_item* items, int32_t max_items, int32_t* n_items,
                        dc_merge_item* merges, int32_t max_merges, int32_t* n_merges, int32_t* n_partials,
                        int32_t* largest_item);

/* Fused decode attention straight from compressed pages: for every work
 * item, score its pages for the n_q GQA query heads of its KV head, take a
 * single-pass online softmax, and mix the value pages; then merge split-K
 * partials by log-sum-exp.  Pages of one item may mix formats (per-page
 * M3 / M0, the selective-key-precision map).
 *   queries : device [n_seqs, n_kv_heads, n_q, head_dim] of queries_dtype
 *             (= [n_seqs, n_q_heads, head_dim] with q_head -> q_head / n_q,
 *             reference dotcache/model_kv_cache.py:85-95), multiplied by
 *             query_scale before use
 *   k_pool, v_pool : pools of the key and value pages; they must share
 *             head_dim and page_capacity and may differ in group size
 *             (one group size per pool); they may be the same pool
 *   k_table, v_table : device int32 [n_seqs, n_kv_heads, table_stride] page
 *             ids into k_pool / v_pool
 *   out     : device fp32 [n_seqs, n_kv_heads, n_q, head_dim]
 *   workspace : device, >= dc_decode_workspace_bytes(n_partials, n_q, head_dim)
 * Replaces reference dotcache/attention_runtime.py:179-315 (decode_step,
 * decode_multi_query_step) and the grouped GPU decode of
 * dotcache/backends/torch_mps.py:4110-4435 behind
 * dotcache/backends/torch_cuda.py:81-158. */
int dc_decode_paged(dc_pool k_pool, dc_pool v_pool, const int32_t* k_table, const int32_t* v_table, int32_t table_stride,
                    const dc_work_item* items, int32_t n_items,
                    const dc_merge_item* merges, int32_t n_merges,
                    const void* queries, int32_t queries_dtype, float query_scale,
                    int32_t n_seqs, int32_t n_kv_heads, int32_t n_q,
                    float* out, void* workspace, int64_t workspace_bytes,
                    dc_stream_t stream);

/* Work items per SIMD that the decode kernel chosen for these pools and
 * n_q runs at once: 2 for the MFMA kernel's instances built for two waves
 * per SIMD (M0 keys at head_dim 128, up to 8 heads per block), else 1.  A
 * planner fills a launch with this many items per SIMD (dc_plan_decode_fill's
 * target_items).  No reference counterpart. */
int32_t dc_decode_waves_per_simd(dc_pool k_pool, dc_pool v_pool, int32_t n_q);

/* Page records for a plan: records[i * rec_stride + s] receives the key and
 * value descriptors of page page_begin + s of work item i, read through
 * k_table / v_table (zeros past the item's pages, or for an id outside
 * its pool).  1 <= rec_stride <= 64.  A snapshot: it stays valid while the
 * items, the tables' entries for those pages and the pools' descriptors of
 * those pages do not change; gather again after any change (an append
 * that changes a page's token count included).  No reference counterpart:
 * it moves the page-table and descriptor reads of the reference's chunked
 * decode (dotcache/backends/torch_mps.py:4110-4273) out of the decode
 * launch, so a decode's waves issue their first page loads one dependent
 * load after their start instead of three. */
int dc_gather_page_records(dc_pool k_pool, dc_pool v_pool, const int32_t* k_table, const int32_t* v_table,
                           int32_t table_stride, const dc_work_item* items, int32_t n_items, int32_t n_seqs,
                           int32_t n_kv_heads, dc_page_record* records, int32_t rec_stride, dc_stream_t stream);

/* dc_decode_paged with the page records of its items (from
 * dc_gather_page_records with the same items, tables and descriptors, and
 * the same rec_stride).  The MFMA kernel reads the descriptors of an item
 * of at most rec_stride pages from its records instead of through the
 * tables; other items, and the generic kernel, read the tables.  records
 * NULL: exactly dc_decode_paged.  Replaces the same reference functions as
 * dc_decode_paged. */
int dc_decode_paged_records(dc_pool k_pool, dc_pool v_pool, const int32_t* k_table, const int32_t* v_table,
                            int32_t table_stride, const dc_work_item* items, int32_t n_items,
                            const dc_merge_item* merges, int32_t n_merges, const void* queries,
                            int32_t queries_dtype, float query_scale, int32_t n_seqs, int32_t n_kv_heads,
                            int32_t n_q, float* out, void* workspace, int64_t workspace_bytes,
                            const dc_page_record* records, int32_t rec_stride, dc_stream_t stream);

int64_t dc_decode_workspace_bytes(int32_t n_partials, int32_t n_q, int32_t head_dim);

/* The split-K merge on its own: for every merge item, combine partials
 * [partial_begin, partial_begin + count) of the workspace by log-sum-exp into
 * out [n_seqs, n_kv_heads, n_q, head_dim].  dc_decode_paged with
 * n_merges = 0 writes the partials and leaves the merge to this call, which
 * lets a caller time or schedule the two kernels apart.  Workspace layout and
 * size as for dc_decode_paged.  Replaces the chunked (m, l) rescale-and-merge
 * of reference dotcache/backends/torch_mps.py:4276-4435 (the online-softmax
 * combine across chunks). */
int dc_lse_merge(const dc_merge_item* merges, int32_t n_merges, const void* workspace, int64_t workspace_bytes,
                 int32_t n_seqs, int32_t n_kv_heads, int32_t n_q, int32_t head_dim, float* out, dc_stream_t stream);

/* dc_lse_merge that also attends, for every merge item m, the fp16 (M3 f16)
 * key and value pages windows[m] of its stream (through the tables, like
 * the decode) before it combines: the window's (m, l, o) joins the
 * item's partials in the log-sum-exp.  A stream's few exact pages (the
 * recent window kept in fp16 among 4-bit pages) then need no decode
 * launch of their own, and the decode launch keeps the kernel instance of
 * the 4-bit pages.  A window holds at most 256 tokens in at most 8 pages;
 * head_dim must be 64, 128 or 256; out and the workspace 16-byte aligned.
 * The windows are device data, so the kernel guards them: a range of more
 * than 8 pages or past table_stride is skipped whole, tokens past a
 * window's 256th and pages of another format are skipped (hosts validate
 * windows first: dotcache_amd.decode.check_windows).
 * records: NULL, or device [n_merges][8] key / value descriptor pairs of
 * each window's pages in order (a host snapshot of the tables and
 * descriptors), read instead of the tables and descriptor arrays.
 * Replaces, for those pages, the same score / softmax / mix as
 * dc_decode_paged (reference dotcache/attention_runtime.py:260-315,
 * dotcache/backends/torch_mps.py:4276-4435). */
int dc_window_merge(dc_pool k_pool, dc_pool v_pool, const int32_t* k_table, const int32_t* v_table,
                    int32_t table_stride, const dc_merge_item* merges, const dc_window_range* windows,
                    int32_t n_merges, const void* queries, int32_t queries_dtype, float query_scale,
                    int32_t n_seqs, int32_t n_kv_heads, int32_t n_q, float* out, const void* workspace,
                    int64_t workspace_bytes, const dc_page_record* records, dc_stream_t stream);

/* dc_decode_paged without a workspace, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  It has no counterpart in the reference.
 * The split-K partials go to a static device array of
 * dc_decode_noalloc_scratch_bytes() bytes (32 MiB) that each GPU the library
 * runs on holds until the process ends; n_partials (from dc_plan_decode) must
 * fit it: n_partials * n_q * (head_dim + 2) * 4 bytes, or the call fails with
 * DC_ESPACE.  The call allocates nothing (its first call on a device looks
 * up that device's array).  Every call on one GPU shares that GPU's array:
 * calls that overlap on one GPU (concurrent streams, threads) race.  All
 * other arguments and results are as for dc_decode_paged. */
int dc_decode_paged_noalloc(dc_pool k_pool, dc_pool v_pool, const int32_t* k_table, const int32_t* v_table,
                            int32_t table_stride, const dc_work_item* items, int32_t n_items,
                            const dc_merge_item* merges, int32_t n_merges, int32_t n_partials,
                            const void* queries, int32_t queries_dtype, float query_scale, int32_t n_seqs,
                            int32_t n_kv_heads, int32_t n_q, float* out, dc_stream_t stream);

/* Bytes of the static scratch array dc_decode_paged_noalloc uses (host only). */
int64_t dc_decode_noalloc_scratch_bytes(void);

/* Process-wide decode kernel choice: 0 (default) runs the MFMA kernel when
 * every page format (M3 fp16 keys and values, M0 4- or 8-bit keys of group
 * 32, M0 4- or 8-bit values of group 32 or 64), head_dim (64/128/256) and
 * n_q <= 16 fit it, and the generic kernel otherwise; 1 always runs the
 * generic kernel (for cross-checking the two); 2 runs only the MFMA kernel
 * and fails with DC_EINVAL where it does not fit (for tests that must know
 * which kernel ran).  Host only; not thread-safe. */
int dc_set_decode_path(int32_t path);

/* Process-wide head block of the MFMA kernel: the 16 MFMA score columns and
 * mix rows hold 16 / nqb copies of nqb query heads, each copy working on
 * its own key / value group, so a launch with n_q <= 4 or <= 8 scales 4 or
 * 2 groups per operand instead of one.  0 (default) picks the smallest
 * block (4, 8 or 16) that holds n_q and that the pool's specialised kernel
 * provides; 4, 8 or 16 sets the smallest block used (16: one group per
 * MFMA operand, for cross-checking the layouts).  No counterpart in the
 * reference (a kernel tuning switch).  Host only; not thread-safe. */
int dc_set_mfma_head_block(int32_t nqb);

#ifdef __cplusplus
}
#endif

#endif /* DOTCACHE_HIP_H */
