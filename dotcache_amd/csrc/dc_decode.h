// Internal interface between the decode entry point and its kernels.
#pragma once

#include "dc_common.h"

namespace dc {

constexpr int kMaxQ = 16;     // GQA query heads per KV head
constexpr int kMaxCap = 256;  // page capacity the decode kernels accept
constexpr float kLog2e = 1.4426950408889634f;

struct DecodeArgs {
  dc_pool kpool;
  dc_pool vpool;
  const int32_t* k_table;
  const int32_t* v_table;
  int32_t table_stride;
  const dc_work_item* items;
  int32_t n_items;
  const void* queries;
  int32_t queries_dtype;
  float q_scale;
  int32_t n_seqs;
  int32_t n_kv_heads;
  int32_t n_q;
  float* out;
  float* part_o;    // [max_partials][n_q][head_dim]
  float* part_ml;   // [max_partials][n_q][2]  (m, l) in the log2 domain
  int64_t max_partials;
  // page records (dc_gather_page_records): [n_items][rec_stride] pairs of
  // (key descriptor, value descriptor), or null
  const dc_page_record* recs;
  int32_t rec_stride;
};

// A work item naming a sequence, KV head or page range outside the call's
// shapes is skipped, not read: a fault guard only (hosts validate plans).
__device__ __forceinline__ bool item_in_bounds(const dc_work_item& it, const DecodeArgs& a) {
  return it.seq >= 0 && it.seq < a.n_seqs && it.kv_head >= 0 && it.kv_head < a.n_kv_heads && it.page_begin >= 0 &&
         it.page_begin <= it.page_end && it.page_end <= a.table_stride && it.chunk_begin >= 0 &&
         it.chunk_begin < (1 << 16) && it.chunk_end >= 0 && it.chunk_end < (1 << 16);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

int launch_decode(const DecodeArgs& a, hipStream_t stream);
int decode_mfma_waves(const DecodeArgs& a);
int launch_decode_generic(const DecodeArgs& a, hipStream_t stream);
// Launches the MFMA kernel when every format in the pools' masks and the
// geometry fit it; *launched tells the caller whether to fall back.
int launch_decode_mfma(const DecodeArgs& a, hipStream_t stream, bool* launched);
int launch_merge(const DecodeArgs& a, const dc_merge_item* merges, int32_t n_merges, hipStream_t stream,
                 const dc_window_range* windows = nullptr);

// Windows a merge attends (dc_window_merge): at most this many tokens in at
// most this many pages.
constexpr int kMaxWinTokens = 256;
constexpr int kMaxWinPages = 8;

}  // namespace dc
