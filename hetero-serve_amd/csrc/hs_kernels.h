// Internal interface between the C-ABI layer (hs_api.hip) and the kernel
// translation units.
#pragma once

#include "hs_common.h"

namespace hs {

// Paged attention over rows: one query vector per (row, head).  Filled by
// hs_api.hip, consumed by the kernels in hs_decode.hip.
struct RowAttnArgs {
  const float* q;         // [rows, H, D]
  const void* k;          // [NB, BS, Hkv, D]
  const void* v;
  const int32_t* bt;      // [B, MB]
  const int32_t* ctx;     // [B]
  const int32_t* cu_q;    // [B + 1] row offsets, or null for S rows per sequence
  float* out;             // [rows, H, D]
  float* part_acc;        // [rows, H, P, D]   un-normalised partial outputs
  float* part_ml;         // [rows, H, P, 2]   partial (max, sum), base-2 domain
  int rows;               // rows in the grid (>= real rows when cu_q is set)
  int S;                  // rows per sequence when cu_q is null
  int B, H, Hkv, BS, MB, NB;
  int mode;               // 0 one pass, 1 fixed partitions, 2 num_splits slices,
                          // 3 one pass per workgroup, keys split over its waves,
                          // 4 even split (16-bit caches, up to 4 query heads per KV head)
  int part_tokens;        // mode 1
  int splits;             // mode 2
  int P;                  // partition slots per (row, head) in the grid
  float qscale;           // scale * log2(e)
  const uint8_t* skip;    // [rows * P] or null: partitions the shared-page kernel serves
  // mode 4: workgroups per unit and state slots per unit (even_m + rows);
  // part_acc / part_ml hold the states as [unit, slot, head of the unit] rows
  int even_m;
  int even_slots;
  int even_min_pages;
};

// Sequence of a row and the end of its key range (exclusive).  Returns false
// for grid rows past the last real row (ragged batches size the grid by the
// longest sequence).
__device__ inline bool row_geometry(const RowAttnArgs& a, int row, int& b, int& end) {
  int s, rows_b;
  if (a.cu_q) {
    if (row >= a.cu_q[a.B]) return false;
    int lo = 0, hi = a.B;  // find b with cu_q[b] <= row < cu_q[b+1]
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (a.cu_q[mid] <= row) lo = mid; else hi = mid;
    }
    b = lo;
    s = row - a.cu_q[b];
    rows_b = a.cu_q[b + 1] - a.cu_q[b];
  } else {
    b = row / a.S;
    s = row - b * a.S;
    rows_b = a.S;
  }
  const int64_t cap = (int64_t)a.MB * a.BS;
  const int64_t e = (int64_t)a.ctx[b] - rows_b + s + 1;
  end = (int)(e < cap ? e : cap);
  return true;
}

// Key range [lo, hi) of partition p; returns false when it is empty.
__device__ inline bool partition_range(const RowAttnArgs& a, int end, int p, int& lo, int& hi,
                                       int& nparts) {
  if (end <= 0) {
    nparts = 0;
    return false;
  }
  int chunk;
  if (a.mode == 0) chunk = end;
  else if (a.mode == 1) chunk = a.part_tokens;
  else chunk = (end + a.splits - 1) / a.splits;
  nparts = (end + chunk - 1) / chunk;
  lo = p * chunk;
  hi = min(lo + chunk, end);
  return p < nparts;
}

// Measurement hook of hs_profile_next_launch: bracket the main kernel of the
// current call with the caller's events (no-ops when none are pending).
void profile_begin(hipStream_t stream);
void profile_end(hipStream_t stream);

// Shared-page decode (hs_decode_shared): where the block ids of a full
// partition are the same in several sequences (prefix caching), the plan
// kernel groups those sequences and a matrix-core kernel reads the pages once
// for up to 32 query slots; the partition kernel skips the grouped
// (sequence, partition) pairs.  Device arrays, in the caller's workspace.
struct SharePlanArgs {
  uint8_t* skip;       // [B * P]  1: (b, p) served by the shared-page kernel
  int32_t* members;    // [P * B]  per partition: the grouped sequences, group by group
  int4* units;         // [P * U]  (first member, members, representative sequence, 0)
  int32_t* n_units;    // [P]
  int U;               // unit slots per partition
  int per_unit;        // sequences per unit (32 query slots / G heads per KV head)
};
bool shared_pages_apply(const RowAttnArgs& a, int kv_dtype, int D);
int64_t share_unit_slots(int B, int per_unit);
void launch_share_plan(const RowAttnArgs& a, const SharePlanArgs& s, hipStream_t stream);
void launch_shared_pages(const RowAttnArgs& a, const SharePlanArgs& s, int kv_dtype, int D,
                         hipStream_t stream);

// Partition kernel + merge; with `shared`, the plan kernel before and the
// shared-page kernel between them.
int launch_row_attn(const RowAttnArgs& a, int kv_dtype, int D, hipStream_t stream,
                    const SharePlanArgs* shared = nullptr);

// Grouped-query decode of bf16 and fp16 caches on the matrix cores with split
// 16-bit operands (hs_decode_splitmm.hip): fp32-grade results, no conversion.
bool splitmm_serves(int kv_dtype, int BS, int D, int H, int Hkv);   // geometry and dtype
bool splitmm_applies(const RowAttnArgs& a, int kv_dtype, int D);     // ... and this launch
int splitmm_waves(int G);                                            // waves per partition
int splitmm_default_partition(int G, int D);                         // tokens, before small-grid cuts
int64_t splitmm_grid(const RowAttnArgs& a);
void launch_splitmm_part(const RowAttnArgs& a, int kv_dtype, int D, hipStream_t stream);
// Even split (mode 4): the split-operand kernel for 2 to 4 query heads per KV
// head, the VALU walk for plain multi-head attention.  The workgroups per
// unit that fill the device once (occupancy of the kernel that serves this
// geometry on the current device), and the workspace its states take.
int splitmm_even_groups(int kv_dtype, int D, int H, int Hkv, int B, int MB);   // 0: not served
int splitmm_even_min_pages();
struct EvenLayout {
  int64_t acc, ml, end;   // byte offsets; end == INT64_MAX when too large
};
EvenLayout splitmm_even_layout(int B, int H, int Hkv, int D, int M);
void launch_splitmm_even(const RowAttnArgs& a, int kv_dtype, int D, hipStream_t stream);

// Query heads one decode wave serves (GQA packing): 1, 2, 4 or 8.
int row_attn_heads_per_wave(int H, int Hkv);

int launch_page_copy(const void* pool, void* buf, bool unpack, int L, int NB, int64_t page_bytes,
                     const int64_t* ids, int n, hipStream_t stream);

int launch_gather_rows(const void* cache, int NB, int BS, int64_t row_bytes, const int32_t* bt,
                       int MB, int B, int length, void* out, hipStream_t stream);

// New K/V rows into the cache (hs_kvwrite.hip): rows of row_elems elements,
// source rows src_row_stride elements apart, cast to the cache dtype.
int launch_kv_scatter(void* k_cache, void* v_cache, int kv_dtype, int64_t num_slots,
                      int64_t row_elems, const int64_t* slots, int64_t n, const void* k_src,
                      const void* v_src, int src_dtype, int64_t src_row_stride, hipStream_t stream);
int launch_block_tables(const int32_t* packed, int B, int width, int32_t* out,
                        hipStream_t stream);
int launch_kv_append(void* k_cache, void* v_cache, int kv_dtype, int NB, int BS,
                     int64_t row_elems, const int32_t* bt, int B, int MB,
                     const int32_t* positions,
                     const int32_t* seq_ids, int64_t n, const void* k_src, const void* v_src,
                     int src_dtype, int64_t src_row_stride, hipStream_t stream);

// Matrix-core causal prefill (hs_prefill_mfma.hip).  cu_q null: S rows per
// sequence, q/out [B, S, H, D]; else ragged rows as in hs_prefill_varlen.
int launch_prefill_mfma(const float* q, const int32_t* cu_q, int S, int max_rows_per_seq,
                        const void* k, const void* v, int kv_dtype, int NB, const int32_t* bt,
                        const int32_t* ctx, float* out, int B, int H, int Hkv, int D, int BS,
                        int MB, float scale, void* workspace, size_t workspace_bytes,
                        hipStream_t stream);

// Launch shape of the MFMA prefill (workgroup width, key-range parts) and the
// workspace a split needs (0 without one).
struct PrefillPlan {
  bool wide;      // 256-row workgroups (head dim 64 and 128)
  int n_split;    // key-range parts per query tile (1: none)
  int stream_ns;  // workgroups per XCD of the persistent kernel (0: grid kernel)
};
PrefillPlan plan_prefill_mfma(int B, int max_rows, int H, int D, int cus, bool can_split);
int64_t prefill_workspace_bytes(const PrefillPlan& p, int B, int max_rows, int H, int D);

}  // namespace hs
