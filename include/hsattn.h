/*
 * hsattn.h -- C ABI of the MI355X (gfx950) paged-attention library libhsattn.so.
 *
 * This is the drop-in boundary for hetero-serve's paged-attention hot path.
 * Each entry point replaces one pybind function that the reference builds
 * with torch.utils.cpp_extension.load_inline from CUDA source embedded in a
 * Python string; the citation above each declaration names that function
 * (paths relative to the reference checkout).  Nothing here uses torch or
 * pybind types: tensors cross as plain device pointers plus sizes, and the
 * stream crosses as an opaque hipStream_t handle (void*).
 *
 * Conventions shared by every entry point
 *   - All pointers are device pointers on the current HIP device, except
 *     where a comment says otherwise.
 *   - Every launch goes on `stream` (NULL = the null stream). Nothing here
 *     synchronises the stream, allocates memory or keeps state between
 *     calls, so calls are re-entrant and may run on several host threads.
 *   - Return value: HS_OK (0) on success, a negative HS_E* code otherwise.
 *     The message for the last failure on the calling thread is returned by
 *     hs_last_error().
 *   - KV pages are token-major, as the reference allocator lays them out
 *     (heteroserve/kv/blocks.py:72-81): a cache is [num_blocks, block_size,
 *     n_kv_heads, head_dim] with the inner three dimensions contiguous.
 *   - Block tables are [B, max_blocks] int32, padded with -1; a position j of
 *     sequence b lives in block block_tables[b][j / block_size] at offset
 *     j % block_size (heteroserve/model/paged_attn_v2.py:124-127).  Entries
 *     outside [0, num_blocks) are read as block 0 (the torch reference clamps
 *     negatives to 0, paged_attn.py:275), so a bad table can never make a
 *     kernel read outside the pool.
 */
#ifndef HSATTN_H
#define HSATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HS_ABI_VERSION 5

/* KV element type codes (the pool dtype). */
#define HS_DTYPE_F32 0
#define HS_DTYPE_F16 1
#define HS_DTYPE_BF16 2

/* Status codes. */
#define HS_OK 0
#define HS_EINVAL (-1)       /* bad argument: shape, pointer, size         */
#define HS_EUNSUPPORTED (-2) /* geometry this library does not serve       */
#define HS_EHIP (-3)         /* the HIP runtime reported an error          */
#define HS_EWORKSPACE (-4)   /* workspace missing or too small             */

/* ABI version of the loaded library; the Python loader refuses a mismatch. */
int hs_abi_version(void);

/* Message of the last failed call on this thread ("" when none).  Valid
 * until the next call into the library from the same thread. */
const char* hs_last_error(void);

/*
 * Measurement hook (no reference counterpart).  The next libhsattn call made
 * from this thread records `start_event` on its stream just before its main
 * kernel (the partition kernel of hs_decode, the attention kernel of
 * hs_prefill*, the copy kernel of hs_kv_*) and `stop_event` just after it, so
 * a benchmark can time that one kernel on the stream it runs on.  The events
 * are hipEvent_t handles owned by the caller; one call consumes them.
 * Passing NULL, NULL cancels a pending request.
 */
int hs_profile_next_launch(void* start_event, void* stop_event);

/* Compute units of HIP device `device` (256 on MI355X); -1 on error. */
int hs_device_cu_count(int device);

/*
 * Split count heuristic of the v3 decode path.
 * Replaces: choose_num_splits, heteroserve/model/paged_attn_v3.py:212-232.
 *   clamp(max(max_context / 32, ceil(CUs * 8 / (num_seqs * num_heads))), 1, 64)
 * with CUs taken from the current HIP device.  Returns -1 on error.
 */
int64_t hs_choose_num_splits(int64_t num_seqs, int64_t num_heads, int64_t max_context);

/*
 * Workspace bytes hs_decode needs for these sizes (0 when it needs none).
 * num_splits and partition_tokens as for hs_decode; Hkv because the default
 * partition size depends on the GQA group (version 2 of the ABI added it).
 * The default also depends on the kv dtype, which this query does not take:
 * it returns the size for the shortest default any dtype gets, enough for
 * every dtype.
 * The default also shrinks for small grids (halved while the launch would
 * have too few waves per CU, down to 32 tokens or one 16-token page per wave
 * of the workgroup that shares a partition, whichever is longer: 64 tokens
 * for the matrix-core decode up to 4 query heads per KV head), and the even
 * split's state slots (see hs_decode) follow the kernel's occupancy, from B,
 * MB and the CU count of the current device: query the size with the device
 * that will run the call current.
 */
size_t hs_decode_workspace_bytes(int B, int H, int Hkv, int D, int BS, int MB, int num_splits,
                                 int partition_tokens);

/*
 * Decode attention, one query token per sequence:
 *   out[b,h,:] = softmax(scale * q[b,h,:] . K[b,j,kvh,:] over j < ctx_b) . V[b,j,kvh,:]
 * with kvh = h / (H / Hkv) and ctx_b = min(context_lens[b], MB * BS).
 * A sequence with ctx_b <= 0 gets a zero output row.
 *
 * Replaces three reference entry points, which compute the same function:
 *   paged_attention     heteroserve/model/paged_attn.py:136-183     (v1)
 *   paged_attention_v2  heteroserve/model/paged_attn_v2.py:159-212  (v2)
 *   paged_attention_v3  heteroserve/model/paged_attn_v3.py:234-303  (v3)
 *
 *   q            [B, H, D] float32
 *   k_cache      [num_blocks, BS, Hkv, D] of kv_dtype (same for v_cache)
 *   block_tables [B, MB] int32;  context_lens [B] int32
 *   out          [B, H, D] float32
 *   D            32, 64, 128 or 256;  H % Hkv == 0
 *   num_splits   1  = one pass per (sequence, head)               (v2)
 *                >1 = the context cut into num_splits slices of
 *                     ceil(ctx_b / num_splits) tokens, then an
 *                     log-sum-exp merge                            (v3)
 *                0  = fixed partitions of partition_tokens tokens
 *                     plus the merge (the fast default; with
 *                     partition_tokens == 0, a small grid of rows of at most
 *                     1024 keys by the table's width instead runs one
 *                     workgroup per (sequence, head group) whose waves split
 *                     the keys and merge in LDS: no merge launch, the
 *                     workspace unused)
 *   partition_tokens  used when num_splits == 0; 0 = library default (512
 *                tokens, fewer for GQA groups and for grids of fewer than 4
 *                waves per CU; fp16 and bf16 caches with 2 or more query
 *                heads per KV head, head dim 64 and 128: 768 tokens up to 4
 *                heads per KV head, 384 up to 8, 256 otherwise and at head
 *                dim 32, cut for grids of fewer than 8 waves per CU up to 4
 *                heads per KV head, 4 above).  A row that one partition
 *                covers is written directly, without the merge.
 *                Must be a multiple of 16.
 *                With num_splits == 0 and partition_tokens == 0, fp16 and
 *                bf16 caches with 16-token pages and 1 to 4 query heads per
 *                KV head take the even split instead where their default
 *                partitions would overflow one round of the device: all
 *                pages of the batch, rows laid end to end, cut into one
 *                equal range per resident workgroup of each KV head (of
 *                each pair of heads without grouping), then a merge of the
 *                rows cut across ranges.  Same function; results agree
 *                with the fixed partitions to fp32 rounding (to the
 *                split-operand precision for grouped heads), not bit for
 *                bit.
 *   workspace    device scratch of hs_decode_workspace_bytes(...) bytes
 *                (may be NULL when that is 0).
 */
int hs_decode(const float* q, const void* k_cache, const void* v_cache, int kv_dtype,
              int num_blocks, const int32_t* block_tables, const int32_t* context_lens,
              float* out, int B, int H, int Hkv, int D, int BS, int MB, float scale,
              int num_splits, int partition_tokens, void* workspace,
              size_t workspace_bytes, void* stream);

/*
 * hs_decode without a workspace argument: the partition states go to a
 * scratch array of HS_NOALLOC_SCRATCH_BYTES (64 MiB) inside the library, one
 * per device, held until the process ends.  Same arguments and result as
 * hs_decode (bit for bit: same kernels, same decomposition); a call whose
 * partition states, planned for its own kv_dtype, need more than the fixed
 * size fails with HS_EWORKSPACE before launching.  (That need can be below
 * hs_decode_workspace_bytes(...), which sizes for the worst dtype.)  It
 * allocates nothing: no hipMalloc, no hipFree, no allocating library call.
 * Every call on a device shares that device's scratch, so calls that overlap
 * in time on one device (two streams, two threads) race and must not be
 * issued.
 * No counterpart in the reference.  It is for callers that cannot allocate
 * device memory: code under HIP graph capture (a capture after one eager
 * call on the device, which looks up the scratch address, replays bit for
 * bit), tight serving loops, harnesses that forbid allocation.
 */
#define HS_NOALLOC_SCRATCH_BYTES (64u << 20)
int hs_decode_noalloc(const float* q, const void* k_cache, const void* v_cache, int kv_dtype,
                      int num_blocks, const int32_t* block_tables, const int32_t* context_lens,
                      float* out, int B, int H, int Hkv, int D, int BS, int MB, float scale,
                      int num_splits, int partition_tokens, void* stream);

/*
 * Decode for batches whose sequences share pages (prefix caching: the same
 * block ids at the same positions of several block tables).  Computes what
 * hs_decode(num_splits = 0, partition_tokens) computes.  A partition of
 * partition_tokens keys that is full in at least 4 sequences with identical
 * block ids is read once for up to 32 (sequence, head) query slots of a KV
 * head, together with the sequences whose context ends inside it on the same
 * pages (each attending to its own keys only), on the matrix cores (K/V as
 * stored, q and the probabilities split
 * into two 16-bit terms each, fp32 accumulation: fp32-grade results); every
 * other partition runs as in hs_decode.  The grouping is found on the device by
 * one small kernel per call.  Serves fp16/bf16 KV with BS == 16, D in
 * {32, 64, 128}, partitions of at most 1024 tokens, at most 16 query heads per
 * KV head and B <= 2048; other calls run hs_decode's path unchanged.
 * No reference counterpart (the reference reads every sequence's pages);
 * version 4 of the ABI added it.
 *   workspace  device scratch of hs_decode_shared_workspace_bytes(...) bytes
 *              (hs_decode's partition states plus the grouping).
 */
size_t hs_decode_shared_workspace_bytes(int B, int H, int Hkv, int D, int BS, int MB,
                                        int partition_tokens);
int hs_decode_shared(const float* q, const void* k_cache, const void* v_cache, int kv_dtype,
                     int num_blocks, const int32_t* block_tables, const int32_t* context_lens,
                     float* out, int B, int H, int Hkv, int D, int BS, int MB, float scale,
                     int partition_tokens, void* workspace, size_t workspace_bytes,
                     void* stream);

/*
 * Workspace bytes hs_prefill / hs_prefill_varlen may use for B sequences of
 * up to max_seqlen_q query rows (S for hs_prefill), for the current HIP
 * device; 0 when they need none.  Only the matrix-core path (use_mfma = 1)
 * uses one: when its query tiles cannot cover every CU, each tile's key range
 * is split over up to 4 workgroups, whose partial results (fp32, (D + 2) * 4
 * bytes per part, row and head) are merged by a second kernel; when they give
 * every CU at least two (head dim 64 or 128, H a multiple of 8, at most 256
 * sequences), a persistent kernel of one workgroup per CU takes them from
 * per-XCD queues whose 256 bytes of counters are the workspace (zeroed by
 * the call itself).  No reference counterpart (the reference's prefill has
 * neither); version 3 of the ABI added the workspace arguments below.
 */
size_t hs_prefill_workspace_bytes(int B, int max_seqlen_q, int H, int D, int use_mfma);

/*
 * Causal chunked prefill over the paged cache.  Query s of sequence b sits at
 * absolute position ctx_b - S + s and attends to keys [0, ctx_b - S + s]; rows
 * whose position is negative (padding in front of a short sequence) are zero.
 * The chunk's own K/V must already be in the pool.
 *
 * Replaces:
 *   use_mfma = 0: paged_attention_prefill,
 *                 heteroserve/model/paged_attn_prefill.py:159-214
 *                 (fp32 VALU arithmetic, any KV dtype, D in {32,64,128,256})
 *   use_mfma = 1: paged_attention_prefill_wmma,
 *                 heteroserve/model/paged_attn_wmma.py:256-318
 *                 (fp16 matrix-core operands with fp32 accumulation; KV dtype
 *                 f16 or bf16, BS == 16, D in {32,64,128}.  A query tile
 *                 whose operands fp16 cannot hold -- a bf16 K/V value of
 *                 magnitude >= 65536, a scaled query >= 65520 -- is
 *                 recomputed with fp32 arithmetic instead; the same holds
 *                 for the matrix-core decode paths below)
 *
 *   q   [B, S, H, D] float32;  out [B, S, H, D] float32
 *   workspace  NULL, or device scratch of hs_prefill_workspace_bytes(B, S, H,
 *              D, use_mfma) bytes.  NULL runs without the key-range split
 *              (narrower workgroups instead) and without the persistent
 *              kernel; a workspace smaller than the plan needs is
 *              HS_EWORKSPACE.  Calls that overlap in time must not share one.
 */
int hs_prefill(const float* q, const void* k_cache, const void* v_cache, int kv_dtype,
               int num_blocks, const int32_t* block_tables, const int32_t* context_lens,
               float* out, int B, int S, int H, int Hkv, int D, int BS, int MB, float scale,
               int use_mfma, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Ragged-batch form of hs_prefill (use_mfma as there): sequence b owns query
 * rows [cu_seqlens_q[b], cu_seqlens_q[b+1]) of q [total, H, D] and out, with
 * S_b = cu_seqlens_q[b+1] - cu_seqlens_q[b] <= max_seqlen_q.  Query i of
 * sequence b sits at position ctx_b - S_b + i.  No reference counterpart: the
 * reference's engine calls prefill with B = 1 per chunk
 * (heteroserve/model/torch_engine.py:292-313), and this entry point runs
 * several such chunks in one launch.  workspace as for hs_prefill, sized by
 * hs_prefill_workspace_bytes(B, max_seqlen_q, H, D, use_mfma).
 */
int hs_prefill_varlen(const float* q, const int32_t* cu_seqlens_q, int max_seqlen_q,
                      const void* k_cache, const void* v_cache, int kv_dtype, int num_blocks,
                      const int32_t* block_tables, const int32_t* context_lens, float* out,
                      int B, int H, int Hkv, int D, int BS, int MB, float scale,
                      int use_mfma, void* workspace, size_t workspace_bytes, void* stream);

/*
 * KV-block pack for migration:
 *   out[i, l, c] = pool[l, c, block_ids[i]]      (c = 0 for K, 1 for V)
 * where one page is page_bytes = BS * Hkv * D * itemsize bytes, pool is
 * [L, 2, NB, page] and out is [n, L, 2, page].  A bitwise copy.
 * Replaces: TorchBlockAllocator.export_blocks_device,
 *           heteroserve/kv/torch_blocks.py:137-148
 * (pool[:, :, idx].permute(2, 0, 1, 3, 4, 5).contiguous()).
 * block_ids is a device int64 array; ids outside [0, NB) are skipped (the
 * Python layer rejects them first, as torch indexing would).
 */
int hs_kv_pack(const void* pool, int L, int NB, int64_t page_bytes, const int64_t* block_ids,
               int n, void* out, void* stream);

/*
 * Inverse of hs_kv_pack:  pool[l, c, block_ids[i]] = in[i, l, c].
 * Replaces: TorchBlockAllocator.write_blocks_device,
 *           heteroserve/kv/torch_blocks.py:150-154 (a Python loop of one
 *           copy per block).  block_ids must not repeat.
 */
int hs_kv_unpack(void* pool, int L, int NB, int64_t page_bytes, const int64_t* block_ids,
                 int n, const void* in, void* stream);

/*
 * Contiguous gather of the first `length` tokens of every sequence:
 *   out[b, t] = cache[block_tables[b][t / BS], t % BS]
 * for one layer's K (or V) cache [NB, BS, row] with row = row_bytes bytes
 * (Hkv * D * itemsize); out is [B, length, row].
 * Replaces: TorchBlockAllocator.gather_kv_batch,
 *           heteroserve/kv/torch_blocks.py:125-135 (the per-layer gather
 *           that the fused decode kernels make unnecessary).
 */
int hs_kv_gather(const void* cache, int NB, int BS, int64_t row_bytes,
                 const int32_t* block_tables, int MB, int B, int length, void* out,
                 void* stream);

/*
 * Write new K and V rows into one layer's cache:
 *   k_cache[slots[i]] = cast(k_src[i]),  v_cache[slots[i]] = cast(v_src[i])
 * for i < n, where a cache is [num_slots, Hkv, D] (the pool view
 * [NB, BS, Hkv, D] with num_slots = NB * BS) and row i of a source starts
 * src_row_stride elements after row i - 1 (a strided view of the fused QKV
 * projection works as is).  Casts round as torch's `.to()` does; equal dtypes
 * copy bits.  Slots outside [0, num_slots) are skipped; slots must not repeat.
 * Replaces: fk[slots] = k.to(dtype); fv[slots] = v.to(dtype),
 *           heteroserve/model/torch_engine.py:239-240 and :306-308, and the
 *           per-layer loop of TorchBlockAllocator.write_kv,
 *           heteroserve/kv/torch_blocks.py:89-106.
 */
int hs_kv_scatter(void* k_cache, void* v_cache, int kv_dtype, int64_t num_slots, int Hkv, int D,
                  const int64_t* slots, int64_t n, const void* k_src, const void* v_src,
                  int src_dtype, int64_t src_row_stride, void* stream);

/*
 * hs_kv_scatter with each row's slot computed on the device from its
 * sequence's block table (int32 [B, MB], -1 padded) and its absolute
 * position:  slot = block_tables[s][pos / BS] * BS + pos % BS,  with
 * s = seq_ids[i] (or s = i when seq_ids is NULL) and pos = positions[i].
 * Rows whose sequence index is outside [0, B), whose position is negative or
 * past the table, or whose table entry is outside [0, NB), are skipped: the
 * kernel reads no table row past B and writes no slot outside the cache.
 * (Version 5 of the ABI added B.)
 * Replaces: the per-sequence slot loop of decode_batch_paged
 *           (heteroserve/model/torch_engine.py:221-227, one .tolist() per
 *           sequence) followed by the scatter at :239-240; and
 *           TorchBlockAllocator.slots_for + write_kv
 *           (heteroserve/kv/torch_blocks.py:68-73, 89-106) for a chunk.
 */
int hs_kv_append(void* k_cache, void* v_cache, int kv_dtype, int NB, int BS, int Hkv, int D,
                 const int32_t* block_tables, int B, int MB, const int32_t* positions,
                 const int32_t* seq_ids, int64_t n, const void* k_src, const void* v_src,
                 int src_dtype, int64_t src_row_stride, void* stream);

/*
 * Build the int32 block-table tensor [B, width], -1 padded, from one device
 * buffer packed = [off[0], ..., off[B], ids...]: row b holds
 * ids[off[b] .. off[b+1]) truncated to `width` entries.  The host uploads
 * the buffer in one copy.
 * Replaces: TorchBlockAllocator.block_table_tensor,
 *           heteroserve/kv/torch_blocks.py:75-85 (one host-to-device copy per
 *           sequence), called every decode step at
 *           heteroserve/model/torch_engine.py:215-216.
 */
int hs_block_tables(const int32_t* packed, int B, int width, int32_t* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* HSATTN_H */
