// extern "C" entry points of libhsattn.so (declared in include/hsattn.h).
//
// This layer validates arguments with the reference's error messages where it
// has one, sizes grids and workspaces, and hands off to the kernel launchers.
// It keeps no mutable state besides a per-device cache of CU counts and the
// thread-local error message.
#include <algorithm>
#include <mutex>
#include <string>
#include <unordered_map>

#include "hs_kernels.h"

namespace hs {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return fail(HS_EHIP, std::string(what) + ": " + hipGetErrorString(e));
  return HS_OK;
}

struct ProfileRequest {
  hipEvent_t start = nullptr;
  hipEvent_t stop = nullptr;
};
static thread_local ProfileRequest g_profile;

// A failed record leaves the event unrecorded; the caller's elapsed-time
// query then reports the error, so the status is not needed here.
void profile_begin(hipStream_t stream) {
  if (g_profile.start) (void)hipEventRecord(g_profile.start, stream);
}

void profile_end(hipStream_t stream) {
  if (g_profile.stop) (void)hipEventRecord(g_profile.stop, stream);
  g_profile = ProfileRequest{};
}

constexpr int kDefaultPartition = 512;
constexpr int kMinDefaultPartition = 32;   // small grids: see default_partition

static int device_cu_count(int device) {
  static std::mutex mu;
  static std::unordered_map<int, int> cache;
  std::lock_guard<std::mutex> lock(mu);
  auto it = cache.find(device);
  if (it != cache.end()) return it->second;
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
    return -1;
  cache[device] = cus;
  return cus;
}

static bool valid_dtype(int t) {
  return t == HS_DTYPE_F32 || t == HS_DTYPE_F16 || t == HS_DTYPE_BF16;
}

static bool valid_row_head_dim(int D) { return D == 32 || D == 64 || D == 128 || D == 256; }

// Shared checks of the paged-attention entry points.
static int check_attn_common(const void* q, const void* k, const void* v, int kv_dtype, int NB,
                             const void* bt, const void* ctx, const void* out, int B, int H,
                             int Hkv, int D, int BS, int MB) {
  if (!q || !k || !v || !bt || !ctx || !out)
    return fail(HS_EINVAL, "null tensor pointer");
  if (!valid_dtype(kv_dtype))
    return fail(HS_EINVAL, "unknown kv dtype code " + std::to_string(kv_dtype));
  if (B < 0 || H <= 0 || Hkv <= 0 || D <= 0 || BS <= 0 || MB <= 0 || NB <= 0)
    return fail(HS_EINVAL, "sizes must be positive");
  if (H % Hkv != 0) return fail(HS_EINVAL, "n_head must be divisible by n_kv_head");
  if (D % 32 != 0) return fail(HS_EINVAL, "head_dim must be a multiple of the warp size");
  return HS_OK;
}

struct DecodePlan {
  int mode, part_tokens, splits, P;
};

// Default partition: 512 tokens, shorter when a wave serves G > 2 query
// heads of a GQA group (fewer waves, each doing G times the work per token):
// measured on C2's geometry with 8 and 4 KV heads, 256 and 128 tokens.  With
// 8 or more query heads per KV head and at most 2 waves' worth of heads per
// row (matrix-core path, 32 heads a wave), 512 again: there the merge of many
// short partitions cost more than the waves it adds (MQA with 32 heads on
// C2's geometry: 65 us at 512 tokens, 90 us at 128).
//
// bf16 and fp16 caches with 2 or more query heads per KV head run the
// split-operand matrix-core decode, whose workgroups of splitmm_waves(G)
// waves share a partition: its own default (splitmm_default_partition: 768,
// 384 or 256 tokens) applies there.
//
// Small grids: the partition is halved (down to 32 tokens, or one page per
// wave, and never below that floor) while the launch, estimated from the
// table's width, has fewer than 4 waves per CU.  Each wave then walks a few
// iterations instead of a long serial chain.  Measured on C1 (8 sequences, 12
// heads, contexts up to 512): 20.1 us per step at 512 tokens, 14.8 at 64, 14.3
// at 32, 15.8 at 16 (the merge grows).
static int shrink_for_small_grid(int pt, int min_pt, int64_t waves_per_part, int BS, int MB,
                                 int waves_per_cu = 4) {
  int dev = 0;
  const int cus = hipGetDevice(&dev) == hipSuccess ? device_cu_count(dev) : 0;
  if (cus <= 0) return pt;
  const int64_t max_ctx = (int64_t)MB * BS;
  while (pt > min_pt &&
         sat_mul(waves_per_part, ceil_div(max_ctx, pt)) < waves_per_cu * (int64_t)cus)
    pt = std::max(min_pt, pt / 2);
  return pt;
}

// The VALU kernel's partition before the small-grid cut.
static int valu_partition(int H, int Hkv) {
  const int G = H / Hkv;
  return G >= 8 && (int64_t)Hkv * (((int64_t)G + 31) / 32) <= 2
             ? kDefaultPartition
             : std::min(kDefaultPartition, 1024 / row_attn_heads_per_wave(H, Hkv));
}

static int default_partition(int B, int H, int Hkv, int BS, int MB, int kv_dtype, int D) {
  const int G = H / Hkv;
  if (splitmm_serves(kv_dtype, BS, D, H, Hkv)) {
    // split-operand matrix-core decode: splitmm_waves(G) waves share a
    // partition.  Up to 4 query heads per KV head the cut goes on to 8 waves
    // per CU (32 query heads, bf16, D 128, step us at 4 / 8 waves per CU:
    // 8 KV heads, B 4: 10.9 / 9.8; B 8 at 2-4k tokens: 29.1 / 27.4; B 16 at
    // 1-2k: 28.7 / 26.8; C2-gqa unchanged), above 4 it stays at 4 (4 KV
    // heads, B 16 at 1-2k: 17.5 / 20.8)
    const int kw = splitmm_waves(G);
    return shrink_for_small_grid(splitmm_default_partition(G, D),
                                 std::max(kMinDefaultPartition, BS * kw),
                                 sat_mul(B, Hkv, ceil_div(G, 16), kw), BS, MB, G <= 4 ? 8 : 4);
  }
  return shrink_for_small_grid(valu_partition(H, Hkv), kMinDefaultPartition,
                               sat_mul(B, Hkv, G / row_attn_heads_per_wave(H, Hkv)), BS, MB);
}

// Rows of at most this many keys (by the table's width) can take mode 3.
constexpr int64_t kWgSplitMaxTokens = 1024;

// The default decomposition of a small grid whose rows are short: instead of
// partitions cut down to a few tokens and a merge launch, one workgroup per
// (row, head group) splits the row's keys over its waves and combines their
// states in LDS (mode 3; the caller's workspace goes unused).  Applies where
// the VALU kernel runs and the partition above was shortened for the grid.
// Measured on C1 (8 sequences, 12 heads, head dim 64, fp16, up to 512
// tokens): step 14.3 us with 32-token partitions and the merge, 12.6 us so.
static bool wg_split_applies(int B, int H, int Hkv, int BS, int MB, int kv_dtype, int D) {
  if (splitmm_serves(kv_dtype, BS, D, H, Hkv)) return false;
  if ((int64_t)MB * BS > kWgSplitMaxTokens) return false;
  return default_partition(B, H, Hkv, BS, MB, kv_dtype, D) < valu_partition(H, Hkv);
}

// The workspace queries take no kv dtype: they size for the shortest default
// partition any dtype gets (most partitions, largest state).
static int default_partition_any_dtype(int B, int H, int Hkv, int BS, int MB, int D) {
  return std::min({default_partition(B, H, Hkv, BS, MB, HS_DTYPE_F32, D),
                   default_partition(B, H, Hkv, BS, MB, HS_DTYPE_F16, D),
                   default_partition(B, H, Hkv, BS, MB, HS_DTYPE_BF16, D)});
}

static int plan_decode(int BS, int MB, int num_splits, int partition_tokens, int default_pt,
                       DecodePlan* plan) {
  if (num_splits < 0) return fail(HS_EINVAL, "num_splits must be >= 0");
  const int64_t max_ctx = (int64_t)MB * BS;
  if (num_splits == 1) {
    *plan = {0, 0, 1, 1};
  } else if (num_splits > 1) {
    *plan = {2, 0, num_splits, num_splits};
  } else {
    const int pt = partition_tokens > 0 ? partition_tokens : default_pt;
    if (pt % 16 != 0) return fail(HS_EINVAL, "partition_tokens must be a multiple of 16");
    const int64_t P = ceil_div(max_ctx, pt);
    if (P > 0x7fffffffLL) return fail(HS_EUNSUPPORTED, "too many partitions per row");
    // fixed partitions stay mode 1 when one covers the row (the partition
    // kernel then writes the output itself, no merge): the grouped-query
    // matrix-core kernel serves mode 1 only, and a one-pass plan sent those
    // rows to the VALU kernel, 7-10x slower for 4 query heads per KV head
    *plan = {1, pt, 0, (int)(P < 1 ? 1 : P)};
  }
  return HS_OK;
}

// Partition states: rows * H * P un-normalised outputs of D floats, padded to
// 256 bytes, then as many (max, sum) pairs.  INT64_MAX when that does not fit.
static int64_t decode_ws_bytes(int64_t rows, int H, int D, int P) {
  if (P <= 1) return 0;
  const int64_t states = sat_mul(rows, H, P);
  const int64_t acc = sat_mul(states, D, (int64_t)sizeof(float));
  const int64_t acc_aligned = sat_add(acc, 255) & ~(int64_t)255;
  return sat_add(acc_aligned, sat_mul(states, 2 * (int64_t)sizeof(float)));
}

// Sizes a query function cannot report (0 means "none needed" there).
constexpr int64_t kTooLarge = INT64_MAX;

// The default decomposition of decode with up to 4 query heads per KV head
// (16-bit caches, 16-token pages; the split-operand matrix cores for grouped
// heads, the VALU walk for plain multi-head attention), on grids large
// enough: the even split (mode 4, hs_decode_splitmm.hip), one equal share of
// all pages per workgroup, then a merge of the rows it cut.  Calls that name
// a partition or a split count keep those decompositions.
static bool even_applies(int kv_dtype, int BS, int D, int B, int H, int Hkv, int MB,
                         int num_splits, int partition_tokens) {
  return num_splits == 0 && partition_tokens == 0 && BS == 16 &&
         splitmm_even_groups(kv_dtype, D, H, Hkv, B, MB) > 0;
}

// Workspace bytes of a decode call with this kv dtype (checked sizes) into
// *need, kTooLarge when they do not fit; returns the planning error, if any.
static int decode_need(int B, int H, int Hkv, int D, int BS, int MB, int kv_dtype,
                       int num_splits, int partition_tokens, int64_t* need) {
  if (even_applies(kv_dtype, BS, D, B, H, Hkv, MB, num_splits, partition_tokens)) {
    *need = splitmm_even_layout(B, H, Hkv, D,
                                splitmm_even_groups(kv_dtype, D, H, Hkv, B, MB)).end;
    return HS_OK;
  }
  DecodePlan plan;
  const int rc = plan_decode(BS, MB, num_splits, partition_tokens,
                             default_partition(B, H, Hkv, BS, MB, kv_dtype, D), &plan);
  if (rc != HS_OK) return rc;
  *need = decode_ws_bytes(B, H, D, plan.P);
  return HS_OK;
}

}  // namespace hs

using namespace hs;

extern "C" {

int hs_abi_version(void) { return HS_ABI_VERSION; }

const char* hs_last_error(void) { return g_last_error.c_str(); }

int hs_device_cu_count(int device) { return device_cu_count(device); }

int hs_profile_next_launch(void* start_event, void* stop_event) {
  if ((start_event == nullptr) != (stop_event == nullptr))
    return fail(HS_EINVAL, "pass both events or neither");
  g_profile.start = static_cast<hipEvent_t>(start_event);
  g_profile.stop = static_cast<hipEvent_t>(stop_event);
  return HS_OK;
}

int64_t hs_choose_num_splits(int64_t num_seqs, int64_t num_heads, int64_t max_context) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    set_error("hipGetDevice failed");
    return -1;
  }
  const int sms = device_cu_count(dev);
  if (sms <= 0) {
    set_error("could not read the device CU count");
    return -1;
  }
  // paged_attn_v3.py:224-231
  if (num_seqs < 0 || num_heads < 0 || max_context < 0) {
    set_error("sizes must be non-negative");
    return -1;
  }
  const int64_t prod = sat_mul(num_seqs, num_heads);
  const int64_t have = prod > 1 ? prod : 1;
  const int64_t by_chain = max_context / 32 > 1 ? max_context / 32 : 1;
  const int64_t fill = ceil_div((int64_t)sms * 8, have);
  const int64_t to_fill = fill > 1 ? fill : 1;
  int64_t s = by_chain > to_fill ? by_chain : to_fill;
  s = s < 64 ? s : 64;
  return s > 1 ? s : 1;
}

size_t hs_decode_workspace_bytes(int B, int H, int Hkv, int D, int BS, int MB, int num_splits,
                                 int partition_tokens) {
  if (B <= 0 || H <= 0 || Hkv <= 0 || H % Hkv != 0 || D <= 0 || BS <= 0 || MB <= 0) return 0;
  // the largest need of the three cache dtypes (this query takes none)
  int64_t need = 0;
  for (int dt : {HS_DTYPE_F32, HS_DTYPE_F16, HS_DTYPE_BF16}) {
    int64_t n = 0;
    if (decode_need(B, H, Hkv, D, BS, MB, dt, num_splits, partition_tokens, &n) != HS_OK ||
        n == kTooLarge)
      return 0;
    need = std::max(need, n);
  }
  return (size_t)need;
}

}  // extern "C"

namespace hs {

// Shared-page plan arrays after the decode workspace: skip [B * P] bytes,
// members [P * B] int32, units [P * U] int4, unit counts [P] int32.  `end` is
// kTooLarge when the sizes do not fit.
struct ShareLayout {
  int64_t skip, members, units, n_units, end;
};

static int64_t align256s(int64_t x) { return sat_add(x, 255) & ~(int64_t)255; }

static ShareLayout share_layout(int64_t base, int B, int P, int64_t U) {
  ShareLayout l;
  l.skip = align256s(base);
  l.members = align256s(sat_add(l.skip, sat_mul(B, P)));
  l.units = align256s(sat_add(l.members, sat_mul(P, B, (int64_t)sizeof(int32_t))));
  l.n_units = align256s(sat_add(l.units, sat_mul(P, U, 4 * (int64_t)sizeof(int32_t))));
  l.end = sat_add(l.n_units, sat_mul(P, (int64_t)sizeof(int32_t)));
  if (l.end >= kTooLarge - 255) l.end = kTooLarge;
  return l;
}

static int share_per_unit(int H, int Hkv) { return 32 / (H / Hkv); }

static int decode_common(const float* q, const void* k_cache, const void* v_cache, int kv_dtype,
                         int num_blocks, const int32_t* block_tables, const int32_t* context_lens,
                         float* out, int B, int H, int Hkv, int D, int BS, int MB, float scale,
                         int num_splits, int partition_tokens, void* workspace,
                         size_t workspace_bytes, void* stream, bool shared_pages) {
  int rc = check_attn_common(q, k_cache, v_cache, kv_dtype, num_blocks, block_tables,
                             context_lens, out, B, H, Hkv, D, BS, MB);
  if (rc != HS_OK) return rc;
  if (!valid_row_head_dim(D))
    return fail(HS_EUNSUPPORTED, "unsupported head_dim " + std::to_string(D));
  if (B == 0) return HS_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (!shared_pages &&
      even_applies(kv_dtype, BS, D, B, H, Hkv, MB, num_splits, partition_tokens)) {
    const int M = splitmm_even_groups(kv_dtype, D, H, Hkv, B, MB);
    const EvenLayout l = splitmm_even_layout(B, H, Hkv, D, M);
    if (l.end == kTooLarge)
      return fail(HS_EUNSUPPORTED, "decode partition states too large for these sizes");
    if (!workspace || workspace_bytes < (size_t)l.end)
      return fail(HS_EWORKSPACE, "decode needs " + std::to_string(l.end) +
                                     " workspace bytes, got " +
                                     std::to_string(workspace ? workspace_bytes : 0));
    char* ws = static_cast<char*>(workspace);
    RowAttnArgs a{};
    a.q = q;
    a.k = k_cache;
    a.v = v_cache;
    a.bt = block_tables;
    a.ctx = context_lens;
    a.out = out;
    a.part_acc = reinterpret_cast<float*>(ws + l.acc);
    a.part_ml = reinterpret_cast<float*>(ws + l.ml);
    a.rows = B;
    a.S = 1;
    a.B = B;
    a.H = H;
    a.Hkv = Hkv;
    a.BS = BS;
    a.MB = MB;
    a.NB = num_blocks;
    a.mode = 4;
    a.P = 1;
    a.even_m = M;
    a.even_slots = M + B;
    a.even_min_pages = splitmm_even_min_pages();
    a.qscale = scale * kLog2e;
    return launch_row_attn(a, kv_dtype, D, st);
  }
  DecodePlan plan;
  if ((rc = plan_decode(BS, MB, num_splits, partition_tokens,
                        default_partition(B, H, Hkv, BS, MB, kv_dtype, D), &plan)) != HS_OK)
    return rc;
  const int64_t need_i = decode_ws_bytes(B, H, D, plan.P);
  if (need_i == kTooLarge)
    return fail(HS_EUNSUPPORTED, "decode partition states too large for these sizes");
  const size_t need = (size_t)need_i;
  if (need > 0 && (!workspace || workspace_bytes < need))
    return fail(HS_EWORKSPACE, "decode needs " + std::to_string(need) + " workspace bytes, got " +
                                   std::to_string(workspace ? workspace_bytes : 0));
  RowAttnArgs a{};
  a.q = q;
  a.k = k_cache;
  a.v = v_cache;
  a.bt = block_tables;
  a.ctx = context_lens;
  a.cu_q = nullptr;
  a.out = out;
  a.part_acc = static_cast<float*>(workspace);
  const size_t acc_bytes = ((size_t)B * H * plan.P * D * sizeof(float) + 255) & ~(size_t)255;
  a.part_ml = need ? reinterpret_cast<float*>(static_cast<char*>(workspace) + acc_bytes) : nullptr;
  a.rows = B;
  a.S = 1;
  a.B = B;
  a.H = H;
  a.Hkv = Hkv;
  a.BS = BS;
  a.MB = MB;
  a.NB = num_blocks;
  a.mode = plan.mode;
  a.part_tokens = plan.part_tokens;
  a.splits = plan.splits;
  a.P = plan.P;
  a.qscale = scale * kLog2e;
  if (!shared_pages || !shared_pages_apply(a, kv_dtype, D)) {
    // the default decomposition of a small grid of short rows: one
    // workgroup per row and head group (the workspace, sized for the
    // partitions above, goes unused)
    if (num_splits == 0 && partition_tokens == 0 &&
        wg_split_applies(B, H, Hkv, BS, MB, kv_dtype, D)) {
      a.mode = 3;
      a.part_tokens = 0;
      a.P = 1;
    }
    return launch_row_attn(a, kv_dtype, D, st);
  }
  SharePlanArgs sp{};
  sp.per_unit = share_per_unit(H, Hkv);
  sp.U = (int)share_unit_slots(B, sp.per_unit);   // B <= 2048 here (shared_pages_apply)
  const ShareLayout l = share_layout((int64_t)need, B, plan.P, sp.U);
  if (l.end == kTooLarge) return fail(HS_EUNSUPPORTED, "shared-page plan too large");
  if (workspace_bytes < (size_t)l.end)
    return fail(HS_EWORKSPACE, "shared-page decode needs " + std::to_string(l.end) +
                                   " workspace bytes, got " + std::to_string(workspace_bytes));
  char* ws = static_cast<char*>(workspace);
  sp.skip = reinterpret_cast<uint8_t*>(ws + l.skip);
  sp.members = reinterpret_cast<int32_t*>(ws + l.members);
  sp.units = reinterpret_cast<int4*>(ws + l.units);
  sp.n_units = reinterpret_cast<int32_t*>(ws + l.n_units);
  a.skip = sp.skip;
  return launch_row_attn(a, kv_dtype, D, st, &sp);
}

}  // namespace hs

extern "C" {

int hs_decode(const float* q, const void* k_cache, const void* v_cache, int kv_dtype,
              int num_blocks, const int32_t* block_tables, const int32_t* context_lens,
              float* out, int B, int H, int Hkv, int D, int BS, int MB, float scale,
              int num_splits, int partition_tokens, void* workspace, size_t workspace_bytes,
              void* stream) {
  return decode_common(q, k_cache, v_cache, kv_dtype, num_blocks, block_tables, context_lens,
                       out, B, H, Hkv, D, BS, MB, scale, num_splits, partition_tokens, workspace,
                       workspace_bytes, stream, false);
}

}  // extern "C"

namespace hs {

// Scratch of hs_decode_noalloc: the decode's partition states live here
// instead of in a caller workspace.  Each device holds its own copy (the
// runtime allocates it when it loads this library's code on that device) until
// the process ends.  In host code `scratch` is only a stand-in symbol; its
// address on a device comes from hipGetSymbolAddress with that device current.
static __device__ __align__(256) uint8_t scratch[HS_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;

// Device address of `scratch` on the current device, looked up once per
// device and kept.
static int noalloc_scratch(void** out) {
  static std::mutex mu;
  static void* ptr[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(HS_EHIP, "hipGetDevice failed");
  if (dev < 0 || dev >= kMaxDevices)
    return fail(HS_EUNSUPPORTED, "device " + std::to_string(dev) + " out of range");
  std::lock_guard<std::mutex> lock(mu);
  if (!ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(HS_EHIP, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
    ptr[dev] = p;
  }
  *out = ptr[dev];
  return HS_OK;
}

}  // namespace hs

extern "C" {

int hs_decode_noalloc(const float* q, const void* k_cache, const void* v_cache, int kv_dtype,
                      int num_blocks, const int32_t* block_tables, const int32_t* context_lens,
                      float* out, int B, int H, int Hkv, int D, int BS, int MB, float scale,
                      int num_splits, int partition_tokens, void* stream) {
  // the partition states this call needs, planned for its own cache dtype
  // (hs_decode_workspace_bytes takes none and sizes for the worst dtype)
  size_t need = 0;
  if (B > 0 && H > 0 && Hkv > 0 && H % Hkv == 0 && D > 0 && BS > 0 && MB > 0 &&
      valid_dtype(kv_dtype)) {
    int64_t n = 0;
    const int rc = decode_need(B, H, Hkv, D, BS, MB, kv_dtype, num_splits, partition_tokens, &n);
    if (rc != HS_OK) return rc;
    if (n == kTooLarge)
      return fail(HS_EUNSUPPORTED, "decode partition states too large for these sizes");
    need = (size_t)n;
  }
  if (need > (size_t)HS_NOALLOC_SCRATCH_BYTES)
    return fail(HS_EWORKSPACE, "hs_decode_noalloc: this call needs " + std::to_string(need) +
                                   " bytes of partition state, more than the library's fixed " +
                                   std::to_string((size_t)HS_NOALLOC_SCRATCH_BYTES) +
                                   "; use hs_decode with a workspace");
  void* ws = nullptr;
  if (need > 0) {
    const int rc = noalloc_scratch(&ws);
    if (rc != HS_OK) return rc;
  }
  return decode_common(q, k_cache, v_cache, kv_dtype, num_blocks, block_tables, context_lens,
                       out, B, H, Hkv, D, BS, MB, scale, num_splits, partition_tokens, ws,
                       need > 0 ? (size_t)HS_NOALLOC_SCRATCH_BYTES : 0, stream, false);
}

size_t hs_decode_shared_workspace_bytes(int B, int H, int Hkv, int D, int BS, int MB,
                                        int partition_tokens) {
  // the fixed-partition states (this entry point never takes the even
  // split), then the plan arrays
  if (B <= 0 || H <= 0 || Hkv <= 0 || H % Hkv != 0 || D <= 0 || BS <= 0 || MB <= 0) return 0;
  DecodePlan plan;
  if (plan_decode(BS, MB, 0, partition_tokens, default_partition_any_dtype(B, H, Hkv, BS, MB, D),
                  &plan) != HS_OK)
    return 0;
  const int64_t base = decode_ws_bytes(B, H, D, plan.P);
  if (base == 0 || base == kTooLarge) return 0;   // one partition per row: nothing to share
  const int pu = H / Hkv <= 32 ? share_per_unit(H, Hkv) : 1;
  const int64_t end = share_layout((int64_t)base, B, plan.P,
                                   share_unit_slots(B, pu > 0 ? pu : 1)).end;
  return end == kTooLarge ? 0 : (size_t)end;
}

int hs_decode_shared(const float* q, const void* k_cache, const void* v_cache, int kv_dtype,
                     int num_blocks, const int32_t* block_tables, const int32_t* context_lens,
                     float* out, int B, int H, int Hkv, int D, int BS, int MB, float scale,
                     int partition_tokens, void* workspace, size_t workspace_bytes,
                     void* stream) {
  return decode_common(q, k_cache, v_cache, kv_dtype, num_blocks, block_tables, context_lens,
                       out, B, H, Hkv, D, BS, MB, scale, 0, partition_tokens, workspace,
                       workspace_bytes, stream, true);
}

static int prefill_common(const float* q, const int32_t* cu_q, int S, int max_rows,
                          const void* k_cache, const void* v_cache, int kv_dtype, int num_blocks,
                          const int32_t* block_tables, const int32_t* context_lens, float* out,
                          int B, int H, int Hkv, int D, int BS, int MB, float scale,
                          int use_mfma, void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_attn_common(q, k_cache, v_cache, kv_dtype, num_blocks, block_tables,
                             context_lens, out, B, H, Hkv, D, BS, MB);
  if (rc != HS_OK) return rc;
  if (S < 0 || max_rows < 0) return fail(HS_EINVAL, "query length must be >= 0");
  if (B == 0 || max_rows == 0) return HS_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (use_mfma) {
    if (kv_dtype != HS_DTYPE_F16 && kv_dtype != HS_DTYPE_BF16)
      return fail(HS_EUNSUPPORTED, "the MFMA path needs an fp16 or bf16 KV cache");
    if (BS != 16)
      return fail(HS_EUNSUPPORTED, "the MFMA path needs block_size == 16 (one page per tile)");
    if (!(D == 32 || D == 64 || D == 128))
      return fail(HS_EUNSUPPORTED, "unsupported head_dim for the MFMA path: " + std::to_string(D));
    // S is the rows of every sequence (padded form) or the longest sequence's
    // rows (ragged form): the MFMA grid is sized per sequence.
    return launch_prefill_mfma(q, cu_q, S, S, k_cache, v_cache, kv_dtype, num_blocks,
                               block_tables, context_lens, out, B, H, Hkv, D, BS, MB, scale,
                               workspace, workspace_bytes, st);
  }
  if (!valid_row_head_dim(D))
    return fail(HS_EUNSUPPORTED, "unsupported head_dim " + std::to_string(D));
  RowAttnArgs a{};
  a.q = q;
  a.k = k_cache;
  a.v = v_cache;
  a.bt = block_tables;
  a.ctx = context_lens;
  a.cu_q = cu_q;
  a.out = out;
  a.rows = max_rows;
  a.S = S;
  a.B = B;
  a.H = H;
  a.Hkv = Hkv;
  a.BS = BS;
  a.MB = MB;
  a.NB = num_blocks;
  a.mode = 0;  // one pass per (row, head): no workspace
  a.splits = 1;
  a.P = 1;
  a.qscale = scale * kLog2e;
  return launch_row_attn(a, kv_dtype, D, st);
}

int hs_prefill(const float* q, const void* k_cache, const void* v_cache, int kv_dtype,
               int num_blocks, const int32_t* block_tables, const int32_t* context_lens,
               float* out, int B, int S, int H, int Hkv, int D, int BS, int MB, float scale,
               int use_mfma, void* workspace, size_t workspace_bytes, void* stream) {
  if ((int64_t)B * S > 0x7fffffffLL) return fail(HS_EINVAL, "B * S too large");
  return prefill_common(q, nullptr, S, B * S, k_cache, v_cache, kv_dtype, num_blocks,
                        block_tables, context_lens, out, B, H, Hkv, D, BS, MB, scale, use_mfma,
                        workspace, workspace_bytes, stream);
}

int hs_prefill_varlen(const float* q, const int32_t* cu_seqlens_q, int max_seqlen_q,
                      const void* k_cache, const void* v_cache, int kv_dtype, int num_blocks,
                      const int32_t* block_tables, const int32_t* context_lens, float* out,
                      int B, int H, int Hkv, int D, int BS, int MB, float scale, int use_mfma,
                      void* workspace, size_t workspace_bytes, void* stream) {
  if (!cu_seqlens_q) return fail(HS_EINVAL, "null cu_seqlens_q");
  // Total rows are needed for the row grid; they are the last prefix sum,
  // which lives on the device.  The caller passes max_seqlen_q, so the grid is
  // sized B * max_seqlen_q and rows past a sequence's end exit early.
  if ((int64_t)B * max_seqlen_q > 0x7fffffffLL) return fail(HS_EINVAL, "B * max_seqlen_q too large");
  return prefill_common(q, cu_seqlens_q, max_seqlen_q, B * max_seqlen_q, k_cache, v_cache,
                        kv_dtype, num_blocks, block_tables, context_lens, out, B, H, Hkv, D, BS,
                        MB, scale, use_mfma, workspace, workspace_bytes, stream);
}

size_t hs_prefill_workspace_bytes(int B, int max_seqlen_q, int H, int D, int use_mfma) {
  if (!use_mfma || B <= 0 || max_seqlen_q <= 0 || H <= 0 || D <= 0) return 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  const int cus = device_cu_count(dev);
  if (cus <= 0) return 0;
  const PrefillPlan plan = plan_prefill_mfma(B, max_seqlen_q, H, D, cus, true);
  const int64_t need = prefill_workspace_bytes(plan, B, max_seqlen_q, H, D);
  return need == INT64_MAX ? 0 : (size_t)need;
}

int hs_kv_pack(const void* pool, int L, int NB, int64_t page_bytes, const int64_t* block_ids,
               int n, void* out, void* stream) {
  if (n < 0 || L <= 0 || NB <= 0 || page_bytes <= 0)
    return fail(HS_EINVAL, "pack sizes must be positive");
  if (n == 0) return HS_OK;
  if (!pool || !block_ids || !out) return fail(HS_EINVAL, "null pointer");
  return launch_page_copy(pool, out, false, L, NB, page_bytes, block_ids, n,
                          static_cast<hipStream_t>(stream));
}

int hs_kv_unpack(void* pool, int L, int NB, int64_t page_bytes, const int64_t* block_ids, int n,
                 const void* in, void* stream) {
  if (n < 0 || L <= 0 || NB <= 0 || page_bytes <= 0)
    return fail(HS_EINVAL, "unpack sizes must be positive");
  if (n == 0) return HS_OK;
  if (!pool || !block_ids || !in) return fail(HS_EINVAL, "null pointer");
  return launch_page_copy(pool, const_cast<void*>(in), true, L, NB, page_bytes, block_ids, n,
                          static_cast<hipStream_t>(stream));
}

int hs_kv_gather(const void* cache, int NB, int BS, int64_t row_bytes, const int32_t* block_tables,
                 int MB, int B, int length, void* out, void* stream) {
  if (B < 0 || length < 0 || NB <= 0 || BS <= 0 || MB <= 0 || row_bytes <= 0)
    return fail(HS_EINVAL, "gather sizes must be positive");
  if ((int64_t)length > (int64_t)MB * BS)
    return fail(HS_EINVAL, "length exceeds the block table's capacity");
  if (B == 0 || length == 0) return HS_OK;
  if (!cache || !block_tables || !out) return fail(HS_EINVAL, "null pointer");
  return launch_gather_rows(cache, NB, BS, row_bytes, block_tables, MB, B, length, out,
                            static_cast<hipStream_t>(stream));
}

static int check_kv_write(void* k_cache, void* v_cache, int kv_dtype, int Hkv, int D,
                          int64_t n, const void* k_src, const void* v_src, int src_dtype,
                          int64_t src_row_stride) {
  if (n < 0 || Hkv <= 0 || D <= 0) return fail(HS_EINVAL, "KV write sizes must be positive");
  if (kv_dtype < HS_DTYPE_F32 || kv_dtype > HS_DTYPE_BF16 || src_dtype < HS_DTYPE_F32 ||
      src_dtype > HS_DTYPE_BF16)
    return fail(HS_EINVAL, "unsupported dtype code");
  if (src_row_stride < (int64_t)Hkv * D)
    return fail(HS_EINVAL, "source row stride is smaller than Hkv * D");
  if (n > 0 && (!k_cache || !v_cache || !k_src || !v_src)) return fail(HS_EINVAL, "null pointer");
  return HS_OK;
}

int hs_kv_scatter(void* k_cache, void* v_cache, int kv_dtype, int64_t num_slots, int Hkv, int D,
                  const int64_t* slots, int64_t n, const void* k_src, const void* v_src,
                  int src_dtype, int64_t src_row_stride, void* stream) {
  const int rc = check_kv_write(k_cache, v_cache, kv_dtype, Hkv, D, n, k_src, v_src, src_dtype,
                                src_row_stride);
  if (rc != HS_OK) return rc;
  if (num_slots <= 0) return fail(HS_EINVAL, "num_slots must be positive");
  if (n == 0) return HS_OK;
  if (!slots) return fail(HS_EINVAL, "null pointer");
  return launch_kv_scatter(k_cache, v_cache, kv_dtype, num_slots, (int64_t)Hkv * D, slots, n,
                           k_src, v_src, src_dtype, src_row_stride,
                           static_cast<hipStream_t>(stream));
}

int hs_kv_append(void* k_cache, void* v_cache, int kv_dtype, int NB, int BS, int Hkv, int D,
                 const int32_t* block_tables, int B, int MB, const int32_t* positions,
                 const int32_t* seq_ids, int64_t n, const void* k_src, const void* v_src,
                 int src_dtype, int64_t src_row_stride, void* stream) {
  const int rc = check_kv_write(k_cache, v_cache, kv_dtype, Hkv, D, n, k_src, v_src, src_dtype,
                                src_row_stride);
  if (rc != HS_OK) return rc;
  if (NB <= 0 || BS <= 0 || B <= 0 || MB <= 0)
    return fail(HS_EINVAL, "append sizes must be positive");
  if (n == 0) return HS_OK;
  if (!block_tables || !positions) return fail(HS_EINVAL, "null pointer");
  return launch_kv_append(k_cache, v_cache, kv_dtype, NB, BS, (int64_t)Hkv * D, block_tables, B,
                          MB,
                          positions, seq_ids, n, k_src, v_src, src_dtype, src_row_stride,
                          static_cast<hipStream_t>(stream));
}

int hs_block_tables(const int32_t* packed, int B, int width, int32_t* out, void* stream) {
  if (B < 0 || width < 0) return fail(HS_EINVAL, "block table sizes must be non-negative");
  if ((int64_t)B * width == 0) return HS_OK;
  if (!packed || !out) return fail(HS_EINVAL, "null pointer");
  return launch_block_tables(packed, B, width, out, static_cast<hipStream_t>(stream));
}

}  // extern "C"
