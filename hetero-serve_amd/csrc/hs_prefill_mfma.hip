// Causal chunked prefill over the paged KV cache on gfx950 matrix cores.
//
// Reference: prefill_wmma_kernel, heteroserve/model/paged_attn_wmma.py:80-254
// (a FlashAttention loop over 16-token pages with an online softmax), and the
// semantics of paged_attention_prefill_torch, paged_attn_prefill.py:281-322:
// query i of a chunk of S_b rows sits at position ctx_b - S_b + i and attends
// to keys [0, that position]; rows at negative positions are zero.
//
// Work decomposition.  A workgroup owns 256 query rows (8 waves x 32 rows; 4
// waves at head dim 32) of one (sequence, head) and walks that head's keys in
// tiles of 64 (four 16-token pages), staging each K/V tile in LDS once for all
// of its waves.  The LDS tiles are double-buffered with one barrier per tile,
// and the global loads of later tiles are in flight while the current one is
// consumed.  The kernel is held to two waves per SIMD (<= 256 registers), one
// workgroup per CU: a wave's softmax (VALU) then runs while the other wave of
// its SIMD issues MFMAs, which measured faster than 64 rows per wave at one
// wave per SIMD, even though each LDS fragment then feeds one MFMA instead of
// two.  A grid too small for the CUs (one chunk of one sequence) splits each
// query tile's keys over up to 4 workgroups whose partial softmax states
// prefill_merge_kernel combines.
// Scores are computed transposed, S^T = K . Q^T, with v_mfma_f32_32x32x16_f16:
// K rows are the A operand (read from LDS), Q^T the B operand (held in
// registers for the whole walk).  The accumulator then has one query per
// lane and 16 keys per lane in registers, which is exactly the layout of the
// B operand of O^T = V^T . P^T, so the probabilities P go from the softmax to
// the second MFMA without leaving registers; V^T (A operand) is read from the
// token-major V tile in LDS with gfx950's transposing ds_read_b64_tr_b16.
// O^T accumulates one query per lane, so the online-softmax rescale is a
// per-lane scalar multiply.
//
// Key order inside a tile.  A 32x32 accumulator gives lane half h the key rows
// 8g + 4h + m (g = 0..3, m = 0..3) in registers 4g + m.  The P.V operand
// wants registers 0..7 of half h to be keys 8h..8h+7 of a 16-key chunk.  The
// two orders differ by swapping bits 2 and 3 of the key index, so K is stored
// in LDS with that swap (row r of a 32-key block holds key swap23(r)); then
// accumulator register r of half h holds key 16*(r/8) + 8h + r%8.
//
// Numerics.  MFMA operands are fp16 (a bf16 cache is widened to fp16, which
// is exact for |x| < 65504); Q is pre-scaled by scale*log2(e) so every
// exponential is one v_exp_f32; scores, the softmax state and O are fp32.
// Masked scores are -inf while the running max starts at a finite -3e38, so
// a masked probability is exp2(-inf) = 0 with no compare or select.
// The running max is only raised (and O rescaled) when a tile's max exceeds
// it by more than 8 (in log2 units), so probabilities stay <= 256, well
// inside fp16, and most tiles skip the rescale.
//
// Scheduling.  Workgroups are handed to the 8 XCDs round-robin; the grid is
// laid out so that every query tile of one (sequence, head) lands on the same
// XCD, consecutively, heaviest (last) tile first, and consecutive (sequence,
// head) pairs alternate XCDs.  The tiles of one head then share its K/V
// through that XCD's L2.
#include "hs_kernels.h"
#include "hs_mfma.h"
#include "hs_rowwalk.h"

#include <algorithm>
#include <cstdlib>
#include <type_traits>

namespace hs {

namespace {

using namespace mfma;

constexpr int kRowsPerWave = 32;             // one 32-row MFMA tile per wave
constexpr int kBN = 64;                      // keys per LDS tile (four pages), a multiple of 32
constexpr int kXcds = 8;
constexpr int kKPad = 8;                     // halves of padding per LDS K row
// Halves of padding per LDS V row.  A transposing read of V^T fragments has
// each 32-lane half of the wave read 4 rows x 64 bytes (two 16-lane groups,
// adjacent 16-dim column blocks); a row stride of 16 or 48 dwords mod 64 puts
// those 4 rows on disjoint 16-bank ranges.
template <int D>
constexpr int v_pad() { return D == 32 ? 0 : 32; }
constexpr float kRescaleSlack = 8.0f;        // log2 units
constexpr int kMaxRanked = 256;              // sequences a workgroup ranks itself
constexpr int kMaxSplit = 4;                 // key-range parts of one query tile

// Workgroup shape: W waves of 32 query rows.  D 128 and 64 run 8 waves (256
// rows, one workgroup per CU; each K/V tile then serves twice the rows of a
// 4-wave workgroup, which measured 3-10% faster on every prefill shape tried).
// When those tiles cannot cover the CUs, the key range is split instead
// (plan_prefill_mfma); without a workspace for that, 4 waves (128 rows) reach
// twice as many CUs.  D 32 has too few 16-byte chunks per tile for 512
// threads and always runs 4 waves.  Four waves move the K/V tiles: the first
// half of 8, all of 4 (2 of 4 at D 32).
template <int D, int W>
struct Shape {
  static constexpr int kWaves = W;
  static constexpr int kThreads = kWaves * 64;
  static constexpr int kBM = kWaves * kRowsPerWave;   // query rows per workgroup
  static constexpr int kProdWaves = D >= 64 ? 4 : W / 2;
};

struct PrefillArgs {
  const float* q;        // [rows, H, D]
  const void* k;         // [NB, 16, Hkv, D]
  const void* v;
  const int32_t* bt;     // [B, MB]
  const int32_t* ctx;    // [B]
  const int32_t* cu_q;   // [B + 1] or null (S rows per sequence)
  float* out;            // [rows, H, D]
  int S, B, H, Hkv, MB, NB;
  int n_qt;              // query tiles per (sequence, head) in the grid
  int slots_per_xcd;     // grid = kXcds * slots_per_xcd
  int ranked;            // 1: query tiles are dispatched longest first (B * n_qt <= kMaxRanked)
  float qscale;          // scale * log2(e)
  // Key-range split (ranked dispatch only): each query tile's key tiles are
  // cut into up to n_split parts run by separate workgroups, which write
  // unnormalised O and (running max, sum) for prefill_merge_kernel.
  int n_split;           // 1: no split, each workgroup writes out itself
  int rows_cap;          // query rows per sequence in the partial arrays
  float* part_o;         // [n_split, B, rows_cap, H, D]
  float2* part_ml;       // [n_split, B, rows_cap, H]
  int* counters;         // persistent kernel: one work counter per XCD (zeroed per launch)
};

// K rows are read as 16-byte fragments (row j by lane j), V rows by the
// transposing read (four rows by each group of 16 lanes); the two paddings
// keep each pattern free of bank conflicts.
template <int D>
struct PrefillTileLds {
  _Float16 k[kBN][D + kKPad];       // K tile, row r holds key swap23(r)
  _Float16 v[kBN][D + v_pad<D>()];  // V tile, row r holds key r
};

// V^T fragment (A operand of the 32x32x16 product) for dims 32 d .. 32 d + 31
// and keys k0 + 8 hh .. k0 + 8 hh + 7: lane (j, hh) gets V[k0 + 8 hh + e][32 d + j],
// e = 0..7.  ds_read_b64_tr_b16 transposes inside each group of 16 lanes:
// lane i supplies 8 bytes of row i / 4 of a 4 x 16 block and receives column
// i (lane layout checked on gfx950); two reads give the eight keys.
template <int D>
__device__ inline half8 vt_fragment(const PrefillTileLds<D>& t, int d, int k0, int j, int hh) {
  typedef __fp16 half4x __attribute__((__vector_size__(4 * sizeof(__fp16))));
  typedef __attribute__((address_space(3))) half4x lds_half4x;
  typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
  const int i = j & 15;
  // C-style casts keep the LDS address arithmetic visible, so the constant
  // part of the address goes into the instructions' offset field
  const lds_half4x* lo_p =
      (const lds_half4x*)(&t.v[k0 + 8 * hh + (i >> 2)][32 * d + (j & 16) + 4 * (i & 3)]);
  const lds_half4x* hi_p =
      (const lds_half4x*)(&t.v[k0 + 8 * hh + 4 + (i >> 2)][32 * d + (j & 16) + 4 * (i & 3)]);
  const half4x lo = __builtin_amdgcn_ds_read_tr16_b64_v4f16(const_cast<lds_half4x*>(lo_p));
  const half4x hi = __builtin_amdgcn_ds_read_tr16_b64_v4f16(const_cast<lds_half4x*>(hi_p));
  return __builtin_shufflevector(__builtin_bit_cast(f16x4, lo), __builtin_bit_cast(f16x4, hi),
                                 0, 1, 2, 3, 4, 5, 6, 7);
}

// The producer: how the first half of a workgroup's waves (256 threads at
// head dim 128) move one K/V tile from the paged cache through registers
// into LDS.  The SIMD arbiter favours older waves, so waves 0..3 would
// otherwise finish each tile early and idle at the barrier while waves 4..7,
// which share their SIMDs, finish alone; moving the whole tile on waves 0..3
// measured 3-6% faster on every prefill shape tried than spreading it over
// all eight (and faster than a 3:1 split).
//   K: chunk c = tid + 256*u is key c / (D/8), dims 8*(c % (D/8)).  16
//      neighbouring lanes read one 256-byte head row, and every load of a
//      wave falls in a single page, so the page base is a scalar and each lane
//      keeps one 32-bit offset for the whole walk.
//   V: the same chunks as K (same pages, same lane offsets), stored
//      token-major.
// The block ids of a tile are fetched by one vector load, a tile ahead: lane
// L holds the id of page L * kG / 16 (kG = 64 / (keys per lane group)).
template <int D, int W>
struct Producer {
  static constexpr int kDC = D / 8;                         // 16-byte chunks per head row
  static constexpr int kThreads = Shape<D, W>::kProdWaves * 64;   // the producing waves
  static constexpr int kKChunks = kBN * D / 8 / kThreads;   // K chunks per thread
  static constexpr int kG = kKChunks;                       // V keys per thread
  static constexpr int kGroups = kBN / kG;                  // V key groups per dim chunk
  static constexpr int kKeysPerU = kThreads / kDC;          // keys between K chunks u, u+1
  static constexpr int kPages = kBN / 16;
  static_assert(kKChunks >= 1 && (kG == 1 || kG == 2 || kG == 4), "tile / thread split");
  static_assert(kKeysPerU % 16 == 0 && 16 % kG == 0, "loads must not straddle pages");
  static constexpr int kChunksPerBlock = (kKChunks + kBN / 32 - 1) / (kBN / 32);

  // One tile in flight from global memory.
  struct Regs {
    uint4 k[kKChunks];
    uint4 v[kKChunks];
  };

  int vid[2];          // page ids of the tiles of parity 0 / 1 (lane L: page vpage(L))
  float chk;           // range check of the fp16 words this thread wrote (bf16 caches)

  // per-thread constants
  uint32_t koff;       // byte offset of this lane's K chunk inside a page (+ head)
  int kpage0;          // page of K chunk 0 (wave-uniform)
  int vpage;           // page whose id this lane fetches
  int64_t tok;         // elements between consecutive tokens of a page

  __device__ inline void init(const PrefillArgs& a, int wave, int kvh) {
    const int tid = threadIdx.x;
    chk = 0.0f;
    tok = (int64_t)a.Hkv * D;
    const int t_k = tid / kDC;
    koff = (uint32_t)(((t_k % 16) * tok + kvh * D + (tid % kDC) * 8) * 2);
    kpage0 = wave * 64 / (16 * kDC);
    vpage = kG * (tid % kGroups) / 16;
  }

  // One vector load per tile: lane L reads the id of the page its V keys are
  // in; K page p's id is read from a lane that holds it.  Tile t's id lives
  // in slot t % 2 and is fetched before the loads of the tile before it, so
  // waiting for it never waits for a K/V load issued later.
  template <int kSlot>
  __device__ inline void fetch_ids(const int32_t* bt, int mb, int kt) {
    vid[kSlot] = bt[min(kt * kPages + vpage, mb - 1)];
  }

  template <typename T, int kSlot>
  __device__ inline void load_k_chunk(const PrefillArgs& a, Regs& r, int u) const {
    const int page = kpage0 + u * (kKeysPerU / 16);              // wave-uniform
    const int kid = __builtin_amdgcn_readlane(vid[kSlot], page * 16 / kG);
    const char* base = reinterpret_cast<const char*>(a.k) +
                       safe_block(kid, a.NB) * tok * 16 * (int64_t)sizeof(T);
    r.k[u] = load16(base + koff);
  }

  template <typename T, int kSlot>
  __device__ inline void load_v(const PrefillArgs& a, Regs& r) const {
#pragma unroll
    for (int u = 0; u < kKChunks; ++u) {
      const int page = kpage0 + u * (kKeysPerU / 16);            // wave-uniform
      const int vid_u = __builtin_amdgcn_readlane(vid[kSlot], page * 16 / kG);
      const char* base = reinterpret_cast<const char*>(a.v) +
                         safe_block(vid_u, a.NB) * tok * 16 * (int64_t)sizeof(T);
      r.v[u] = load16(base + koff);
    }
  }

  template <typename T, int kSlot>
  __device__ inline void load_tile(const PrefillArgs& a, Regs& r) const {
#pragma unroll
    for (int u = 0; u < kKChunks; ++u) load_k_chunk<T, kSlot>(a, r, u);
    load_v<T, kSlot>(a, r);
  }

  // Registers -> LDS (fp16; K with the bit-2/3 row swap, V in key order).
  // Only a bf16 cache can hold values fp16 cannot; those words are checked.
  // The empty asm pins each check next to its conversion: left free, the
  // compiler sinks the checks into the next tile and keeps the converted
  // words alive until then (+14 VGPRs for K's, +16 for V's, measured).
  __device__ inline void fold_check(float x) {
    chk += x;
    asm volatile("" : "+v"(chk));
  }
  template <typename T>
  __device__ inline void store_k_chunk(PrefillTileLds<D>& s, const Regs& r, int u) {
    const int t_k = threadIdx.x / kDC;
    const int row0 = (t_k & ~31) | swap_bits23(t_k & 31);
    const uint4 h = to_f16x8<T>(r.k[u]);
    if constexpr (std::is_same_v<T, Bf16>) fold_check(f16_check(h, 0.0f));
    *reinterpret_cast<uint4*>(&s.k[row0 + u * kKeysPerU][(threadIdx.x % kDC) * 8]) = h;
  }

  template <typename T>
  __device__ inline void store_v(PrefillTileLds<D>& s, const Regs& r) {
    const int t_k = threadIdx.x / kDC;
#pragma unroll
    for (int u = 0; u < kKChunks; ++u) {
      const uint4 h = to_f16x8<T>(r.v[u]);
      if constexpr (std::is_same_v<T, Bf16>) fold_check(f16_check(h, 0.0f));
      *reinterpret_cast<uint4*>(&s.v[t_k + u * kKeysPerU][(threadIdx.x % kDC) * 8]) = h;
    }
  }

  template <typename T>
  __device__ inline void store_tile(PrefillTileLds<D>& s, const Regs& r) {
#pragma unroll
    for (int u = 0; u < kKChunks; ++u) store_k_chunk<T>(s, r, u);
    store_v<T>(s, r);
  }
};

// S^T for the 32 keys of block kb of an LDS tile against this wave's 32
// queries.  All K fragments are read before the first MFMA (the scheduler is
// fenced from sinking the reads), so LDS latency is paid once per block.
template <int D>
__device__ inline float16x qk_block(const PrefillTileLds<D>& t, int kb, const half8* qf, int j,
                                    int hh) {
  constexpr int kDC16 = D / 16;
  half8 kf[kDC16];
#pragma unroll
  for (int c = 0; c < kDC16; ++c)
    kf[c] = *reinterpret_cast<const half8*>(&t.k[kb * 32 + j][16 * c + 8 * hh]);
  __builtin_amdgcn_sched_barrier(0);
  float16x s;
#pragma unroll
  for (int r = 0; r < 16; ++r) s[r] = 0.0f;
#pragma unroll
  for (int c = 0; c < kDC16; ++c) s = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[c], qf[c], s, 0, 0, 0);
  return s;
}

// Longest-first dispatch.  Every workgroup ranks the batch's sequences by the
// keys their last (heaviest) query tile walks, descending, and lays out the
// query tiles sequence by sequence in that order, each sequence's tiles
// heaviest first; the workgroup takes the tile of rank `slot / nh` for its
// slot.  Head h runs on XCD h % 8, so the query tiles of one (sequence, head)
// run close together on one XCD and share its L2, and each XCD gets the same
// mix of work.  Ranking sequences rather than single tiles keeps that
// sharing: tiles of equal length from different sequences would otherwise
// interleave and evict each other's K/V.  Returns false when the slot has no
// tile.
struct RankScratch {
  int keys[kMaxRanked];      // keys walked by each sequence's last tile
  int tiles[kMaxRanked];     // query tiles of each sequence
  int ctx[kMaxRanked];       // context length, first row and rows of each
  int row0[kMaxRanked];      // sequence, kept so that the chosen one's need
  int rows[kMaxRanked];      // no second trip to memory
  int b, qt;
};

__device__ inline int seq_rows(const PrefillArgs& a, int b) {
  return a.cu_q ? a.cu_q[b + 1] - a.cu_q[b] : a.S;
}

template <int kBM>
__device__ inline bool ranked_tile(const PrefillArgs& a, RankScratch& rs, int& b, int& h, int& qt,
                                   int& part) {
  const int xcd = blockIdx.x % kXcds;
  const int slot = blockIdx.x / kXcds;
  const int nh = a.H > xcd ? (a.H - xcd + kXcds - 1) / kXcds : 0;   // heads on this XCD
  if (nh == 0) return false;
  const int r = slot / (nh * a.n_split);   // slot = (r * n_split + part) * nh + head
  const int tid = threadIdx.x;
  if (tid < a.B) {
    const int rows = seq_rows(a, tid);
    const int ctx = a.ctx[tid];
    rs.keys[tid] = rows > 0 ? min(a.MB * 16, ctx) : -1;
    rs.tiles[tid] = (rows + kBM - 1) / kBM;
    rs.ctx[tid] = ctx;
    rs.row0[tid] = a.cu_q ? a.cu_q[tid] : tid * a.S;
    rs.rows[tid] = rows;
  }
  if (tid == 0) rs.b = -1;
  __syncthreads();
  // Sequence tid's first slot in the ranked layout is the tile count of the
  // sequences ranked before it; the thread whose range holds slot r claims it.
  if (tid < a.B) {
    const int k = rs.keys[tid];
    int start = 0;
    for (int q = 0; q < a.B; ++q) {
      const int kq = rs.keys[q];
      start += ((kq > k) | ((kq == k) & (q < tid))) ? rs.tiles[q] : 0;
    }
    const int n = rs.tiles[tid];
    if (r >= start && r < start + n) {
      rs.b = tid;
      rs.qt = n - 1 - (r - start);
    }
  }
  __syncthreads();
  b = rs.b;
  if (b < 0) return false;
  qt = rs.qt;
  h = xcd + kXcds * (slot % nh);
  part = (slot / nh) % a.n_split;
  return true;
}

// The rows of one wave in fp32 (RowWalk, the VALU decode arithmetic), for a
// workgroup whose fp16 operands overflowed: rows w_first .. w_first + 31 of
// sequence b, head h, keys [key_lo, key_hi) of the row's causal range.  It
// writes what the matrix-core loop would have: the normalised output row, or
// with a key-range split the part's un-normalised state.  One row at a time
// with the whole wave on it: slow, and only taken for such inputs.
template <typename T, int D>
__device__ inline void prefill_rows_fp32(const PrefillArgs& a, int b, int h,
                                                            int kvh, int row0, int S_b,
                                                            int base_pos, int cap, int w_first,
                                                            int key_lo, int key_hi, int part) {
  using Walk = RowWalk<T, D, true, 1>;   // 16-token pages: a load group never straddles one
  const KvPages kv{a.k, a.v, a.Hkv, 16, a.NB};
  const int32_t* bt = a.bt + (int64_t)b * a.MB;
  for (int j = 0; j < kRowsPerWave; ++j) {
    const int i = w_first + j;
    if (i >= S_b || (a.n_split > 1 && i >= a.rows_cap)) break;
    const int hi = min(key_hi, min(base_pos + i, cap - 1) + 1);
    const float* q = a.q + ((int64_t)(row0 + i) * a.H + h) * D;
    Walk w;
    if (key_lo < hi) {
      w.run(kv, q, a.qscale, kvh, bt, key_lo, hi);
    } else {   // no keys: a zero row, or an empty part (weight 0 in the merge)
      w.m[0] = kNegBig;
      w.l[0] = 0.0f;
#pragma unroll
      for (int e = 0; e < Walk::kVec; ++e) w.acc[0][e] = 0.0f;
    }
    if (a.n_split > 1) {
      const int64_t pair = ((int64_t)(part * a.B + b) * a.rows_cap + i) * a.H + h;
      w.store_state(0, a.part_o + pair * D, a.part_ml + pair);
    } else {
      w.store_out(0, a.out + ((int64_t)(row0 + i) * a.H + h) * D);
    }
  }
}

template <typename T, int D, int W>
__global__ __launch_bounds__((Shape<D, W>::kThreads)) __attribute__((amdgpu_waves_per_eu(2)))
void prefill_mfma_kernel(PrefillArgs a) {
  using Sh = Shape<D, W>;
  constexpr int kBM = Sh::kBM;
  constexpr int kDC16 = D / 16;   // 16-dim chunks (QK MFMA k-steps)
  constexpr int kDB = D / 32;     // 32-dim output blocks
  constexpr int kNKB = kBN / 32;  // 32-key blocks per tile
  __shared__ PrefillTileLds<D> lds[2];
  __shared__ int range_fail;      // some fp16 operand of this workgroup was inf or NaN

  // ---- which (sequence, head, query tile) -------------------------------
  int b, h, qt, row0, S_b, ctx_b, part = 0;
  if (a.ranked) {
    __shared__ RankScratch rank_scratch;
    if (!ranked_tile<kBM>(a, rank_scratch, b, h, qt, part)) return;
    row0 = rank_scratch.row0[b];
    S_b = rank_scratch.rows[b];
    ctx_b = rank_scratch.ctx[b];
  } else {
    // all query tiles of one (sequence, head) on one XCD, heaviest first
    const int xcd = blockIdx.x % kXcds;
    const int slot = blockIdx.x / kXcds;
    const int pair = (slot / a.n_qt) * kXcds + xcd;     // (b * H + h)
    if (pair >= a.B * a.H) return;
    qt = a.n_qt - 1 - slot % a.n_qt;
    b = pair / a.H;
    h = pair - b * a.H;
    if (a.cu_q) {
      row0 = a.cu_q[b];
      S_b = a.cu_q[b + 1] - row0;
    } else {
      row0 = b * a.S;
      S_b = a.S;
    }
    ctx_b = a.ctx[b];
  }
  if (qt * kBM >= S_b) return;
  if (threadIdx.x == 0) range_fail = 0;   // ordered before any write by the walk's barriers

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 31;          // query of this lane within the wave's 32
  const int hh = lane >> 5;         // lane half
  const int kvh = h / (a.H / a.Hkv);
  const int cap = a.MB * 16;        // keys the block table can address
  const int base_pos = ctx_b - S_b;     // position of row 0 of the chunk

  // This lane's query row and its inclusive key limit (-1: padding row).
  const int w_first = qt * kBM + wave * kRowsPerWave;
  const int i_row = w_first + j;
  const bool row_ok = i_row < S_b;
  const int lim = row_ok ? min(base_pos + i_row, cap - 1) : -1;
  const int last_row = min(qt * kBM + kBM, S_b) - 1;
  const int kend = min(cap, base_pos + last_row + 1);           // keys the workgroup needs
  // This workgroup's key tiles [kt0, kt1): all of them, or its part of a
  // split.  Every query tile of a sequence cuts at the same key tiles (parts
  // of ceil(T / n_split) tiles, T = the sequence's last tile's count), so the
  // workgroups of one part stream the same K/V at the same time; the longest
  // tile's parts set the span either way.
  const int kt_all = kend > 0 ? (kend + kBN - 1) / kBN : 0;
  // (a negative context, invalid input, counts as empty: kt0 and the table
  // offset below stay >= 0)
  const int kt_seq = (max(0, min(cap, ctx_b)) + kBN - 1) / kBN;
  const int per_part = (kt_seq + a.n_split - 1) / a.n_split;
  const int kt0 = min(kt_all, part * per_part);
  const int kt1 = min(kt_all, kt0 + per_part);
  // Block table from tile kt0 on.  A non-empty part has kt0 * 4 < MB (since
  // kt_all * 64 < MB * 16 + 64); an empty one consumes no tile, and its
  // prologue loads stay in the table through the clamp.
  const int pg0 = min(kt0, (a.MB - 1) / (kBN / 16)) * (kBN / 16);
  const int32_t* bt = a.bt + (int64_t)b * a.MB + pg0;
  const int mb = a.MB - pg0;
  const int w_lim_min = min(base_pos + w_first, cap - 1);       // first row of the wave
  const int w_lim_max = w_first < S_b ? min(base_pos + min(w_first + kRowsPerWave, S_b) - 1,
                                            cap - 1)
                                      : -1;

  // Q^T fragments: lane (j, hh) holds q[row][16c + 8hh .. +7] (loaded in the
  // prologue below, beside the first tile's loads)
  half8 qf[kDC16];

  float16x o[kDB];
#pragma unroll
  for (int d = 0; d < kDB; ++d)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[d][r] = 0.0f;
  float m = kNegBig;   // running max (shared by lanes j and j + 32)
  float l = 0.0f;      // this lane's share of the running sum

  // ---- key tiles: double-buffered LDS, one barrier per tile ---------------
  // Tiles pass through one register set of the producing waves and two LDS
  // buffers (tile t in buffer t % 2).  While tile kt is consumed from LDS,
  // tile kt+1 is written from the register set into the idle buffer and the
  // set is refilled with tile kt+2, so a load has one tile of compute to
  // arrive (two tiles ahead measured the same).  Block ids run one tile ahead
  // of the loads.  The loop is instantiated twice: with the producer's work
  // for waves 0..kWaves/2-1 and without it for the others; both run one
  // barrier per tile.
  auto run = [&](auto prod_tag) {
    constexpr bool kProd = decltype(prod_tag)::value;
    using P = Producer<D, W>;
    const int n_kt = kt1 - kt0;
    P pr;
    pr.init(a, wave, kvh);
    typename P::Regs rg;
    float qchk = 0.0f;   // range check of this lane's fp16 query words
    // In the main loop every load and block-id fetch is unconditional, so that
    // the compiler counts outstanding loads exactly and waits only for the tile
    // it is about to store (a load issued under a condition makes it wait for
    // all of them).  The last tile pairs run a tail copy of the step that loads
    // only what is still needed.
    // The prologue is ordered so that its memory round trips overlap: block
    // ids of tiles 0 and 1, then Q, then tile 0's K/V (waiting for the ids
    // only), then Q's conversion, tile 0's LDS store and tile 1's loads.  Its
    // loads are unconditional too: ids are clamped to the table, so a tile past
    // the end reads a valid page, and a padding row reads the chunk's last row
    // (scaled to zero).
    if constexpr (kProd) {
      pr.template fetch_ids<0>(bt, mb, 0);
      pr.template fetch_ids<1>(bt, mb, 1);
    }
    {
      float4 x[2 * kDC16];
      const float* qp = a.q + ((int64_t)(row0 + min(i_row, S_b - 1)) * a.H + h) * D + 8 * hh;
#pragma unroll
      for (int c = 0; c < kDC16; ++c) {
        x[2 * c] = *reinterpret_cast<const float4*>(qp + 16 * c);
        x[2 * c + 1] = *reinterpret_cast<const float4*>(qp + 16 * c + 4);
      }
      if constexpr (kProd) pr.template load_tile<T, 0>(a, rg);
      const float sc = row_ok ? a.qscale : 0.0f;   // padding rows: q = 0
#pragma unroll
      for (int c = 0; c < kDC16; ++c) {
        const float4 x0 = x[2 * c], x1 = x[2 * c + 1];
        const uint4 w = make_uint4(pack_f16(x0.x * sc, x0.y * sc), pack_f16(x0.z * sc, x0.w * sc),
                                   pack_f16(x1.x * sc, x1.y * sc), pack_f16(x1.z * sc, x1.w * sc));
        qchk = f16_check(w, qchk);
        qf[c] = __builtin_bit_cast(half8, w);
      }
    }
    if constexpr (kProd) {
      pr.template store_tile<T>(lds[0], rg);
      pr.template fetch_ids<0>(bt, mb, 2);
      pr.template load_tile<T, 1>(a, rg);
    }
    __syncthreads();

    // One tile: consume tile kt from buffer kSet ^ 1, write tile kt+1 from the
    // register set into buffer kSet, refill the set with tile kt+2 (block ids of
    // tile t in slot t % 2).
    auto tile_step = [&](auto set_tag, auto main_tag, int kt) {
      constexpr int kSet = decltype(set_tag)::value;
      constexpr bool kMain = decltype(main_tag)::value;   // loads known to be needed
      const bool load = kMain || kt + 2 < n_kt;   // tile kt+2 is needed
      typename P::Regs& r = rg;
      PrefillTileLds<D>& nxt = lds[kSet];
      const PrefillTileLds<D>& t = lds[kSet ^ 1];
      const bool fill = kt + 1 < n_kt;        // tile kt+1 sits in set kSet
      const int tile_key0 = (kt0 + kt) * kBN;
      // 32-key blocks of this tile that reach this wave's rows (wave-uniform);
      // none in the padding step after an odd tile count, whose keys may still
      // reach the rows when the range is one part of a split
      const bool live = kMain || kt < n_kt;
      const int nkb = !live || w_lim_max < tile_key0
                          ? 0
                          : min(kNKB, (w_lim_max - tile_key0) / 32 + 1);

      half8 kn[kDC16];   // K fragments of the next block of this tile
  #pragma unroll
      for (int kb = 0; kb < kNKB; ++kb) {
        // Producer share of this block: V at block 0, K chunks spread over the
        // blocks; each store frees registers for the matching load of tile kt+2.
        if (kProd && kb == 0) {
          if (kMain || kt + 3 < n_kt) pr.template fetch_ids<kSet>(bt, mb, kt + 3);
          if (fill) pr.template store_v<T>(nxt, r);
          if (load) pr.template load_v<T, kSet ^ 1>(a, r);      // tile kt+2
        }
  #pragma unroll
        for (int cc = 0; cc < P::kChunksPerBlock; ++cc) {
          const int u = kb * P::kChunksPerBlock + cc;
          if (kProd && u < P::kKChunks) {
            if (fill) pr.template store_k_chunk<T>(nxt, r, u);
            if (load) pr.template load_k_chunk<T, kSet ^ 1>(a, r, u);
          }
        }
        if (kb >= nkb) continue;

        // S^T of block 0 reads its K fragments here; those of block 1 were read
        // during block 0's softmax (measured +2% on C4, bit-identical)
        float16x s;
        if (kb == 0) {
          s = qk_block<D>(t, kb, qf, j, hh);
        } else {
  #pragma unroll
          for (int r = 0; r < 16; ++r) s[r] = 0.0f;
  #pragma unroll
          for (int c = 0; c < kDC16; ++c) s = __builtin_amdgcn_mfma_f32_32x32x16_f16(kn[c], qf[c], s, 0, 0, 0);
        }

        // V^T fragments of this block, read before the softmax so that their
        // latency hides behind it.
        half8 vf[2][kDB];
  #pragma unroll
        for (int kc = 0; kc < 2; ++kc)
  #pragma unroll
          for (int d = 0; d < kDB; ++d)
            vf[kc][d] = vt_fragment<D>(t, d, kb * 32 + kc * 16, j, hh);
        if (kb + 1 < kNKB) {
  #pragma unroll
          for (int c = 0; c < kDC16; ++c)
            kn[c] = *reinterpret_cast<const half8*>(&t.k[(kb + 1) * 32 + j][16 * c + 8 * hh]);
        }

        // mask: accumulator register r of half hh holds key key0 + 16*(r/8) + 8*hh + r%8
        const int key0 = tile_key0 + kb * 32;
        if (key0 + 31 > w_lim_min) {
  #pragma unroll
          for (int r = 0; r < 16; ++r)
            if (key0 + 16 * (r >> 3) + 8 * hh + (r & 7) > lim) s[r] = -INFINITY;
        }

        // online softmax; the max is only raised when it grows by > 8
        float mx = s[0];
  #pragma unroll
        for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s[r]);
        mx = max_halves(mx);
        if (__builtin_amdgcn_ballot_w64(mx > m + kRescaleSlack) != 0) {
          const float m_new = fmaxf(m, mx);
          const float corr = fast_exp2(m - m_new);
          l *= corr;
  #pragma unroll
          for (int d = 0; d < kDB; ++d)
  #pragma unroll
            for (int r = 0; r < 16; ++r) o[d][r] *= corr;
          m = m_new;
        }
        half8 p[2];
  #pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
          uint32_t w[4];
  #pragma unroll
          for (int i = 0; i < 4; ++i) {
            // masked scores are -inf: exp2(-inf) = 0
            w[i] = pack_f16(fast_exp2(s[8 * hf + 2 * i] - m), fast_exp2(s[8 * hf + 2 * i + 1] - m));
            // the row sum adds the fp16 probabilities P.V will use
            l = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2x, w[i]),
                                       (half2x){(_Float16)1.0f, (_Float16)1.0f}, l, false);
          }
          p[hf] = __builtin_bit_cast(half8, make_uint4(w[0], w[1], w[2], w[3]));
        }

        // O^T += V^T . P^T over the two 16-key chunks of this block
  #pragma unroll
        for (int kc = 0; kc < 2; ++kc)
  #pragma unroll
          for (int d = 0; d < kDB; ++d)
            o[d] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[kc][d], p[kc], o[d], 0, 0, 0);
      }
      __syncthreads();   // buffer kSet is complete; buffer kSet ^ 1 is consumed
    };

    // Pairs of steps (so that register sets and LDS buffers are static); an
    // odd count ends with one empty step (nothing consumed or stored).
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    using Main = std::true_type;
    using Tail = std::false_type;
    int kt = 0;
    for (; kt + 4 < n_kt; kt += 2) {
      tile_step(S1{}, Main{}, kt);
      tile_step(S0{}, Main{}, kt + 1);
    }
    for (; kt < n_kt; kt += 2) {
      tile_step(S1{}, Tail{}, kt);
      tile_step(S0{}, Tail{}, kt + 1);
    }
    return f16_check_failed(pr.chk + qchk);
  };
  const bool my_fail = wave < Sh::kProdWaves ? run(std::true_type{}) : run(std::false_type{});

  // Operands fp16 cannot hold (a bf16 K/V value of magnitude >= 65536 among the
  // keys this workgroup walked, or a scaled query >= 65520) make the
  // matrix-core result unusable: the workgroup recomputes its rows in fp32.
  if (my_fail) range_fail = 1;
  __syncthreads();
  if (range_fail) {
    prefill_rows_fp32<T, D>(a, b, h, kvh, row0, S_b, base_pos, cap, w_first, kt0 * kBN,
                            kt1 * kBN, part);
    return;
  }

  // ---- normalise and store: lane (j, hh) owns query j and dims
  // d*32 + 8*g + 4*hh + (0..3) ----
  const float lsum = sum_halves(l);
  if (!row_ok) return;
  float inv;
  float* op;
  if (a.n_split > 1) {
    // one part of a split: unnormalised O and (running max, sum) for the merge
    // (rows past rows_cap, which a too-small max_seqlen_q leaves, have no slot)
    if (i_row >= a.rows_cap) return;
    const int64_t pair = ((int64_t)(part * a.B + b) * a.rows_cap + i_row) * a.H + h;
    if (hh == 0) a.part_ml[pair] = make_float2(m, lsum);
    inv = 1.0f;
    op = a.part_o + pair * D + 4 * hh;
  } else {
    inv = lsum > 0.0f ? 1.0f / lsum : 0.0f;
    op = a.out + ((int64_t)(row0 + i_row) * a.H + h) * D + 4 * hh;
  }
#pragma unroll
  for (int d = 0; d < kDB; ++d)
#pragma unroll
    for (int g = 0; g < 4; ++g)
      *reinterpret_cast<float4*>(op + d * 32 + 8 * g) =
          make_float4(o[d][4 * g] * inv, o[d][4 * g + 1] * inv, o[d][4 * g + 2] * inv,
                      o[d][4 * g + 3] * inv);
}

// ---------------------------------------------------------------------------
// Pipelined kernel: 8 waves of 32 query rows, head dim 64 and 128.
//
// Per 64-key tile and SIMD the two resident waves issue 2 x 32 MFMAs (2048
// cycles of the matrix pipe); everything else has to fit beside them.  Three
// choices keep it there:
//  * V is stored d-major in LDS (V^T, one 64-key row per dim), transposed by
//    the producer while it widens bf16 to fp16 (the same instruction count
//    as the widening alone), so every MFMA fragment is one ds_read_b128;
//  * every wave moves one eighth of each tile (the keys of half a page, K and
//    V), so no wave carries the producer alone;
//  * three LDS buffers: while tile t is consumed, tile t+1 is complete and
//    tile t+2 is being written.  Each wave runs a software pipeline over its
//    32-key blocks, S^T of block b+1 (including the first block of the next
//    tile) on the MFMA pipe beside the softmax of block b, and P.V of block b
//    beside its producer share.
// The softmax subtracts the running max inside the QK product (the
// accumulator starts at -m, a register block kept per wave), and replaces
// the per-block row max by a check of the block's probability sum: a block
// whose fp16 probabilities could exceed 65504 (a new max more than ~15
// above m, in log2 units) takes a rare path that raises m, rescales O and
// redoes the block.  So a steady-state block costs 16 exponentials, 8
// conversions and 8 dot products per lane.
// ---------------------------------------------------------------------------

constexpr int kPipeWaves = 8;
// Fourth word of a raw (unformatted, unswizzled) buffer resource on gfx9-family
// GPUs, gfx950 included.
constexpr int kBufferRsrcWord3 = 0x00020000;
constexpr int kPipeBufs = 3;
constexpr float kPMax = 65504.0f;            // largest finite fp16

// One tile in LDS.  K rows as in PrefillTileLds (row r of a 32-key block holds
// key swap23(r)); V^T row d holds V[key][d] of the tile's 64 keys in key
// order, its 16-byte chunk c (keys 8c .. 8c+7) stored at chunk
// c ^ vt_swz<D>(d).  Layouts measured on gfx950 with the LDS bank-conflict
// counter (ds_read_b128 / ds_write_b128, every row stride from 128 to 384
// bytes against several chunk swizzles): for the fragment reads (32
// consecutive rows, one chunk per lane half) and the producer's writes (rows
// 2l, 2l + 1 of lane l at D 128; row l at D 64) both to be conflict-free,
// D 128 takes unpadded 128-byte rows with the chunk XORed by (d >> 1) & 7,
// and D 64 144-byte rows with no swizzle.
template <int D>
constexpr int vt_pad() { return D == 128 ? 0 : 8; }
template <int D>
__device__ inline int vt_swz(int d) { return D == 128 ? (d >> 1) & 7 : 0; }

template <int D>
struct PipeTile {
  _Float16 k[kBN][D + kKPad];
  _Float16 vt[D][kBN + vt_pad<D>()];
};

// The producer share of wave w: the keys 8w .. 8w+7 of each tile (half of
// page w / 2), K and V.  V: lane l loads the D / 64 dims kVD * l .. of each of
// the 8 keys (one coalesced token row per load instruction), widens and
// transposes them into kVD V^T rows of 8 keys (one 16-byte LDS write each).
// K: 16-byte chunks, kKC lanes per token row, kKU chunks per lane, written
// row by row.  The page base is wave-uniform (one block id per wave and tile).
template <typename T, int D>
struct PipeProducer {
  static constexpr int kVD = D / 64;
  static constexpr int kKC = D / 8;
  static constexpr int kKU = kKC / 8;
  static constexpr int kKeysPerKU = 64 / kKC;
  static_assert(kVD >= 1 && kKU >= 1, "head dim 64 or 128");

  uint32_t v[8];      // V words of the tile in flight: key u in v[u]
  uint4 k[kKU];       // K chunks of the tile in flight
  int ids;            // lanes 0..3 (mod 4): block ids of the 4 pages of one tile
  const char* kpage;  // K page of the tile whose V load_v issued (wave-uniform)
  float chk;          // range check of the converted K words (bf16 caches)

  int64_t page_bytes;  // bytes of one page of the cache
  uint32_t v_off;      // byte offset of this lane's V word in its page (key 0 of the wave)
  uint32_t k_off;      // byte offset of this lane's K chunk (u = 0)
  uint32_t tok_bytes;  // bytes between consecutive tokens of a page
  int wave, lane;

  __device__ inline void init(const PrefillArgs& a, int wave_, int kvh) {
    wave = wave_;
    lane = threadIdx.x & 63;
    chk = 0.0f;
    tok_bytes = (uint32_t)(a.Hkv * D * (int)sizeof(T));
    page_bytes = (int64_t)tok_bytes * 16;
    const uint32_t head = (uint32_t)(kvh * D * (int)sizeof(T));
    const uint32_t tok0 = (uint32_t)(8 * (wave & 1));
    v_off = tok0 * tok_bytes + head + (uint32_t)(kVD * lane * (int)sizeof(T));
    k_off = (tok0 + (uint32_t)(lane / kKC)) * tok_bytes + head +
            (uint32_t)(8 * (lane % kKC) * (int)sizeof(T));
  }

  // Block ids of tile `tile` (clamped to the table, which has mb >= 1
  // entries; a part without tiles asks for tile -1): one vector load.
  __device__ inline void fetch_ids(const int32_t* bt, int mb, int tile) {
    ids = bt[min(max(tile * 4 + (lane & 3), 0), mb - 1)];
  }

  __device__ inline const char* page(const PrefillArgs& a, const void* base) const {
    const int id = __builtin_amdgcn_readlane(ids, wave >> 1);
    return reinterpret_cast<const char*>(base) + safe_block(id, a.NB) * page_bytes;
  }

  // Buffer resource of one page (base, unstrided, page_bytes long): loads
  // take the lane's offset in a VGPR and the key's in an SGPR, so a tile's
  // loads share one 64-bit page base instead of computing an address each.
  __device__ inline __amdgpu_buffer_rsrc_t page_rsrc(const char* page) const {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(page), (short)0,
                                             (int)page_bytes, kBufferRsrcWord3);
  }

  // V of the tile whose ids are in `ids`; also keeps that tile's K page, so
  // that `ids` can take the next tile's ids before load_k
  __device__ inline void load_v(const PrefillArgs& a) {
    kpage = page(a, a.k);
    const __amdgpu_buffer_rsrc_t r = page_rsrc(page(a, a.v));
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if constexpr (kVD == 2) {
        v[u] = __builtin_amdgcn_raw_buffer_load_b32(r, (int)v_off, (int)(u * tok_bytes), 0);
      } else {
        v[u] = __builtin_amdgcn_raw_buffer_load_b16(r, (int)v_off, (int)(u * tok_bytes), 0);
      }
    }
  }

  __device__ inline void load_k() {
    const __amdgpu_buffer_rsrc_t r = page_rsrc(kpage);
#pragma unroll
    for (int u = 0; u < kKU; ++u) {
      typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
      const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(
          r, (int)k_off, (int)(u * kKeysPerKU * tok_bytes), 0);
      k[u] = make_uint4(x[0], x[1], x[2], x[3]);
    }
  }

  // fp16 word of keys (u, u+1) of dim e (0: low half of the loaded word)
  __device__ inline uint32_t vpair(int u, int e) const {
    if constexpr (std::is_same_v<T, Bf16>) {
      const float x0 = __uint_as_float(e ? (v[u] & 0xffff0000u) : (v[u] << 16));
      const float x1 = __uint_as_float(e ? (v[u + 1] & 0xffff0000u) : (v[u + 1] << 16));
      return pack_f16(x0, x1);
    } else {
      return e ? __builtin_amdgcn_perm(v[u + 1], v[u], 0x07060302u)
               : __builtin_amdgcn_perm(v[u + 1], v[u], 0x05040100u);
    }
  }

  __device__ inline void store_v(PipeTile<D>& t) const {
#pragma unroll
    for (int e = 0; e < kVD; ++e) {
      const int d = kVD * lane + e;
      const uint4 w = make_uint4(vpair(0, e), vpair(2, e), vpair(4, e), vpair(6, e));
      *reinterpret_cast<uint4*>(&t.vt[d][8 * (wave ^ vt_swz<D>(d))]) = w;
    }
  }

  __device__ inline void store_k(PipeTile<D>& t) {
#pragma unroll
    for (int u = 0; u < kKU; ++u) {
      const int key = 8 * wave + kKeysPerKU * u + lane / kKC;
      const int row = (key & ~31) | swap_bits23(key & 31);
      const uint4 h = to_f16x8<T>(k[u]);
      if constexpr (std::is_same_v<T, Bf16>) {
        chk = f16_check(h, chk);
        asm volatile("" : "+v"(chk));
      }
      *reinterpret_cast<uint4*>(&t.k[row][8 * (lane % kKC)]) = h;
    }
  }
};

template <typename T, int D>
__global__ __launch_bounds__(kPipeWaves * 64) __attribute__((amdgpu_waves_per_eu(2)))
void prefill_pipe_kernel(PrefillArgs a) {
  constexpr int kBM = kPipeWaves * kRowsPerWave;
  constexpr int kDC16 = D / 16;   // QK MFMA k-steps
  constexpr int kDB = D / 32;     // 32-dim output blocks
  using Prod = PipeProducer<T, D>;
  __shared__ PipeTile<D> lds[kPipeBufs];
  __shared__ int range_fail;

  // ---- which (sequence, head, query tile) -------------------------------
  int b, h, qt, row0, S_b, ctx_b, part = 0;
  if (a.ranked) {
    __shared__ RankScratch rank_scratch;
    if (!ranked_tile<kBM>(a, rank_scratch, b, h, qt, part)) return;
    row0 = rank_scratch.row0[b];
    S_b = rank_scratch.rows[b];
    ctx_b = rank_scratch.ctx[b];
  } else {
    const int xcd = blockIdx.x % kXcds;
    const int slot = blockIdx.x / kXcds;
    const int pair = (slot / a.n_qt) * kXcds + xcd;
    if (pair >= a.B * a.H) return;
    qt = a.n_qt - 1 - slot % a.n_qt;
    b = pair / a.H;
    h = pair - b * a.H;
    if (a.cu_q) {
      row0 = a.cu_q[b];
      S_b = a.cu_q[b + 1] - row0;
    } else {
      row0 = b * a.S;
      S_b = a.S;
    }
    ctx_b = a.ctx[b];
  }
  if (qt * kBM >= S_b) return;
  if (threadIdx.x == 0) range_fail = 0;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 31;
  const int hh = lane >> 5;
  const int kvh = h / (a.H / a.Hkv);
  const int cap = a.MB * 16;
  const int base_pos = ctx_b - S_b;

  const int w_first = qt * kBM + wave * kRowsPerWave;
  const int i_row = w_first + j;
  const bool row_ok = i_row < S_b;
  const int lim = row_ok ? min(base_pos + i_row, cap - 1) : -1;
  const int last_row = min(qt * kBM + kBM, S_b) - 1;
  const int kend = min(cap, base_pos + last_row + 1);
  const int kt_all = kend > 0 ? (kend + kBN - 1) / kBN : 0;
  const int kt_seq = (max(0, min(cap, ctx_b)) + kBN - 1) / kBN;
  const int per_part = (kt_seq + a.n_split - 1) / a.n_split;
  const int kt0 = min(kt_all, part * per_part);
  const int kt1 = min(kt_all, kt0 + per_part);
  const int n_kt = kt1 - kt0;
  const int pg0 = min(kt0, (a.MB - 1) / (kBN / 16)) * (kBN / 16);
  const int32_t* bt = a.bt + (int64_t)b * a.MB + pg0;
  const int mb = a.MB - pg0;
  const int key_base = kt0 * kBN;
  const int w_lim_min = min(base_pos + w_first, cap - 1);
  const int w_lim_max = w_first < S_b ? min(base_pos + min(w_first + kRowsPerWave, S_b) - 1,
                                            cap - 1)
                                      : -1;
  // this wave's live 32-key blocks of the part (wave-uniform); blocks from
  // `mask_from` on reach past the wave's first row and need the causal mask
  const int nb_w = w_lim_max < key_base ? 0 : min(2 * n_kt, (w_lim_max - key_base) / 32 + 1);
  const int mask_x = w_lim_min - key_base - 31;
  const int mask_from = mask_x < 0 ? 0 : mask_x / 32 + 1;
  const int t_w = (nb_w + 1) / 2;   // tiles with compute

  // ---- prologue: Q^T fragments, tiles 0 and 1 into buffers 0 and 1, tile
  // 2 in flight.  Tiles 0 and 1 load through two register sets at once, so
  // the prologue pays two memory round trips (ids, then K/V), not four.
  half8 qf[kDC16];
  float qchk = 0.0f;
  Prod pr, pr1;
  pr.init(a, wave, kvh);
  pr1 = pr;
  pr.fetch_ids(bt, mb, 0);
  pr1.fetch_ids(bt, mb, min(1, n_kt - 1));
  {
    float4 x[2 * kDC16];
    const float* qp = a.q + ((int64_t)(row0 + min(i_row, S_b - 1)) * a.H + h) * D + 8 * hh;
#pragma unroll
    for (int c = 0; c < kDC16; ++c) {
      x[2 * c] = *reinterpret_cast<const float4*>(qp + 16 * c);
      x[2 * c + 1] = *reinterpret_cast<const float4*>(qp + 16 * c + 4);
    }
    pr.load_v(a);
    pr.load_k();
    pr1.load_v(a);
    pr1.load_k();
    pr.fetch_ids(bt, mb, min(2, n_kt - 1));
    const float sc = row_ok ? a.qscale : 0.0f;
#pragma unroll
    for (int c = 0; c < kDC16; ++c) {
      const float4 x0 = x[2 * c], x1 = x[2 * c + 1];
      const uint4 w = make_uint4(pack_f16(x0.x * sc, x0.y * sc), pack_f16(x0.z * sc, x0.w * sc),
                                 pack_f16(x1.x * sc, x1.y * sc), pack_f16(x1.z * sc, x1.w * sc));
      qchk = f16_check(w, qchk);
      qf[c] = __builtin_bit_cast(half8, w);
    }
  }
  pr.store_v(lds[0]);
  pr.store_k(lds[0]);
  pr1.store_v(lds[1]);
  pr1.store_k(lds[1]);
  pr.chk += pr1.chk;
  pr.load_v(a);
  pr.fetch_ids(bt, mb, min(3, n_kt - 1));
  pr.load_k();
  __syncthreads();

  float16x o[kDB];
#pragma unroll
  for (int d = 0; d < kDB; ++d)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[d][r] = 0.0f;
  float m = kNegBig;    // running max (lanes j and j + 32 agree)
  float l = 0.0f;       // this lane's share of the running sum
  float16x bias;        // -m in every register: the QK accumulator's start
  float16x s_cur, s_nxt;
  half8 kf[kDC16];      // K fragments of the next QK block
  half8 vf[2][kDB];     // V^T fragments of the next P.V block
  half8 p[2];           // probabilities of the block in P.V

  auto read_k = [&](const PipeTile<D>& t, int kb) __attribute__((always_inline)) {
#pragma unroll
    for (int c = 0; c < kDC16; ++c)
      kf[c] = *reinterpret_cast<const half8*>(&t.k[kb * 32 + j][16 * c + 8 * hh]);
  };
  // accumulator register r of half hh holds key key0 + 16 (r / 8) + 8 hh + r % 8
  auto mask = [&](float16x& s, int blk) __attribute__((always_inline)) {
    const int key0 = key_base + 32 * blk;
#pragma unroll
    for (int r = 0; r < 16; ++r)
      if (key0 + 16 * (r >> 3) + 8 * hh + (r & 7) > lim) s[r] = -INFINITY;
  };
  const int vsw = hh ^ vt_swz<D>(j);   // this lane's chunk swizzle (the same for rows 32 db + j)
  // V^T fragment i (16-key chunk i / kDB, dims 32 (i % kDB) ..) of block kb
  auto read_v1 = [&](const PipeTile<D>& t, int kb, int i) __attribute__((always_inline)) {
    vf[i / kDB][i % kDB] = *reinterpret_cast<const half8*>(
        &t.vt[32 * (i % kDB) + j][8 * ((4 * kb + 2 * (i / kDB)) ^ vsw)]);
  };
  // probabilities of pair i (registers 2i, 2i+1) of s; returns the running
  // block sum
  auto prob2 = [&](const float16x& s, int i, uint32_t* w, float lb) __attribute__((always_inline)) {
    w[i] = pack_f16(fast_exp2(s[2 * i]), fast_exp2(s[2 * i + 1]));
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2x, w[i]),
                                  (half2x){(_Float16)1.0f, (_Float16)1.0f}, lb, false);
  };
  auto probs = [&](const float16x& s) __attribute__((always_inline)) {
    uint32_t w[8];
    float lb = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) lb = prob2(s, i, w, lb);
    p[0] = __builtin_bit_cast(half8, make_uint4(w[0], w[1], w[2], w[3]));
    p[1] = __builtin_bit_cast(half8, make_uint4(w[4], w[5], w[6], w[7]));
    return lb;
  };
  // One QK/softmax phase: S of the next block (when kQk) on the MFMA pipe,
  // the probabilities of `sm` on the VALU, the V^T fragments of block `vkb`
  // of `tv` from LDS, in that interleave: pair i of the softmax and V
  // fragment i follow QK k-step i.
  auto phase_qs = [&](auto qk_tag, float16x& s_out, const float16x& sm, const PipeTile<D>& tv,
                      int vkb) __attribute__((always_inline)) {
    constexpr bool kQk = decltype(qk_tag)::value;
    uint32_t w[8];
    float lb = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if constexpr (kQk) {
        if (i < kDC16)
          s_out = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[i], qf[i], i == 0 ? bias : s_out, 0,
                                                         0, 0);
      }
      if (i < 2 * kDB) read_v1(tv, vkb, i);
      lb = prob2(sm, i, w, lb);
    }
    p[0] = __builtin_bit_cast(half8, make_uint4(w[0], w[1], w[2], w[3]));
    p[1] = __builtin_bit_cast(half8, make_uint4(w[4], w[5], w[6], w[7]));
    if constexpr (kQk) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // LDS read
        __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);   // VALU
      }
    }
    return lb;
  };
  // the rare path after a softmax: some probability of block s could leave
  // fp16.  Raise m by the block's max above it, rescale O, l and the bias,
  // shift s and (when already computed) the next block's scores, and redo
  // the probabilities.
  auto settle = [&](float lb, float16x& s, float16x& nxt, bool has_nxt) __attribute__((always_inline)) {
    if (__builtin_amdgcn_ballot_w64(!(lb <= kPMax)) != 0) {
      float mx = s[0];
#pragma unroll
      for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s[r]);
      mx = max_halves(mx);
      const float dlt = mx > 0.0f ? mx : 0.0f;
      const float corr = fast_exp2(-dlt);
      m += dlt;
      l *= corr;
#pragma unroll
      for (int d = 0; d < kDB; ++d)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[d][r] *= corr;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        bias[r] -= dlt;
        s[r] -= dlt;
      }
      if (has_nxt) {
#pragma unroll
        for (int r = 0; r < 16; ++r) nxt[r] -= dlt;
      }
      lb = probs(s);
    }
    l += lb;
  };
  // One P.V phase: O += V^T . P^T on the MFMA pipe, the K fragments of the
  // next QK block (when kRead) from LDS, and the producer's share `prod`.
  auto phase_pv = [&](auto read_tag, const PipeTile<D>& tk, int kkb, auto&& prod) __attribute__((always_inline)) {
    constexpr bool kRead = decltype(read_tag)::value;
#pragma unroll
    for (int i = 0; i < 2 * kDB; ++i) {
      o[i % kDB] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[i / kDB][i % kDB], p[i / kDB],
                                                          o[i % kDB], 0, 0, 0);
      if constexpr (kRead) {
        if (i < kDC16)
          kf[i] = *reinterpret_cast<const half8*>(&tk.k[kkb * 32 + j][16 * i + 8 * hh]);
      }
    }
    prod();
    if constexpr (kRead) {
#pragma unroll
      for (int i = 0; i < 2 * kDB; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);   // MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 1);   // LDS read
        __builtin_amdgcn_sched_group_barrier(0x002, 3, 1);   // VALU
      }
    }
  };
  using Yes = std::true_type;
  using No = std::false_type;

  // ---- the walk ------------------------------------------------------------
  // Period t consumes tile t (buffer t % 3) and the first block of tile t+1,
  // writes tile t+2 (loaded during period t-1) and loads tile t+3 (block ids
  // of tile t+4 fetched between its V and K loads).  A wave with no live
  // blocks left only produces.  Every wave runs n_kt periods, one barrier
  // each.
  if (t_w > 0) {
    // first block: its max sets m and the bias
    read_k(lds[0], 0);
    float16x zero;
#pragma unroll
    for (int r = 0; r < 16; ++r) zero[r] = 0.0f;
    s_cur = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[0], qf[0], zero, 0, 0, 0);
#pragma unroll
    for (int c = 1; c < kDC16; ++c)
      s_cur = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[c], qf[c], s_cur, 0, 0, 0);
    if (mask_from == 0) mask(s_cur, 0);
    float mx = s_cur[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s_cur[r]);
    m = fmaxf(kNegBig, max_halves(mx));
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      bias[r] = -m;
      s_cur[r] -= m;
    }
    read_k(lds[0], 1);
  }
  auto prod_v = [&](PipeTile<D>& tw, int t) __attribute__((always_inline)) {
    return [&pr, &tw, &a, bt, mb, t, n_kt]() {
      pr.store_v(tw);
      pr.load_v(a);
      pr.fetch_ids(bt, mb, min(t + 4, n_kt - 1));
    };
  };
  auto prod_k = [&](PipeTile<D>& tw) __attribute__((always_inline)) {
    return [&pr, &tw]() {
      pr.store_k(tw);
      pr.load_k();
    };
  };
  int t = 0;
  // full periods: blocks 2t, 2t+1 and 2t+2 are live
  for (; t + 1 < t_w; ++t) {
    const PipeTile<D>& tc = lds[t % kPipeBufs];
    const PipeTile<D>& tn = lds[(t + 1) % kPipeBufs];
    PipeTile<D>& tw = lds[(t + 2) % kPipeBufs];
    // A: S of block 2t+1 beside the softmax of block 2t
    if (2 * t >= mask_from) mask(s_cur, 2 * t);
    float lb = phase_qs(Yes{}, s_nxt, s_cur, tc, 0);
    settle(lb, s_cur, s_nxt, true);
    // B: P.V of block 2t beside the V share of tile t+2
    phase_pv(Yes{}, tn, 0, prod_v(tw, t));
    // C: S of block 2t+2 beside the softmax of block 2t+1
    if (2 * t + 1 >= mask_from) mask(s_nxt, 2 * t + 1);
    lb = phase_qs(Yes{}, s_cur, s_nxt, tc, 1);
    settle(lb, s_nxt, s_cur, true);
    // D: P.V of block 2t+1 beside the K share of tile t+2
    phase_pv(Yes{}, tn, 1, prod_k(tw));
    __syncthreads();
  }
  if (t < t_w) {   // the last period with compute: no QK of a next tile
    const PipeTile<D>& tc = lds[t % kPipeBufs];
    PipeTile<D>& tw = lds[(t + 2) % kPipeBufs];
    const bool second = 2 * t + 1 < nb_w;
    if (2 * t >= mask_from) mask(s_cur, 2 * t);
    if (second) {
      s_nxt = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[0], qf[0], bias, 0, 0, 0);
#pragma unroll
      for (int c = 1; c < kDC16; ++c)
        s_nxt = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[c], qf[c], s_nxt, 0, 0, 0);
    }
    float lb = phase_qs(No{}, s_nxt, s_cur, tc, 0);
    settle(lb, s_cur, s_nxt, second);
    phase_pv(No{}, tc, 0, prod_v(tw, t));
    if (second) {
      if (2 * t + 1 >= mask_from) mask(s_nxt, 2 * t + 1);
      lb = phase_qs(No{}, s_cur, s_nxt, tc, 1);
      settle(lb, s_nxt, s_cur, false);
      phase_pv(No{}, tc, 1, prod_k(tw));
    } else {
      prod_k(tw)();
    }
    __syncthreads();
    ++t;
  }
  for (; t < n_kt; ++t) {   // producer only
    PipeTile<D>& tw = lds[(t + 2) % kPipeBufs];
    prod_v(tw, t)();
    prod_k(tw)();
    __syncthreads();
  }

  // ---- range check, normalise and store ------------------------------------
  // fp16 operands that overflowed (a bf16 K value >= 65536 among the walked
  // keys, a scaled query >= 65520) fail the K and Q checks; a V value that
  // overflowed makes O infinite or NaN (0 x inf for a zero probability).
  bool my_fail = f16_check_failed(pr.chk + qchk);
  {
    float oc = 0.0f;
#pragma unroll
    for (int d = 0; d < kDB; ++d)
#pragma unroll
      for (int r = 0; r < 16; ++r) oc += o[d][r] * 0.0f;
    my_fail = my_fail || !(oc == 0.0f);
  }
  if (my_fail) range_fail = 1;
  __syncthreads();
  if (range_fail) {
    prefill_rows_fp32<T, D>(a, b, h, kvh, row0, S_b, base_pos, cap, w_first, kt0 * kBN,
                            kt1 * kBN, part);
    return;
  }
  const float lsum = sum_halves(l);
  if (!row_ok) return;
  float inv;
  float* op;
  if (a.n_split > 1) {
    if (i_row >= a.rows_cap) return;
    const int64_t pair = ((int64_t)(part * a.B + b) * a.rows_cap + i_row) * a.H + h;
    if (hh == 0) a.part_ml[pair] = make_float2(m, lsum);
    inv = 1.0f;
    op = a.part_o + pair * D + 4 * hh;
  } else {
    inv = lsum > 0.0f ? 1.0f / lsum : 0.0f;
    op = a.out + ((int64_t)(row0 + i_row) * a.H + h) * D + 4 * hh;
  }
#pragma unroll
  for (int d = 0; d < kDB; ++d)
#pragma unroll
    for (int g = 0; g < 4; ++g)
      *reinterpret_cast<float4*>(op + d * 32 + 8 * g) =
          make_float4(o[d][4 * g] * inv, o[d][4 * g + 1] * inv, o[d][4 * g + 2] * inv,
                      o[d][4 * g + 3] * inv);
}

// ---------------------------------------------------------------------------
// Persistent form of the pipelined kernel (prefill_stream_kernel): one
// workgroup per CU takes query tiles from a per-XCD queue, and its producer
// streams the K/V tiles of consecutive query tiles without a break.
//
// The grid kernel pays, for every 256-row query tile, the ranking of the
// batch, two dependent memory round trips (block ids, then K/V) before its
// first tile is in LDS, an epilogue and the gap until the next workgroup
// starts on the CU: ~11 us per query tile on C4 (one tile of the key walk
// is ~1.7 us).  Here the ranking runs once per workgroup, and the producer
// treats the key tiles of a workgroup's consecutive query tiles as one
// stream: while the last tiles of one query tile are consumed, the first
// tiles of the next are already loaded, converted and stored.  The next
// tile's Q loads are issued before the epilogue that stores the current
// tile's output.
//
// Queue.  Query tiles are ranked as in the grid kernel (sequences longest
// first, each sequence's tiles heaviest first; head h on XCD h % 8).  XCD x
// serves its items in that order from one counter in the caller's workspace
// (zeroed by prefill_stream_reset_kernel before the launch), so a workgroup
// that finishes early takes the next heaviest item; per-tile costs vary with
// how much K/V the XCD's L2 shares, and a static deal of the same items left
// 26 us of idle tail on C4.  Each workgroup knows its current item and the
// next one: the next is taken (one atomic) while the current one's Q loads
// are in flight and published to all waves before its first period.  The
// producer may only enter items already published; when an item is so short
// that the stream reaches the end of the published ones, the producer holds
// on the last tile and the stream restarts (the kernel's prologue) at the
// item it could not enter.
// ---------------------------------------------------------------------------

constexpr int kStreamMaxRanked = 2048;     // ranked query tiles (all sequences)
constexpr int kStreamRing = 4;             // item slots: previous, current, next
constexpr size_t kStreamWorkspaceBytes = 256;   // one work counter per XCD
constexpr int kStreamNone = 0x7fffffff;

struct StreamScratch {
  int keys[kMaxRanked];
  int tiles[kMaxRanked];
  int ctx[kMaxRanked];
  int row0[kMaxRanked];
  int rows[kMaxRanked];
  int2 tab[kStreamMaxRanked];     // ranked tile r: {b | qt << 8, key tiles}
  int4 ring[kStreamRing];         // item j in slot j % 4: {b, h, qt, key tiles}; b < 0: none
};

// Key tiles walked by query tile qt of a sequence (rows S_b, context ctx_b):
// the causal range of its last row, capped at the table's capacity.
__device__ inline int stream_tile_keys(int S_b, int ctx_b, int qt, int cap) {
  constexpr int kBM = kPipeWaves * kRowsPerWave;
  const int last_row = min(qt * kBM + kBM, S_b) - 1;
  const int kend = min(cap, ctx_b - S_b + last_row + 1);
  return kend > 0 ? (kend + kBN - 1) / kBN : 0;
}

// Ranks the batch and fills the table of ranked tiles; returns the number of
// items of this XCD's queue (ranked tiles x heads on the XCD).
__device__ inline int stream_rank(const PrefillArgs& a, StreamScratch& s) {
  constexpr int kBM = kPipeWaves * kRowsPerWave;
  const int tid = threadIdx.x;
  const int cap = a.MB * 16;
  if (tid < a.B) {
    const int rows = seq_rows(a, tid);
    const int ctx = a.ctx[tid];
    s.keys[tid] = rows > 0 ? min(cap, ctx) : -1;
    s.tiles[tid] = (rows + kBM - 1) / kBM;
    s.ctx[tid] = ctx;
    s.row0[tid] = a.cu_q ? a.cu_q[tid] : tid * a.S;
    s.rows[tid] = rows;
  }
  __syncthreads();
  if (tid < a.B) {
    const int k = s.keys[tid];
    int start = 0;
    for (int q = 0; q < a.B; ++q) {
      const int kq = s.keys[q];
      start += ((kq > k) | ((kq == k) & (q < tid))) ? s.tiles[q] : 0;
    }
    const int n = s.tiles[tid];
    for (int t = 0; t < n && start + t < kStreamMaxRanked; ++t) {
      const int qt = n - 1 - t;
      s.tab[start + t] = make_int2(tid | (qt << 8),
                                   stream_tile_keys(s.rows[tid], s.ctx[tid], qt, cap));
    }
  }
  int R = 0;
  for (int q = 0; q < a.B; ++q) R += s.tiles[q];
  __syncthreads();
  return min(R, kStreamMaxRanked) * (a.H / kXcds);   // the host bounds R by the same limit
}

// Item k of this XCD's queue: {b, h, qt, key tiles}, or none.
__device__ inline int4 stream_item(const PrefillArgs& a, const StreamScratch& s, int k, int K) {
  if (k >= K) return make_int4(-1, 0, 0, 0);
  const int nh = a.H / kXcds;
  const int2 e = s.tab[k / nh];
  return make_int4(e.x & 0xff, (int)(blockIdx.x % kXcds) + kXcds * (k % nh), e.x >> 8, e.y);
}

// The producer's position in the tile stream (wave-uniform, the same in every
// wave): key tile `kt` of the workgroup's item `it`.  Items below `allowed`
// are published; the stream enters no other.  Where it cannot go on it holds
// on its tile (the loads that run ahead then read that tile again) and, when
// the reason was an unpublished item, records it in `stall_at`.
struct StreamCursor {
  int it, kt, nkt, row, head;
  int allowed, stall_at;

  template <int kHeadBytes>
  __device__ inline void enter(const PrefillArgs& a, int j, const int4& e) {
    it = j;
    kt = 0;
    nkt = e.w;
    row = e.x * a.MB;
    head = e.y / (a.H / a.Hkv) * kHeadBytes;
  }
  // first published item >= j that walks keys; false when there is none yet
  template <int kHeadBytes>
  __device__ inline bool seek(const PrefillArgs& a, const StreamScratch& s, int j) {
    for (int nx = j;; ++nx) {
      if (nx >= allowed) {
        stall_at = min(stall_at, nx);
        return false;
      }
      const int4 e = s.ring[nx % kStreamRing];
      const int b = __builtin_amdgcn_readfirstlane(e.x);
      if (b < 0) return false;
      const int n = __builtin_amdgcn_readfirstlane(e.w);
      if (n > 0) {
        enter<kHeadBytes>(a, nx, make_int4(b, __builtin_amdgcn_readfirstlane(e.y), 0, n));
        return true;
      }
    }
  }
  template <int kHeadBytes>
  __device__ inline void advance(const PrefillArgs& a, const StreamScratch& s) {
    if (kt + 1 < nkt) {
      ++kt;
      return;
    }
    if (stall_at != kStreamNone) return;
    seek<kHeadBytes>(a, s, it + 1);   // on failure the cursor is unchanged
  }
};

// PipeProducer's moves with the head of each tile taken from the stream: the
// head's byte offset goes into the page base (the buffer resource then covers
// the rest of the page), the lanes' offsets stay those of head 0.
template <typename T, int D>
struct StreamProducer {
  static constexpr int kVD = D / 64;
  static constexpr int kKC = D / 8;
  static constexpr int kKU = kKC / 8;
  static constexpr int kKeysPerKU = 64 / kKC;

  uint32_t v[8];
  uint4 k[kKU];
  int ids;            // lanes 0..3 (mod 4): block ids of the 4 pages of one tile
  int ids_head;       // head bytes of the tile whose ids are in `ids`
  const char* kpage;  // K page + head of the tile whose V load_v issued
  int k_head;
  float chk;

  int64_t page_bytes;
  uint32_t v_off, k_off, tok_bytes;
  int wave, lane;

  __device__ inline void init(const PrefillArgs& a, int wave_) {
    wave = wave_;
    lane = threadIdx.x & 63;
    chk = 0.0f;
    tok_bytes = (uint32_t)(a.Hkv * D * (int)sizeof(T));
    page_bytes = (int64_t)tok_bytes * 16;
    const uint32_t tok0 = (uint32_t)(8 * (wave & 1));
    v_off = tok0 * tok_bytes + (uint32_t)(kVD * lane * (int)sizeof(T));
    k_off = (tok0 + (uint32_t)(lane / kKC)) * tok_bytes +
            (uint32_t)(8 * (lane % kKC) * (int)sizeof(T));
  }

  __device__ inline void fetch_ids(const PrefillArgs& a, const StreamCursor& c) {
    ids = a.bt[(int64_t)c.row + min(c.kt * 4 + (lane & 3), a.MB - 1)];
    ids_head = c.head;
  }

  __device__ inline const char* page(const PrefillArgs& a, const void* base) const {
    const int id = __builtin_amdgcn_readlane(ids, wave >> 1);
    return reinterpret_cast<const char*>(base) + safe_block(id, a.NB) * page_bytes + ids_head;
  }

  __device__ inline __amdgpu_buffer_rsrc_t rsrc(const char* p, int head) const {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(p), (short)0,
                                             (int)(page_bytes - head), kBufferRsrcWord3);
  }

  __device__ inline void load_v(const PrefillArgs& a) {
    kpage = page(a, a.k);
    k_head = ids_head;
    const __amdgpu_buffer_rsrc_t r = rsrc(page(a, a.v), ids_head);
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if constexpr (kVD == 2) {
        v[u] = __builtin_amdgcn_raw_buffer_load_b32(r, (int)v_off, (int)(u * tok_bytes), 0);
      } else {
        v[u] = __builtin_amdgcn_raw_buffer_load_b16(r, (int)v_off, (int)(u * tok_bytes), 0);
      }
    }
  }

  __device__ inline void load_k() {
    const __amdgpu_buffer_rsrc_t r = rsrc(kpage, k_head);
#pragma unroll
    for (int u = 0; u < kKU; ++u) {
      typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
      const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(
          r, (int)k_off, (int)(u * kKeysPerKU * tok_bytes), 0);
      k[u] = make_uint4(x[0], x[1], x[2], x[3]);
    }
  }

  __device__ inline uint32_t vpair(int u, int e) const {
    if constexpr (std::is_same_v<T, Bf16>) {
      const float x0 = __uint_as_float(e ? (v[u] & 0xffff0000u) : (v[u] << 16));
      const float x1 = __uint_as_float(e ? (v[u + 1] & 0xffff0000u) : (v[u + 1] << 16));
      return pack_f16(x0, x1);
    } else {
      return e ? __builtin_amdgcn_perm(v[u + 1], v[u], 0x07060302u)
               : __builtin_amdgcn_perm(v[u + 1], v[u], 0x05040100u);
    }
  }

  __device__ inline void store_v(PipeTile<D>& t) const {
#pragma unroll
    for (int e = 0; e < kVD; ++e) {
      const int d = kVD * lane + e;
      const uint4 w = make_uint4(vpair(0, e), vpair(2, e), vpair(4, e), vpair(6, e));
      *reinterpret_cast<uint4*>(&t.vt[d][8 * (wave ^ vt_swz<D>(d))]) = w;
    }
  }

  __device__ inline void store_k(PipeTile<D>& t) {
#pragma unroll
    for (int u = 0; u < kKU; ++u) {
      const int key = 8 * wave + kKeysPerKU * u + lane / kKC;
      const int row = (key & ~31) | swap_bits23(key & 31);
      const uint4 h = to_f16x8<T>(k[u]);
      if constexpr (std::is_same_v<T, Bf16>) {
        chk = f16_check(h, chk);
        asm volatile("" : "+v"(chk));
      }
      *reinterpret_cast<uint4*>(&t.k[row][8 * (lane % kKC)]) = h;
    }
  }
};

// This lane's index, computed where it is used: the compiler cannot hoist
// it, so values derived from it for one query tile are not kept in registers
// across the whole item loop.
__device__ inline int opaque_lane() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

__global__ void prefill_stream_reset_kernel(int* counters) {
  if (threadIdx.x < kXcds) counters[threadIdx.x] = 0;
}

template <typename T, int D>
__global__ __launch_bounds__(kPipeWaves * 64) __attribute__((amdgpu_waves_per_eu(2)))
void prefill_stream_kernel(PrefillArgs a) {
  constexpr int kBM = kPipeWaves * kRowsPerWave;
  constexpr int kDC16 = D / 16;
  constexpr int kDB = D / 32;
  constexpr int kHeadBytes = D * (int)sizeof(T);
  using Prod = StreamProducer<T, D>;
  __shared__ PipeTile<D> lds[kPipeBufs];
  __shared__ StreamScratch ss;
  __shared__ int fail[3];   // per item, rotating: some fp16 operand was inf or NaN

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane & 31;
  const int hh = lane >> 5;
  const int cap = a.MB * 16;
  int* counter = a.counters + blockIdx.x % kXcds;
  if (tid < 3) fail[tid] = 0;   // ordered by the barriers below

  const int K = stream_rank(a, ss);
  if (tid == 0) ss.ring[0] = stream_item(a, ss, atomicAdd(counter, 1), K);
  __syncthreads();
  if (__builtin_amdgcn_readfirstlane(ss.ring[0].x) < 0) return;

  Prod pr;
  pr.init(a, wave);
  StreamCursor cur;
  cur.allowed = 1;
  cur.stall_at = kStreamNone;
  // The stream from item j on, at stream position g: tiles g and g + 1 into
  // their buffers, tile g + 2 in flight, the ids of tile g + 3 fetched.
  auto prologue = [&](int jj, int g) __attribute__((always_inline)) {
    cur.stall_at = kStreamNone;
    if (cur.seek<kHeadBytes>(a, ss, jj)) {
      Prod pr1 = pr;
      pr1.chk = 0.0f;
      pr.fetch_ids(a, cur);
      cur.advance<kHeadBytes>(a, ss);
      pr1.fetch_ids(a, cur);
      cur.advance<kHeadBytes>(a, ss);
      pr.load_v(a);
      pr.load_k();
      pr1.load_v(a);
      pr1.load_k();
      pr.fetch_ids(a, cur);
      cur.advance<kHeadBytes>(a, ss);
      pr.store_v(lds[g % kPipeBufs]);
      pr.store_k(lds[g % kPipeBufs]);
      pr1.store_v(lds[(g + 1) % kPipeBufs]);
      pr1.store_k(lds[(g + 1) % kPipeBufs]);
      pr.chk += pr1.chk;
      pr.load_v(a);
      pr.fetch_ids(a, cur);
      cur.advance<kHeadBytes>(a, ss);
      pr.load_k();
    }
    __syncthreads();
  };

  float4 qx[2 * kDC16];   // this item's fp32 Q rows in flight

  // Q rows of item e: this lane's row, or the tile's last row past its end
  auto load_q = [&](const int4& e) __attribute__((always_inline)) {
    const int ln = opaque_lane();
    const int S_b = __builtin_amdgcn_readfirstlane(ss.rows[e.x]);
    const int row0 = __builtin_amdgcn_readfirstlane(ss.row0[e.x]);
    const int i_row = e.z * kBM + wave * kRowsPerWave + (ln & 31);
    const float* qp = a.q + ((int64_t)(row0 + min(i_row, S_b - 1)) * a.H + e.y) * D + 8 * (ln >> 5);
#pragma unroll
    for (int c = 0; c < kDC16; ++c) {
      qx[2 * c] = *reinterpret_cast<const float4*>(qp + 16 * c);
      qx[2 * c + 1] = *reinterpret_cast<const float4*>(qp + 16 * c + 4);
    }
  };

  prologue(0, 0);

  // Each iteration: the atomic that takes the next item and this item's Q
  // loads, the next item published, this item, its output stores.
  // (Variants that kept the Q rows or the output rows live around the loop's
  // back edge, to overlap the Q round trip with the stores, made the
  // allocator spill heavily.)
  int g = 0;   // stream position of the next tile to consume
  int slow_from = -1;
  for (int jj = 0;; ++jj) {
    const int4 item = ss.ring[jj % kStreamRing];
    const int b = __builtin_amdgcn_readfirstlane(item.x);
    const int h = __builtin_amdgcn_readfirstlane(item.y);
    const int qt = __builtin_amdgcn_readfirstlane(item.z);
    if (b < 0) break;
    load_q(make_int4(b, h, qt, 0));
    const int n_kt = __builtin_amdgcn_readfirstlane(item.w);
    const int row0 = __builtin_amdgcn_readfirstlane(ss.row0[b]);
    const int S_b = __builtin_amdgcn_readfirstlane(ss.rows[b]);
    const int ctx_b = __builtin_amdgcn_readfirstlane(ss.ctx[b]);
    const int base_pos = ctx_b - S_b;
    const int w_first = qt * kBM + wave * kRowsPerWave;
    const int ln = opaque_lane();
    const int i_row = w_first + (ln & 31);
    const bool row_ok = i_row < S_b;

    // Q^T fragments
    half8 qf[kDC16];
    float16x o[kDB];
    float l;
    float qchk = 0.0f;
    {
      const float sc = row_ok ? a.qscale : 0.0f;
#pragma unroll
      for (int c = 0; c < kDC16; ++c) {
        const float4 x0 = qx[2 * c], x1 = qx[2 * c + 1];
        const uint4 w = make_uint4(pack_f16(x0.x * sc, x0.y * sc), pack_f16(x0.z * sc, x0.w * sc),
                                   pack_f16(x1.x * sc, x1.y * sc), pack_f16(x1.z * sc, x1.w * sc));
        qchk = f16_check(w, qchk);
        qf[c] = __builtin_bit_cast(half8, w);
      }
    }
    if (jj == cur.stall_at) prologue(jj, g);   // the stream broke before this item

    const int lim = (row_ok ? min(base_pos + i_row, cap - 1) : -1) - 8 * (ln >> 5);
    const int w_lim_min = min(base_pos + w_first, cap - 1);
    const int w_lim_max = w_first < S_b ? min(base_pos + min(w_first + kRowsPerWave, S_b) - 1,
                                              cap - 1)
                                        : -1;
    const int nb_w = w_lim_max < 0 ? 0 : min(2 * n_kt, w_lim_max / 32 + 1);
    const int mask_x = w_lim_min - 31;
    const int mask_from = mask_x < 0 ? 0 : mask_x / 32 + 1;
    const int t_w = (nb_w + 1) / 2;
    // The period that takes the next item from the queue: the latest one
    // whose publication (the period after) still lets the stream enter the
    // next item without a stop (it needs it at the end of period n_kt - 5),
    // ~7 key tiles before this item ends.  The queue so hands out items
    // close to the time a workgroup needs one, as a longest-first deal would.
    const int fetch_t = max(0, n_kt - 7);
    int next_k;   // thread 0 only

    float16x bias;
    float16x s_cur, s_nxt;
    half8 kf[kDC16];
    half8 vf[2][kDB];
    half8 p[2];
    float m;
    auto read_k = [&](const PipeTile<D>& t, int kb) __attribute__((always_inline)) {
  #pragma unroll
      for (int c = 0; c < kDC16; ++c)
        kf[c] = *reinterpret_cast<const half8*>(&t.k[kb * 32 + j][16 * c + 8 * hh]);
    };
    // lim is the row's last key minus 8 hh (the lane half's key offset), so
    // that one register carries both
    auto mask = [&](float16x& s, int blk) __attribute__((always_inline)) {
      const int key0 = 32 * blk;
  #pragma unroll
      for (int r = 0; r < 16; ++r)
        if (key0 + 16 * (r >> 3) + (r & 7) > lim) s[r] = -INFINITY;
    };
    const int vsw = hh ^ vt_swz<D>(j);
    auto read_v1 = [&](const PipeTile<D>& t, int kb, int i) __attribute__((always_inline)) {
      vf[i / kDB][i % kDB] = *reinterpret_cast<const half8*>(
          &t.vt[32 * (i % kDB) + j][8 * ((4 * kb + 2 * (i / kDB)) ^ vsw)]);
    };
    auto prob2 = [&](const float16x& s, int i, uint32_t* w, float lb) __attribute__((always_inline)) {
      w[i] = pack_f16(fast_exp2(s[2 * i]), fast_exp2(s[2 * i + 1]));
      return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2x, w[i]),
                                    (half2x){(_Float16)1.0f, (_Float16)1.0f}, lb, false);
    };
    auto probs = [&](const float16x& s) __attribute__((always_inline)) {
      uint32_t w[8];
      float lb = 0.0f;
  #pragma unroll
      for (int i = 0; i < 8; ++i) lb = prob2(s, i, w, lb);
      p[0] = __builtin_bit_cast(half8, make_uint4(w[0], w[1], w[2], w[3]));
      p[1] = __builtin_bit_cast(half8, make_uint4(w[4], w[5], w[6], w[7]));
      return lb;
    };
    auto phase_qs = [&](auto qk_tag, float16x& s_out, const float16x& sm, const PipeTile<D>& tv,
                        int vkb) __attribute__((always_inline)) {
      constexpr bool kQk = decltype(qk_tag)::value;
      uint32_t w[8];
      float lb = 0.0f;
  #pragma unroll
      for (int i = 0; i < 8; ++i) {
        if constexpr (kQk) {
          if (i < kDC16)
            s_out = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[i], qf[i], i == 0 ? bias : s_out, 0,
                                                           0, 0);
        }
        if (i < 2 * kDB) read_v1(tv, vkb, i);
        lb = prob2(sm, i, w, lb);
      }
      p[0] = __builtin_bit_cast(half8, make_uint4(w[0], w[1], w[2], w[3]));
      p[1] = __builtin_bit_cast(half8, make_uint4(w[4], w[5], w[6], w[7]));
      if constexpr (kQk) {
  #pragma unroll
        for (int i = 0; i < 8; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
        }
      }
      return lb;
    };
    auto settle = [&](float lb, float16x& s, float16x& nxt, bool has_nxt) __attribute__((always_inline)) {
      if (__builtin_amdgcn_ballot_w64(!(lb <= kPMax)) != 0) {
        float mx = s[0];
  #pragma unroll
        for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s[r]);
        mx = max_halves(mx);
        const float dlt = mx > 0.0f ? mx : 0.0f;
        const float corr = fast_exp2(-dlt);
        m += dlt;
        l *= corr;
  #pragma unroll
        for (int d = 0; d < kDB; ++d)
  #pragma unroll
          for (int r = 0; r < 16; ++r) o[d][r] *= corr;
  #pragma unroll
        for (int r = 0; r < 16; ++r) {
          bias[r] -= dlt;
          s[r] -= dlt;
        }
        if (has_nxt) {
  #pragma unroll
          for (int r = 0; r < 16; ++r) nxt[r] -= dlt;
        }
        lb = probs(s);
      }
      l += lb;
    };
    auto phase_pv = [&](auto read_tag, const PipeTile<D>& tk, int kkb, auto&& prod) __attribute__((always_inline)) {
      constexpr bool kRead = decltype(read_tag)::value;
  #pragma unroll
      for (int i = 0; i < 2 * kDB; ++i) {
        o[i % kDB] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[i / kDB][i % kDB], p[i / kDB],
                                                            o[i % kDB], 0, 0, 0);
        if constexpr (kRead) {
          if (i < kDC16)
            kf[i] = *reinterpret_cast<const half8*>(&tk.k[kkb * 32 + j][16 * i + 8 * hh]);
        }
      }
      prod();
      if constexpr (kRead) {
  #pragma unroll
        for (int i = 0; i < 2 * kDB; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 1);
          __builtin_amdgcn_sched_group_barrier(0x002, 3, 1);
        }
      }
    };
    using Yes = std::true_type;
    using No = std::false_type;
    // the producer's share of a period: V of the tile two ahead into LDS, the
    // next tile's V loads, the ids of the tile after it; then K likewise
    // The next item is taken from the queue in period fetch_t (thread 0's
    // atomic, just before the period's V loads) and published in the next
    // period, after store_v has waited for those loads and with them for the
    // atomic.
    auto prod_v = [&](PipeTile<D>& tw, int t) __attribute__((always_inline)) {
      return [&pr, &tw, &a, &cur, &next_k, counter, K, t, fetch_t, jj, tid]() {
        pr.store_v(tw);
        if (t == fetch_t + 1 && tid == 0)
          ss.ring[(jj + 1) % kStreamRing] = stream_item(a, ss, next_k, K);
        if (t == fetch_t && tid == 0) next_k = atomicAdd(counter, 1);
        pr.load_v(a);
        pr.fetch_ids(a, cur);
      };
    };
    auto prod_k = [&](PipeTile<D>& tw) __attribute__((always_inline)) {
      return [&pr, &tw]() {
        pr.store_k(tw);
        pr.load_k();
      };
    };
    // end of a period: the cursor moves to the tile whose ids the next period
    // fetches (its LDS reads are covered by the barrier's wait)
    auto end_period = [&](int t) __attribute__((always_inline)) {
      cur.advance<kHeadBytes>(a, ss);
      __syncthreads();
      if (t == fetch_t + 1) cur.allowed = jj + 2;
    };

#pragma unroll
    for (int d = 0; d < kDB; ++d)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[d][r] = 0.0f;
    m = kNegBig;
    l = 0.0f;
    if (t_w > 0) {
      const PipeTile<D>& t0 = lds[g % kPipeBufs];
      read_k(t0, 0);
      float16x zero;
#pragma unroll
      for (int r = 0; r < 16; ++r) zero[r] = 0.0f;
      s_cur = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[0], qf[0], zero, 0, 0, 0);
#pragma unroll
      for (int c = 1; c < kDC16; ++c)
        s_cur = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[c], qf[c], s_cur, 0, 0, 0);
      if (mask_from == 0) mask(s_cur, 0);
      float mx = s_cur[0];
#pragma unroll
      for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s_cur[r]);
      m = fmaxf(kNegBig, max_halves(mx));
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        bias[r] = -m;
        s_cur[r] -= m;
      }
      read_k(t0, 1);
    }

    // the item's periods: stream tile g + t consumed, g + t + 2 written,
    // g + t + 3 loaded, ids of g + t + 4 fetched
    int t = 0;
    for (; t + 1 < t_w; ++t) {
      const PipeTile<D>& tc = lds[(g + t) % kPipeBufs];
      const PipeTile<D>& tn = lds[(g + t + 1) % kPipeBufs];
      PipeTile<D>& tw = lds[(g + t + 2) % kPipeBufs];
      if (2 * t >= mask_from) mask(s_cur, 2 * t);
      float lb = phase_qs(Yes{}, s_nxt, s_cur, tc, 0);
      settle(lb, s_cur, s_nxt, true);
      phase_pv(Yes{}, tn, 0, prod_v(tw, t));
      if (2 * t + 1 >= mask_from) mask(s_nxt, 2 * t + 1);
      lb = phase_qs(Yes{}, s_cur, s_nxt, tc, 1);
      settle(lb, s_nxt, s_cur, true);
      phase_pv(Yes{}, tn, 1, prod_k(tw));
      end_period(t);
    }
    if (t < t_w) {
      const PipeTile<D>& tc = lds[(g + t) % kPipeBufs];
      PipeTile<D>& tw = lds[(g + t + 2) % kPipeBufs];
      const bool second = 2 * t + 1 < nb_w;
      if (2 * t >= mask_from) mask(s_cur, 2 * t);
      if (second) {
        s_nxt = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[0], qf[0], bias, 0, 0, 0);
#pragma unroll
        for (int c = 1; c < kDC16; ++c)
          s_nxt = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[c], qf[c], s_nxt, 0, 0, 0);
      }
      float lb = phase_qs(No{}, s_nxt, s_cur, tc, 0);
      settle(lb, s_cur, s_nxt, second);
      phase_pv(No{}, tc, 0, prod_v(tw, t));
      if (second) {
        if (2 * t + 1 >= mask_from) mask(s_nxt, 2 * t + 1);
        lb = phase_qs(No{}, s_cur, s_nxt, tc, 1);
        settle(lb, s_nxt, s_cur, false);
        phase_pv(No{}, tc, 1, prod_k(tw));
      } else {
        prod_k(tw)();
      }
      end_period(t);
      ++t;
    }
    for (; t < n_kt; ++t) {
      PipeTile<D>& tw = lds[(g + t + 2) % kPipeBufs];
      prod_v(tw, t)();
      prod_k(tw)();
      end_period(t);
    }
    g += n_kt;
    if (fetch_t + 1 >= n_kt) {
      // an item of at most one period: its successor is taken here (the
      // stream will have stopped short of it and restarts there)
      if (tid == 0) {
        if (n_kt == 0) next_k = atomicAdd(counter, 1);
        ss.ring[(jj + 1) % kStreamRing] = stream_item(a, ss, next_k, K);
      }
      __syncthreads();
      cur.allowed = jj + 2;
    }

    // ---- range check (the rows are stored at the top of the next
    // iteration).  The conversion check covers every tile this wave converted
    // so far, which includes this item's; a failure therefore also sends the
    // items after it to the fp32 path.
    bool my_fail = f16_check_failed(pr.chk + qchk);
    {
      float oc = 0.0f;
#pragma unroll
      for (int d = 0; d < kDB; ++d)
#pragma unroll
        for (int r = 0; r < 16; ++r) oc += o[d][r] * 0.0f;
      my_fail = my_fail || !(oc == 0.0f);
    }
    // fail[jj % 3]: set by any wave of item jj, read after the barrier,
    // cleared by thread 0 two items later (every read of it is then past a
    // barrier that thread 0 has also passed)
    if (my_fail) fail[jj % 3] = 1;
    if (tid == 0) fail[(jj + 1) % 3] = 0;
    __syncthreads();
    if (fail[jj % 3] != 0) {
      slow_from = jj;   // this item and every later one: fp32, below
      break;
    }
    {   // the normalised rows
      const float lsum = sum_halves(l);
      const int le = opaque_lane();
      const int i_out = w_first + (le & 31);
      if (i_out < S_b) {
        const float inv = lsum > 0.0f ? 1.0f / lsum : 0.0f;
        float* op = a.out + ((int64_t)(row0 + i_out) * a.H + h) * D + 4 * (le >> 5);
#pragma unroll
        for (int d = 0; d < kDB; ++d)
#pragma unroll
          for (int gq = 0; gq < 4; ++gq)
            *reinterpret_cast<float4*>(op + d * 32 + 8 * gq) =
                make_float4(o[d][4 * gq] * inv, o[d][4 * gq + 1] * inv, o[d][4 * gq + 2] * inv,
                            o[d][4 * gq + 3] * inv);
      }
    }
  }
  // the loads that ran ahead of the last period are not consumed; let them
  // land before the waves end
  __builtin_amdgcn_s_waitcnt(0);
  if (slow_from < 0) return;

  // Some fp16 operand of item slow_from was out of range.  The conversion
  // check accumulates over all tiles a wave converted, so the matrix-core
  // loop is left for good: this item and the workgroup's remaining ones are
  // computed with fp32 arithmetic, one at a time (the next item is already
  // published; each later one is taken from the queue here).
  for (int jj = slow_from;; ++jj) {
    const int4 item = ss.ring[jj % kStreamRing];
    const int b = __builtin_amdgcn_readfirstlane(item.x);
    if (b < 0) break;
    const int h = __builtin_amdgcn_readfirstlane(item.y);
    const int qt = __builtin_amdgcn_readfirstlane(item.z);
    const int n_kt = __builtin_amdgcn_readfirstlane(item.w);
    const int row0 = __builtin_amdgcn_readfirstlane(ss.row0[b]);
    const int S_b = __builtin_amdgcn_readfirstlane(ss.rows[b]);
    const int ctx_b = __builtin_amdgcn_readfirstlane(ss.ctx[b]);
    prefill_rows_fp32<T, D>(a, b, h, h / (a.H / a.Hkv), row0, S_b, ctx_b - S_b, cap,
                            qt * kBM + wave * kRowsPerWave, 0, n_kt * kBN, 0);
    const bool more = __builtin_amdgcn_readfirstlane(ss.ring[(jj + 1) % kStreamRing].x) >= 0;
    if (tid == 0 && more)
      ss.ring[(jj + 2) % kStreamRing] = stream_item(a, ss, atomicAdd(counter, 1), K);
    __syncthreads();
  }
}

// Merge of a split prefill: for row i of sequence b and head h,
//   out = sum_p w_p O_p / sum_p w_p l_p,  w_p = exp2(m_p - max_p m_p)
// over the n_split parts (a part without keys for the row has m_p = -3e38 and
// weight 0; a row without keys gets zeros, as in the unsplit kernel).  One
// thread per 4 dims; the partial arrays are read once, out written once.
template <int D>
__global__ __launch_bounds__(256) void prefill_merge_kernel(PrefillArgs a) {
  constexpr int kC = D / 4;
  const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t n_pairs = (int64_t)a.B * a.rows_cap * a.H;   // pairs per part
  const int64_t pair = g / kC;
  if (pair >= n_pairs) return;
  const int c = (int)(g - pair * kC);
  const int h = (int)(pair % a.H);
  const int64_t bi = pair / a.H;
  const int i = (int)(bi % a.rows_cap);
  const int b = (int)(bi / a.rows_cap);
  if (i >= seq_rows(a, b)) return;
  const int64_t row0 = a.cu_q ? a.cu_q[b] : (int64_t)b * a.S;
  float2 ml[kMaxSplit];
  float mx = kNegBig;
#pragma unroll
  for (int p = 0; p < kMaxSplit; ++p) {
    if (p < a.n_split) {
      ml[p] = a.part_ml[p * n_pairs + pair];
      mx = fmaxf(mx, ml[p].x);
    }
  }
  float lsum = 0.0f;
  float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
  for (int p = 0; p < kMaxSplit; ++p) {
    if (p < a.n_split) {
      const float w = fast_exp2(ml[p].x - mx);
      const float4 o = reinterpret_cast<const float4*>(a.part_o)[(p * n_pairs + pair) * kC + c];
      lsum += w * ml[p].y;
      acc.x += w * o.x;
      acc.y += w * o.y;
      acc.z += w * o.z;
      acc.w += w * o.w;
    }
  }
  const float inv = lsum > 0.0f ? 1.0f / lsum : 0.0f;
  reinterpret_cast<float4*>(a.out)[((row0 + i) * a.H + h) * kC + c] =
      make_float4(acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv);
}

// Grid plan for one head dim and width: query tiles of W * 32 rows, longest
// first when the batch has at most kMaxRanked sequences; a split multiplies
// each ranked tile's slots by n_split (parts next to each other).
template <typename T, int D, int W>
int launch_typed(PrefillArgs a, int max_rows_per_seq, int stream_ns, hipStream_t stream) {
  constexpr int kBM = Shape<D, W>::kBM;
  a.n_qt = (max_rows_per_seq + kBM - 1) / kBM;
  const int64_t pairs = (int64_t)a.B * a.H;
  a.ranked = a.B <= kMaxRanked;
  if (a.n_split > 1 && !a.ranked) return fail(HS_EUNSUPPORTED, "split prefill needs ranked tiles");
  const int64_t slots = a.ranked ? sat_mul(a.B, a.n_qt, ceil_div(a.H, kXcds), a.n_split)
                                 : sat_mul(ceil_div(pairs, kXcds), a.n_qt);
  if (sat_mul(slots, kXcds) > 0x7fffffffLL) return fail(HS_EUNSUPPORTED, "prefill grid too large");
  a.slots_per_xcd = (int)slots;
  const dim3 grid((unsigned)(kXcds * a.slots_per_xcd)), block(Shape<D, W>::kThreads);
  // 8-wave workgroups at head dim 64 and 128 take the pipelined kernel; the
  // 4-wave shape (small grids without a workspace, head dim 32) the other
  if constexpr (W == kPipeWaves && D >= 64) {
    if (stream_ns > 0) {   // its queue counters were zeroed by the caller
      hipLaunchKernelGGL((prefill_stream_kernel<T, D>), dim3((unsigned)(kXcds * stream_ns)), block,
                         0, stream, a);
    } else {
      hipLaunchKernelGGL((prefill_pipe_kernel<T, D>), grid, block, 0, stream, a);
    }
  } else {
    hipLaunchKernelGGL((prefill_mfma_kernel<T, D, W>), grid, block, 0, stream, a);
  }
  if (a.n_split > 1) {
    // the workspace of B * rows_cap * H * (D + 2) floats per part exists, so
    // this product fits; the grid must still fit one launch
    const int64_t groups = ceil_div(sat_mul(a.B, a.rows_cap, a.H, D / 4), 256);
    if (groups > 0x7fffffffLL) return fail(HS_EUNSUPPORTED, "prefill merge grid too large");
    hipLaunchKernelGGL((prefill_merge_kernel<D>), dim3((unsigned)groups), dim3(256), 0, stream, a);
  }
  return HS_OK;
}

template <typename T>
int launch_dim(const PrefillArgs& a, int D, bool wide, int max_rows_per_seq, int stream_ns,
               hipStream_t stream) {
  switch (D) {
    case 32: return launch_typed<T, 32, 4>(a, max_rows_per_seq, 0, stream);
    case 64:
      return wide ? launch_typed<T, 64, 8>(a, max_rows_per_seq, stream_ns, stream)
                  : launch_typed<T, 64, 4>(a, max_rows_per_seq, 0, stream);
    case 128:
      return wide ? launch_typed<T, 128, 8>(a, max_rows_per_seq, stream_ns, stream)
                  : launch_typed<T, 128, 4>(a, max_rows_per_seq, 0, stream);
    default: return fail(HS_EUNSUPPORTED, "unsupported head_dim for the MFMA path: " +
                                              std::to_string(D));
  }
}

}  // namespace

// Launch shape of the MFMA prefill for B sequences of up to max_rows query
// rows on a device with `cus` CUs.  Full-width workgroups (256 rows; 128 at
// head dim 32) when their query tiles cover every CU.  Otherwise, with a
// workspace, each tile's key range is split over floor(cus / tiles) <= 4
// workgroups (a 1024-row chunk of 32 heads: 128 tiles, 2 parts); without one,
// 128-row workgroups, which run one wave per SIMD but reach twice as many CUs.
//
// With a workspace, full-width grids of at least two query tiles per CU run
// the persistent kernel instead (stream_ns workgroups per XCD, one per CU):
// it needs whole XCDs of heads (H % 8 == 0), the ranked dispatch and at most
// kStreamMaxRanked ranked tiles.  HETEROSERVE_PREFILL_GRID=1 keeps the grid
// kernel (for comparisons).
PrefillPlan plan_prefill_mfma(int B, int max_rows, int H, int D, int cus, bool can_split) {
  const int bm = D >= 64 ? 256 : 128;
  const int64_t tiles = sat_mul(B, ceil_div(max_rows, bm), H);
  PrefillPlan p{true, 1, 0};
  if (tiles >= cus) {
    const char* env = std::getenv("HETEROSERVE_PREFILL_GRID");
    const bool grid_only = env && env[0] == '1';
    const int64_t ranked = sat_mul(B, ceil_div(max_rows, bm));
    if (can_split && !grid_only && D >= 64 && B <= kMaxRanked && H % kXcds == 0 &&
        ranked <= kStreamMaxRanked && tiles >= 2 * (int64_t)cus && cus >= kXcds)
      p.stream_ns = cus / kXcds;
    return p;
  }
  const int64_t splits = std::min<int64_t>(kMaxSplit, tiles > 0 ? cus / tiles : 1);
  if (can_split && splits >= 2 && B <= kMaxRanked) p.n_split = (int)splits;
  else p.wide = false;
  return p;
}

// INT64_MAX when the sizes do not fit
int64_t prefill_workspace_bytes(const PrefillPlan& p, int B, int max_rows, int H, int D) {
  if (p.stream_ns > 0) return (int64_t)kStreamWorkspaceBytes;
  if (p.n_split < 2) return 0;
  const int64_t pairs = sat_mul(p.n_split, B, max_rows, H);
  const int64_t o_bytes = sat_add(sat_mul(pairs, D, (int64_t)sizeof(float)), 255) / 256 * 256;
  return sat_add(o_bytes, sat_mul(pairs, (int64_t)sizeof(float2)));
}

int launch_prefill_mfma(const float* q, const int32_t* cu_q, int S, int max_rows_per_seq,
                        const void* k, const void* v, int kv_dtype, int NB, const int32_t* bt,
                        const int32_t* ctx, float* out, int B, int H, int Hkv, int D, int BS,
                        int MB, float scale, void* workspace, size_t workspace_bytes,
                        hipStream_t stream) {
  (void)BS;  // validated to be 16 by the caller
  PrefillArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.bt = bt;
  a.ctx = ctx;
  a.cu_q = cu_q;
  a.out = out;
  a.S = S;
  a.B = B;
  a.H = H;
  a.Hkv = Hkv;
  a.MB = MB;
  a.NB = NB;
  a.qscale = scale * kLog2e;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(HS_EHIP, "hipGetDevice failed");
  const int cus = hs_device_cu_count(dev);
  if (cus <= 0) return fail(HS_EHIP, "could not read the device CU count");
  PrefillPlan plan = plan_prefill_mfma(B, max_rows_per_seq, H, D, cus, workspace != nullptr);
  a.n_split = plan.n_split;
  a.rows_cap = max_rows_per_seq;
  if (plan.stream_ns > 0) {
    if (workspace_bytes < kStreamWorkspaceBytes)
      return fail(HS_EWORKSPACE, "prefill workspace too small: " +
                                     std::to_string(kStreamWorkspaceBytes) + " bytes needed");
    if (sat_mul(B, MB) > 0x7fffffffLL) plan.stream_ns = 0;   // table rows as int: grid kernel
    a.counters = static_cast<int*>(workspace);
  }
  if (plan.n_split > 1) {
    const int64_t need_i = prefill_workspace_bytes(plan, B, max_rows_per_seq, H, D);
    if (need_i == INT64_MAX) return fail(HS_EUNSUPPORTED, "prefill split too large");
    const size_t need = (size_t)need_i;
    if (workspace_bytes < need)
      return fail(HS_EWORKSPACE, "prefill workspace too small: " + std::to_string(need) +
                                     " bytes needed");
    const size_t o_bytes = need - (size_t)plan.n_split * B * max_rows_per_seq * H * sizeof(float2);
    a.part_o = static_cast<float*>(workspace);
    a.part_ml = reinterpret_cast<float2*>(static_cast<char*>(workspace) + o_bytes);
  }
  // the persistent kernel's queue counters, zeroed before the launch (and
  // before the profiling bracket, which then times the kernel alone)
  if (plan.stream_ns > 0)
    hipLaunchKernelGGL(prefill_stream_reset_kernel, dim3(1), dim3(64), 0, stream, a.counters);
  profile_begin(stream);
  int rc;
  if (kv_dtype == HS_DTYPE_F16)
    rc = launch_dim<_Float16>(a, D, plan.wide, max_rows_per_seq, plan.stream_ns, stream);
  else
    rc = launch_dim<Bf16>(a, D, plan.wide, max_rows_per_seq, plan.stream_ns, stream);
  profile_end(stream);
  if (rc != HS_OK) return rc;
  return check_launch("MFMA prefill");
}

}  // namespace hs
