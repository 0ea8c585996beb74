// Shared pages (prefix caching) on gfx950 matrix cores, at fp32 accuracy.
//
// Reference: paged_attn_v2.py:75-157 (one query row per head, KV head
// h / (H / Hkv), online softmax) and paged_attn_v3.py:75-208 (partitions
// merged by log-sum-exp).  Sequences whose partition has the same block ids
// (a shared prefix) read the same K/V; share_plan_kernel finds such groups on
// the device, and shared_pages_kernel reads each grouped partition once for
// up to 32 query slots, (sequence, head) pairs of one KV head.  There is no
// reference counterpart (the reference reads every sequence's pages).
//
// The wave code (gqa_wave_run) walks a partition in blocks of 32 tokens:
//   S^T = K . Q^T   v_mfma_f32_32x32x16_{bf16,f16}, K rows (tokens) the A
//                   operand, Q^T (query slots) the B operand, held in
//                   registers;
//   O^T += V^T . P^T  the accumulator of the first product is already the B
//                   operand layout of the second (lane = slot), so P stays in
//                   registers; V^T is read from the token-major V rows with
//                   the transposing LDS read ds_read_b64_tr_b16.
// K and V are loaded with 16 lanes per 256-byte token row (loading K straight
// into the operand layout, one token per lane, touched 32 rows per load
// instruction and measured 4x slower per block) and staged, as stored,
// through the wave's own LDS.
// Token order: the accumulator gives lane half h the token rows 8g + 4h + m
// in registers 4g + m, while the P.V operand wants registers 0..7 of half h
// to be tokens 8h..8h+7 of a 16-token chunk; the two differ by a swap of bits
// 2 and 3 of the token index, so K's LDS row r holds token swap23(r).
//
// Numerics: split operands, as in the grouped-query decode
// (hs_decode_splitmm.hip).  K and V go to the MFMAs as stored; the query and
// the probabilities are fp32, each split into two terms of the cache's type
// (x = hi + lo, hi = T(x), lo = T(x - hi)), and every product is taken
// against both terms.  Products of 16-bit values are exact in the fp32
// accumulators, so scores and outputs match fp32 arithmetic to about 2^-16
// relative (bf16) or better (fp16), and no input value needs a fallback.  For
// fp16 caches each slot's scaled query is first multiplied by a power of two
// that puts its largest element in [2^14, 2^15) (the scores are multiplied
// back, exactly), and the probabilities are taken 2^7 larger: neither term
// overflows fp16.  Scores and the softmax state are fp32 in base 2
// (scale * log2(e) folded into q), and the running max is raised lazily
// (only when a block's max exceeds it by more than 8), as in the MFMA
// prefill.  The partition states (m, l, un-normalised acc) have the layout
// and meaning of the VALU kernel's, so the same merge kernel combines them.
//
// A partition's block ids (at most 64 pages) are fetched once by one vector
// load; every K/V load is unconditional (ids clamped to the table, pages past
// the end masked), so the compiler's wait counts stay exact, and the next
// block's loads are in flight while the current block is computed.
#include "hs_kernels.h"
#include "hs_mfma.h"

namespace hs {

namespace {

using namespace mfma;

constexpr int kGqaWaves = 4;        // waves per workgroup: consecutive head units
constexpr int kHeadsPerWave = 32;   // MFMA N dimension
constexpr int kBlock = 32;          // tokens per block
constexpr float kSlack = 8.0f;      // lazy-rescale slack, log2 units

constexpr int kKPad = 8;            // 16-bit words of padding per K row
// Padding per V row: a transposing read of V^T fragments has each 32-lane
// half of the wave read 4 rows x 64 bytes (two 16-lane groups, adjacent
// 16-dim column blocks); a row stride of 16 or 48 dwords mod 64 puts those 4
// rows on disjoint 16-bank ranges.
template <int D>
constexpr int v_pad() { return D == 32 ? 0 : 32; }

// One block of K and V as stored in the cache (16-bit words).
template <int D>
struct GqaWaveLds {
  uint16_t k[kBlock][D + kKPad];       // K, row r holds token swap23(r)
  uint16_t v[kBlock][D + v_pad<D>()];  // V, token-major
};

// The cache's element type and its 32x32x16 product.  kPBias: the
// probabilities go to the P.V product as 2^kPBias p (fp16: p <= 2^8 under the
// lazy rescale, so 2^15 at most); kScaleQ: each slot's query is brought to
// [2^14, 2^15) by a power of two before it is split.
template <typename T>
struct Split32;

template <>
struct Split32<Bf16> {
  typedef __bf16 E;
  typedef __bf16 E8 __attribute__((ext_vector_type(8)));
  static constexpr float kPBias = 0.0f;
  static constexpr bool kScaleQ = false;
  __device__ static float16x mm(E8 x, E8 y, float16x c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(x, y, c, 0, 0, 0);
  }
};

template <>
struct Split32<_Float16> {
  typedef _Float16 E;
  typedef half8 E8;
  static constexpr float kPBias = 7.0f;
  static constexpr bool kScaleQ = true;
  __device__ static float16x mm(E8 x, E8 y, float16x c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(x, y, c, 0, 0, 0);
  }
};

// V^T fragment (A operand of the 32x32x16 product) for dims 32 d .. 32 d + 31
// and tokens k0 + 8 hh .. k0 + 8 hh + 7: lane (j, hh) gets V[k0 + 8 hh + e][32 d + j],
// e = 0..7.  ds_read_b64_tr_b16 transposes inside each group of 16 lanes:
// lane i supplies 8 bytes of row i / 4 of a 4 x 16 block and receives column
// i (lane layout checked on gfx950); two reads give the eight tokens.
template <typename E8, int D>
__device__ inline E8 vt_fragment(const GqaWaveLds<D>& w, int d, int k0, int j, int hh) {
  typedef short short4x __attribute__((ext_vector_type(4)));
  typedef short short8x __attribute__((ext_vector_type(8)));
  typedef __attribute__((address_space(3))) short4x lds_short4x;
  const int i = j & 15;
  // C-style casts keep the LDS address arithmetic visible, so the constant
  // part of the address goes into the instructions' offset field
  const lds_short4x* lo_p =
      (const lds_short4x*)(&w.v[k0 + 8 * hh + (i >> 2)][32 * d + (j & 16) + 4 * (i & 3)]);
  const lds_short4x* hi_p =
      (const lds_short4x*)(&w.v[k0 + 8 * hh + 4 + (i >> 2)][32 * d + (j & 16) + 4 * (i & 3)]);
  const short4x lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(const_cast<lds_short4x*>(lo_p));
  const short4x hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(const_cast<lds_short4x*>(hi_p));
  const short8x x = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(E8, x);
}

// One wave's partition pass: up to 32 query slots that read the same KV
// head and the same pages, keys [lo, hi) of block table row `bt`.  Lane
// (j, hh) serves slot j: its query starts at element q_off of a.q, and it
// sees only keys below slot_hi (a member whose context ends inside the
// partition).  Slots j >= gc are padding (zero query, nothing written by the
// caller).  Returns
// the state in o / m / l in the ordinary units (m minus kPBias: o and l
// carry the 2^kPBias factor of the probabilities); l is this lane's share of
// the sum.
template <typename T, int D>
__device__ inline void gqa_wave_run(const RowAttnArgs& a, GqaWaveLds<D>& w, int lane, int kvh,
                                    int gc, const int32_t* bt, int lo, int hi, int slot_hi,
                                    int64_t q_off, float16x (&o)[D / 32], float& m, float& l) {
  using Ops = Split32<T>;
  using E = typename Ops::E;
  using E8 = typename Ops::E8;
  constexpr int kDC16 = D / 16;     // QK k-steps
  constexpr int kDB = D / 32;       // 32-dim output blocks
  constexpr int kDC = D / 8;        // 16-byte chunks per head row
  constexpr int kTpi = 64 / kDC;    // tokens per wave-wide load (kDC lanes per row)
  constexpr int kLi = kBlock / kTpi;   // loads per block, for K and for V
  static_assert(kTpi <= 16 && kLi >= 2, "head_dim");
  const int j = lane & 31;
  const int hh = lane >> 5;

  // Block ids of the partition's pages: lane i holds page lo / 16 + i
  // (clamped to the table); 1024 tokens are at most 64 pages.
  const int page0 = lo >> 4;
  const int idv = bt[min(page0 + lane, a.MB - 1)];

  // Q^T fragments, split: lane (j, hh) holds slot j, dims 16c + 8hh .. +7.
  // qexp: the power of two the query was multiplied by (kScaleQ), taken back
  // out of every score.
  E8 qh[kDC16], ql[kDC16];
  int qexp = 0;
  {
    const float sc = j < gc ? a.qscale : 0.0f;
    const float* qp = a.q + q_off + 8 * hh;
    float xq[kDC16][8];
    float amax = 0.0f;
#pragma unroll
    for (int c = 0; c < kDC16; ++c) {
      const float4 x0 = *reinterpret_cast<const float4*>(qp + 16 * c);
      const float4 x1 = *reinterpret_cast<const float4*>(qp + 16 * c + 4);
      const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        xq[c][e] = xs[e] * sc;
        amax = fmaxf(amax, fabsf(xq[c][e]));
      }
    }
    if constexpr (Ops::kScaleQ) {
      // the slot's largest |element| (its dims are split over lanes j and
      // j + 32); 2^qexp * amax lands in [2^14, 2^15), and a zero or
      // non-finite query keeps qexp = 0
      amax = max_halves(amax);
      if (amax > 0.0f && __builtin_isfinite(amax)) qexp = 15 - __builtin_amdgcn_frexp_expf(amax);
    }
#pragma unroll
    for (int c = 0; c < kDC16; ++c) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = Ops::kScaleQ ? ldexpf(xq[c][e], qexp) : xq[c][e];
        const E h = (E)x;
        qh[c][e] = h;
        ql[c][e] = (E)(x - (float)h);
      }
    }
    // Keep the split query in registers: without this anchor the compiler
    // may re-load and re-split it on every block to save registers.
#pragma unroll
    for (int c = 0; c < kDC16; ++c) {
      uint4& uh = reinterpret_cast<uint4&>(qh[c]);
      uint4& ul = reinterpret_cast<uint4&>(ql[c]);
      asm volatile("" : "+v"(uh.x), "+v"(uh.y), "+v"(uh.z), "+v"(uh.w));
      asm volatile("" : "+v"(ul.x), "+v"(ul.y), "+v"(ul.z), "+v"(ul.w));
    }
  }
  const int64_t tok = (int64_t)a.Hkv * D;           // elements between tokens of a page
  // Loads are coalesced: kDC neighbouring lanes read one token's head row.
  // Lane L holds chunk L % kDC of token slot L / kDC; load u of K and of V
  // covers tokens kTpi*u + slot, which stay inside one 16-token page
  // (wave-uniform block id).
  const int ck = lane % kDC;
  const int slot = lane / kDC;
  const uint16_t* kbase = reinterpret_cast<const uint16_t*>(a.k) + kvh * D + 8 * ck;
  const uint16_t* vbase = reinterpret_cast<const uint16_t*>(a.v) + kvh * D + 8 * ck;

  uint4 kr[kLi], vr[kLi];
  // Loads of the block whose first page is relative page pg.
  auto load_block = [&](int pg) {
    pg = min(pg, 62);                                  // a block past the end reads valid pages
    const int64_t b0 = safe_block(__builtin_amdgcn_readlane(idv, pg), a.NB) * 16;
    const int64_t b1 = safe_block(__builtin_amdgcn_readlane(idv, pg + 1), a.NB) * 16;
#pragma unroll
    for (int u = 0; u < kLi; ++u) {
      const int t = kTpi * u + slot;                   // token in the block
      kr[u] = load16_stream(kbase + ((t < 16 ? b0 : b1) + (t & 15)) * tok);
    }
#pragma unroll
    for (int u = 0; u < kLi; ++u) {
      const int t = kTpi * u + slot;
      vr[u] = load16_stream(vbase + ((t < 16 ? b0 : b1) + (t & 15)) * tok);
    }
  };
  // Registers -> LDS as stored: K rows in swapped order, V rows in order.
  auto store_block = [&](GqaWaveLds<D>& w) {
#pragma unroll
    for (int u = 0; u < kLi; ++u) {
      const int t = kTpi * u + slot;
      *reinterpret_cast<uint4*>(&w.k[swap_bits23(t)][8 * ck]) = kr[u];
      *reinterpret_cast<uint4*>(&w.v[t][8 * ck]) = vr[u];
    }
  };

#pragma unroll
  for (int d = 0; d < kDB; ++d)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[d][r] = 0.0f;
  m = kNegBig;   // running max of slot j (shared by lanes j, j + 32)
  l = 0.0f;      // this lane's share of the running sum
  const int lim = min(hi, slot_hi);   // this slot's keys end here

  load_block(0);
  for (int t0 = lo; t0 < hi; t0 += kBlock) {
    // this block into LDS, then the next block's loads (in flight while this
    // one is computed); a wave's LDS operations complete in order, so its
    // own reads below see these writes
    store_block(w);
    load_block(((t0 - lo) >> 4) + 2);

    E8 kf[kDC16];
#pragma unroll
    for (int c = 0; c < kDC16; ++c) kf[c] = *reinterpret_cast<const E8*>(&w.k[j][16 * c + 8 * hh]);
    float16x s = Ops::mm(kf[0], qh[0], (float16x)0.0f);
    s = Ops::mm(kf[0], ql[0], s);
#pragma unroll
    for (int c = 1; c < kDC16; ++c) {
      s = Ops::mm(kf[c], qh[c], s);
      s = Ops::mm(kf[c], ql[c], s);
    }
    if constexpr (Ops::kScaleQ) {
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] = ldexpf(s[r], -qexp);
    }
    // register r of half hh holds token t0 + 16 * (r / 8) + 8 * hh + r % 8
    if (__builtin_amdgcn_ballot_w64(t0 + kBlock > lim) != 0) {
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (t0 + 16 * (r >> 3) + 8 * hh + (r & 7) >= lim) s[r] = -INFINITY;
    }
    float mx = s[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s[r]);
    mx = max_halves(mx);
    // Each slot decides for itself (the wave only skips the rescale when no
    // slot needs it): a slot's result never depends on the other slots of its
    // wave, whichever sequences or heads share it.
    const float m_new = mx > m + kSlack ? mx : m;
    if (__builtin_amdgcn_ballot_w64(m_new != m) != 0) {
      const float corr = fast_exp2(m - m_new);   // 1 for slots that keep m
      l *= corr;
#pragma unroll
      for (int d = 0; d < kDB; ++d)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[d][r] *= corr;
      m = m_new;
    }
    E8 ph[2], pl[2];
    const float mb = m - Ops::kPBias;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float p = fast_exp2(s[r] - mb);       // masked tokens: exp2(-inf) = 0
      l += p;
      const E h = (E)p;
      ph[r >> 3][r & 7] = h;
      pl[r >> 3][r & 7] = (E)(p - (float)h);
    }
#pragma unroll
    for (int kc = 0; kc < 2; ++kc)
#pragma unroll
      for (int d = 0; d < kDB; ++d) {
        const E8 vf = vt_fragment<E8, D>(w, d, 16 * kc, j, hh);
        o[d] = Ops::mm(vf, ph[kc], o[d]);
        o[d] = Ops::mm(vf, pl[kc], o[d]);
      }
  }
  m -= Ops::kPBias;
}

// Result of slot j of a wave: lane (j, hh) owns dims d*32 + 8g + 4hh + 0..3.
template <int D>
__device__ inline void gqa_wave_store(const RowAttnArgs& a, int lane, int gc,
                                      const float16x (&o)[D / 32], float m, float l, bool direct,
                                      int64_t out_off, int64_t pi) {
  constexpr int kDB = D / 32;
  const int j = lane & 31;
  const int hh = lane >> 5;
  const float lsum = sum_halves(l);
  if (j >= gc) return;
  if (direct) {
    const float inv = lsum > 0.0f ? 1.0f / lsum : 0.0f;
    float* op = a.out + out_off + 4 * hh;
#pragma unroll
    for (int d = 0; d < kDB; ++d)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *reinterpret_cast<float4*>(op + d * 32 + 8 * g) =
            make_float4(o[d][4 * g] * inv, o[d][4 * g + 1] * inv, o[d][4 * g + 2] * inv,
                        o[d][4 * g + 3] * inv);
  } else {
    float* op = a.part_acc + pi * D + 4 * hh;
#pragma unroll
    for (int d = 0; d < kDB; ++d)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *reinterpret_cast<float4*>(op + d * 32 + 8 * g) =
            make_float4(o[d][4 * g], o[d][4 * g + 1], o[d][4 * g + 2], o[d][4 * g + 3]);
    if (hh == 0) *reinterpret_cast<float2*>(a.part_ml + 2 * pi) = make_float2(m, lsum);
  }
}


// ---------------------------------------------------------------------------
// Shared pages (prefix caching): sequences whose full partition p has the
// same block ids read the same K/V.  The plan kernel groups them; one wave of
// the shared-page kernel then serves up to 32 query slots, (sequence, head)
// pairs of one KV head, with gqa_wave, reading the pages once.
// ---------------------------------------------------------------------------

constexpr int kShareMaxB = 2048;   // sequences the plan kernel can group
constexpr int kShareMin = 4;       // sequences that must hold a partition to group it

constexpr int kShareMaxPages = 64; // pages of a partition (1024 tokens): one per lane

// splitmix64 finaliser: a well-mixed 64-bit image of one (position, id).
__device__ inline uint64_t mix64(uint64_t x) {
  x ^= x >> 30;
  x *= 0xbf58476d1ce4e5b9ull;
  x ^= x >> 27;
  x *= 0x94d049bb133111ebull;
  return x ^ (x >> 31);
}

constexpr int kShareSlots = 2 * kShareMaxB;   // hash-table slots (a power of two)

constexpr int kPlanWaves = 16;      // waves of a plan workgroup
constexpr int kPlanBatch = 16;      // sequences whose loads a wave issues together

// One workgroup per partition index p.  Its waves take batches of
// kPlanBatch sequences, all of a batch's loads in flight together, the 64
// lanes reading one sequence's block ids of the partition at once (up to 64
// pages, one coalesced load).  A sequence's partition p is a candidate when
// it is full (all part_tokens keys below its context); its hash is the
// wave's sum of mix64(position, id).  The representative is the first
// sequence with the same hash, found through an open-addressing table in LDS
// and confirmed id by id (a hash collision leaves the sequence on its own).
// Sequences whose context ends inside partition p then join a group whose
// representative holds their pages there (below).  Groups of at least
// kShareMin full holders get a range of members[] and of units by atomic
// allocation, so the order of groups, and of sequences inside a group, may
// differ between calls; no result depends on it (every query slot of the
// matrix-core wave is computed on its own, its running max included).
__global__ __launch_bounds__(kPlanWaves * 64) void share_plan_kernel(RowAttnArgs a,
                                                                     SharePlanArgs s) {
  constexpr int kThreads = kPlanWaves * 64;
  __shared__ uint64_t key[kShareSlots];       // hash of the slot's partition (~0: empty)
  __shared__ int first[kShareSlots];          // lowest sequence with that hash
  __shared__ uint64_t hsh[kShareMaxB];
  __shared__ int rep[kShareMaxB];
  __shared__ int cnt[kShareMaxB];             // sequences per representative
  __shared__ int moff[kShareMaxB];            // representative: its members[] offset
  __shared__ int uoff[kShareMaxB];            // representative: its first unit
  __shared__ int fill[kShareMaxB];            // representative: members placed so far
  __shared__ int fid[kShareMaxB];             // block id of the partition's first page
  __shared__ int npart[kShareMaxB];           // pages of a partition the context ends in, else 0
  __shared__ int members_used, units_used;
  const int p = blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int pages = a.part_tokens / 16;       // <= 64: one per lane
  const int64_t cap = (int64_t)a.MB * a.BS;
  const int col = min(p * pages + min(lane, pages - 1), a.MB - 1);   // this lane's table entry
  for (int i = tid; i < kShareSlots; i += kThreads) {
    key[i] = ~0ull;
    first[i] = 0x7fffffff;
  }
  for (int b = tid; b < a.B; b += kThreads) {
    cnt[b] = 0;
    fill[b] = 0;
  }
  if (tid == 0) {
    members_used = 0;
    units_used = 0;
  }
  __syncthreads();
  for (int b0 = wave * kPlanBatch; b0 < a.B; b0 += kPlanWaves * kPlanBatch) {
    int id[kPlanBatch], ctx[kPlanBatch];
#pragma unroll
    for (int k = 0; k < kPlanBatch; ++k) {
      const int b = min(b0 + k, a.B - 1);
      id[k] = a.bt[(int64_t)b * a.MB + col];
      ctx[k] = a.ctx[b];
    }
    // lane k ends with the hash of sequence b0 + k, the id of its first page
    // of the partition, and its page count there when its context ends
    // inside the partition
    uint64_t mine = ~0ull;
    int my_fid = 0, my_np = 0;
#pragma unroll
    for (int k = 0; k < kPlanBatch; ++k) {
      const int64_t end = ctx[k] < cap ? ctx[k] : cap;
      const int64_t p_lo = (int64_t)p * a.part_tokens;
      const bool full = p_lo + a.part_tokens <= end;
      uint64_t h = lane < pages ? mix64(((uint64_t)lane << 32) | (uint32_t)id[k]) : 0;
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) h += __shfl_xor(h, off);
      if (!full || h == ~0ull) h = ~0ull;
      const int f0 = __builtin_amdgcn_readfirstlane(id[k]);
      if (lane == k) {
        mine = h;
        my_fid = f0;
        my_np = !full && end > p_lo ? (int)((end - p_lo + 15) / 16) : 0;
      }
    }
    // the batch's inserts in parallel, one lane per sequence: claim an empty
    // slot or find this hash's, then lower its index
    const int b = b0 + lane;
    if (lane < kPlanBatch && b < a.B) {
      hsh[b] = mine;
      fid[b] = my_fid;
      npart[b] = my_np;
      if (mine != ~0ull) {
        for (int i = (int)(mine & (kShareSlots - 1));; i = (i + 1) & (kShareSlots - 1)) {
          const uint64_t old = atomicCAS(&key[i], ~0ull, mine);
          if (old == ~0ull || old == mine) {
            atomicMin(&first[i], b);
            break;
          }
        }
      }
    }
  }
  __syncthreads();
  for (int b0 = wave * kPlanBatch; b0 < a.B; b0 += kPlanWaves * kPlanBatch) {
    // lane k looks up sequence b0 + k's representative
    int rl = -1;
    if (lane < kPlanBatch && b0 + lane < a.B) {
      const uint64_t h = hsh[b0 + lane];
      if (h != ~0ull) {
        int i = (int)(h & (kShareSlots - 1));
        while (key[i] != h) i = (i + 1) & (kShareSlots - 1);
        rl = first[i];
      }
    }
    int r[kPlanBatch], mine[kPlanBatch], other[kPlanBatch];
#pragma unroll
    for (int k = 0; k < kPlanBatch; ++k) {
      const int b = min(b0 + k, a.B - 1);
      r[k] = __builtin_amdgcn_readlane(rl, k);
      mine[k] = a.bt[(int64_t)b * a.MB + col];
      other[k] = a.bt[(int64_t)max(r[k], 0) * a.MB + col];
    }
#pragma unroll
    for (int k = 0; k < kPlanBatch; ++k) {
      const int b = b0 + k;
      if (b >= a.B) break;                     // wave-uniform
      int rk = r[k];
      if (rk >= 0 && rk != b && __builtin_amdgcn_ballot_w64(mine[k] != other[k]) != 0) rk = b;
      if (lane == 0) rep[b] = rk;
    }
  }
  __syncthreads();
  // a sequence that fell back to itself after a collision is not counted
  // with the group of the hash's first sequence.  A group's members mostly
  // share waves, so each wave adds its count per representative with one
  // atomic (one atomic per sequence serialised on the group's counter).
  for (int b0 = wave * 64; b0 < a.B; b0 += kThreads) {   // wave-uniform
    const int b = b0 + lane;
    int r = b < a.B ? rep[b] : -1;
    if (r >= 0 && rep[r] != r) r = -1;
    for (uint64_t todo = __builtin_amdgcn_ballot_w64(r >= 0); todo != 0;) {
      const int rl = __builtin_amdgcn_readlane(r, __builtin_ctzll(todo));
      const uint64_t same = __builtin_amdgcn_ballot_w64(r == rl);
      if (lane == __builtin_ctzll(todo)) atomicAdd(&cnt[rl], __builtin_popcountll(same));
      todo &= ~same;
    }
  }
  __syncthreads();
  // Members whose context ends inside the partition: such a sequence joins
  // a group when its pages there are the representative's first pages (a
  // shared prefix that the sequence has not yet grown past).  Groups are
  // found by the id of the partition's first page (a table from that id to
  // the group's representative, in the hash table's storage), then every
  // page of the sequence is compared; the shared-page kernel masks each
  // member's keys at its own context.
  for (int i = tid; i < kShareSlots; i += kThreads) {
    key[i] = ~0ull;
    first[i] = 0x7fffffff;
  }
  __syncthreads();
  for (int r = tid; r < a.B; r += kThreads) {
    if (rep[r] != r || cnt[r] < kShareMin) continue;
    const uint64_t id0 = (uint32_t)fid[r];
    for (int i = (int)(mix64(id0) & (kShareSlots - 1));; i = (i + 1) & (kShareSlots - 1)) {
      const uint64_t old = atomicCAS(&key[i], ~0ull, id0);
      if (old == ~0ull || old == id0) {
        atomicMin(&first[i], r);
        break;
      }
    }
  }
  __syncthreads();
  for (int b0 = wave * kPlanBatch; b0 < a.B; b0 += kPlanWaves * kPlanBatch) {
    int rl = -1, nl = 0;                       // lane k: sequence b0 + k
    if (lane < kPlanBatch && b0 + lane < a.B && npart[b0 + lane] > 0) {
      const uint64_t id0 = (uint32_t)fid[b0 + lane];
      int i = (int)(mix64(id0) & (kShareSlots - 1));
      while (key[i] != ~0ull && key[i] != id0) i = (i + 1) & (kShareSlots - 1);
      if (key[i] == id0) {
        rl = first[i];
        nl = npart[b0 + lane];
      }
    }
    int r[kPlanBatch], np[kPlanBatch], mine[kPlanBatch], other[kPlanBatch];
#pragma unroll
    for (int k = 0; k < kPlanBatch; ++k) {
      const int b = min(b0 + k, a.B - 1);
      r[k] = __builtin_amdgcn_readlane(rl, k);
      np[k] = __builtin_amdgcn_readlane(nl, k);
      mine[k] = r[k] >= 0 ? a.bt[(int64_t)b * a.MB + col] : 0;
      other[k] = r[k] >= 0 ? a.bt[(int64_t)r[k] * a.MB + col] : 0;
    }
#pragma unroll
    for (int k = 0; k < kPlanBatch; ++k) {
      if (r[k] < 0) continue;                  // wave-uniform
      if (__builtin_amdgcn_ballot_w64(lane < np[k] && mine[k] != other[k]) == 0 && lane == 0) {
        rep[b0 + k] = r[k];
        atomicAdd(&cnt[r[k]], 1);
      }
    }
  }
  __syncthreads();
  for (int r = tid; r < a.B; r += kThreads) {
    if (rep[r] != r || cnt[r] < kShareMin) continue;
    const int n = cnt[r];
    const int nu = (n + s.per_unit - 1) / s.per_unit;
    const int off = atomicAdd(&members_used, n);
    const int u0 = atomicAdd(&units_used, nu);
    moff[r] = off;
    uoff[r] = u0;
    for (int k = 0; k < nu; ++k)
      s.units[(int64_t)p * s.U + u0 + k] =
          make_int4(off + k * s.per_unit, min(s.per_unit, n - k * s.per_unit), r, 0);
  }
  __syncthreads();
  // members[]: a wave reserves its members of a group with one atomic and
  // places them in lane order
  for (int b0 = wave * 64; b0 < a.B; b0 += kThreads) {   // wave-uniform
    const int b = b0 + lane;
    int g = -1;
    if (b < a.B) {
      const int r = rep[b];
      const bool grouped = r >= 0 && rep[r] == r && cnt[r] >= kShareMin;
      s.skip[(int64_t)b * a.P + p] = grouped ? 1 : 0;
      if (grouped) g = r;
    }
    for (uint64_t todo = __builtin_amdgcn_ballot_w64(g >= 0); todo != 0;) {
      const int leader = __builtin_ctzll(todo);
      const int rl = __builtin_amdgcn_readlane(g, leader);
      const uint64_t same = __builtin_amdgcn_ballot_w64(g == rl);
      int base = 0;
      if (lane == leader) base = atomicAdd(&fill[rl], __builtin_popcountll(same));
      base = __builtin_amdgcn_readlane(base, leader);
      if (g == rl)
        s.members[(int64_t)p * a.B + moff[rl] + base +
                  __builtin_popcountll(same & ((1ull << lane) - 1))] = b;
      todo &= ~same;
    }
  }
  if (tid == 0) s.n_units[p] = units_used;
}

constexpr int kShareGroups = 256;   // workgroups of the shared-page grid

// A fixed grid of workgroups strides over the work items (partition, unit,
// KV head), KV head fastest; each prefix of partitions' unit counts comes
// from n_units (partitions are at most 64: one per lane).  Slot j of a unit
// is member j / G of the group with query head kvh * G + j % G.  The four
// waves of a workgroup take a quarter of the partition's keys each, and
// their states are combined through LDS, so that a shared partition costs a
// quarter of a wave's walk of it.  The grid is one wave per SIMD, so the
// kernel may use the whole register file of one.
template <typename T, int D>
__global__ __launch_bounds__(kGqaWaves * 64) __attribute__((amdgpu_waves_per_eu(1)))
void shared_pages_kernel(RowAttnArgs a, SharePlanArgs s) {
  constexpr int kDB = D / 32;
  constexpr int kState = 16 * kDB + 2;           // floats per lane: o, m, l
  static_assert(kState * 64 * sizeof(float) <= sizeof(GqaWaveLds<D>), "state exchange");
  __shared__ GqaWaveLds<D> lds[kGqaWaves];
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int j = lane & 31;
  int pre = lane < a.P ? s.n_units[lane] : 0;   // inclusive prefix over partitions
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int x = __shfl_up(pre, off);
    if (lane >= off) pre += x;
  }
  const int total = __shfl(pre, 63);
  const int G = a.H / a.Hkv;
  const int64_t cap = (int64_t)a.MB * a.BS;
  const int span = a.part_tokens / kGqaWaves / 16 * 16;   // keys per wave, page-aligned
  // Slot j of work item `item`: its unit, member sequence and query row
  // (recomputed after the key walk rather than held through it).
  struct Slot {
    int p, kvh, gc, mb;
    int4 un;
    int64_t row_h;
  };
  auto slot_of = [&](int item) {
    Slot t;
    t.kvh = item % a.Hkv;
    const int k = item / a.Hkv;                  // unit number over all partitions
    t.p = __popcll(__builtin_amdgcn_ballot_w64(lane < a.P && pre <= k));
    const int u = k - (t.p > 0 ? __shfl(pre, t.p - 1) : 0);
    t.un = s.units[(int64_t)t.p * s.U + u];
    t.gc = t.un.y * G;
    const int js = min(j, t.gc - 1);
    t.mb = s.members[(int64_t)t.p * a.B + t.un.x + js / G];
    t.row_h = (int64_t)t.mb * a.H + t.kvh * G + js % G;
    return t;
  };
  for (int item = blockIdx.x; item < total * a.Hkv; item += gridDim.x) {   // workgroup-uniform
    float16x o[kDB];
    float m, l;
    {
      const Slot t = slot_of(item);
      const int lo = t.p * a.part_tokens + wv * span;
      const int hi = wv == kGqaWaves - 1 ? (t.p + 1) * a.part_tokens : lo + span;
      const int64_t end = a.ctx[t.mb] < cap ? a.ctx[t.mb] : cap;   // member's own keys
      gqa_wave_run<T, D>(a, lds[wv], lane, t.kvh, t.gc, a.bt + (int64_t)t.un.z * a.MB, lo, hi,
                         (int)min(end, (int64_t)hi), t.row_h * D, o, m, l);
    }
    __syncthreads();   // every wave is done with its K/V tiles
    float* xs = reinterpret_cast<float*>(&lds[wv]);
    if (wv > 0) {
#pragma unroll
      for (int d = 0; d < kDB; ++d)
#pragma unroll
        for (int r = 0; r < 16; ++r) xs[(16 * d + r) * 64 + lane] = o[d][r];
      xs[16 * kDB * 64 + lane] = m;
      xs[(16 * kDB + 1) * 64 + lane] = l;
    }
    __syncthreads();
    if (wv == 0) {
      float mm = m;
#pragma unroll
      for (int w = 1; w < kGqaWaves; ++w)
        mm = fmaxf(mm, reinterpret_cast<const float*>(&lds[w])[16 * kDB * 64 + lane]);
      const float c0 = fast_exp2(m - mm);
      l *= c0;
#pragma unroll
      for (int d = 0; d < kDB; ++d)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[d][r] *= c0;
#pragma unroll
      for (int w = 1; w < kGqaWaves; ++w) {
        // one wave's state at a time (the fence keeps the scheduler from
        // loading all of them ahead of the sums)
        __builtin_amdgcn_sched_barrier(0);
        const float* xw = reinterpret_cast<const float*>(&lds[w]);
        const float cw = fast_exp2(xw[16 * kDB * 64 + lane] - mm);
        l += cw * xw[(16 * kDB + 1) * 64 + lane];
#pragma unroll
        for (int d = 0; d < kDB; ++d)
#pragma unroll
          for (int r = 0; r < 16; ++r) o[d][r] += cw * xw[(16 * d + r) * 64 + lane];
      }
      const Slot t = slot_of(item);
      const int64_t end = a.ctx[t.mb] < cap ? a.ctx[t.mb] : cap;
      gqa_wave_store<D>(a, lane, t.gc, o, mm, l, end <= a.part_tokens, t.row_h * D,
                        t.row_h * a.P + t.p);
    }
    __syncthreads();   // the exchange area is free for the next item
  }
}

}  // namespace

bool shared_pages_apply(const RowAttnArgs& a, int kv_dtype, int D) {
  const int G = a.H / a.Hkv;
  return (kv_dtype == HS_DTYPE_F16 || kv_dtype == HS_DTYPE_BF16) && a.BS == 16 &&
         (D == 32 || D == 64 || D == 128) && a.mode == 1 && a.part_tokens <= 16 * kShareMaxPages &&
         a.P > 1 && a.P <= 64 && G <= kHeadsPerWave / 2 && a.B <= kShareMaxB &&
         a.cu_q == nullptr &&
         a.S == 1;
}

int64_t share_unit_slots(int B, int per_unit) {
  return ceil_div(B, kShareMin) + ceil_div(B, per_unit);
}

void launch_share_plan(const RowAttnArgs& a, const SharePlanArgs& s, hipStream_t stream) {
  hipLaunchKernelGGL(share_plan_kernel, dim3((unsigned)a.P), dim3(kPlanWaves * 64), 0, stream,
                     a, s);
}

void launch_shared_pages(const RowAttnArgs& a, const SharePlanArgs& s, int kv_dtype, int D,
                         hipStream_t stream) {
  const dim3 grid(kShareGroups), block(kGqaWaves * 64);
  if (kv_dtype == HS_DTYPE_F16) {
    switch (D) {
      case 32: hipLaunchKernelGGL((shared_pages_kernel<_Float16, 32>), grid, block, 0, stream, a, s); break;
      case 64: hipLaunchKernelGGL((shared_pages_kernel<_Float16, 64>), grid, block, 0, stream, a, s); break;
      default: hipLaunchKernelGGL((shared_pages_kernel<_Float16, 128>), grid, block, 0, stream, a, s); break;
    }
  } else {
    switch (D) {
      case 32: hipLaunchKernelGGL((shared_pages_kernel<Bf16, 32>), grid, block, 0, stream, a, s); break;
      case 64: hipLaunchKernelGGL((shared_pages_kernel<Bf16, 64>), grid, block, 0, stream, a, s); break;
      default: hipLaunchKernelGGL((shared_pages_kernel<Bf16, 128>), grid, block, 0, stream, a, s); break;
    }
  }
}

}  // namespace hs
