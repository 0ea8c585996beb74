// Grouped-query decode for bf16 and fp16 caches on gfx950 matrix cores, at
// fp32 accuracy.
//
// Reference: paged_attn_v2.py:75-157 (one query row per head, KV head
// h / (H / Hkv), online softmax) and paged_attn_v3.py:75-208 (partitions
// merged by log-sum-exp).  Same function as the VALU decode kernel
// (hs_decode.hip); this one serves 16-bit caches when two or more query heads
// share a KV head.
//
// Why matrix cores here.  With G query heads per KV head, the VALU kernel's
// per-token work grows with G (G dot products and G softmax states per
// 16-byte load) while the bytes read stay the same; at G = 4 it is bound by
// that arithmetic, not by HBM.  On the matrix cores the G dot products of a
// token are one column block of an MFMA, and the kernel does a few VALU
// instructions per page instead.  Measured on MI355X, C2's batch and contexts
// with 32 query heads (whole decode call, bf16, D = 128): 2 / 4 / 8 / 16 / 32
// heads per KV head 217 / 124 / 78 / 51 / 50 us, against 232 / 148 us for
// the VALU kernel and 125 / 95 / 64 us for an fp16-operand matrix-core kernel
// (q and the probabilities rounded to fp16, ~1e-3 error) that this one
// replaced.
//
// Numerics.  K and V go to the MFMAs as they are stored (no conversion).  The
// query and the probabilities are fp32; each is split into two terms of the
// cache's type, x = hi + lo with hi = T(x) and lo = T(x - hi), and every
// product is taken against both terms (as two MFMA columns for up to 8 heads
// per KV head, as two products above that).  Products of 16-bit values are
// exact in the fp32 accumulators, so the result matches fp32 arithmetic to
// about 2^-16 relative for bf16 (hi + lo carries 16 significant bits) and
// better for fp16 (22 bits).  fp16 has a narrow exponent range, so for fp16
// caches each head's scaled query is first multiplied by a power of two that
// puts its largest element in [2^14, 2^15) (the scores are multiplied back,
// exactly, after the product), and the probabilities are taken 2^7 times
// larger (at most 2^15 under the lazy rescale below): neither term then
// overflows, and the lo terms stay clear of fp16's subnormals.
//
// Work decomposition.  A workgroup serves up to 16 query heads of one KV head
// for one (row, partition); its kW waves (4 for up to 4 heads per KV head, 2
// above) take the partition's 16-token pages in turn, and each wave computes
// per page:
//   S^T = K . Q^T    v_mfma_f32_16x16x32_{bf16,f16}, K (16 tokens x 32 dims,
//                    from LDS) the A operand, Q^T (heads) the B operand, held
//                    in registers as hi and lo terms; D / 32 k-steps
//   O^T += V^T . P^T v_mfma_f32_16x16x16_{bf16,f16}, V^T (16 dims x 16 tokens,
//                    read transposed from the token-major LDS copy by
//                    ds_read_b64_tr_b16) the A operand, P^T the B operand.  The S^T
//                    accumulator gives lane l the tokens 4(l/16) + i of column
//                    l % 16, which is exactly the B-operand layout of the
//                    second product, so probabilities never leave registers;
//                    and O^T has column l % 16 in lane l too, so the online
//                    rescale and the final normalisation are per-lane scalars.
// Pages are loaded coalesced (D / 8 lanes per head row of one token, 16 bytes
// each) into registers one page ahead of the one being computed, then
// written to the wave's own LDS token-major as they came (no conversion); a
// wave's LDS operations complete in order, so the walk needs no barriers.  At
// the end the waves combine their (m, l, O) through LDS (two barriers) and
// the workgroup writes one partition state: a quarter (or half) of the
// states that one-wave partitions of the same length would write, which is
// most of what separated this kernel from its own loads (measured on MI355X,
// 8 KV heads: 16 of 122 us went to the states).
//
// Grid order.  The hardware deals workgroups to the eight XCDs round-robin by
// workgroup id, and workgroups are numbered unit-fastest (unit = KV head and
// head chunk), so the units of one (row, partition) land on different XCDs
// and every XCD gets an equal share of each row.  Four one-KV-head waves per
// workgroup instead made the XCD depend on the partition index, and the
// early partitions (live in every row) piled up on a few XCDs (160 against
// 138 us).
//
// The partition states (m, l, un-normalised acc) have the VALU kernel's
// layout and meaning, and the same merge kernel combines them; they are
// written through LDS so each head's D floats go out as whole 128-byte lines.
#include <algorithm>
#include <map>
#include <mutex>
#include <utility>

#include "hs_kernels.h"
#include "hs_rowwalk.h"

namespace hs {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef short short4x __attribute__((ext_vector_type(4)));
typedef float float4x __attribute__((ext_vector_type(4)));

constexpr int kSlots = 16;         // query heads per wave (MFMA N)
constexpr int kPage = 16;          // tokens per page (block_size)
constexpr float kSlack = 8.0f;     // lazy-rescale slack, log2 units
constexpr int kMaxPages = 64;      // pages of a fixed partition
constexpr int kWindow = 64;        // block ids held at a time: one per lane

// One page of K and of V, both token-major as in the cache.  Row paddings:
// K rows are read as 16-byte MFMA fragments (row j by lane j), V rows by the
// transposing read below (four rows by each group of 16 lanes).  With K rows
// of D + 8 and V rows of D + 16 halves, the 16 lanes of a group land on
// disjoint banks at D = 32, 64 and 128 (K: 16 spans of 4 banks at stride
// (D + 8) / 2 dwords; V: 4 rows x 4 pairs at stride (D + 16) / 2), and the
// 16-byte row stores stay whole.
template <int D>
struct PageLds {
  static constexpr int kKRow = D + 8;
  static constexpr int kVRow = D + 16;
  alignas(16) uint16_t k[kPage][kKRow];
  alignas(16) uint16_t v[kPage][kVRow];
};

// V^T fragment of the 16x16x16 product for dims 16 dt .. 16 dt + 15: lane
// (j, g) gets V[4 g + e][16 dt + j], e = 0..3.  ds_read_b64_tr_b16 transposes
// within each group of 16 lanes: lane i supplies 8 bytes of row i / 4 of a
// 4 x 16 block and receives column i (lane layout checked on gfx950).
template <int D>
__device__ inline short4x read_vt(const PageLds<D>& w, int dt, int j, int g) {
  typedef __attribute__((address_space(3))) short4x lds_short4x;
  // a C-style cast keeps the LDS address arithmetic visible, so the constant
  // part of the address goes into the instruction's offset field
  const lds_short4x* p = (const lds_short4x*)(&w.v[4 * g + (j >> 2)][16 * dt + 4 * (j & 3)]);
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(const_cast<lds_short4x*>(p));
}

// The cache's element type and its two products.  kPBias: the probabilities
// go to the P.V product as 2^kPBias p (fp16: p <= 2^8 under the lazy rescale,
// so 2^15 at most); kScaleQ: each head's query is brought to [2^14, 2^15)
// by a power of two before it is split.
struct Bf16Ops {
  typedef __bf16 E;
  typedef bf16x8 E8;
  static constexpr float kPBias = 0.0f;
  static constexpr bool kScaleQ = false;
  __device__ static float4x qk(E8 k, E8 q, float4x c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(k, q, c, 0, 0, 0);
  }
  __device__ static float4x pv(short4x v, short4x p, float4x c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(v, p, c, 0, 0, 0);
  }
};

struct F16Ops {
  typedef _Float16 E;
  typedef half8 E8;
  static constexpr float kPBias = 7.0f;
  static constexpr bool kScaleQ = true;
  __device__ static float4x qk(E8 k, E8 q, float4x c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(k, q, c, 0, 0, 0);
  }
  __device__ static float4x pv(short4x v, short4x p, float4x c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(half4, v),
                                                 __builtin_bit_cast(half4, p), c, 0, 0, 0);
  }
};

// x = hi + lo with hi, lo of type E (RNE); returns their bit patterns.
template <typename E>
__device__ inline void split16(float x, uint16_t& hi, uint16_t& lo) {
  const E h = (E)x;
  hi = __builtin_bit_cast(uint16_t, h);
  lo = __builtin_bit_cast(uint16_t, (E)(x - (float)h));
}

// Both values of x across lanes l and l ^ 16, and across l and l ^ 32.
__device__ inline float max_across_groups(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ inline float sum_across_groups(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

template <int D>
struct PageWalk {
  static constexpr int kDC = D / 8;           // 16-byte chunks per head row
  static constexpr int kTpi = 64 / kDC;       // tokens per wave-wide load
  static constexpr int kLi = kPage / kTpi;    // loads per page, for K and for V
  static constexpr int kKS = D / 32;          // QK k-steps
  static constexpr int kDT = D / 16;          // O^T dim tiles
  static_assert(kLi >= 1 && kTpi * kLi == kPage, "head_dim");

  struct Regs {
    uint4 k[kLi];    // K load u: token kTpi * u + slot, chunk ck
    uint4 v[kLi];    // V load u: the same token and chunk
  };
};

// One wave's pass over pages first, first + step, ... of keys [lo, hi) (lo a
// multiple of 16) of block-table row `bt`, for query slots j < gc whose
// queries start at element q_off of a.q (slot j at q_off + j * D); no pages
// (first past the end) leaves the empty state.  Returns the state in o / m /
// l: lane l holds column l % 16, dims 16 * dt + 4 * (l / 16) + i of o[dt][i];
// m is the running max (log2 units), l this lane's share of the sum (tokens
// 4 * (l / 16) + i of every page); the caller reduces l across the four lane
// groups.
//
// kCols (gc <= 8): the hi and lo terms are separate MFMA columns instead of
// separate products: column c < 8 carries the hi term of head c, column
// c + 8 its lo term, so each product is taken once.  A score is the sum of
// its two columns (lanes j and j ^ 8, one DPP rotate); both lanes then hold
// the same score and softmax state, lane j < 8 feeds the hi term of the
// probability and lane j + 8 the lo term, and o of head c is the sum of
// columns c and c + 8 (added by the caller).  Without kCols, column j is head
// j and every product is taken twice, against hi and against lo.
//
// The state is in the ordinary units (m minus kPBias: o and l carry the
// 2^kPBias factor of the probabilities).
template <typename Ops, int D, bool kCols>
__device__ inline void page_walk(const RowAttnArgs& a, PageLds<D>& w, int kvh, int gc,
                                 const int32_t* bt, int lo, int hi, int first, int step,
                                 int64_t q_off, float4x (&o)[D / 16], float& m, float& l) {
  using W = PageWalk<D>;
  using E = typename Ops::E;
  using E8 = typename Ops::E8;
  constexpr int kDC = W::kDC, kTpi = W::kTpi, kLi = W::kLi, kKS = W::kKS, kDT = W::kDT;
  constexpr int kQS = kCols ? 1 : 2;               // products per page and operand
  const int lane = threadIdx.x & 63;
  const int j = lane & 15;          // MFMA column of this lane
  const int g = lane >> 4;          // lane group: tokens 4g .. 4g + 3 of a page
  const int hj = kCols ? (j & 7) : j;   // query slot (head) of column j
  const bool lo_col = kCols && j >= 8;
  const int ck = lane % kDC;        // loads: chunk of the head row
  const int slot = lane / kDC;      // loads: token slot

  // Block ids of the range's pages, 64 at a time: lane i of idv holds page
  // page0 + 64 win + i, and idn those of the next window, loaded one window
  // ahead so that crossing into it waits for nothing.  (A fixed partition has
  // at most 64 pages and never leaves window 0.)
  const int page0 = lo / kPage;
  const int npages = (hi - lo + kPage - 1) / kPage;
  int idv = bt[min(page0 + lane, a.MB - 1)];
  int idn = npages > kWindow ? bt[min(page0 + kWindow + lane, a.MB - 1)] : 0;
  int win = 0;

  // Q^T fragments, split: lane l holds column j's dims 32 st + 8 g .. + 7.
  // qexp: the power of two the query was multiplied by (kScaleQ), taken back
  // out of every score.
  E8 qf[kQS][kKS];
  int qexp = 0;
  {
    const float sc = hj < gc ? a.qscale : 0.0f;
    const float* qp = a.q + q_off + (int64_t)min(hj, gc - 1) * D + 8 * g;
    float xq[kKS][8];
    float amax = 0.0f;
#pragma unroll
    for (int st = 0; st < kKS; ++st) {
      const float4 x0 = *reinterpret_cast<const float4*>(qp + 32 * st);
      const float4 x1 = *reinterpret_cast<const float4*>(qp + 32 * st + 4);
      const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        xq[st][e] = xs[e] * sc;
        amax = fmaxf(amax, fabsf(xq[st][e]));
      }
    }
    if constexpr (Ops::kScaleQ) {
      // the head's largest |element| (its D dims are spread over the four
      // lane groups of column j); 2^qexp * amax lands in [2^14, 2^15), and
      // a zero or non-finite head keeps qexp = 0
      amax = max_across_groups(amax);
      if (amax > 0.0f && __builtin_isfinite(amax)) qexp = 15 - __builtin_amdgcn_frexp_expf(amax);
    }
#pragma unroll
    for (int st = 0; st < kKS; ++st) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = Ops::kScaleQ ? ldexpf(xq[st][e], qexp) : xq[st][e];
        const E h = (E)x;
        const E r = (E)(x - (float)h);
        if constexpr (kCols) {
          qf[0][st][e] = lo_col ? r : h;
        } else {
          qf[0][st][e] = h;
          qf[1][st][e] = r;
        }
      }
    }
    // Keep the split query in registers: without this anchor the compiler
    // re-loads and re-splits it on every page to save registers.
#pragma unroll
    for (int q = 0; q < kQS; ++q)
#pragma unroll
      for (int st = 0; st < kKS; ++st) {
        uint4& u = reinterpret_cast<uint4&>(qf[q][st]);
        asm volatile("" : "+v"(u.x), "+v"(u.y), "+v"(u.z), "+v"(u.w));
      }
  }

  const int64_t tok = (int64_t)a.Hkv * D;          // elements between tokens of a page
  // Page addresses: a wave-uniform base (scalar registers) plus one 32-bit
  // lane offset shared by all loads of a page.
  const uint16_t* kbase = reinterpret_cast<const uint16_t*>(a.k) + kvh * D;
  const uint16_t* vbase = reinterpret_cast<const uint16_t*>(a.v) + kvh * D;
  const uint32_t loff = (uint32_t)(slot * tok + 8 * ck) * 2u;   // bytes; < 16 * tok * 2

  typename W::Regs rg;
  // Loads of page pg of the range (pg < npages).  A wave's pages increase by
  // step < kWindow, so they enter the windows one at a time.
  auto load_page = [&](typename W::Regs& r, int pg) {
    if (pg / kWindow != win) {   // wave-uniform
      win = pg / kWindow;
      idv = idn;
      idn = kWindow * (win + 1) < npages
                ? bt[min(page0 + kWindow * (win + 1) + lane, a.MB - 1)] : 0;
    }
    const int64_t b0 =
        safe_block(__builtin_amdgcn_readlane(idv, pg % kWindow), a.NB) * kPage;
    const char* kp = reinterpret_cast<const char*>(kbase + b0 * tok);
    const char* vp = reinterpret_cast<const char*>(vbase + b0 * tok);
#pragma unroll
    for (int u = 0; u < kLi; ++u)
      r.k[u] = load16_stream(kp + (int64_t)u * kTpi * tok * 2 + loff);
#pragma unroll
    for (int u = 0; u < kLi; ++u)
      r.v[u] = load16_stream(vp + (int64_t)u * kTpi * tok * 2 + loff);
  };
  // Registers -> LDS, rows as loaded.
  auto store_page = [&](const typename W::Regs& r) {
#pragma unroll
    for (int u = 0; u < kLi; ++u) {
      *reinterpret_cast<uint4*>(&w.k[kTpi * u + slot][8 * ck]) = r.k[u];
      *reinterpret_cast<uint4*>(&w.v[kTpi * u + slot][8 * ck]) = r.v[u];
    }
  };

#pragma unroll
  for (int d = 0; d < kDT; ++d)
#pragma unroll
    for (int i = 0; i < 4; ++i) o[d][i] = 0.0f;
  m = kNegBig;
  l = 0.0f;

  if (first < npages) load_page(rg, first);
  for (int pg = first; pg < npages; pg += step) {
    store_page(rg);
    // the next page's loads fly during this page's arithmetic; none past
    // the last page
    if (pg + step < npages) load_page(rg, pg + step);   // wave-uniform

    // S^T: lane l gets tokens 4g + i of this page for column j
    float4x sa[kQS];
#pragma unroll
    for (int q = 0; q < kQS; ++q) sa[q] = float4x{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int st = 0; st < kKS; ++st) {
      const E8 kf = *reinterpret_cast<const E8*>(&w.k[j][32 * st + 8 * g]);
#pragma unroll
      for (int q = 0; q < kQS; ++q) sa[q] = Ops::qk(kf, qf[q][st], sa[q]);
    }
    float s[4];
    const int t0 = lo + pg * kPage + 4 * g;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float x = kCols ? sa[0][i] + dpp<kDppRowRor8>(sa[0][i]) : sa[0][i] + sa[kQS - 1][i];
      if constexpr (Ops::kScaleQ) x = ldexpf(x, -qexp);
      s[i] = t0 + i < hi ? x : -INFINITY;
    }

    // online softmax of column j; the max is raised only when it grows by > 8
    float mx = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
    mx = max_across_groups(mx);
    const float m_new = mx > m + kSlack ? mx : m;
    if (__builtin_amdgcn_ballot_w64(m_new != m) != 0) {
      const float corr = fast_exp2(m - m_new);    // 1 for heads that keep m
      l *= corr;
#pragma unroll
      for (int d = 0; d < kDT; ++d)
#pragma unroll
        for (int i = 0; i < 4; ++i) o[d][i] *= corr;
      m = m_new;
    }
    short4x pf[kQS];
    const float mb = m - Ops::kPBias;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float p = fast_exp2(s[i] - mb);       // masked tokens: exp2(-inf) = 0
      l += p;
      uint16_t h16, l16;
      split16<E>(p, h16, l16);
      if constexpr (kCols) {
        pf[0][i] = (short)(lo_col ? l16 : h16);
      } else {
        pf[0][i] = (short)h16;
        pf[1][i] = (short)l16;
      }
    }

    // O^T += V^T . P^T, dims 16 d .. 16 d + 15 per tile
#pragma unroll
    for (int d = 0; d < kDT; ++d) {
      const short4x vf = read_vt(w, d, j, g);
#pragma unroll
      for (int q = 0; q < kQS; ++q) o[d] = Ops::pv(vf, pf[q], o[d]);
    }
  }
  m -= Ops::kPBias;
}

// The kW wave states of one (row, key range, unit) combined into one: the
// weight of each wave is 2^(m - M) with M the workgroup's max for the
// column.  Lane (j, g) owns dims 16 d + 4 g .. + 3 of head j of the unit.
// Each wave's rows go to its own page buffers (free once the walk is done),
// weighted (and normalised when `single`: the range is the whole row); then
// the workgroup sums the kW copies of a head row with D / 4 lanes per row and
// writes it: to out_rows + hh * D when single, else to acc_rows + hh *
// acc_stride floats, with (m, l) of head j at ml + 2 j * ml_stride.  Every
// wave of the workgroup calls it (it holds barriers); the page buffers and
// wave_m / wave_l are free again when it returns.
template <int D, bool kCols, int kW>
__device__ inline void write_unit_state(float4x (&o)[D / 16], float m, float l, int gc,
                                        bool single, float* out_rows, float* acc_rows,
                                        int64_t acc_stride, float* ml, int64_t ml_stride,
                                        PageLds<D> (&lds)[kW], float (&wave_m)[kW][kSlots],
                                        float (&wave_l)[kW][kSlots]) {
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int j = lane & 15;
  const int g = lane >> 4;
  float lsum = sum_across_groups(l);
  if constexpr (kCols) {   // head j < 8: hi column j plus lo column j + 8
#pragma unroll
    for (int d = 0; d < D / 16; ++d)
#pragma unroll
      for (int i = 0; i < 4; ++i) o[d][i] += dpp<kDppRowRor8>(o[d][i]);
  }
  float sc = 1.0f;
  if constexpr (kW > 1) {
    if (g == 0) {
      wave_m[wv][j] = m;
      wave_l[wv][j] = lsum;
    }
    __syncthreads();
    float mm = wave_m[0][j];
#pragma unroll
    for (int w = 1; w < kW; ++w) mm = fmaxf(mm, wave_m[w][j]);
    float ll = 0.0f;
#pragma unroll
    for (int w = 0; w < kW; ++w) ll += wave_l[w][j] * fast_exp2(wave_m[w][j] - mm);
    sc = fast_exp2(m - mm);
    m = mm;
    lsum = ll;
  }
  constexpr int kSt = D + 4;                          // floats per staged row
  static_assert(kSlots * kSt * sizeof(float) <= sizeof(PageLds<D>), "staging fits");
  if (single) sc *= lsum > 0.0f ? 1.0f / lsum : 0.0f;
  float* st = reinterpret_cast<float*>(&lds[wv]);
#pragma unroll
  for (int d = 0; d < D / 16; ++d)
    *reinterpret_cast<float4*>(&st[j * kSt + 16 * d + 4 * g]) =
        make_float4(o[d][0] * sc, o[d][1] * sc, o[d][2] * sc, o[d][3] * sc);
  if (!single && wv == 0 && g == 0 && j < gc)
    *reinterpret_cast<float2*>(ml + 2 * (int64_t)j * ml_stride) = make_float2(m, lsum);
  if constexpr (kW > 1) __syncthreads();
  constexpr int kLr = D / 4;                          // lanes per head row
  constexpr int kHp = 64 / kLr;                       // head rows per wave and pass
  const int c4 = lane % kLr;
  for (int hb = wv * kHp; hb < gc; hb += kW * kHp) {  // wave-uniform
    const int hh = hb + lane / kLr;
    if (hh < gc) {
      float4 x = *reinterpret_cast<const float4*>(
          &reinterpret_cast<const float*>(&lds[0])[hh * kSt + 4 * c4]);
#pragma unroll
      for (int w = 1; w < kW; ++w) {
        const float4 y = *reinterpret_cast<const float4*>(
            &reinterpret_cast<const float*>(&lds[w])[hh * kSt + 4 * c4]);
        x = make_float4(x.x + y.x, x.y + y.y, x.z + y.z, x.w + y.w);
      }
      float* dst = single ? out_rows + (int64_t)hh * D : acc_rows + (int64_t)hh * acc_stride;
      *reinterpret_cast<float4*>(dst + 4 * c4) = x;
    }
  }
  __syncthreads();   // staging read by every wave before the buffers are reused
}

// One workgroup per (row, partition, KV head, head chunk): kW waves take the
// partition's pages in turn (wave w: pages w, w + kW, ...), then combine
// their states through LDS, so the partition writes one state however many
// waves read it.  Every early return below is workgroup-uniform (it depends
// on blockIdx only), so all waves reach the barriers.
template <typename Ops, int D, bool kCols, int kW>
__global__ __launch_bounds__(64 * kW) void splitmm_part_kernel(RowAttnArgs a) {
  __shared__ PageLds<D> lds[kW];
  __shared__ float wave_m[kW][kSlots], wave_l[kW][kSlots];
  const int wv = threadIdx.x >> 6;
  const int G = a.H / a.Hkv;
  const int n_hc = (G + kSlots - 1) / kSlots;          // head chunks per KV head
  const int n_units = a.Hkv * n_hc;
  // Workgroups are numbered unit-fastest over (row, partition, unit).
  const int64_t gw = blockIdx.x;
  if (gw >= (int64_t)a.rows * a.P * n_units) return;
  const int unit = (int)(gw % n_units);
  const int kvh = unit / n_hc;
  const int hc = unit - kvh * n_hc;
  const int h0 = kvh * G + hc * kSlots;
  const int gc = min(kSlots, G - hc * kSlots);          // heads of this unit
  const int64_t rp = gw / n_units;
  const int row = (int)(rp / a.P);
  const int p = (int)(rp - (int64_t)row * a.P);
  if (a.skip && a.skip[rp]) return;                     // served by the shared-page kernel

  int b, end;
  if (!row_geometry(a, row, b, end)) return;
  int lo = 0, hi = 0, nparts = 0;
  const bool live = partition_range(a, end, p, lo, hi, nparts);
  const int64_t orow0 = ((int64_t)row * a.H + h0) * D;
  if (!live) {
    if (end <= 0 && p == 0) {   // nothing to attend to: zero rows
      for (int d = threadIdx.x; d < gc * D; d += 64 * kW) a.out[orow0 + d] = 0.0f;
    }
    return;
  }
  float4x o[D / 16];
  float m, l;
  page_walk<Ops, D, kCols>(a, lds[wv], kvh, gc, a.bt + (int64_t)b * a.MB, lo, hi, wv, kW, orow0,
                           o, m, l);
  const int64_t pi0 = ((int64_t)row * a.H + h0) * a.P + p;   // state of head h0
  write_unit_state<D, kCols, kW>(o, m, l, gc, nparts == 1, a.out + orow0,
                                 a.part_acc + pi0 * D, (int64_t)a.P * D, a.part_ml + 2 * pi0,
                                 a.P, lds, wave_m, wave_l);
}

// ---------------------------------------------------------------------------
// Even split (mode 4): the decode's pages cut into equal shares
// ---------------------------------------------------------------------------
//
// A unit's work is every page of every row: with the rows' pages laid end to
// end (row b's pages start at R_b = pages of rows 0 .. b - 1), the Tp pages
// are cut into M ranges of Q = ceil(Tp / M) pages, one per workgroup, and M
// workgroups per unit fill the chip about once.  A range that crosses a row
// boundary is walked one row piece ("segment") at a time.  So every
// workgroup reads the same number of bytes, whatever the mix of context
// lengths, and the grid drains all at once: fixed partitions leave a last,
// partly filled round of workgroups (C2's batch: 1816 workgroups of 768
// tokens on 1024 slots).
//
// A segment that is a whole row writes the normalised output.  Otherwise it
// writes its state to slot (unit, w + b) (w the workgroup's range, b the row:
// distinct for every segment, M + B slots per unit), and even_merge_kernel,
// launched next, combines the segments of each such row.  (Merging in the
// same kernel, by the last segment to arrive, needs an agent-scope release
// and acquire per segment to cross the XCDs' separate L2s; measured on
// MI355X that made the C2-gqa decode 3.5x slower.)

// Pages of sequence b: ceil(end / 16), end = ctx clamped to [0, MB * BS].
__device__ inline int row_pages(const RowAttnArgs& a, int b) {
  const int64_t cap = (int64_t)a.MB * a.BS;
  int64_t e = a.ctx[b];
  e = e < 0 ? 0 : (e < cap ? e : cap);
  return (int)((e + kPage - 1) / kPage);
}

// Lane l's value of x, as a wave-uniform (scalar) value.
__device__ inline int64_t lane_value64(int64_t x, int l) {
  const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)x, l);
  const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)((uint64_t)x >> 32), l);
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

__device__ inline int64_t wave_sum64(int64_t x) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) x += __shfl_xor(x, off);
  return lane_value64(x, 0);
}

// Tp: the pages of all rows (each wave of the caller computes it).
__device__ inline int64_t total_pages(const RowAttnArgs& a) {
  const int lane = threadIdx.x & 63;
  int64_t tp = 0;
  for (int c = 0; c < a.B; c += 64) tp += wave_sum64(c + lane < a.B ? row_pages(a, c + lane) : 0);
  return tp;
}

// Q, the pages of a range: Tp cut into at most even_m ranges of at least
// even_min_pages pages (a small decode takes fewer workgroups, the rest of
// the grid finds its range empty).
__device__ inline int64_t range_pages(const RowAttnArgs& a, int64_t tp) {
  const int64_t m = max((int64_t)1, min((int64_t)a.even_m,
                                        (tp + a.even_min_pages - 1) / a.even_min_pages));
  return max((int64_t)1, (tp + m - 1) / m);
}

// Range wr of the even split: pages [s, e) of the rows laid end to end,
// and its first row r with R_r, the pages of the rows before it (R_r <= s <
// R_{r+1}).  Every lane computes the same (scalar) values; false for an
// empty range.  (The first 64 rows' pages stay in registers between the two
// passes.)
__device__ inline bool even_range(const RowAttnArgs& a, int wr, int64_t& s, int64_t& e, int& r,
                                  int64_t& Rr) {
  const int lane = threadIdx.x & 63;
  const int64_t v0 = lane < a.B ? row_pages(a, lane) : 0;
  int64_t tp = wave_sum64(v0);
  for (int c = 64; c < a.B; c += 64)
    tp += wave_sum64(c + lane < a.B ? row_pages(a, c + lane) : 0);
  const int64_t Q = range_pages(a, tp);
  s = (int64_t)wr * Q;
  e = min(s + Q, tp);
  if (s >= e) return false;
  r = a.B;
  Rr = tp;
  int64_t base = 0;
  for (int c = 0; c < a.B; c += 64) {
    const int64_t v = c == 0 ? v0 : (c + lane < a.B ? row_pages(a, c + lane) : 0);
    int64_t inc = v;                                    // inclusive scan over the chunk
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int64_t y = __shfl_up(inc, off);
      if (lane >= off) inc += y;
    }
    const uint64_t hit = __builtin_amdgcn_ballot_w64(c + lane < a.B && base + inc > s);
    if (hit != 0) {
      const int l0 = __builtin_ctzll(hit);
      r = c + l0;
      Rr = base + lane_value64(inc - v, l0);
      break;
    }
    base += lane_value64(inc, 63);
  }
  return true;
}

template <typename Ops, int D, bool kCols, int kW>
__global__ __launch_bounds__(64 * kW) void splitmm_even_kernel(RowAttnArgs a) {
  __shared__ PageLds<D> lds[kW];
  __shared__ float wave_m[kW][kSlots], wave_l[kW][kSlots];
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int G = a.H / a.Hkv;
  const int n_hc = (G + kSlots - 1) / kSlots;
  const int n_units = a.Hkv * n_hc;
  const int kg = min(G, kSlots);                        // state rows per slot
  const int unit = (int)(blockIdx.x % n_units);         // unit-fastest: units spread over XCDs
  const int wr = (int)(blockIdx.x / n_units);           // this workgroup's range, < M
  const int kvh = unit / n_hc;
  const int hc = unit - kvh * n_hc;
  const int h0 = kvh * G + hc * kSlots;
  const int gc = min(kSlots, G - hc * kSlots);

  int64_t s, e, Rr;
  int r;
  if (!even_range(a, wr, s, e, r, Rr)) return;          // workgroup-uniform

  float4x o[D / 16];
  float m, l;
  for (; r < a.B && Rr < e; ++r) {                      // workgroup-uniform
    const int pr = row_pages(a, r);
    const int64_t Rn = Rr + pr;
    if (pr > 0) {
      const int64_t pa = max(s, Rr), pb = min(e, Rn);   // pa < pb: this row's segment
      const int64_t cap = (int64_t)a.MB * a.BS;
      const int end = (int)min((int64_t)a.ctx[r], cap);
      const int lo = (int)(pa - Rr) * kPage;
      const int hi = (int)min((pb - Rr) * kPage, (int64_t)end);
      const int64_t orow0 = ((int64_t)r * a.H + h0) * D;
      page_walk<Ops, D, kCols>(a, lds[wv], kvh, gc, a.bt + (int64_t)r * a.MB, lo, hi, wv, kW,
                               orow0, o, m, l);
      const int64_t slot = ((int64_t)unit * a.even_slots + wr + r) * kg;   // head h0's state
      write_unit_state<D, kCols, kW>(o, m, l, gc, pa == Rr && pb == Rn, a.out + orow0,
                                     a.part_acc + slot * D, D, a.part_ml + 2 * slot, 1, lds,
                                     wave_m, wave_l);
    }
    Rr = Rn;
  }
}

// The even split for plain multi-head attention (one query head per KV head)
// on the VALU walk: a workgroup is kEvenValuWaves adjacent heads (each its
// own unit: the merge's slot layout with one state row per slot) and one
// range wr; each wave walks its head's pieces of the range with RowWalk
// (hs_rowwalk.h), the fixed-partition kernel's arithmetic, and writes a whole
// row's output or a cut row's state.  Adjacent heads read adjacent 256-byte
// pieces of each token row, as in the partition kernel.
constexpr int kEvenValuWaves = 2;

template <typename T, int D>
__global__ __launch_bounds__(64 * kEvenValuWaves)
__attribute__((amdgpu_waves_per_eu(D > 128 ? 3 : 4))) void row_attn_even_kernel(RowAttnArgs a) {
  const int lane = threadIdx.x & 63;
  const int n_hp = (a.H + kEvenValuWaves - 1) / kEvenValuWaves;
  const int hp = (int)(blockIdx.x % n_hp);              // head pairs fastest: token rows together
  const int wr = (int)(blockIdx.x / n_hp);
  const int h = hp * kEvenValuWaves + (int)(threadIdx.x >> 6);
  if (h >= a.H) return;                                 // the waves share nothing
  int64_t s, e, Rr;
  int r;
  if (!even_range(a, wr, s, e, r, Rr)) return;
  const int64_t cap = (int64_t)a.MB * a.BS;
  for (; r < a.B && Rr < e; ++r) {                      // wave-uniform
    const int pr = row_pages(a, r);
    const int64_t Rn = Rr + pr;
    if (pr > 0) {
      const int64_t pa = max(s, Rr), pb = min(e, Rn);   // pa < pb: this row's piece
      const int end = (int)min((int64_t)a.ctx[r], cap);
      const int lo = (int)(pa - Rr) * kPage;
      const int hi = (int)min((pb - Rr) * kPage, (int64_t)end);
      const int64_t orow = ((int64_t)r * a.H + h) * D;
      RowWalk<T, D, true, 1> w;
      w.run(KvPages{a.k, a.v, a.Hkv, a.BS, a.NB}, a.q + orow, a.qscale, h, a.bt + (int64_t)r * a.MB,
            lo, hi);
      if (w.slot(lane) == 0) {
        if (pa == Rr && pb == Rn) {
          w.store_out(0, a.out + orow);
        } else {
          const int64_t slot = (int64_t)h * a.even_slots + wr + r;
          w.store_state(0, a.part_acc + slot * D, reinterpret_cast<float2*>(a.part_ml) + slot);
        }
      }
    }
    Rr = Rn;
  }
}

// One wave per (row, head): a row cut over several ranges gets the
// log-sum-exp merge of its segments' states (the merge kernel's arithmetic,
// hs_decode.hip), a row without keys a zero output; a row inside one range
// was written by the even-split kernel.  Latency-bound (a few MB in all): one
// pass over the context lengths gives Tp and R_r, lane p reads segment p's
// (max, sum), and the partial outputs are read 8 segments at a time, each
// weight taken from the lane that computed it.
template <int D>
__global__ __launch_bounds__(256) void even_merge_kernel(RowAttnArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t wg = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (wg >= (int64_t)a.B * a.H) return;
  const int r = (int)(wg / a.H);
  const int h = (int)(wg - (int64_t)r * a.H);
  float* dst = a.out + wg * D;
  constexpr int kPer = (D + 63) / 64;
  int64_t tp = 0, Rr = 0;                               // all pages; pages of rows before r
  for (int c = 0; c < a.B; c += 64) {
    const int b = c + lane;
    const int64_t v = b < a.B ? row_pages(a, b) : 0;
    tp += wave_sum64(v);
    Rr += wave_sum64(b < r ? v : 0);
  }
  const int pr = row_pages(a, r);
  if (pr == 0) {
#pragma unroll
    for (int i = 0; i < kPer; ++i)
      if (lane + 64 * i < D) dst[lane + 64 * i] = 0.0f;
    return;
  }
  const int64_t Q = range_pages(a, tp);
  const int64_t w_first = Rr / Q, w_last = (Rr + pr - 1) / Q;
  if (w_first == w_last) return;
  const int G = a.H / a.Hkv;
  const int n_hc = (G + kSlots - 1) / kSlots;
  const int kg = min(G, kSlots);
  const int kvh = h / G, hc = (h - kvh * G) / kSlots;
  const int jh = h - kvh * G - hc * kSlots;             // head within its unit
  const int64_t unit = (int64_t)kvh * n_hc + hc;
  // segment w's state row: slot (unit, w + r), head jh
  const int64_t s0 = (unit * a.even_slots + w_first + r) * kg + jh;
  const int n = (int)(w_last - w_first + 1);
  const float2* ml = reinterpret_cast<const float2*>(a.part_ml);
  const float2 none = make_float2(kNegBig, 0.0f);
  const float2 st0 = lane < n ? ml[s0 + (int64_t)lane * kg] : none;
  float mm = st0.x;
  for (int p = 64 + lane; p < n; p += 64) mm = fmaxf(mm, ml[s0 + (int64_t)p * kg].x);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) mm = fmaxf(mm, __shfl_xor(mm, off));
  constexpr int kBatch = 8;
  float acc[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) acc[i] = 0.0f;
  float lsum = 0.0f;
  for (int p0 = 0; p0 < n; p0 += 64) {
    const int nn = min(64, n - p0);
    const float2 st = p0 == 0 ? st0 : (lane < nn ? ml[s0 + (int64_t)(p0 + lane) * kg] : none);
    const float wt = lane < nn ? fast_exp2(st.x - mm) : 0.0f;
    lsum = fmaf(st.y, wt, lsum);
    const float* pa = a.part_acc + (s0 + (int64_t)p0 * kg) * D;
    for (int p = 0; p < nn; p += kBatch) {
      float v[kBatch][kPer];
#pragma unroll
      for (int u = 0; u < kBatch; ++u)
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
          const int d = lane + 64 * i;
          v[u][i] = (p + u < nn && d < D) ? pa[(int64_t)(p + u) * kg * D + d] : 0.0f;
        }
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const float wu = __builtin_bit_cast(
            float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wt), min(p + u, 63)));
#pragma unroll
        for (int i = 0; i < kPer; ++i) acc[i] = fmaf(v[u][i], wu, acc[i]);
      }
    }
  }
  lsum = group_sum<64>(lsum);
  const float inv = lsum > 0.0f ? 1.0f / lsum : 0.0f;
#pragma unroll
  for (int i = 0; i < kPer; ++i)
    if (lane + 64 * i < D) dst[lane + 64 * i] = acc[i] * inv;
}

}  // namespace

bool splitmm_serves(int kv_dtype, int BS, int D, int H, int Hkv) {
  return (kv_dtype == HS_DTYPE_BF16 || kv_dtype == HS_DTYPE_F16) && BS == kPage &&
         (D == 32 || D == 64 || D == 128) && H / Hkv >= 2;
}

bool splitmm_applies(const RowAttnArgs& a, int kv_dtype, int D) {
  return splitmm_serves(kv_dtype, a.BS, D, a.H, a.Hkv) && a.mode == 1 &&
         a.part_tokens <= kPage * kMaxPages;
}

// Waves per partition and the default partition.  Groups of at most 4 query
// heads (the least arithmetic per byte) share a partition between 4 waves,
// larger groups between 2, so a quarter (half) of the partition states reach
// HBM.  Measured on C2's batch and contexts, 32 query heads, bf16 (step, us,
// waves x partition tokens):
//   G = 2:  226 (1 x 256)  217 (2 x 512)  213 (4 x 512)
//   G = 4:  129 (1 x 256)  126 (2 x 512)  123 (4 x 512)
//   G = 8:   80 (1 x 256)   77 (2 x 256)   78 (4 x 256)
//   G = 16:  52 (1 x 128)   50 (2 x 256)   53 (4 x 256)
//   G = 32:  51 (1 x 128)   49 (2 x 256)   53 (4 x 256)
// The partition length is best at about 12 pages per wave (step, us, same
// batch, partition tokens 256 / 384 / 512 / 640 / 768 / 896 / 1024):
//   G = 2, D 128:  226 216 215 211 208 216 215
//   G = 4, D 128:  126 119 122 117 117 121 138
//   G = 8, D 128:   78  69  83  78  81  83 110
//   G = 4, D 64:    72  69  75  69  68  73  89
//   G = 2, D 64:   124 127 129 123 125 134 136
// so 768 tokens for 4 waves and 384 for 2 (G = 8); G > 8 keeps 256.  At head
// dim 32 (1-KB head pages) 256 tokens measured best or within 4% for every G
// (C2 contexts, fp16, 32 query heads: G = 2 / 4 / 8: 119 / 65 / 40 us).
int splitmm_waves(int G) { return G <= 4 ? 4 : 2; }
int splitmm_default_partition(int G, int D) {
  if (D == 32 || G > 8) return 256;
  return G <= 4 ? 768 : 384;
}

int64_t splitmm_grid(const RowAttnArgs& a) {
  const int G = a.H / a.Hkv;
  return sat_mul(a.rows, a.P, a.Hkv, ceil_div(G, kSlots));
}

template <typename Ops, int D, int kW>
static void launch_waves(const RowAttnArgs& a, hipStream_t stream) {
  const dim3 grid((unsigned)splitmm_grid(a)), block(64 * kW);
  if (a.H / a.Hkv <= 8)   // one head chunk of at most 8 heads: hi/lo as columns
    hipLaunchKernelGGL((splitmm_part_kernel<Ops, D, true, kW>), grid, block, 0, stream, a);
  else
    hipLaunchKernelGGL((splitmm_part_kernel<Ops, D, false, kW>), grid, block, 0, stream, a);
}

template <typename Ops>
static void launch_for(const RowAttnArgs& a, int D, hipStream_t stream) {
  const bool four = splitmm_waves(a.H / a.Hkv) == 4;
  if (D == 32) {
    if (four) launch_waves<Ops, 32, 4>(a, stream);
    else launch_waves<Ops, 32, 2>(a, stream);
  } else if (D == 64) {
    if (four) launch_waves<Ops, 64, 4>(a, stream);
    else launch_waves<Ops, 64, 2>(a, stream);
  } else {
    if (four) launch_waves<Ops, 128, 4>(a, stream);
    else launch_waves<Ops, 128, 2>(a, stream);
  }
}

void launch_splitmm_part(const RowAttnArgs& a, int kv_dtype, int D, hipStream_t stream) {
  if (kv_dtype == HS_DTYPE_F16) launch_for<F16Ops>(a, D, stream);
  else launch_for<Bf16Ops>(a, D, stream);
}

// ---------------------------------------------------------------------------
// even split: host side
// ---------------------------------------------------------------------------

// The even split serves groups of at most 4 query heads per KV head (one
// 4-wave workgroup per unit, hi and lo terms as MFMA columns) on grids whose
// fixed partitions would take more than one round of the device.  Measured
// on MI355X against fixed partitions (whole call, us): C2-gqa 109 / 113, 300
// sequences of 16..3000 tokens 328 / 378, 64 x 4096 tokens 177 / 189, C2
// contexts at head dim 64 (fp16) 66 / 69.  It lost with 8 query heads per KV
// head (C2 contexts, 4 KV heads: 74 / 69 at 16-page ranges, 70 / 69 at 32)
// and where the partitions fit one round (64 rows of 100..700 tokens, one
// 768-token partition each: 31.8 / 24.0; 8 rows of 1-4k tokens: 25.5 /
// 24.8): there the merge launch costs more than the last round's idle slots.
constexpr int kEvenMaxGroup = 4;
constexpr int kEvenWaves = 4;
// Workgroups of the device's occupancy per CU taken by the grid: filled once
// (C2-gqa: 109 us; twice 114, three times 116), and the least pages of a
// range (16: 4 a wave; 32 measured the same on C2-gqa).
constexpr int kEvenRounds = 1;
constexpr int kEvenMinPages = 16;

template <typename Ops>
static const void* even_kernel_t(int D) {
  if (D == 32) return (const void*)splitmm_even_kernel<Ops, 32, true, kEvenWaves>;
  if (D == 64) return (const void*)splitmm_even_kernel<Ops, 64, true, kEvenWaves>;
  return (const void*)splitmm_even_kernel<Ops, 128, true, kEvenWaves>;
}

static const void* even_kernel(int kv_dtype, int D) {
  return kv_dtype == HS_DTYPE_F16 ? even_kernel_t<F16Ops>(D) : even_kernel_t<Bf16Ops>(D);
}

int splitmm_even_min_pages() { return kEvenMinPages; }

// Plain multi-head attention (H == Hkv) on 16-bit caches with 16-token
// pages: the VALU even split, against the VALU kernel's fixed 512-token
// partitions.
constexpr int kValuFixedPartition = 512;

static bool even_valu_serves(int kv_dtype, int D, int H, int Hkv) {
  return H == Hkv && (kv_dtype == HS_DTYPE_BF16 || kv_dtype == HS_DTYPE_F16) &&
         (D == 32 || D == 64 || D == 128 || D == 256);
}

template <typename T>
static const void* even_valu_kernel_t(int D) {
  if (D == 32) return (const void*)row_attn_even_kernel<T, 32>;
  if (D == 64) return (const void*)row_attn_even_kernel<T, 64>;
  if (D == 128) return (const void*)row_attn_even_kernel<T, 128>;
  return (const void*)row_attn_even_kernel<T, 256>;
}

static const void* even_valu_kernel(int kv_dtype, int D) {
  return kv_dtype == HS_DTYPE_F16 ? even_valu_kernel_t<_Float16>(D) : even_valu_kernel_t<Bf16>(D);
}

// Resident workgroups of the kernel per CU and the CU count, on the current
// device; looked up once per (device, kernel).
static void even_occupancy(const void* fn, int block, int* occ, int* cus) {
  static std::mutex mu;
  static std::map<std::pair<int, const void*>, std::pair<int, int>> cache;
  int dev = 0;
  *occ = 0;
  *cus = 0;
  if (hipGetDevice(&dev) != hipSuccess) return;
  std::lock_guard<std::mutex> lock(mu);
  auto it = cache.find({dev, fn});
  if (it == cache.end()) {
    int n = 0, c = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fn, block, 0) != hipSuccess) n = 0;
    if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) c = 0;
    it = cache.emplace(std::make_pair(dev, fn), std::make_pair(n, c)).first;
  }
  *occ = it->second.first;
  *cus = it->second.second;
}

// M, the workgroups per unit: the device's resident workgroups (kEvenRounds
// times over) split between the units.  0 when the even split does not
// serve the call: more than kEvenMaxGroup query heads per KV head, or fixed
// default partitions that fit one round (B rows of the table's width, a
// bound on the real count, at most M partitions per unit).
int splitmm_even_groups(int kv_dtype, int D, int H, int Hkv, int B, int MB) {
  const int G = H / Hkv;
  int occ = 0, cus = 0;
  int64_t groups, part;   // workgroups sharing a range; the fixed plan's partition
  if (even_valu_serves(kv_dtype, D, H, Hkv)) {
    even_occupancy(even_valu_kernel(kv_dtype, D), 64 * kEvenValuWaves, &occ, &cus);
    groups = ceil_div(H, kEvenValuWaves);
    part = kValuFixedPartition;
  } else if (splitmm_serves(kv_dtype, kPage, D, H, Hkv) && G <= kEvenMaxGroup) {
    even_occupancy(even_kernel(kv_dtype, D), 64 * kEvenWaves, &occ, &cus);
    groups = Hkv;
    part = splitmm_default_partition(G, D);
  } else {
    return 0;
  }
  if (occ <= 0 || cus <= 0) return 0;
  const int64_t fill = ceil_div((int64_t)cus * occ * kEvenRounds, groups);
  const int64_t parts = sat_mul(B, ceil_div((int64_t)MB * kPage, part));
  if (parts <= fill) return 0;
  return (int)std::min<int64_t>(fill, 1 << 20);
}

EvenLayout splitmm_even_layout(int B, int H, int Hkv, int D, int M) {
  const int G = H / Hkv;
  const int64_t n_units = (int64_t)Hkv * ceil_div(G, kSlots);
  const int64_t states = sat_mul(n_units, sat_add(M, B), std::min(G, kSlots));
  EvenLayout l;
  l.acc = 0;
  l.ml = sat_add(sat_mul(states, D, (int64_t)sizeof(float)), 255) & ~(int64_t)255;
  l.end = sat_add(l.ml, sat_mul(states, 2 * (int64_t)sizeof(float)));
  if (l.end >= INT64_MAX - 255) l.end = INT64_MAX;
  return l;
}

template <typename Ops>
static void launch_even_for(const RowAttnArgs& a, int D, hipStream_t stream) {
  const dim3 grid((unsigned)((int64_t)a.Hkv * a.even_m)), block(64 * kEvenWaves);
  if (D == 32)
    hipLaunchKernelGGL((splitmm_even_kernel<Ops, 32, true, kEvenWaves>), grid, block, 0, stream, a);
  else if (D == 64)
    hipLaunchKernelGGL((splitmm_even_kernel<Ops, 64, true, kEvenWaves>), grid, block, 0, stream, a);
  else
    hipLaunchKernelGGL((splitmm_even_kernel<Ops, 128, true, kEvenWaves>), grid, block, 0, stream,
                       a);
}

// The even-split kernel, then the merge of the rows it cut (which also
// zeroes rows without keys).  Needs a.rows == a.B (one query row per
// sequence) and a.H / a.Hkv <= kEvenMaxGroup.
template <typename T>
static void launch_even_valu_for(const RowAttnArgs& a, int D, hipStream_t stream) {
  const dim3 grid((unsigned)(ceil_div(a.H, kEvenValuWaves) * (int64_t)a.even_m)),
      block(64 * kEvenValuWaves);
  if (D == 32) hipLaunchKernelGGL((row_attn_even_kernel<T, 32>), grid, block, 0, stream, a);
  else if (D == 64) hipLaunchKernelGGL((row_attn_even_kernel<T, 64>), grid, block, 0, stream, a);
  else if (D == 128) hipLaunchKernelGGL((row_attn_even_kernel<T, 128>), grid, block, 0, stream, a);
  else hipLaunchKernelGGL((row_attn_even_kernel<T, 256>), grid, block, 0, stream, a);
}

void launch_splitmm_even(const RowAttnArgs& a, int kv_dtype, int D, hipStream_t stream) {
  profile_begin(stream);
  if (even_valu_serves(kv_dtype, D, a.H, a.Hkv)) {
    if (kv_dtype == HS_DTYPE_F16) launch_even_valu_for<_Float16>(a, D, stream);
    else launch_even_valu_for<Bf16>(a, D, stream);
  } else if (kv_dtype == HS_DTYPE_F16) {
    launch_even_for<F16Ops>(a, D, stream);
  } else {
    launch_even_for<Bf16Ops>(a, D, stream);
  }
  profile_end(stream);
  const dim3 grid((unsigned)(((int64_t)a.B * a.H + 3) / 4)), block(256);
  if (D == 32) hipLaunchKernelGGL(even_merge_kernel<32>, grid, block, 0, stream, a);
  else if (D == 64) hipLaunchKernelGGL(even_merge_kernel<64>, grid, block, 0, stream, a);
  else if (D == 128) hipLaunchKernelGGL(even_merge_kernel<128>, grid, block, 0, stream, a);
  else hipLaunchKernelGGL(even_merge_kernel<256>, grid, block, 0, stream, a);
}

}  // namespace hs
