// Grouped-query decode on gfx950 matrix cores.
//
// Reference: paged_attn_v2.py:75-157 (one query row per head, KV head
// h / (H / Hkv), online softmax) and paged_attn_v3.py:75-208 (partitions
// merged by log-sum-exp).  When G = H / Hkv query heads share a KV head, the
// per-token work of the VALU kernel (hs_decode.hip) grows with G while the
// bytes read stay the same; here it goes to the matrix cores instead.
//
// One wave serves up to 32 query heads of one KV group for one (row,
// partition) and walks the partition in blocks of 32 tokens:
//   S^T = K . Q^T   v_mfma_f32_32x32x16_f16, K rows (tokens) the A operand,
//                   Q^T (heads) the B operand, held in registers;
//   O^T += V^T . P^T  the accumulator of the first product is already the B
//                   operand layout of the second (lane = head), so P stays in
//                   registers.
// K and V are loaded with 16 lanes per 256-byte token row (loading K straight
// into the operand layout, one token per lane, touched 32 rows per load
// instruction and measured 4x slower per block) and staged through the
// wave's own LDS: K row-major, V transposed.
// Token order: the accumulator gives lane half h the token rows 8g + 4h + m
// in registers 4g + m, while the P.V operand wants registers 0..7 of half h
// to be tokens 8h..8h+7 of a 16-token chunk; the two differ by a swap of bits
// 2 and 3 of the token index, so K's LDS row r holds token swap23(r).
//
// Operands are fp16 (bf16 KV is widened exactly for |x| < 65504; fp32 KV
// keeps the VALU kernel), scores and the softmax state are fp32 in base 2
// (scale * log2(e) folded into q), and the running max is raised lazily (only
// when a block's max exceeds it by more than 8), as in the MFMA prefill.
// The partition states (m, l, un-normalised acc) have the layout and meaning
// of the VALU kernel's, so the same merge kernel combines them.
//
// Used for paged caches with 16-token blocks, fixed partitions of at most
// 1024 tokens, head_dim 32, 64 or 128 and at least 8 query heads per KV
// head (at 4 the VALU kernel's packed heads measured faster: 169 against
// 197 us on C2's geometry with 8 KV heads); every other case runs the VALU
// kernel.  A partition's block ids (at
// most 64 pages) are fetched once by one vector load; every K/V load is
// unconditional (ids clamped to the table, pages past the end masked), so the
// compiler's wait counts stay exact, and the next block's loads are in flight
// while the current block is computed.
#include "hs_kernels.h"
#include "hs_mfma.h"

namespace hs {

namespace {

using namespace mfma;

constexpr int kGqaWaves = 4;        // waves per workgroup: consecutive head units
constexpr int kHeadsPerWave = 32;   // MFMA N dimension
constexpr int kBlock = 32;          // tokens per block
constexpr int kVtPad = 8;           // halves of padding per V^T row
constexpr float kSlack = 8.0f;      // lazy-rescale slack, log2 units

constexpr int kKPad = 8;            // halves of padding per K row

template <int D>
struct GqaWaveLds {
  _Float16 k[kBlock][D + kKPad];    // K of one block, row r holds token swap23(r)
  _Float16 vt[D][kBlock + kVtPad];  // V of one block, transposed
};

template <typename T, int D>
__global__ __launch_bounds__(kGqaWaves * 64) __attribute__((amdgpu_waves_per_eu(2)))
void gqa_mfma_part_kernel(RowAttnArgs a) {
  constexpr int kDC16 = D / 16;     // QK k-steps
  constexpr int kDB = D / 32;       // 32-dim output blocks
  constexpr int kDC = D / 8;        // 16-byte chunks per head row
  constexpr int kTpi = 64 / kDC;    // tokens per wave-wide load (kDC lanes per row)
  constexpr int kLi = kBlock / kTpi;   // loads per block, for K and for V
  constexpr int kG = kLi / 2;       // consecutive V tokens per lane and page
  static_assert(kTpi <= 16 && kG >= 1, "head_dim");
  __shared__ GqaWaveLds<D> lds[kGqaWaves];

  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int j = lane & 31;
  const int hh = lane >> 5;
  const int G = a.H / a.Hkv;
  const int n_hc = (G + kHeadsPerWave - 1) / kHeadsPerWave;   // head chunks per KV head
  const int n_units = a.Hkv * n_hc;
  // Waves are numbered unit-fastest over (row, partition, unit), so the waves
  // of a workgroup read neighbouring KV heads of the same tokens, and take
  // further (row, partition) pairs when a row has fewer than kGqaWaves units.
  const int64_t gw = (int64_t)blockIdx.x * kGqaWaves + wv;
  if (gw >= (int64_t)a.rows * a.P * n_units) return;   // no barriers below
  const int unit = (int)(gw % n_units);
  const int kvh = unit / n_hc;
  const int hc = unit - kvh * n_hc;
  const int h0 = kvh * G + hc * kHeadsPerWave;
  const int gc = min(kHeadsPerWave, G - hc * kHeadsPerWave);   // heads of this wave
  const int64_t rp = gw / n_units;
  const int row = (int)(rp / a.P);
  const int p = (int)(rp - (int64_t)row * a.P);

  int b, end;
  if (!row_geometry(a, row, b, end)) return;
  int lo = 0, hi = 0, nparts = 0;
  const bool live = partition_range(a, end, p, lo, hi, nparts);
  const int64_t orow0 = ((int64_t)row * a.H + h0) * D;
  if (!live) {
    if (end <= 0 && p == 0) {   // nothing to attend to: zero rows
      for (int d = lane; d < gc * D; d += 64) a.out[orow0 + d] = 0.0f;
    }
    return;
  }

  // Block ids of the partition's pages: lane i holds page lo / 16 + i
  // (clamped to the table); 1024 tokens are at most 64 pages.
  const int32_t* bt = a.bt + (int64_t)b * a.MB;
  const int page0 = lo >> 4;
  const int idv = bt[min(page0 + lane, a.MB - 1)];

  // Q^T fragments: lane (j, hh) holds head h0 + j, dims 16c + 8hh .. +7.
  half8 qf[kDC16];
  {
    const float sc = j < gc ? a.qscale : 0.0f;
    const float* qp = a.q + orow0 + (int64_t)min(j, gc - 1) * D + 8 * hh;
#pragma unroll
    for (int c = 0; c < kDC16; ++c) {
      const float4 x0 = *reinterpret_cast<const float4*>(qp + 16 * c);
      const float4 x1 = *reinterpret_cast<const float4*>(qp + 16 * c + 4);
      qf[c] = __builtin_bit_cast(
          half8, make_uint4(pack_f16(x0.x * sc, x0.y * sc), pack_f16(x0.z * sc, x0.w * sc),
                            pack_f16(x1.x * sc, x1.y * sc), pack_f16(x1.z * sc, x1.w * sc)));
    }
  }

  const int64_t tok = (int64_t)a.Hkv * D;           // elements between tokens of a page
  // Loads are coalesced: kDC neighbouring lanes read one token's head row.
  // Lane L holds chunk L % kDC of token slot L / kDC.  K load u covers
  // tokens kTpi*u + slot; V load u of page half ph covers tokens
  // 16*ph + kG*slot + u % kG, so that each lane ends up with kG consecutive
  // tokens of the same 8 dims for its transposed LDS store.  Every load
  // stays inside one 16-token page (wave-uniform block id).
  const int ck = lane % kDC;
  const int slot = lane / kDC;
  const T* kbase = reinterpret_cast<const T*>(a.k) + kvh * D + 8 * ck;
  const T* vbase = reinterpret_cast<const T*>(a.v) + kvh * D + 8 * ck;

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
      const int ph = u / kG;
      const int t = kG * slot + u % kG;                // token in the page
      vr[u] = load16_stream(vbase + ((ph == 0 ? b0 : b1) + t) * tok);
    }
  };
  // Registers -> LDS: K rows in swapped order, V transposed.
  auto store_block = [&](GqaWaveLds<D>& w) {
#pragma unroll
    for (int u = 0; u < kLi; ++u) {
      const int t = kTpi * u + slot;
      *reinterpret_cast<uint4*>(&w.k[swap_bits23(t)][8 * ck]) = to_f16x8<T>(kr[u]);
    }
#pragma unroll
    for (int ph = 0; ph < 2; ++ph)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        _Float16* dst = &w.vt[8 * ck + e][16 * ph + kG * slot];
        const uint4* x = vr + kG * ph;
        if constexpr (kG == 4) {
          *reinterpret_cast<uint2*>(dst) =
              make_uint2(pack_col<T>(x[0], x[1], e), pack_col<T>(x[2], x[3], e));
        } else if constexpr (kG == 2) {
          *reinterpret_cast<uint32_t*>(dst) = pack_col<T>(x[0], x[1], e);
        } else {
          *dst = (_Float16)elem_f32<T>(x[0], e);
        }
      }
  };

  float16x o[kDB];
#pragma unroll
  for (int d = 0; d < kDB; ++d)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[d][r] = 0.0f;
  float m = kNegBig;   // running max of head j (shared by lanes j, j + 32)
  float l = 0.0f;      // this lane's share of the running sum
  GqaWaveLds<D>& w = lds[wv];

  load_block(0);
  for (int t0 = lo; t0 < hi; t0 += kBlock) {
    // this block into LDS, then the next block's loads (in flight while this
    // one is computed); a wave's LDS operations complete in order, so its
    // own reads below see these writes
    store_block(w);
    load_block(((t0 - lo) >> 4) + 2);

    half8 kf[kDC16];
#pragma unroll
    for (int c = 0; c < kDC16; ++c)
      kf[c] = *reinterpret_cast<const half8*>(&w.k[j][16 * c + 8 * hh]);
    float16x s = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[0], qf[0], (float16x)0.0f, 0, 0, 0);
#pragma unroll
    for (int c = 1; c < kDC16; ++c) s = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[c], qf[c], s, 0, 0, 0);
    // register r of half hh holds token t0 + 16 * (r / 8) + 8 * hh + r % 8
    if (t0 + kBlock > hi) {
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (t0 + 16 * (r >> 3) + 8 * hh + (r & 7) >= hi) s[r] = -INFINITY;
    }
    float mx = s[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s[r]);
    mx = max_halves(mx);
    if (__builtin_amdgcn_ballot_w64(mx > m + kSlack) != 0) {
      const float m_new = fmaxf(m, mx);
      const float corr = fast_exp2(m - m_new);
      l *= corr;
#pragma unroll
      for (int d = 0; d < kDB; ++d)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[d][r] *= corr;
      m = m_new;
    }
    half8 pk[2];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      uint32_t w[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        w[i] = pack_f16(fast_exp2(s[8 * hf + 2 * i] - m), fast_exp2(s[8 * hf + 2 * i + 1] - m));
        l = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2x, w[i]),
                                   (half2x){(_Float16)1.0f, (_Float16)1.0f}, l, false);
      }
      pk[hf] = __builtin_bit_cast(half8, make_uint4(w[0], w[1], w[2], w[3]));
    }
#pragma unroll
    for (int kc = 0; kc < 2; ++kc)
#pragma unroll
      for (int d = 0; d < kDB; ++d) {
        const half8 vf =
            *reinterpret_cast<const half8*>(&w.vt[d * 32 + j][kc * 16 + 8 * hh]);
        o[d] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pk[kc], o[d], 0, 0, 0);
      }
  }

  // Partition state of head h0 + j: lane (j, hh) owns dims d*32 + 8g + 4hh + 0..3.
  const float lsum = sum_halves(l);
  if (j >= gc) return;
  if (nparts == 1) {
    const float inv = lsum > 0.0f ? 1.0f / lsum : 0.0f;
    float* op = a.out + orow0 + (int64_t)j * D + 4 * hh;
#pragma unroll
    for (int d = 0; d < kDB; ++d)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *reinterpret_cast<float4*>(op + d * 32 + 8 * g) =
            make_float4(o[d][4 * g] * inv, o[d][4 * g + 1] * inv, o[d][4 * g + 2] * inv,
                        o[d][4 * g + 3] * inv);
  } else {
    const int64_t pi = ((int64_t)row * a.H + h0 + j) * a.P + p;
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

int64_t grid_size(const RowAttnArgs& a) {
  const int G = a.H / a.Hkv;
  const int64_t waves = (int64_t)a.rows * a.P * a.Hkv * ((G + kHeadsPerWave - 1) / kHeadsPerWave);
  return (waves + kGqaWaves - 1) / kGqaWaves;
}

template <typename T, int D>
void launch_typed(const RowAttnArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL((gqa_mfma_part_kernel<T, D>), dim3((unsigned)grid_size(a)),
                     dim3(kGqaWaves * 64), 0, stream, a);
}

}  // namespace

bool gqa_mfma_applies(const RowAttnArgs& a, int kv_dtype, int D) {
  return (kv_dtype == HS_DTYPE_F16 || kv_dtype == HS_DTYPE_BF16) && a.BS == 16 &&
         (D == 32 || D == 64 || D == 128) && a.H / a.Hkv >= 8 && a.mode == 1 &&
         a.part_tokens <= 1024;
}

int64_t gqa_mfma_grid(const RowAttnArgs& a) { return grid_size(a); }

void launch_gqa_mfma_part(const RowAttnArgs& a, int kv_dtype, int D, hipStream_t stream) {
  if (kv_dtype == HS_DTYPE_F16) {
    switch (D) {
      case 32: launch_typed<_Float16, 32>(a, stream); break;
      case 64: launch_typed<_Float16, 64>(a, stream); break;
      default: launch_typed<_Float16, 128>(a, stream); break;
    }
  } else {
    switch (D) {
      case 32: launch_typed<Bf16, 32>(a, stream); break;
      case 64: launch_typed<Bf16, 64>(a, stream); break;
      default: launch_typed<Bf16, 128>(a, stream); break;
    }
  }
}

}  // namespace hs
