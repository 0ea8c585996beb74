// Causal chunked prefill over the paged KV cache on gfx950 matrix cores.
//
// Reference: prefill_wmma_kernel, heteroserve/model/paged_attn_wmma.py:80-254
// (a FlashAttention loop over 16-token pages with an online softmax), and the
// semantics of paged_attention_prefill_torch, paged_attn_prefill.py:281-322:
// query i of a chunk of S_b rows sits at position ctx_b - S_b + i and attends
// to keys [0, that position]; rows at negative positions are zero.
//
// Work decomposition.  A workgroup owns 128 query rows (4 waves x 32 rows) of
// one (sequence, head) and walks that head's keys in tiles of 64 (four
// 16-token pages), staging each K/V tile in LDS once for all four waves.  The
// LDS tiles are double-buffered with one barrier per tile, and the next
// tile's global loads are in flight while the current one is consumed.  The
// kernel is held to two waves per SIMD (<= 256 registers), so one wave's
// softmax overlaps the other's MFMAs; measured on C4 this beat 64 rows per
// wave at one wave per SIMD by 1.8x, even though each LDS fragment then feeds
// one MFMA instead of two.
// Scores are computed transposed, S^T = K . Q^T, with v_mfma_f32_32x32x16_f16:
// K rows are the A operand (read from LDS), Q^T the B operand (held in
// registers for the whole walk).  The accumulator then has one query per
// lane and 16 keys per lane in registers, which is exactly the layout of the
// B operand of O^T = V^T . P^T, so the probabilities P go from the softmax to
// the second MFMA without leaving registers; V^T (A operand) comes from a
// transposed copy of the V tile in LDS.  O^T accumulates one query per lane,
// so the online-softmax rescale is a per-lane scalar multiply.
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

namespace hs {

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2x __attribute__((ext_vector_type(2)));
typedef float float16x __attribute__((ext_vector_type(16)));
typedef float float2x __attribute__((ext_vector_type(2)));

constexpr int kWaves = 4;
constexpr int kMTiles = 1;                   // 32-row MFMA tiles per wave
constexpr int kRowsPerWave = 32 * kMTiles;
constexpr int kBM = kWaves * kRowsPerWave;   // query rows per workgroup
constexpr int kBN = 64;                      // keys per LDS tile (four pages)
constexpr int kThreads = kWaves * 64;
constexpr int kXcds = 8;
constexpr int kKPad = 8;                     // halves of padding per LDS K row
constexpr int kVPad = 8;                     // halves of padding per LDS V^T row
constexpr float kRescaleSlack = 8.0f;        // log2 units

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
  float qscale;          // scale * log2(e)
};

template <int D>
struct PrefillTileLds {
  _Float16 k[kBN][D + kKPad];       // K tile, row r holds key swap23(r)
  _Float16 vt[D][kBN + kVPad];      // V tile transposed
};

__device__ inline int swap_bits23(int r) {
  return (r & ~12) | ((r & 4) << 1) | ((r & 8) >> 1);
}

__device__ inline uint32_t pack_f16(float a, float b) {
  const half2x h = __builtin_convertvector((float2x){a, b}, half2x);  // v_cvt_pk_f16_f32, RNE
  return __builtin_bit_cast(uint32_t, h);
}

// Element e (0..7) of 8 packed 16-bit KV values, widened to fp32 (exact).
template <typename T>
__device__ inline float elem_f32(const uint4& w, int e);

template <>
__device__ inline float elem_f32<Bf16>(const uint4& w, int e) {
  const uint32_t d = e < 2 ? w.x : e < 4 ? w.y : e < 6 ? w.z : w.w;
  return __uint_as_float((e & 1) ? (d & 0xffff0000u) : (d << 16));
}

template <>
__device__ inline float elem_f32<_Float16>(const uint4& w, int e) {
  const uint32_t d = e < 2 ? w.x : e < 4 ? w.y : e < 6 ? w.z : w.w;
  const half2x h = __builtin_bit_cast(half2x, d);
  return (float)h[e & 1];
}

// 8 KV elements -> 8 fp16.
template <typename T>
__device__ inline uint4 to_f16x8(const uint4& w) {
  return make_uint4(pack_f16(elem_f32<T>(w, 0), elem_f32<T>(w, 1)),
                    pack_f16(elem_f32<T>(w, 2), elem_f32<T>(w, 3)),
                    pack_f16(elem_f32<T>(w, 4), elem_f32<T>(w, 5)),
                    pack_f16(elem_f32<T>(w, 6), elem_f32<T>(w, 7)));
}

template <>
__device__ inline uint4 to_f16x8<_Float16>(const uint4& w) {
  return w;
}

// One thread's share of a K/V tile in flight from global memory.
//   K: chunk c = tid + 256*u is key c / (D/8), dims 8*(c % (D/8)): 16
//      neighbouring lanes read one 256-byte head row.
//   V: the thread owns kG consecutive keys kG*(tid % (64/kG)) of the 8 dims
//      8*(tid / (64/kG)), so that its transposed LDS store for one dim is one
//      kG*2-byte write and 64/kG neighbouring lanes fill one V^T row segment.
template <int D>
struct TileRegs {
  static constexpr int kKChunks = kBN * D / 8 / kThreads;  // D=128: 4
  static constexpr int kG = kKChunks;                      // keys per thread in V
  uint4 k[kKChunks];
  uint4 v[kG];
};

template <typename T, int D>
__device__ inline void load_tile(const PrefillArgs& a, TileRegs<D>& r, const int32_t* bt,
                                 int kvh, int kt) {
  constexpr int kDC = D / 8;
  constexpr int kG = TileRegs<D>::kG;
  constexpr int kGroups = kBN / kG;
  const int tid = threadIdx.x;
  const int64_t tok = (int64_t)a.Hkv * D;
  const int64_t blk = tok * 16;
  const T* kb = reinterpret_cast<const T*>(a.k) + kvh * D;
  const T* vb = reinterpret_cast<const T*>(a.v) + kvh * D;
#pragma unroll
  for (int u = 0; u < TileRegs<D>::kKChunks; ++u) {
    const int c = tid + kThreads * u;
    const int key = c / kDC;
    const int page = min(kt * 4 + key / 16, a.MB - 1);
    const int64_t off = safe_block(bt[page], a.NB) * blk + (key % 16) * tok + (c % kDC) * 8;
    r.k[u] = load16(kb + off);
  }
  const int key0 = kG * (tid % kGroups);
  const int dc = tid / kGroups;
#pragma unroll
  for (int g = 0; g < kG; ++g) {
    const int key = key0 + g;
    const int page = min(kt * 4 + key / 16, a.MB - 1);
    const int64_t off = safe_block(bt[page], a.NB) * blk + (key % 16) * tok + dc * 8;
    r.v[g] = load16(vb + off);
  }
}

template <typename T, int D>
__device__ inline void store_tile(PrefillTileLds<D>& s, const TileRegs<D>& r) {
  constexpr int kDC = D / 8;
  constexpr int kG = TileRegs<D>::kG;
  constexpr int kGroups = kBN / kG;
  const int tid = threadIdx.x;
#pragma unroll
  for (int u = 0; u < TileRegs<D>::kKChunks; ++u) {
    const int c = tid + kThreads * u;
    const int key = c / kDC;
    const int row = (key & ~31) | swap_bits23(key & 31);
    *reinterpret_cast<uint4*>(&s.k[row][(c % kDC) * 8]) = to_f16x8<T>(r.k[u]);
  }
  const int key0 = kG * (tid % kGroups);
  const int dc = tid / kGroups;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    _Float16* dst = &s.vt[dc * 8 + e][key0];
    if constexpr (kG == 4) {
      *reinterpret_cast<uint2*>(dst) =
          make_uint2(pack_f16(elem_f32<T>(r.v[0], e), elem_f32<T>(r.v[1], e)),
                     pack_f16(elem_f32<T>(r.v[2], e), elem_f32<T>(r.v[3], e)));
    } else if constexpr (kG == 2) {
      *reinterpret_cast<uint32_t*>(dst) = pack_f16(elem_f32<T>(r.v[0], e), elem_f32<T>(r.v[1], e));
    } else {
      *dst = (_Float16)elem_f32<T>(r.v[0], e);
    }
  }
}

template <typename T, int D>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2)))
void prefill_mfma_kernel(PrefillArgs a) {
  constexpr int kDC16 = D / 16;   // 16-dim chunks (QK MFMA k-steps)
  constexpr int kDB = D / 32;     // 32-dim output blocks
  __shared__ PrefillTileLds<D> lds[2];

  // ---- which (sequence, head, query tile) -------------------------------
  const int xcd = blockIdx.x % kXcds;
  const int slot = blockIdx.x / kXcds;
  const int pair = (slot / a.n_qt) * kXcds + xcd;     // (b * H + h)
  if (pair >= a.B * a.H) return;
  const int qt = a.n_qt - 1 - slot % a.n_qt;          // heaviest tile first
  const int b = pair / a.H;
  const int h = pair - b * a.H;
  int row0, S_b;
  if (a.cu_q) {
    row0 = a.cu_q[b];
    S_b = a.cu_q[b + 1] - row0;
  } else {
    row0 = b * a.S;
    S_b = a.S;
  }
  if (qt * kBM >= S_b) return;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int j = lane & 31;          // query of this lane within a 32-row tile
  const int hh = lane >> 5;         // lane half
  const int kvh = h / (a.H / a.Hkv);
  const int cap = a.MB * 16;        // keys the block table can address
  const int base_pos = a.ctx[b] - S_b;   // position of row 0 of the chunk
  const int32_t* bt = a.bt + (int64_t)b * a.MB;

  // Rows of this lane (one per M tile) and their inclusive key limits (-1 =
  // padding row that attends to nothing).
  const int w_first = qt * kBM + wave * kRowsPerWave;
  int i_row[kMTiles], lim[kMTiles];
#pragma unroll
  for (int mt = 0; mt < kMTiles; ++mt) {
    i_row[mt] = w_first + 32 * mt + j;
    lim[mt] = i_row[mt] < S_b ? min(base_pos + i_row[mt], cap - 1) : -1;
  }
  const int last_row = min(qt * kBM + kBM, S_b) - 1;
  const int kend = min(cap, base_pos + last_row + 1);           // keys the workgroup needs
  const int w_lim_min = min(base_pos + w_first, cap - 1);       // first row of the wave
  const int w_lim_max = w_first < S_b ? min(base_pos + min(w_first + kRowsPerWave, S_b) - 1,
                                            cap - 1)
                                      : -1;

  // ---- Q^T fragments: lane (j, hh) holds q[row][16c + 8hh .. +7] ---------
  half8 qf[kMTiles][kDC16];
#pragma unroll
  for (int mt = 0; mt < kMTiles; ++mt) {
    const bool ok = i_row[mt] < S_b;
    const float* qp =
        a.q + ((int64_t)(row0 + min(i_row[mt], S_b - 1)) * a.H + h) * D + 8 * hh;
#pragma unroll
    for (int c = 0; c < kDC16; ++c) {
      float4 x0 = make_float4(0.f, 0.f, 0.f, 0.f), x1 = x0;
      if (ok) {
        x0 = *reinterpret_cast<const float4*>(qp + 16 * c);
        x1 = *reinterpret_cast<const float4*>(qp + 16 * c + 4);
      }
      const float s = a.qscale;
      qf[mt][c] = __builtin_bit_cast(
          half8, make_uint4(pack_f16(x0.x * s, x0.y * s), pack_f16(x0.z * s, x0.w * s),
                            pack_f16(x1.x * s, x1.y * s), pack_f16(x1.z * s, x1.w * s)));
    }
  }

  float16x o[kMTiles][kDB];
#pragma unroll
  for (int mt = 0; mt < kMTiles; ++mt)
#pragma unroll
    for (int d = 0; d < kDB; ++d)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[mt][d][r] = 0.0f;
  float m[kMTiles], l[kMTiles];   // running max (shared by lanes j, j+32), own partial sum
#pragma unroll
  for (int mt = 0; mt < kMTiles; ++mt) {
    m[mt] = kNegBig;
    l[mt] = 0.0f;
  }

  // ---- key tiles: double-buffered LDS, one barrier per tile ---------------
  // Tile kt+1 is written to the idle buffer at the top of iteration kt (its
  // loads were issued during iteration kt-1), then tile kt+2's loads are
  // issued, then tile kt is consumed.
  const int n_kt = kend > 0 ? (kend + kBN - 1) / kBN : 0;
  TileRegs<D> regs;
  if (n_kt > 0) {
    load_tile<T, D>(a, regs, bt, kvh, 0);
    store_tile<T, D>(lds[0], regs);
    if (n_kt > 1) load_tile<T, D>(a, regs, bt, kvh, 1);
    __syncthreads();
  }

  for (int kt = 0; kt < n_kt; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < n_kt) {
      store_tile<T, D>(lds[cur ^ 1], regs);
      if (kt + 2 < n_kt) load_tile<T, D>(a, regs, bt, kvh, kt + 2);
    }
    const PrefillTileLds<D>& t = lds[cur];

#pragma unroll
    for (int kb = 0; kb < kBN / 32; ++kb) {
      const int key0 = kt * kBN + kb * 32;
      if (key0 > w_lim_max) break;          // every key past this wave's rows

      // S^T = K . Q^T for 32 keys x (2 x 32) queries
      float16x s[kMTiles];
#pragma unroll
      for (int mt = 0; mt < kMTiles; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) s[mt][r] = 0.0f;
#pragma unroll
      for (int c = 0; c < kDC16; ++c) {
        const half8 ka = *reinterpret_cast<const half8*>(&t.k[kb * 32 + j][16 * c + 8 * hh]);
#pragma unroll
        for (int mt = 0; mt < kMTiles; ++mt)
          s[mt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, qf[mt][c], s[mt], 0, 0, 0);
      }

      // accumulator register r of half hh holds key key0 + 16*(r/8) + 8*hh + r%8
      if (key0 + 31 > w_lim_min) {
#pragma unroll
        for (int mt = 0; mt < kMTiles; ++mt)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (key0 + 16 * (r >> 3) + 8 * hh + (r & 7) > lim[mt]) s[mt][r] = kNegBig;
      }

      half8 p[kMTiles][2];
#pragma unroll
      for (int mt = 0; mt < kMTiles; ++mt) {
        float mx = kNegBig;
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[mt][r]);
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        if (__builtin_amdgcn_ballot_w64(mx > m[mt] + kRescaleSlack) != 0) {
          const float m_new = fmaxf(m[mt], mx);
          const float corr = fast_exp2(m[mt] - m_new);
          l[mt] *= corr;
#pragma unroll
          for (int d = 0; d < kDB; ++d)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[mt][d][r] *= corr;
          m[mt] = m_new;
        }
        float pf[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          pf[r] = s[mt][r] > kNegBig ? fast_exp2(s[mt][r] - m[mt]) : 0.0f;
          l[mt] += pf[r];
        }
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
          p[mt][hf] = __builtin_bit_cast(
              half8, make_uint4(pack_f16(pf[8 * hf + 0], pf[8 * hf + 1]),
                                pack_f16(pf[8 * hf + 2], pf[8 * hf + 3]),
                                pack_f16(pf[8 * hf + 4], pf[8 * hf + 5]),
                                pack_f16(pf[8 * hf + 6], pf[8 * hf + 7])));
      }

      // O^T += V^T . P^T over the two 16-key chunks of this block
#pragma unroll
      for (int kc = 0; kc < 2; ++kc)
#pragma unroll
        for (int d = 0; d < kDB; ++d) {
          const half8 va =
              *reinterpret_cast<const half8*>(&t.vt[d * 32 + j][kb * 32 + kc * 16 + 8 * hh]);
#pragma unroll
          for (int mt = 0; mt < kMTiles; ++mt)
            o[mt][d] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, p[mt][kc], o[mt][d], 0, 0, 0);
        }
    }
    __syncthreads();   // the idle buffer is complete; this tile is consumed
  }

  // ---- normalise and store: lane (j, hh) owns query j of each M tile and
  // dims d*32 + 8*g + 4*hh + (0..3) ----
#pragma unroll
  for (int mt = 0; mt < kMTiles; ++mt) {
    const float lsum = l[mt] + __shfl_xor(l[mt], 32);
    if (i_row[mt] >= S_b) continue;
    const float inv = lsum > 0.0f ? 1.0f / lsum : 0.0f;
    float* op = a.out + ((int64_t)(row0 + i_row[mt]) * a.H + h) * D + 4 * hh;
#pragma unroll
    for (int d = 0; d < kDB; ++d)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *reinterpret_cast<float4*>(op + d * 32 + 8 * g) =
            make_float4(o[mt][d][4 * g] * inv, o[mt][d][4 * g + 1] * inv,
                        o[mt][d][4 * g + 2] * inv, o[mt][d][4 * g + 3] * inv);
  }
}

template <typename T, int D>
void launch_typed(const PrefillArgs& a, hipStream_t stream) {
  const dim3 grid((unsigned)(kXcds * a.slots_per_xcd)), block(kThreads);
  hipLaunchKernelGGL((prefill_mfma_kernel<T, D>), grid, block, 0, stream, a);
}

template <typename T>
int launch_dim(const PrefillArgs& a, int D, hipStream_t stream) {
  switch (D) {
    case 32: launch_typed<T, 32>(a, stream); break;
    case 64: launch_typed<T, 64>(a, stream); break;
    case 128: launch_typed<T, 128>(a, stream); break;
    default: return fail(HS_EUNSUPPORTED, "unsupported head_dim for the MFMA path: " +
                                              std::to_string(D));
  }
  return HS_OK;
}

}  // namespace

int launch_prefill_mfma(const float* q, const int32_t* cu_q, int S, int max_rows_per_seq,
                        const void* k, const void* v, int kv_dtype, int NB, const int32_t* bt,
                        const int32_t* ctx, float* out, int B, int H, int Hkv, int D, int BS,
                        int MB, float scale, hipStream_t stream) {
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
  a.n_qt = (max_rows_per_seq + kBM - 1) / kBM;
  const int64_t pairs = (int64_t)B * H;
  const int64_t slots = (pairs + kXcds - 1) / kXcds * a.n_qt;
  if (slots * kXcds > 0x7fffffffLL) return fail(HS_EUNSUPPORTED, "prefill grid too large");
  a.slots_per_xcd = (int)slots;
  a.qscale = scale * kLog2e;
  profile_begin(stream);
  int rc;
  if (kv_dtype == HS_DTYPE_F16) rc = launch_dim<_Float16>(a, D, stream);
  else rc = launch_dim<Bf16>(a, D, stream);
  profile_end(stream);
  if (rc != HS_OK) return rc;
  return check_launch("MFMA prefill");
}

}  // namespace hs
