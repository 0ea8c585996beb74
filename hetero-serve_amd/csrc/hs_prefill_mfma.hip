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
// one MFMA instead of two.  Two 64-key tiles take 70 KiB of LDS, so two
// workgroups share a CU and one's pipeline fill overlaps the other's compute
// (measured: 8-wave workgroups with 128-key tiles, one per CU, were 20-30%
// slower on every prefill shape tried).
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

namespace hs {

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2x __attribute__((ext_vector_type(2)));
typedef float float16x __attribute__((ext_vector_type(16)));
typedef float float2x __attribute__((ext_vector_type(2)));

constexpr int kWaves = 4;
constexpr int kRowsPerWave = 32;             // one 32-row MFMA tile per wave
constexpr int kBM = kWaves * kRowsPerWave;   // query rows per workgroup
constexpr int kBN = 64;                      // keys per LDS tile (four pages), a multiple of 32
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
  static_assert(kKChunks >= 1 && (kG == 1 || kG == 2 || kG == 4), "tile / thread split");
  static constexpr int kChunksPerBlock = (kKChunks + kBN / 32 - 1) / (kBN / 32);
  uint4 k[kKChunks];
  uint4 v[kG];
};

// Block ids of the pages a thread's loads of tile kt touch, fetched one tile
// ahead of the loads themselves so that the block-table round trip never
// sits in front of the K/V loads.
template <int D>
struct TileIds {
  int k[TileRegs<D>::kKChunks];
  int v[TileRegs<D>::kG];
};

template <int D>
__device__ inline void tile_ids(const PrefillArgs& a, TileIds<D>& ids, const int32_t* bt, int kt) {
  constexpr int kDC = D / 8;
  constexpr int kG = TileRegs<D>::kG;
  constexpr int kGroups = kBN / kG;
  const int tid = threadIdx.x;
#pragma unroll
  for (int u = 0; u < TileRegs<D>::kKChunks; ++u) {
    const int key = (tid + kThreads * u) / kDC;
    ids.k[u] = bt[min(kt * (kBN / 16) + key / 16, a.MB - 1)];
  }
#pragma unroll
  for (int g = 0; g < kG; ++g) {
    const int key = kG * (tid % kGroups) + g;
    ids.v[g] = bt[min(kt * (kBN / 16) + key / 16, a.MB - 1)];
  }
}

template <typename T, int D>
__device__ inline void load_k_chunk(const PrefillArgs& a, TileRegs<D>& r, const TileIds<D>& ids,
                                    int kvh, int u) {
  constexpr int kDC = D / 8;
  const int c = threadIdx.x + kThreads * u;
  const int key = c / kDC;
  const int64_t tok = (int64_t)a.Hkv * D;
  const int64_t off = safe_block(ids.k[u], a.NB) * tok * 16 + (key % 16) * tok + kvh * D +
                      (c % kDC) * 8;
  r.k[u] = load16(reinterpret_cast<const T*>(a.k) + off);
}

template <typename T, int D>
__device__ inline void load_v(const PrefillArgs& a, TileRegs<D>& r, const TileIds<D>& ids,
                              int kvh) {
  constexpr int kG = TileRegs<D>::kG;
  constexpr int kGroups = kBN / kG;
  const int key0 = kG * (threadIdx.x % kGroups);
  const int dc = threadIdx.x / kGroups;
  const int64_t tok = (int64_t)a.Hkv * D;
#pragma unroll
  for (int g = 0; g < kG; ++g) {
    const int key = key0 + g;
    const int64_t off = safe_block(ids.v[g], a.NB) * tok * 16 + (key % 16) * tok + kvh * D +
                        dc * 8;
    r.v[g] = load16(reinterpret_cast<const T*>(a.v) + off);
  }
}

template <typename T, int D>
__device__ inline void load_tile(const PrefillArgs& a, TileRegs<D>& r, const TileIds<D>& ids,
                                 int kvh) {
#pragma unroll
  for (int u = 0; u < TileRegs<D>::kKChunks; ++u) load_k_chunk<T, D>(a, r, ids, kvh, u);
  load_v<T, D>(a, r, ids, kvh);
}

// Registers -> LDS (fp16; K with the bit-2/3 row swap, V transposed).
template <typename T, int D>
__device__ inline void store_k_chunk(PrefillTileLds<D>& s, const TileRegs<D>& r, int u) {
  constexpr int kDC = D / 8;
  const int c = threadIdx.x + kThreads * u;
  const int key = c / kDC;
  const int row = (key & ~31) | swap_bits23(key & 31);
  *reinterpret_cast<uint4*>(&s.k[row][(c % kDC) * 8]) = to_f16x8<T>(r.k[u]);
}

// V^T: the thread owns kG consecutive keys of 8 dims, so each of its 8
// stores (one per dim) is a kG*2-byte write, and the kBN/kG lanes that share
// a dim chunk fill one contiguous V^T row segment.
template <typename T, int D>
__device__ inline void store_v(PrefillTileLds<D>& s, const TileRegs<D>& r) {
  constexpr int kG = TileRegs<D>::kG;
  constexpr int kGroups = kBN / kG;
  const int key0 = kG * (threadIdx.x % kGroups);
  const int dc = threadIdx.x / kGroups;
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
__device__ inline void store_tile(PrefillTileLds<D>& s, const TileRegs<D>& r) {
#pragma unroll
  for (int u = 0; u < TileRegs<D>::kKChunks; ++u) store_k_chunk<T, D>(s, r, u);
  store_v<T, D>(s, r);
}

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

template <typename T, int D>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2)))
void prefill_mfma_kernel(PrefillArgs a) {
  constexpr int kDC16 = D / 16;   // 16-dim chunks (QK MFMA k-steps)
  constexpr int kDB = D / 32;     // 32-dim output blocks
  constexpr int kNKB = kBN / 32;  // 32-key blocks per tile
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
  const int j = lane & 31;          // query of this lane within the wave's 32
  const int hh = lane >> 5;         // lane half
  const int kvh = h / (a.H / a.Hkv);
  const int cap = a.MB * 16;        // keys the block table can address
  const int base_pos = a.ctx[b] - S_b;   // position of row 0 of the chunk
  const int32_t* bt = a.bt + (int64_t)b * a.MB;

  // This lane's query row and its inclusive key limit (-1: padding row).
  const int w_first = qt * kBM + wave * kRowsPerWave;
  const int i_row = w_first + j;
  const bool row_ok = i_row < S_b;
  const int lim = row_ok ? min(base_pos + i_row, cap - 1) : -1;
  const int last_row = min(qt * kBM + kBM, S_b) - 1;
  const int kend = min(cap, base_pos + last_row + 1);           // keys the workgroup needs
  const int w_lim_min = min(base_pos + w_first, cap - 1);       // first row of the wave
  const int w_lim_max = w_first < S_b ? min(base_pos + min(w_first + kRowsPerWave, S_b) - 1,
                                            cap - 1)
                                      : -1;

  // ---- Q^T fragments: lane (j, hh) holds q[row][16c + 8hh .. +7] ---------
  half8 qf[kDC16];
  {
    const float* qp = a.q + ((int64_t)(row0 + min(i_row, S_b - 1)) * a.H + h) * D + 8 * hh;
    const float sc = a.qscale;
#pragma unroll
    for (int c = 0; c < kDC16; ++c) {
      float4 x0 = make_float4(0.f, 0.f, 0.f, 0.f), x1 = x0;
      if (row_ok) {
        x0 = *reinterpret_cast<const float4*>(qp + 16 * c);
        x1 = *reinterpret_cast<const float4*>(qp + 16 * c + 4);
      }
      qf[c] = __builtin_bit_cast(
          half8, make_uint4(pack_f16(x0.x * sc, x0.y * sc), pack_f16(x0.z * sc, x0.w * sc),
                            pack_f16(x1.x * sc, x1.y * sc), pack_f16(x1.z * sc, x1.w * sc)));
    }
  }

  float16x o[kDB];
#pragma unroll
  for (int d = 0; d < kDB; ++d)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[d][r] = 0.0f;
  float m = kNegBig;   // running max (shared by lanes j and j + 32)
  float l = 0.0f;      // this lane's share of the running sum

  // ---- key tiles: double-buffered LDS, one barrier per tile ---------------
  // While tile kt is consumed from one buffer, tile kt+1 (loaded during
  // iteration kt-1) is written into the other, and tile kt+2 is loaded;
  // tile kt+3's block ids are fetched at the end of the tile.
  const int n_kt = kend > 0 ? (kend + kBN - 1) / kBN : 0;
  TileRegs<D> regs;
  TileIds<D> ids;
  if (n_kt > 0) {
    tile_ids<D>(a, ids, bt, 0);
    load_tile<T, D>(a, regs, ids, kvh);
    if (n_kt > 1) tile_ids<D>(a, ids, bt, 1);
    store_tile<T, D>(lds[0], regs);
    if (n_kt > 1) load_tile<T, D>(a, regs, ids, kvh);
    if (n_kt > 2) tile_ids<D>(a, ids, bt, 2);
    __syncthreads();
  }

  for (int kt = 0; kt < n_kt; ++kt) {
    const int cur = kt & 1;
    const bool fill = kt + 1 < n_kt;        // tile kt+1 sits in registers
    const bool fetch = kt + 2 < n_kt;       // tile kt+2's loads go out now
    const PrefillTileLds<D>& t = lds[cur];
    const int tile_key0 = kt * kBN;
    // 32-key blocks of this tile that reach this wave's rows
    const int nkb = w_lim_max < tile_key0 ? 0 : min(kNKB, (w_lim_max - tile_key0) / 32 + 1);

    // Software pipeline: the MFMAs of block kb+1's scores are issued before
    // block kb's softmax, so they run while the VALU works on the softmax.
    float16x s_cur;
    if (nkb > 0) s_cur = qk_block<D>(t, 0, qf, j, hh);

#pragma unroll
    for (int kb = 0; kb < kNKB; ++kb) {
      // Producer share of this block: write part of tile kt+1 into the idle
      // buffer (V at block 0, K chunks spread over the blocks) and re-use the freed
      // registers for the matching loads of tile kt+2, which then have a
      // whole tile of compute to arrive.
      if (fill) {
        if (kb == 0) {
          store_v<T, D>(lds[cur ^ 1], regs);
          if (fetch) load_v<T, D>(a, regs, ids, kvh);
        }
#pragma unroll
        for (int cc = 0; cc < TileRegs<D>::kChunksPerBlock; ++cc) {
          const int u = kb * TileRegs<D>::kChunksPerBlock + cc;
          if (u < TileRegs<D>::kKChunks) {
            store_k_chunk<T, D>(lds[cur ^ 1], regs, u);
            if (fetch) load_k_chunk<T, D>(a, regs, ids, kvh, u);
          }
        }
      }
      if (kb == kNKB - 1 && fetch && kt + 3 < n_kt) tile_ids<D>(a, ids, bt, kt + 3);
      if (kb >= nkb) continue;

      const bool more = kb + 1 < nkb;
      float16x s_next;
      if (more) s_next = qk_block<D>(t, kb + 1, qf, j, hh);

      // V^T fragments of this block, read before the softmax so that their
      // latency hides behind it.
      half8 vf[2][kDB];
#pragma unroll
      for (int kc = 0; kc < 2; ++kc)
#pragma unroll
        for (int d = 0; d < kDB; ++d)
          vf[kc][d] =
              *reinterpret_cast<const half8*>(&t.vt[d * 32 + j][kb * 32 + kc * 16 + 8 * hh]);

      // mask: accumulator register r of half hh holds key key0 + 16*(r/8) + 8*hh + r%8
      const int key0 = tile_key0 + kb * 32;
      if (key0 + 31 > w_lim_min) {
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (key0 + 16 * (r >> 3) + 8 * hh + (r & 7) > lim) s_cur[r] = -INFINITY;
      }

      // online softmax; the max is only raised when it grows by > 8
      float mx = kNegBig;
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s_cur[r]);
      mx = fmaxf(mx, __shfl_xor(mx, 32));
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
          w[i] = pack_f16(fast_exp2(s_cur[8 * hf + 2 * i] - m),
                          fast_exp2(s_cur[8 * hf + 2 * i + 1] - m));
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

      if (more) s_cur = s_next;
    }
    __syncthreads();   // the idle buffer is complete; this tile is consumed
  }

  // ---- normalise and store: lane (j, hh) owns query j and dims
  // d*32 + 8*g + 4*hh + (0..3) ----
  const float lsum = l + __shfl_xor(l, 32);
  if (!row_ok) return;
  const float inv = lsum > 0.0f ? 1.0f / lsum : 0.0f;
  float* op = a.out + ((int64_t)(row0 + i_row) * a.H + h) * D + 4 * hh;
#pragma unroll
  for (int d = 0; d < kDB; ++d)
#pragma unroll
    for (int g = 0; g < 4; ++g)
      *reinterpret_cast<float4*>(op + d * 32 + 8 * g) =
          make_float4(o[d][4 * g] * inv, o[d][4 * g + 1] * inv, o[d][4 * g + 2] * inv,
                      o[d][4 * g + 3] * inv);
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
