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
// 16-token pages), staging each K/V tile in LDS once for all four waves.
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
constexpr int kRowsPerWave = 32;
constexpr int kBM = kWaves * kRowsPerWave;  // query rows per workgroup
constexpr int kBN = 64;                     // keys per tile
constexpr int kThreads = kWaves * 64;
constexpr int kXcds = 8;
constexpr int kKPad = 8;                    // halves of padding per LDS K row
constexpr int kVPad = 8;                    // halves of padding per LDS V^T row
constexpr float kRescaleSlack = 8.0f;       // log2 units

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
struct PrefillLds {
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

// 8 KV elements (16 bytes) -> 8 fp16 (16 bytes).
template <typename T>
__device__ inline uint4 to_f16x8(const uint4& w);

template <>
__device__ inline uint4 to_f16x8<_Float16>(const uint4& w) {
  return w;
}

template <>
__device__ inline uint4 to_f16x8<Bf16>(const uint4& w) {
  float f[8];
  Elem<Bf16>::to_f32(w, f);
  return make_uint4(pack_f16(f[0], f[1]), pack_f16(f[2], f[3]), pack_f16(f[4], f[5]),
                    pack_f16(f[6], f[7]));
}

// Element e (0..7) of 8 packed 16-bit values, widened to fp32.
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

// Per-thread share of one K/V tile: kChunks 16-byte pieces of K and of V.
template <int D>
struct TileRegs {
  static constexpr int kChunks = kBN * D / 8 / kThreads;  // D=128: 4
  uint4 k[kChunks];
  uint4 v[kChunks];
};

// Global -> registers for tile kt.  K: chunk c = tid + 256*u covers key
// c / (D/8), dims 8*(c % (D/8)), so 16 neighbouring lanes read one 256-byte
// head row.  V: piece p = tid + 256*u covers key 4*((p/4) % 16) + p % 4 and
// dims 8*(p / 64), so the lanes of a wave hold consecutive keys of the same
// 8 dims and the transposed LDS stores below are contiguous.
template <typename T, int D>
__device__ inline void load_tile(const PrefillArgs& a, TileRegs<D>& r, const int32_t* bt,
                                 int kvh, int kt) {
  constexpr int kDC = D / 8;                     // 16-byte chunks per row
  const int tid = threadIdx.x;
  const int64_t tok = (int64_t)a.Hkv * D;
  const int64_t blk = tok * 16;
  const T* kb = reinterpret_cast<const T*>(a.k) + kvh * D;
  const T* vb = reinterpret_cast<const T*>(a.v) + kvh * D;
#pragma unroll
  for (int u = 0; u < TileRegs<D>::kChunks; ++u) {
    const int c = tid + kThreads * u;
    const int key = c / kDC;
    const int page = min(kt * 4 + key / 16, a.MB - 1);
    const int64_t off = safe_block(bt[page], a.NB) * blk + (key % 16) * tok + (c % kDC) * 8;
    r.k[u] = load16(kb + off);
  }
  // V: 64 keys x kDC chunks = kThreads * kChunks pieces; thread -> (quad, dchunk)
  constexpr int kQuads = kBN / 4;                // 16 key quads per tile
#pragma unroll
  for (int u = 0; u < TileRegs<D>::kChunks; ++u) {
    const int piece = tid + kThreads * u;        // piece -> (dchunk, quad, i)
    const int i = piece & 3;                     // key within the quad
    const int quad = (piece >> 2) % kQuads;
    const int dc = (piece >> 2) / kQuads;
    const int key = quad * 4 + i;
    const int page = min(kt * 4 + key / 16, a.MB - 1);
    const int64_t off = safe_block(bt[page], a.NB) * blk + (key % 16) * tok + dc * 8;
    r.v[u] = load16(vb + off);
  }
}

// Registers -> LDS (fp16; K with the bit-2/3 row swap, V transposed).
template <typename T, int D>
__device__ inline void store_tile(PrefillLds<D>& s, const TileRegs<D>& r) {
  constexpr int kDC = D / 8;
  constexpr int kQuads = kBN / 4;
  const int tid = threadIdx.x;
#pragma unroll
  for (int u = 0; u < TileRegs<D>::kChunks; ++u) {
    const int c = tid + kThreads * u;
    const int key = c / kDC;
    const int row = (key & ~31) | swap_bits23(key & 31);
    *reinterpret_cast<uint4*>(&s.k[row][(c % kDC) * 8]) = to_f16x8<T>(r.k[u]);
  }
  // V^T: the 64 lanes of a wave hold 64 consecutive keys of one dchunk, so
  // each 2-byte store instruction writes 128 contiguous bytes of a V^T row.
#pragma unroll
  for (int u = 0; u < TileRegs<D>::kChunks; ++u) {
    const int piece = tid + kThreads * u;
    const int i = piece & 3;
    const int quad = (piece >> 2) % kQuads;
    const int dc = (piece >> 2) / kQuads;
    const int key = quad * 4 + i;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x = elem_f32<T>(r.v[u], e);
      s.vt[dc * 8 + e][key] = (_Float16)x;
    }
  }
}

template <typename T, int D>
__global__ __launch_bounds__(kThreads) void prefill_mfma_kernel(PrefillArgs a) {
  constexpr int kDC16 = D / 16;   // 16-dim chunks (QK MFMA k-steps)
  constexpr int kDB = D / 32;     // 32-dim output blocks
  __shared__ PrefillLds<D> lds;

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
  const int ctx = a.ctx[b];
  const int base_pos = ctx - S_b;   // position of row 0 of the chunk
  const int32_t* bt = a.bt + (int64_t)b * a.MB;

  // Key limit of this lane's query (inclusive), -1 when the row is padding.
  const int i_row = qt * kBM + wave * kRowsPerWave + j;
  const bool row_ok = i_row < S_b;
  const int lim = row_ok ? min(base_pos + i_row, cap - 1) : -1;

  // Keys the workgroup needs and the per-wave bounds.
  const int last_row = min(qt * kBM + kBM, S_b) - 1;
  const int kend = min(cap, base_pos + last_row + 1);
  const int w_first = qt * kBM + wave * kRowsPerWave;
  const int w_last = min(w_first + kRowsPerWave, S_b) - 1;
  const int w_lim_min = min(base_pos + w_first, cap - 1);
  const int w_lim_max = w_first < S_b ? min(base_pos + w_last, cap - 1) : -1;

  // ---- Q^T fragments: lane (j, hh) holds q[row][16c + 8hh .. +7] ---------
  half8 qf[kDC16];
  {
    const float* qp = a.q + ((int64_t)(row0 + min(i_row, S_b - 1)) * a.H + h) * D + 8 * hh;
#pragma unroll
    for (int c = 0; c < kDC16; ++c) {
      float4 x0 = make_float4(0.f, 0.f, 0.f, 0.f), x1 = x0;
      if (row_ok) {
        x0 = *reinterpret_cast<const float4*>(qp + 16 * c);
        x1 = *reinterpret_cast<const float4*>(qp + 16 * c + 4);
      }
      const float s = a.qscale;
      qf[c] = __builtin_bit_cast(
          half8, make_uint4(pack_f16(x0.x * s, x0.y * s), pack_f16(x0.z * s, x0.w * s),
                            pack_f16(x1.x * s, x1.y * s), pack_f16(x1.z * s, x1.w * s)));
    }
  }

  float16x o[kDB];
#pragma unroll
  for (int d = 0; d < kDB; ++d)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[d][r] = 0.0f;
  float m = kNegBig;   // running max (shared by the lane pair j, j + 32)
  float l = 0.0f;      // this lane's share of the running sum

  const int n_kt = kend > 0 ? (kend + kBN - 1) / kBN : 0;
  TileRegs<D> regs;
  if (n_kt > 0) load_tile<T, D>(a, regs, bt, kvh, 0);

  for (int kt = 0; kt < n_kt; ++kt) {
    __syncthreads();                      // previous tile fully consumed
    store_tile<T, D>(lds, regs);
    __syncthreads();
    if (kt + 1 < n_kt) load_tile<T, D>(a, regs, bt, kvh, kt + 1);

    const int k0 = kt * kBN;
    if (k0 > w_lim_max) continue;         // every key past this wave's rows

    // ---- S^T = K . Q^T, two 32-key blocks ----
    float16x s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) s[kb][r] = 0.0f;
#pragma unroll
      for (int c = 0; c < kDC16; ++c) {
        const half8 ka = *reinterpret_cast<const half8*>(&lds.k[kb * 32 + j][16 * c + 8 * hh]);
        s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, qf[c], s[kb], 0, 0, 0);
      }
    }

    // ---- mask (only tiles that reach past some row's limit) ----
    if (k0 + kBN - 1 > w_lim_min) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = k0 + kb * 32 + 16 * (r >> 3) + 8 * hh + (r & 7);
          if (key > lim) s[kb][r] = kNegBig;
        }
    }

    // ---- online softmax ----
    float mx = kNegBig;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kb][r]);
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const bool raise = mx > m + kRescaleSlack;
    if (__builtin_amdgcn_ballot_w64(raise) != 0) {   // wave-uniform decision
      const float m_new = fmaxf(m, mx);
      const float corr = fast_exp2(m - m_new);
      l *= corr;
#pragma unroll
      for (int d = 0; d < kDB; ++d)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[d][r] *= corr;
      m = m_new;
    }
    half8 p[4];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      float pf[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        pf[r] = s[kb][r] > kNegBig ? fast_exp2(s[kb][r] - m) : 0.0f;
        l += pf[r];
      }
#pragma unroll
      for (int half = 0; half < 2; ++half)
        p[kb * 2 + half] = __builtin_bit_cast(
            half8, make_uint4(pack_f16(pf[8 * half + 0], pf[8 * half + 1]),
                              pack_f16(pf[8 * half + 2], pf[8 * half + 3]),
                              pack_f16(pf[8 * half + 4], pf[8 * half + 5]),
                              pack_f16(pf[8 * half + 6], pf[8 * half + 7])));
    }

    // ---- O^T += V^T . P^T over four 16-key chunks ----
#pragma unroll
    for (int kc = 0; kc < 4; ++kc) {
#pragma unroll
      for (int d = 0; d < kDB; ++d) {
        const half8 va = *reinterpret_cast<const half8*>(&lds.vt[d * 32 + j][kc * 16 + 8 * hh]);
        o[d] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, p[kc], o[d], 0, 0, 0);
      }
    }
  }

  // ---- normalise and store: lane (j, hh) owns query j, dims
  // d*32 + 8*(r/4) + 4*hh + r%4 ----
  if (!row_ok) return;
  const float lsum = l + __shfl_xor(l, 32);
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
