// The fp32 key walk of one wave over a paged KV cache: G query heads of one KV
// head attend to keys [lo, hi) of one block-table row with an online softmax.
//
// This is the arithmetic of the VALU decode kernel (hs_decode.hip) and of the
// VALU prefill path.  The matrix-core prefill (hs_prefill_mfma.hip) calls it
// too, as its exact-range fallback: it feeds fp16 operands to the MFMAs, and
// a workgroup whose operands do not fit fp16 is recomputed here from the same
// cache in fp32.  (The matrix-core decodes take split operands of the cache's
// own type and need no fallback.)
//
// Wave layout (gfx950, wave64).  A 16-byte load holds kVec KV elements, so one
// token's head row of D elements is spread over kLpt = D / kVec lanes, and one
// wave-wide load instruction covers kTpl = 64 / kLpt tokens.  For bf16 at
// D = 128 that is 16 lanes per token and 4 tokens per load: a token's dot
// product is reduced inside one 16-lane DPP row, with no LDS traffic.  Each
// group of kLpt lanes ("slot") runs its own online softmax over the tokens it
// loads; the kTpl slot states are merged at the end.  The softmax runs in
// base 2 with scale * log2(e) folded into q.
#pragma once

#include "hs_common.h"

namespace hs {

// The paged cache a walk reads: [NB, BS, Hkv, D] for K and for V.
struct KvPages {
  const void* k;
  const void* v;
  int Hkv, BS, NB;
};

constexpr float kWalkSlack = 8.0f;   // lazy raise of the running max, log2 units

// kPaged: BS % kTpl == 0, so a load group never straddles a page and its
// block id is wave-uniform.
template <typename T, int D, bool kPaged, int G>
struct RowWalk {
  static constexpr int kVec = Elem<T>::kVec;
  static constexpr int kLpt = D / kVec;           // lanes per token
  static constexpr int kTpl = 64 / kLpt;          // tokens per wave-wide load
  static constexpr int kU0 = kTpl >= 32 ? 1 : (32 / kTpl < 8 ? 32 / kTpl : 8);
  static constexpr int kU = kU0 / G > 1 ? kU0 / G : 1;   // loads in flight (registers shrink with G)
  static constexpr int kStep = kTpl * kU;         // tokens per loop iteration
  static_assert(kLpt >= 1 && kLpt <= 64 && 64 % kLpt == 0, "head_dim / lane split");

  // State after run(): every lane holds the merged (m, l) of each head and
  // the un-normalised output of its element chunk, dims
  // chunk(lane) * kVec .. + kVec - 1.  m is in log2 units (kNegBig when the
  // range is empty).
  float m[G], l[G];
  float acc[G][kVec];

  __device__ static inline int chunk(int lane) { return lane % kLpt; }
  __device__ static inline int slot(int lane) { return lane / kLpt; }

  // q: the G query rows, D floats apart (heads h0 .. h0 + G - 1 of one row).
  // Needs lo < hi.
  __device__ inline void run(const KvPages& kv, const float* q, float qscale, int kvh,
                             const int32_t* bt, int lo, int hi) {
    const int lane = threadIdx.x & 63;
    const int r = slot(lane);
    const int c = chunk(lane);
    const int64_t tok_stride = (int64_t)kv.Hkv * D;
    const int64_t blk_stride = tok_stride * kv.BS;
    const T* kp = reinterpret_cast<const T*>(kv.k) + kvh * D + c * kVec;
    const T* vp = reinterpret_cast<const T*>(kv.v) + kvh * D + c * kVec;

    float qv[G][kVec];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float4* q4 = reinterpret_cast<const float4*>(q + g * D + c * kVec);
#pragma unroll
      for (int i = 0; i < kVec / 4; ++i) {
        const float4 x = q4[i];
        qv[g][4 * i + 0] = x.x * qscale;
        qv[g][4 * i + 1] = x.y * qscale;
        qv[g][4 * i + 2] = x.z * qscale;
        qv[g][4 * i + 3] = x.w * qscale;
      }
    }

#pragma unroll
    for (int g = 0; g < G; ++g) {
      m[g] = kNegBig;
      l[g] = 0.0f;
#pragma unroll
      for (int e = 0; e < kVec; ++e) acc[g][e] = 0.0f;
    }

    // Groups of kTpl tokens start at multiples of kTpl.  Addresses of groups
    // past the range are clamped to the last group that holds a live token;
    // their scores are masked below.
    const int t_begin = lo - (lo % kTpl);
    const int last_group = (hi - 1) - ((hi - 1) % kTpl);

    for (int t0 = t_begin; t0 < hi; t0 += kStep) {
      uint4 kr[kU], vr[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int tg = min(t0 + u * kTpl, last_group);
        int64_t off;
        if constexpr (kPaged) {
          off = safe_block(bt[tg / kv.BS], kv.NB) * blk_stride +
                (int64_t)(tg % kv.BS + r) * tok_stride;
        } else {
          const int t = min(tg + r, hi - 1);
          off = safe_block(bt[t / kv.BS], kv.NB) * blk_stride + (int64_t)(t % kv.BS) * tok_stride;
        }
        kr[u] = load16_stream(kp + off);
        vr[u] = load16_stream(vp + off);
      }

      bool ok[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int t = t0 + u * kTpl + r;
        ok[u] = (t >= lo) && (t < hi);
      }
      float pu[G][kU];
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float sc[kU];
        float mx = kNegBig;
#pragma unroll
        for (int u = 0; u < kU; ++u) {
          float kf[kVec];
          Elem<T>::to_f32(kr[u], kf);
          float d = 0.0f;
#pragma unroll
          for (int e = 0; e < kVec; ++e) d = fmaf(qv[g][e], kf[e], d);
          d = group_sum<kLpt>(d);
          sc[u] = ok[u] ? d : kNegBig;
          mx = fmaxf(mx, sc[u]);
        }
        // The running max is raised only when this step's max exceeds it by
        // more than kWalkSlack (log2 units): probabilities stay <= 2^slack in
        // fp32 and the G accumulators are rescaled on few steps.
        if (__builtin_amdgcn_ballot_w64(mx > m[g] + kWalkSlack) != 0) {
          const float m_new = fmaxf(m[g], mx);
          const float corr = fast_exp2(m[g] - m_new);
          l[g] *= corr;
#pragma unroll
          for (int e = 0; e < kVec; ++e) acc[g][e] *= corr;
          m[g] = m_new;
        }
        float psum = 0.0f;
#pragma unroll
        for (int u = 0; u < kU; ++u) {
          pu[g][u] = ok[u] ? fast_exp2(sc[u] - m[g]) : 0.0f;
          psum += pu[g][u];
        }
        l[g] += psum;
      }
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        float vf[kVec];
        Elem<T>::to_f32(vr[u], vf);
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
          for (int e = 0; e < kVec; ++e) acc[g][e] = fmaf(pu[g][u], vf[e], acc[g][e]);
      }
    }

    // Merge the kTpl slot states: lanes with the same chunk c, different slot.
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int off = kLpt; off < 64; off <<= 1) {
        const float m_o = __shfl_xor(m[g], off);
        const float l_o = __shfl_xor(l[g], off);
        const float mm = fmaxf(m[g], m_o);
        const float w_s = fast_exp2(m[g] - mm);
        const float w_o = fast_exp2(m_o - mm);
        l[g] = l[g] * w_s + l_o * w_o;
#pragma unroll
        for (int e = 0; e < kVec; ++e)
          acc[g][e] = acc[g][e] * w_s + __shfl_xor(acc[g][e], off) * w_o;
        m[g] = mm;
      }
    }
  }

  // Head g's result on the lanes of slot 0: normalised into out (dims
  // chunk * kVec ..), or un-normalised with (m, l) as a partition state.
  __device__ inline void store_out(int g, float* out_row) const {
    const int lane = threadIdx.x & 63;
    if (slot(lane) != 0) return;
    const float inv = l[g] > 0.0f ? 1.0f / l[g] : 0.0f;
    float4* o4 = reinterpret_cast<float4*>(out_row + chunk(lane) * kVec);
#pragma unroll
    for (int i = 0; i < kVec / 4; ++i)
      o4[i] = make_float4(acc[g][4 * i] * inv, acc[g][4 * i + 1] * inv, acc[g][4 * i + 2] * inv,
                          acc[g][4 * i + 3] * inv);
  }

  __device__ inline void store_state(int g, float* acc_row, float2* ml) const {
    const int lane = threadIdx.x & 63;
    if (slot(lane) != 0) return;
    float4* o4 = reinterpret_cast<float4*>(acc_row + chunk(lane) * kVec);
#pragma unroll
    for (int i = 0; i < kVec / 4; ++i)
      o4[i] = make_float4(acc[g][4 * i], acc[g][4 * i + 1], acc[g][4 * i + 2], acc[g][4 * i + 3]);
    if (chunk(lane) == 0) *ml = make_float2(m[g], l[g]);
  }
};

}  // namespace hs
