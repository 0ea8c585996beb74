// Paged attention over "rows": one query vector per (row, head) attending to
// a prefix [0, end) of its sequence's paged KV.  Decode is B rows with
// end = ctx_b; the VALU prefill path is B*S rows with end = ctx_b - S + s + 1.
//
// Algorithm (reference: paged_attn_v2.py:75-157 for the single pass,
// paged_attn_v3.py:75-208 for split + merge): an online softmax over the
// row's keys, optionally cut into partitions whose un-normalised states
// (m, l, acc) are combined by a log-sum-exp merge.  The softmax runs in base 2
// with scale * log2(e) folded into q, so every exponential is one v_exp_f32.
//
// The walk of one wave (16-lane token slots, DPP reductions, per-slot softmax
// states merged at the end) is RowWalk, hs_rowwalk.h.
// A workgroup is kDecodeWaves waves = consecutive heads (or GQA head groups)
// of the same (row, partition), and the head group is the fastest-varying grid
// index, so the
// workgroups in flight together stream whole token rows (all heads of a token
// are adjacent in the page) instead of one head's narrow column of many rows.
// KV loads are non-temporal: every byte is read once, so it should not
// displace anything in L2.  Measured on MI355X (C2 decode): the head-major
// grid order took the kernel from 3.5 to 5.3 TB/s, non-temporal loads to
// 5.8 TB/s, 32 tokens of loads in flight per wave and 512-token partitions
// to ~6 TB/s.
#include "hs_kernels.h"
#include "hs_rowwalk.h"

namespace hs {

constexpr int kDecodeWaves = 2;  // waves per workgroup

// One wave = G query heads of one KV group for one (row, partition): each
// 16-byte K/V load feeds G dot products, so a GQA group's pages are read once
// instead of once per query head.  G = 1 is plain multi-head attention.  The
// arithmetic of each head is the same for every G (same slots, token order
// and reduction order), so packing does not change results.
template <typename T, int D, bool kPaged, int G>
__global__ __launch_bounds__(kDecodeWaves * 64)
__attribute__((amdgpu_waves_per_eu(G >= 8 ? 2 : (D > 128 ? 3 : 4)))) void row_attn_part_kernel(RowAttnArgs a) {
  const int lane = threadIdx.x & 63;
  const int n_hw = a.H / G;                                     // head groups of G
  const int n_groups = (n_hw + kDecodeWaves - 1) / kDecodeWaves;
  const int64_t wg = blockIdx.x;
  const int hw = (int)(wg % n_groups) * kDecodeWaves + (threadIdx.x >> 6);
  if (hw >= n_hw) return;
  const int h0 = hw * G;                   // first query head of this wave
  const int64_t rp = wg / n_groups;        // row * P + partition
  const int row = (int)(rp / a.P);
  const int p = (int)(rp - (int64_t)row * a.P);
  if (a.skip && a.skip[rp]) return;        // served by the shared-page kernel

  int b, end;
  if (!row_geometry(a, row, b, end)) return;
  int lo = 0, hi = 0, nparts = 0;
  const bool live = partition_range(a, end, p, lo, hi, nparts);
  const int64_t orow0 = ((int64_t)row * a.H + h0) * D;
  if (!live) {
    if (end <= 0 && p == 0) {  // nothing to attend to: zero rows
      for (int d = lane; d < G * D; d += 64) a.out[orow0 + d] = 0.0f;
    }
    return;
  }

  RowWalk<T, D, kPaged, G> w;
  w.run(KvPages{a.k, a.v, a.Hkv, a.BS, a.NB}, a.q + orow0, a.qscale, h0 / (a.H / a.Hkv),
        a.bt + (int64_t)b * a.MB, lo, hi);
  if (w.slot(lane) != 0) return;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int h = h0 + g;
    if (nparts == 1) {
      w.store_out(g, a.out + orow0 + g * D);
    } else {
      const int64_t pi = ((int64_t)row * a.H + h) * a.P + p;
      w.store_state(g, a.part_acc + pi * D, reinterpret_cast<float2*>(a.part_ml) + pi);
    }
  }
}

// Small grids (mode 3): one workgroup per (row, head group of G) walks the
// whole row, its W waves on W contiguous slices of the keys, and the waves'
// states are combined through LDS, so a batch too small to fill the CUs gets
// W times the waves without partition states or a merge launch.  Each wave
// runs the same RowWalk as the partition kernel; the combine is the
// log-sum-exp merge of paged_attn_v3.py:170-208 over the slices.
template <typename T, int D, bool kPaged, int G, int W>
__global__ __launch_bounds__(W * 64) void row_attn_wg_kernel(RowAttnArgs a) {
  using Walk = RowWalk<T, D, kPaged, G>;
  __shared__ float s_m[W][G], s_l[W][G];
  __shared__ float s_acc[W][G][D];
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int n_hw = a.H / G;
  const int row = (int)(blockIdx.x / n_hw);
  const int h0 = (int)(blockIdx.x % n_hw) * G;
  int b, end;
  if (!row_geometry(a, row, b, end)) return;       // workgroup-uniform
  const int64_t orow0 = ((int64_t)row * a.H + h0) * D;
  if (end <= 0) {                                  // nothing to attend to: zero rows
    for (int d = threadIdx.x; d < G * D; d += W * 64) a.out[orow0 + d] = 0.0f;
    return;
  }
  // slices of whole load groups, so that no two waves load the same group
  const int chunk = ((end + W - 1) / W + Walk::kTpl - 1) / Walk::kTpl * Walk::kTpl;
  const int lo = wv * chunk;
  const int hi = min(end, lo + chunk);
  Walk w;
  if (lo < hi) {
    w.run(KvPages{a.k, a.v, a.Hkv, a.BS, a.NB}, a.q + orow0, a.qscale, h0 / (a.H / a.Hkv),
          a.bt + (int64_t)b * a.MB, lo, hi);
  } else {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      w.m[g] = kNegBig;
      w.l[g] = 0.0f;
#pragma unroll
      for (int e = 0; e < Walk::kVec; ++e) w.acc[g][e] = 0.0f;
    }
  }
  if (Walk::slot(lane) == 0) {
    const int c = Walk::chunk(lane);
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int e = 0; e < Walk::kVec; ++e) s_acc[wv][g][c * Walk::kVec + e] = w.acc[g][e];
      if (c == 0) {
        s_m[wv][g] = w.m[g];
        s_l[wv][g] = w.l[g];
      }
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < G * D; i += W * 64) {
    const int g = i / D, d = i - g * D;
    float mm = s_m[0][g];
#pragma unroll
    for (int v = 1; v < W; ++v) mm = fmaxf(mm, s_m[v][g]);
    float l = 0.0f, o = 0.0f;
#pragma unroll
    for (int v = 0; v < W; ++v) {
      const float wt = fast_exp2(s_m[v][g] - mm);   // an empty slice: exp2(-3e38 - mm) = 0
      l = fmaf(s_l[v][g], wt, l);
      o = fmaf(s_acc[v][g][d], wt, o);
    }
    a.out[orow0 + i] = l > 0.0f ? o / l : 0.0f;
  }
}

// Log-sum-exp merge of the partition states of every (row, head) that has
// more than one non-empty partition (reference: merge_splits_kernel,
// paged_attn_v3.py:170-208).  One wave per (row, head), lanes over D.  The
// kernel is latency-bound (a few MB in all), so its memory round trips are
// batched: lane p reads partition p's (max, sum), 64 partitions per load, and
// the partial outputs are read 8 partitions at a time, each weight taken from
// the lane that computed it.
template <int D>
__global__ __launch_bounds__(256) void row_attn_merge_kernel(RowAttnArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t w = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (w >= (int64_t)a.rows * a.H) return;
  const int row = (int)(w / a.H);
  int b, end;
  if (!row_geometry(a, row, b, end)) return;
  int lo, hi, nparts;
  partition_range(a, end, 0, lo, hi, nparts);
  if (nparts <= 1) return;  // written directly by the partition kernel

  const float2* ml = reinterpret_cast<const float2*>(a.part_ml) + w * a.P;
  const float2 none = make_float2(kNegBig, 0.0f);
  const float2 st0 = lane < nparts ? ml[lane] : none;
  float mm = st0.x;
  for (int p0 = 64; p0 < nparts; p0 += 64)
    if (p0 + lane < nparts) mm = fmaxf(mm, ml[p0 + lane].x);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) mm = fmaxf(mm, __shfl_xor(mm, off));

  constexpr int kPer = (D + 63) / 64;
  constexpr int kBatch = 8;
  float acc[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) acc[i] = 0.0f;
  float lsum = 0.0f;   // this lane's partitions; summed over the wave below
  for (int p0 = 0; p0 < nparts; p0 += 64) {
    const int n = min(64, nparts - p0);
    const float2 st = p0 == 0 ? st0 : (lane < n ? ml[p0 + lane] : none);
    const float wt = lane < n ? fast_exp2(st.x - mm) : 0.0f;
    lsum = fmaf(st.y, wt, lsum);
    const float* pa = a.part_acc + (w * a.P + p0) * D;
    for (int p = 0; p < n; p += kBatch) {
      float v[kBatch][kPer];
#pragma unroll
      for (int u = 0; u < kBatch; ++u)
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
          const int d = lane + 64 * i;
          v[u][i] = (p + u < n && d < D) ? pa[(p + u) * D + d] : 0.0f;
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
  for (int i = 0; i < kPer; ++i) {
    const int d = lane + 64 * i;
    if (d < D) a.out[w * D + d] = acc[i] * inv;
  }
}

// ---------------------------------------------------------------------------
// host launch
// ---------------------------------------------------------------------------

static int elem_vec(int kv_dtype) { return kv_dtype == HS_DTYPE_F32 ? 4 : 8; }

// Tokens one wave-wide load covers for this dtype and head_dim.
int row_attn_tokens_per_load(int kv_dtype, int D) { return 64 / (D / elem_vec(kv_dtype)); }

// Query heads per wave: the largest of 1, 2, 4, 8 dividing the GQA group.
int row_attn_heads_per_wave(int H, int Hkv) {
  const int group = H / Hkv;
  int g = 1;
  while (g < 8 && group % (2 * g) == 0) g *= 2;
  return g;
}

static void launch_merge(const RowAttnArgs& a, int D, hipStream_t stream) {
  const int64_t waves = (int64_t)a.rows * a.H;
  const dim3 grid((unsigned)((waves + 3) / 4)), block(256);
  switch (D) {
    case 32: hipLaunchKernelGGL((row_attn_merge_kernel<32>), grid, block, 0, stream, a); break;
    case 64: hipLaunchKernelGGL((row_attn_merge_kernel<64>), grid, block, 0, stream, a); break;
    case 128: hipLaunchKernelGGL((row_attn_merge_kernel<128>), grid, block, 0, stream, a); break;
    default: hipLaunchKernelGGL((row_attn_merge_kernel<256>), grid, block, 0, stream, a); break;
  }
}

template <typename T, int D, int G>
static void launch_part(const RowAttnArgs& a, hipStream_t stream) {
  const int tpl = 64 / (D / Elem<T>::kVec);
  const int64_t gx = sat_mul(a.rows, a.P, ceil_div(a.H / G, kDecodeWaves));   // checked by the caller
  const dim3 grid((unsigned)gx), block(kDecodeWaves * 64);
  if (a.BS % tpl == 0)
    hipLaunchKernelGGL((row_attn_part_kernel<T, D, true, G>), grid, block, 0, stream, a);
  else
    hipLaunchKernelGGL((row_attn_part_kernel<T, D, false, G>), grid, block, 0, stream, a);
}

// Waves of a mode-3 workgroup: 16 (4 per SIMD, at most 128 VGPRs each), or 8
// where the walk holds more state (G = 8 heads, or head dim 256), as the
// partition kernel's occupancy hints allow.  The waves' states take
// W * G * D floats of LDS, 64 KiB at most.
constexpr int wg_waves(int G, int D) { return G >= 8 || D > 128 ? 8 : 16; }

template <typename T, int D, int G>
static void launch_wg(const RowAttnArgs& a, hipStream_t stream) {
  constexpr int W = wg_waves(G, D);
  const int tpl = 64 / (D / Elem<T>::kVec);
  // the grid size is checked by the caller
  const dim3 grid((unsigned)((int64_t)a.rows * (a.H / G))), block(W * 64);
  if (a.BS % tpl == 0)
    hipLaunchKernelGGL((row_attn_wg_kernel<T, D, true, G, W>), grid, block, 0, stream, a);
  else
    hipLaunchKernelGGL((row_attn_wg_kernel<T, D, false, G, W>), grid, block, 0, stream, a);
}

template <typename T, int D, int G>
static void launch_mode(const RowAttnArgs& a, hipStream_t stream) {
  if (a.mode == 3) launch_wg<T, D, G>(a, stream);
  else launch_part<T, D, G>(a, stream);
}

template <typename T, int D>
static void launch_typed(const RowAttnArgs& a, hipStream_t stream) {
  profile_begin(stream);
  switch (row_attn_heads_per_wave(a.H, a.Hkv)) {
    case 8: launch_mode<T, D, 8>(a, stream); break;
    case 4: launch_mode<T, D, 4>(a, stream); break;
    case 2: launch_mode<T, D, 2>(a, stream); break;
    default: launch_mode<T, D, 1>(a, stream); break;
  }
  profile_end(stream);
}

template <typename T>
static int launch_dim(const RowAttnArgs& a, int D, hipStream_t stream) {
  switch (D) {
    case 32: launch_typed<T, 32>(a, stream); break;
    case 64: launch_typed<T, 64>(a, stream); break;
    case 128: launch_typed<T, 128>(a, stream); break;
    case 256: launch_typed<T, 256>(a, stream); break;
    default: return fail(HS_EUNSUPPORTED, "unsupported head_dim " + std::to_string(D));
  }
  return check_launch("paged attention");
}

// Launch the partition kernel (+ merge when P > 1).  Arguments are validated
// by the caller.  Grouped-query calls on 16-bit caches with 16-token pages
// and fixed partitions go to the split-operand matrix-core kernel
// (hs_decode_splitmm.hip); the rest run the VALU kernel above.  With
// `shared`: the plan kernel, then the shared-page kernel, then the partition
// kernel (which skips the grouped partitions), then the merge.  The shared
// kernel runs first, alone: beside the partition kernel its large workgroups
// waited for whole CUs to drain and finished last.
int launch_row_attn(const RowAttnArgs& a, int kv_dtype, int D, hipStream_t stream,
                    const SharePlanArgs* shared) {
  if (a.mode == 4) {   // even split, then the merge of the rows it cut (hs_decode_splitmm.hip)
    const int64_t gx = sat_mul(a.Hkv, ceil_div(a.H / a.Hkv, 16), a.even_m);
    if (gx > 0x7fffffffLL) return fail(HS_EUNSUPPORTED, "grid too large");
    launch_splitmm_even(a, kv_dtype, D, stream);
    return check_launch("paged attention");
  }
  const bool splitmm = splitmm_applies(a, kv_dtype, D);
  int64_t gx;
  if (splitmm) {
    gx = splitmm_grid(a);
  } else {
    const int G = row_attn_heads_per_wave(a.H, a.Hkv);
    gx = a.mode == 3 ? sat_mul(a.rows, a.H / G)
                     : sat_mul(a.rows, a.P, ceil_div(a.H / G, kDecodeWaves));
  }
  if (gx <= 0) return HS_OK;
  if (gx > 0x7fffffffLL)
    return fail(HS_EUNSUPPORTED, "grid too large: rows * partitions * head groups = " +
                                     std::to_string(gx));
  if (kv_dtype != HS_DTYPE_F32 && kv_dtype != HS_DTYPE_F16 && kv_dtype != HS_DTYPE_BF16)
    return fail(HS_EINVAL, "unknown kv dtype code " + std::to_string(kv_dtype));
  if (shared) {
    launch_share_plan(a, *shared, stream);
    launch_shared_pages(a, *shared, kv_dtype, D, stream);
  }

  int rc = HS_OK;
  if (splitmm) {
    profile_begin(stream);
    launch_splitmm_part(a, kv_dtype, D, stream);
    profile_end(stream);
  } else if (kv_dtype == HS_DTYPE_F32) {
    rc = launch_dim<float>(a, D, stream);
  } else if (kv_dtype == HS_DTYPE_F16) {
    rc = launch_dim<_Float16>(a, D, stream);
  } else {
    rc = launch_dim<Bf16>(a, D, stream);
  }
  if (rc != HS_OK) return rc;
  if (a.P > 1) launch_merge(a, D, stream);
  return check_launch("paged attention");
}

}  // namespace hs
