// Device helpers shared by the gfx950 kernels of libhsattn.so.
//
// Everything here is written for CDNA4 wave64: DPP row operations work on
// 16-lane rows, and a 16-byte global load is the unit every kernel streams
// KV pages with.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/hsattn.h"

namespace hs {

// Finite stand-in for -inf in running maxima.  Scores are kept finite so that
// (m - m_new) never becomes (-inf) - (-inf); masked scores get p = 0 by an
// explicit predicate rather than through exp2(-inf).
constexpr float kNegBig = -3.0e38f;
constexpr float kLog2e = 1.4426950408889634f;

// ---------------------------------------------------------------------------
// 16-byte vector of KV elements -> fp32
// ---------------------------------------------------------------------------

template <typename T>
struct Elem;

template <>
struct Elem<float> {
  static constexpr int kVec = 4;  // elements in one 16-byte load
  static constexpr int kCode = HS_DTYPE_F32;
  __device__ static inline void to_f32(const uint4& w, float* f) {
    f[0] = __uint_as_float(w.x);
    f[1] = __uint_as_float(w.y);
    f[2] = __uint_as_float(w.z);
    f[3] = __uint_as_float(w.w);
  }
};

template <>
struct Elem<_Float16> {
  static constexpr int kVec = 8;
  static constexpr int kCode = HS_DTYPE_F16;
  __device__ static inline void pair(uint32_t u, float* f) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    h2 v = __builtin_bit_cast(h2, u);
    f[0] = (float)v[0];
    f[1] = (float)v[1];
  }
  __device__ static inline void to_f32(const uint4& w, float* f) {
    pair(w.x, f);
    pair(w.y, f + 2);
    pair(w.z, f + 4);
    pair(w.w, f + 6);
  }
};

// bf16 is the top half of an fp32: widening is a shift or a mask.
struct Bf16 {
  uint16_t bits;
};

template <>
struct Elem<Bf16> {
  static constexpr int kVec = 8;
  static constexpr int kCode = HS_DTYPE_BF16;
  __device__ static inline void pair(uint32_t u, float* f) {
    f[0] = __uint_as_float(u << 16);
    f[1] = __uint_as_float(u & 0xffff0000u);
  }
  __device__ static inline void to_f32(const uint4& w, float* f) {
    pair(w.x, f);
    pair(w.y, f + 2);
    pair(w.z, f + 4);
    pair(w.w, f + 6);
  }
};

__device__ inline uint4 load16(const void* p) { return *reinterpret_cast<const uint4*>(p); }

// 16-byte load with the non-temporal hint, for data read exactly once.
__device__ inline uint4 load16_stream(const void* p) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 x = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(x[0], x[1], x[2], x[3]);
}

// 16-byte store with the non-temporal hint, for data written once and not
// read back by this kernel.
__device__ inline void store16_stream(void* p, const uint4& v) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 x = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(x, reinterpret_cast<u32x4*>(p));
}

// ---------------------------------------------------------------------------
// Wave reductions
// ---------------------------------------------------------------------------

// DPP controls (GCN/CDNA encoding).
constexpr int kDppQuadXor1 = 0xB1;     // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;     // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;
constexpr int kDppRowRor8 = 0x128;    // row_ror:8, lane i of a row reads lane i ^ 8

template <int kCtrl>
__device__ inline float dpp(float x) {
  return __builtin_amdgcn_update_dpp(0.0f, x, kCtrl, 0xF, 0xF, false);
}

// Sum over aligned groups of N lanes (N a power of two, 1..64); every lane of
// a group gets the group total.  Up to 16 lanes this stays inside one DPP row
// (quad swaps, then half-row and row mirrors); wider groups add cross-row
// exchanges.
template <int N>
__device__ inline float group_sum(float x) {
  if constexpr (N >= 2) x += dpp<kDppQuadXor1>(x);
  if constexpr (N >= 4) x += dpp<kDppQuadXor2>(x);
  if constexpr (N >= 8) x += dpp<kDppRowHalfMirror>(x);
  if constexpr (N >= 16) x += dpp<kDppRowMirror>(x);
  if constexpr (N >= 32) x += __shfl_xor(x, 16);
  if constexpr (N >= 64) x += __shfl_xor(x, 32);
  return x;
}

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Clamp a block-table entry to a readable block.  The torch reference clamps
// negative entries to 0 (paged_attn.py:275); ids past the pool, which torch
// would reject, are also read as block 0 so that no kernel leaves the pool.
__device__ inline int64_t safe_block(int32_t blk, int num_blocks) {
  return (blk < 0 || blk >= num_blocks) ? 0 : (int64_t)blk;
}

// ---------------------------------------------------------------------------
// Host-side size arithmetic: a product or sum of non-negative sizes that would
// overflow int64_t saturates to INT64_MAX, so the caller's "too large" check
// rejects it instead of wrapping (signed overflow is undefined in C++).
// ---------------------------------------------------------------------------

inline int64_t sat_mul(int64_t a, int64_t b) {
  int64_t r;
  return __builtin_mul_overflow(a, b, &r) ? INT64_MAX : r;
}

inline int64_t sat_add(int64_t a, int64_t b) {
  int64_t r;
  return __builtin_add_overflow(a, b, &r) ? INT64_MAX : r;
}

inline int64_t sat_mul(int64_t a, int64_t b, int64_t c) { return sat_mul(sat_mul(a, b), c); }

inline int64_t sat_mul(int64_t a, int64_t b, int64_t c, int64_t d) {
  return sat_mul(sat_mul(a, b), sat_mul(c, d));
}

// ceil(a / b) for a >= 0, b > 0, without forming a + b - 1
inline int64_t ceil_div(int64_t a, int64_t b) { return a / b + (a % b != 0); }

// ---------------------------------------------------------------------------
// Host-side error reporting (thread-local, read back by hs_last_error)
// ---------------------------------------------------------------------------

void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int check_launch(const char* what);

}  // namespace hs
