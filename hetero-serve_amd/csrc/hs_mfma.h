// Helpers shared by the 32x32 matrix-core kernels (hs_prefill_mfma.hip,
// hs_decode_gqa.hip): the prefill's fp16 operand packing and range check, and
// the lane-half reductions of a 32x32 MFMA accumulator.
#pragma once

#include "hs_common.h"

#include <type_traits>

namespace hs {
namespace mfma {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2x __attribute__((ext_vector_type(2)));
typedef float float16x __attribute__((ext_vector_type(16)));
typedef float float2x __attribute__((ext_vector_type(2)));

__device__ inline int swap_bits23(int r) {
  return (r & ~12) | ((r & 4) << 1) | ((r & 8) >> 1);
}

__device__ inline uint32_t pack_f16(float a, float b) {
  const half2x h = __builtin_convertvector((float2x){a, b}, half2x);  // v_cvt_pk_f16_f32, RNE
  return __builtin_bit_cast(uint32_t, h);
}

// Range check of fp16 MFMA operands.  fp16 holds magnitudes up to 65504: a
// bf16 cache value of magnitude >= 65536, or a scaled query >= 65520, rounds
// to inf.  The kernels fold every operand word they convert into an fp32
// v_dot2_f32_f16 sum: products of finite halves stay below 2^33, so the sum
// is finite unless some half was inf or NaN.  One instruction per one or two
// words (f16_check(w, w, acc) checks a single word).
__device__ inline float f16_check(uint32_t x, uint32_t y, float acc) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2x, x), __builtin_bit_cast(half2x, y), acc,
                                false);
}

__device__ inline float f16_check(const uint4& w, float acc) {
  return f16_check(w.z, w.w, f16_check(w.x, w.y, acc));
}

__device__ inline bool f16_check_failed(float acc) { return !__builtin_isfinite(acc); }

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

// Both lane halves' values of x: {lanes 0-31, lanes 32-63} seen from each lane.
__device__ inline float sum_halves(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ inline float max_halves(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

}  // namespace mfma
}  // namespace hs
