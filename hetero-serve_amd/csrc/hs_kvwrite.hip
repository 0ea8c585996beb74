// Writing new K/V rows into the paged cache: the step just before attention.
//
// Reference: the engine's `fk[slots] = k.to(pool dtype)` / `fv[slots] = ...`
// (heteroserve/model/torch_engine.py:239-240 for decode, :306-308 for a
// prefill chunk) and TorchBlockAllocator.write_kv (kv/torch_blocks.py:89-106,
// the same scatter per layer), with slots from slots_for (:68-73):
//   slot = table[pos // BS] * BS + pos % BS.
//
// One token row is Hkv * D elements.  A thread converts and moves 8
// elements (16 bytes of a 16-bit cache), so a D = 128 head row is one
// 16-lane group and a wave covers 4 heads; K and V are grid.y = 0 / 1 of one
// launch.  The source may be a strided view (rows of the fused QKV output),
// so the source row stride is a parameter.  Casts round like torch's
// `.to()`: fp32 -> bf16 and -> fp16 to nearest even, NaN to the canonical
// quiet NaN torch produces; equal types are copied bit for bit.
//
// A row whose slot is outside the cache (or whose table entry / position is
// invalid in the append form) is skipped: the kernel never writes outside
// the cache.  Rows must not share a slot (the engine never writes two tokens
// to one slot in a step; which of two duplicates survives is unspecified, as
// for torch's index_put).
#include "hs_kernels.h"

#include <type_traits>

namespace hs {

namespace {

constexpr int kWriteThreads = 256;

// ---- element codecs: 8 elements <-> 8 fp32 ------------------------------
template <typename T>
struct Codec;

template <>
struct Codec<float> {
  static constexpr int kBytes = 4;
  __device__ static void load8(const uint8_t* p, float* x) {
    const uint4 a = load16(p), b = load16(p + 16);
    x[0] = __uint_as_float(a.x); x[1] = __uint_as_float(a.y);
    x[2] = __uint_as_float(a.z); x[3] = __uint_as_float(a.w);
    x[4] = __uint_as_float(b.x); x[5] = __uint_as_float(b.y);
    x[6] = __uint_as_float(b.z); x[7] = __uint_as_float(b.w);
  }
  __device__ static void store8(uint8_t* p, const float* x) {
    *reinterpret_cast<uint4*>(p) = make_uint4(__float_as_uint(x[0]), __float_as_uint(x[1]),
                                              __float_as_uint(x[2]), __float_as_uint(x[3]));
    *reinterpret_cast<uint4*>(p + 16) = make_uint4(__float_as_uint(x[4]), __float_as_uint(x[5]),
                                                   __float_as_uint(x[6]), __float_as_uint(x[7]));
  }
  __device__ static float load1(const uint8_t* p) { return *reinterpret_cast<const float*>(p); }
  __device__ static void store1(uint8_t* p, float x) { *reinterpret_cast<float*>(p) = x; }
};

// fp32 -> bf16 bits, round to nearest even; NaN -> 0x7FC0 (c10::BFloat16).
__device__ inline uint32_t f32_to_bf16_bits(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

// fp32 -> fp16 bits, round to nearest even (v_cvt_f16_f32); NaN -> sign | 0x7E00
// as torch's CPU conversion gives.
__device__ inline uint32_t f32_to_f16_bits(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return ((u >> 16) & 0x8000u) | 0x7e00u;
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

template <>
struct Codec<Bf16> {
  static constexpr int kBytes = 2;
  __device__ static void load8(const uint8_t* p, float* x) {
    const uint4 a = load16(p);
    const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = __uint_as_float(w[i] << 16);
      x[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
  __device__ static void store8(uint8_t* p, const float* x) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = f32_to_bf16_bits(x[2 * i]) | (f32_to_bf16_bits(x[2 * i + 1]) << 16);
    *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
  }
  __device__ static float load1(const uint8_t* p) {
    return __uint_as_float((uint32_t)*reinterpret_cast<const uint16_t*>(p) << 16);
  }
  __device__ static void store1(uint8_t* p, float x) {
    *reinterpret_cast<uint16_t*>(p) = (uint16_t)f32_to_bf16_bits(x);
  }
};

template <>
struct Codec<_Float16> {
  static constexpr int kBytes = 2;
  __device__ static void load8(const uint8_t* p, float* x) {
    const uint4 a = load16(p);
    const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[i] & 0xffffu));
      x[2 * i + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[i] >> 16));
    }
  }
  __device__ static void store8(uint8_t* p, const float* x) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = f32_to_f16_bits(x[2 * i]) | (f32_to_f16_bits(x[2 * i + 1]) << 16);
    *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
  }
  __device__ static float load1(const uint8_t* p) {
    return (float)*reinterpret_cast<const _Float16*>(p);
  }
  __device__ static void store1(uint8_t* p, float x) {
    *reinterpret_cast<uint16_t*>(p) = (uint16_t)f32_to_f16_bits(x);
  }
};

// Where row i goes: an explicit slot, or the slot of (sequence, position)
// through the block table.  Returns -1 for a row that must be skipped.
struct RowMap {
  const int64_t* slots;        // scatter form (null in the append form)
  const int32_t* bt;           // append form: [B, MB] tables
  const int32_t* positions;    //              [n] absolute positions
  const int32_t* seq_ids;      //              [n] row -> sequence, or null (row i = sequence i)
  int64_t num_slots;           // NB * BS
  int NB, BS, B, MB;           // B: table rows; a sequence index must be below it

  __device__ int64_t slot(int64_t i) const {
    if (slots) {
      const int64_t s = slots[i];
      return (s >= 0 && s < num_slots) ? s : -1;
    }
    const int64_t b = seq_ids ? seq_ids[i] : i;
    const int pos = positions[i];
    if (b < 0 || b >= B || pos < 0 || pos / BS >= MB) return -1;
    const int blk = bt[b * MB + pos / BS];
    if (blk < 0 || blk >= NB) return -1;
    return (int64_t)blk * BS + pos % BS;
  }
};

// grid.x covers n rows x (row / 8) chunks; grid.y = 0 (K) / 1 (V).
template <typename S, typename C>
__global__ __launch_bounds__(kWriteThreads) void kv_write_kernel(
    uint8_t* k_cache, uint8_t* v_cache, const uint8_t* k_src, const uint8_t* v_src,
    int64_t src_stride_bytes, int64_t row_elems, int64_t n, RowMap map) {
  const int64_t chunks = row_elems / 8;
  const int64_t g = (int64_t)blockIdx.x * kWriteThreads + threadIdx.x;
  if (g >= n * chunks) return;
  const int64_t i = g / chunks;
  const int64_t c = g - i * chunks;
  const int64_t slot = map.slot(i);
  if (slot < 0) return;
  const uint8_t* src = (blockIdx.y ? v_src : k_src) + i * src_stride_bytes + c * 8 * Codec<S>::kBytes;
  uint8_t* dst = (blockIdx.y ? v_cache : k_cache) + (slot * row_elems + c * 8) * Codec<C>::kBytes;
  float x[8];
  Codec<S>::load8(src, x);
  Codec<C>::store8(dst, x);
}

// Any alignment: one element per thread.
template <typename S, typename C>
__global__ __launch_bounds__(kWriteThreads) void kv_write_scalar_kernel(
    uint8_t* k_cache, uint8_t* v_cache, const uint8_t* k_src, const uint8_t* v_src,
    int64_t src_stride_bytes, int64_t row_elems, int64_t n, RowMap map) {
  const int64_t g = (int64_t)blockIdx.x * kWriteThreads + threadIdx.x;
  if (g >= n * row_elems) return;
  const int64_t i = g / row_elems;
  const int64_t e = g - i * row_elems;
  const int64_t slot = map.slot(i);
  if (slot < 0) return;
  const uint8_t* src = (blockIdx.y ? v_src : k_src) + i * src_stride_bytes + e * Codec<S>::kBytes;
  uint8_t* dst = (blockIdx.y ? v_cache : k_cache) + (slot * row_elems + e) * Codec<C>::kBytes;
  Codec<C>::store1(dst, Codec<S>::load1(src));
}

// Equal types: bit copy (NaN payloads included), 16 bytes per thread.
template <int kBytes>
__global__ __launch_bounds__(kWriteThreads) void kv_copy_kernel(
    uint8_t* k_cache, uint8_t* v_cache, const uint8_t* k_src, const uint8_t* v_src,
    int64_t src_stride_bytes, int64_t row_elems, int64_t n, RowMap map) {
  const int64_t row_bytes = row_elems * kBytes;
  const int64_t pieces = row_bytes / 16;
  const int64_t g = (int64_t)blockIdx.x * kWriteThreads + threadIdx.x;
  if (g >= n * pieces) return;
  const int64_t i = g / pieces;
  const int64_t c = g - i * pieces;
  const int64_t slot = map.slot(i);
  if (slot < 0) return;
  const uint8_t* src = (blockIdx.y ? v_src : k_src) + i * src_stride_bytes + c * 16;
  uint8_t* dst = (blockIdx.y ? v_cache : k_cache) + slot * row_bytes + c * 16;
  *reinterpret_cast<uint4*>(dst) = load16(src);
}

template <typename S, typename C>
void launch_pair(uint8_t* kc, uint8_t* vc, const uint8_t* ks, const uint8_t* vs,
                 int64_t stride_bytes, int64_t row_elems, int64_t n, const RowMap& map,
                 bool vec, hipStream_t stream) {
  if (vec) {
    if (std::is_same<S, C>::value && (row_elems * Codec<C>::kBytes) % 16 == 0) {
      const int64_t work = n * (row_elems * Codec<C>::kBytes / 16);
      const dim3 grid((unsigned)((work + kWriteThreads - 1) / kWriteThreads), 2);
      hipLaunchKernelGGL((kv_copy_kernel<Codec<C>::kBytes>), grid, dim3(kWriteThreads), 0, stream, kc,
                         vc, ks, vs, stride_bytes, row_elems, n, map);
    } else {
      const int64_t work = n * (row_elems / 8);
      const dim3 grid((unsigned)((work + kWriteThreads - 1) / kWriteThreads), 2);
      hipLaunchKernelGGL((kv_write_kernel<S, C>), grid, dim3(kWriteThreads), 0, stream, kc, vc,
                         ks, vs, stride_bytes, row_elems, n, map);
    }
  } else {
    const int64_t work = n * row_elems;
    const dim3 grid((unsigned)((work + kWriteThreads - 1) / kWriteThreads), 2);
    hipLaunchKernelGGL((kv_write_scalar_kernel<S, C>), grid, dim3(kWriteThreads), 0, stream, kc,
                       vc, ks, vs, stride_bytes, row_elems, n, map);
  }
}

template <typename S>
int launch_src(int kv_dtype, uint8_t* kc, uint8_t* vc, const uint8_t* ks, const uint8_t* vs,
               int64_t stride_bytes, int64_t row_elems, int64_t n, const RowMap& map, bool vec,
               hipStream_t stream) {
  switch (kv_dtype) {
    case HS_DTYPE_F32: launch_pair<S, float>(kc, vc, ks, vs, stride_bytes, row_elems, n, map, vec, stream); break;
    case HS_DTYPE_F16: launch_pair<S, _Float16>(kc, vc, ks, vs, stride_bytes, row_elems, n, map, vec, stream); break;
    case HS_DTYPE_BF16: launch_pair<S, Bf16>(kc, vc, ks, vs, stride_bytes, row_elems, n, map, vec, stream); break;
    default: return fail(HS_EINVAL, "unsupported KV cache dtype code " + std::to_string(kv_dtype));
  }
  return HS_OK;
}

int dtype_bytes(int code) { return code == HS_DTYPE_F32 ? 4 : 2; }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

int launch_kv_write(void* k_cache, void* v_cache, int kv_dtype, const void* k_src,
                    const void* v_src, int src_dtype, int64_t src_row_stride, int64_t row_elems,
                    int64_t n, const RowMap& map, hipStream_t stream) {
  if (n == 0) return HS_OK;
  const int64_t sb = dtype_bytes(src_dtype), cb = dtype_bytes(kv_dtype);
  const int64_t stride_bytes = sat_mul(src_row_stride, sb);
  if (stride_bytes == INT64_MAX || sat_mul(n, stride_bytes) == INT64_MAX ||
      sat_mul(map.num_slots, row_elems, cb) == INT64_MAX)
    return fail(HS_EUNSUPPORTED, "KV write sizes too large for 64-bit offsets");
  // the vector kernels need 16-byte aligned 8-element groups on both sides
  const bool vec = row_elems % 8 == 0 && aligned16(k_src) && aligned16(v_src) &&
                   aligned16(k_cache) && aligned16(v_cache) && stride_bytes % 16 == 0 &&
                   (row_elems * cb) % 16 == 0;
  const int64_t work = sat_mul(n, row_elems);
  if (ceil_div(work, kWriteThreads) > 0x7fffffffLL)
    return fail(HS_EUNSUPPORTED, "KV write too large for one launch");
  auto* kc = static_cast<uint8_t*>(k_cache);
  auto* vc = static_cast<uint8_t*>(v_cache);
  const auto* ks = static_cast<const uint8_t*>(k_src);
  const auto* vs = static_cast<const uint8_t*>(v_src);
  int rc;
  profile_begin(stream);
  switch (src_dtype) {
    case HS_DTYPE_F32: rc = launch_src<float>(kv_dtype, kc, vc, ks, vs, stride_bytes, row_elems, n, map, vec, stream); break;
    case HS_DTYPE_F16: rc = launch_src<_Float16>(kv_dtype, kc, vc, ks, vs, stride_bytes, row_elems, n, map, vec, stream); break;
    case HS_DTYPE_BF16: rc = launch_src<Bf16>(kv_dtype, kc, vc, ks, vs, stride_bytes, row_elems, n, map, vec, stream); break;
    default: rc = fail(HS_EINVAL, "unsupported source dtype code " + std::to_string(src_dtype));
  }
  profile_end(stream);
  if (rc != HS_OK) return rc;
  return check_launch("KV write");
}

}  // namespace

// out[b, j] = ids[off[b] + j] for j < off[b+1] - off[b] (capped at width), else
// -1; packed = [off[0..B], ids...] uploaded in one copy.
__global__ __launch_bounds__(kWriteThreads) void block_tables_kernel(const int32_t* packed, int B,
                                                                    int width, int32_t* out) {
  const int64_t g = (int64_t)blockIdx.x * kWriteThreads + threadIdx.x;
  if (g >= (int64_t)B * width) return;
  const int b = (int)(g / width);
  const int j = (int)(g - (int64_t)b * width);
  const int off = packed[b];
  const int len = packed[b + 1] - off;
  out[g] = j < len ? packed[B + 1 + off + j] : -1;
}

int launch_block_tables(const int32_t* packed, int B, int width, int32_t* out,
                        hipStream_t stream) {
  const int64_t work = (int64_t)B * width;   // both are int: no overflow
  if (work == 0) return HS_OK;
  if (ceil_div(work, kWriteThreads) > 0x7fffffffLL)
    return fail(HS_EUNSUPPORTED, "block table too large for one launch");
  hipLaunchKernelGGL(block_tables_kernel, dim3((unsigned)((work + kWriteThreads - 1) / kWriteThreads)),
                     dim3(kWriteThreads), 0, stream, packed, B, width, out);
  return check_launch("block table build");
}

int launch_kv_scatter(void* k_cache, void* v_cache, int kv_dtype, int64_t num_slots,
                      int64_t row_elems, const int64_t* slots, int64_t n, const void* k_src,
                      const void* v_src, int src_dtype, int64_t src_row_stride,
                      hipStream_t stream) {
  RowMap map{};
  map.slots = slots;
  map.num_slots = num_slots;
  return launch_kv_write(k_cache, v_cache, kv_dtype, k_src, v_src, src_dtype, src_row_stride,
                         row_elems, n, map, stream);
}

int launch_kv_append(void* k_cache, void* v_cache, int kv_dtype, int NB, int BS,
                     int64_t row_elems, const int32_t* bt, int B, int MB,
                     const int32_t* positions,
                     const int32_t* seq_ids, int64_t n, const void* k_src, const void* v_src,
                     int src_dtype, int64_t src_row_stride, hipStream_t stream) {
  RowMap map{};
  map.bt = bt;
  map.positions = positions;
  map.seq_ids = seq_ids;
  map.num_slots = (int64_t)NB * BS;
  map.NB = NB;
  map.BS = BS;
  map.B = B;
  map.MB = MB;
  return launch_kv_write(k_cache, v_cache, kv_dtype, k_src, v_src, src_dtype, src_row_stride,
                         row_elems, n, map, stream);
}

}  // namespace hs
