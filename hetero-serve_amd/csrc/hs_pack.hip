// Bitwise KV page movement: migration pack / unpack and the contiguous
// per-sequence gather.
//
// All three are HBM-bound copies of whole pages (pack/unpack) or whole token
// rows (gather).  A workgroup copies one 4 KiB piece (256 lanes x one 16-byte
// load and store); every byte is moved once, so loads and stores carry the
// non-temporal hint (measured on the C5 pack: 5.25 -> 5.89 TB/s).  Pieces are
// numbered page-major, and the hardware deals workgroups to the 8 XCDs
// round-robin by id, so the grid is renumbered to give each XCD one
// contiguous run of pieces (whole pages) instead of every eighth piece.
// Measured on the C5 pack / unpack (4096 random 128-KiB pages each way):
// 16-KiB pieces in grid order 5.71 / 5.31 TB/s, 4-KiB pieces 6.41 / 6.16,
// 4-KiB pieces with contiguous runs per XCD 6.52 / 6.41 (8-KiB 6.27 / 6.16).
// A page or row whose size or base is not a multiple of 16 bytes takes a
// byte-granular kernel instead.
#include "hs_kernels.h"

namespace hs {

constexpr int kCopyThreads = 256;
constexpr int kCopyUnroll = 1;
constexpr int64_t kCopyPiece = (int64_t)kCopyThreads * kCopyUnroll * 16;  // bytes per workgroup
constexpr int kXcds = 8;   // MI355X: workgroup b runs on XCD b % 8

// Piece handled by workgroup b of a grid of n: XCD x = b % 8 takes the
// contiguous run [start_x, start_x + count_x) of the n pieces, in order.
__device__ inline int64_t xcd_run_piece(int64_t b, int64_t n) {
  const int64_t x = b % kXcds, q = n / kXcds, r = n % kXcds;
  return x * q + (x < r ? x : r) + b / kXcds;
}

__device__ inline void copy_piece16(const uint8_t* src, uint8_t* dst, int64_t bytes,
                                    int64_t piece) {
  const int64_t base = piece * kCopyPiece + (int64_t)threadIdx.x * 16;
  uint4 v[kCopyUnroll];
#pragma unroll
  for (int u = 0; u < kCopyUnroll; ++u) {
    const int64_t off = base + (int64_t)u * kCopyThreads * 16;
    if (off < bytes) v[u] = load16_stream(src + off);
  }
#pragma unroll
  for (int u = 0; u < kCopyUnroll; ++u) {
    const int64_t off = base + (int64_t)u * kCopyThreads * 16;
    if (off < bytes) store16_stream(dst + off, v[u]);
  }
}

__device__ inline void copy_piece1(const uint8_t* src, uint8_t* dst, int64_t bytes,
                                   int64_t piece) {
  const int64_t end = min(bytes, (piece + 1) * kCopyPiece);
  for (int64_t off = piece * kCopyPiece + threadIdx.x; off < end; off += kCopyThreads)
    dst[off] = src[off];
}

// Page copy between the pool [L, 2, NB, page] and the pack buffer
// [n, L, 2, page].  Workgroup w copies piece (w % pieces) of pack page
// (w / pieces), whose index is (i * L + l) * 2 + c.
template <bool kUnpack, bool kVec16>
__global__ __launch_bounds__(kCopyThreads) void page_copy_kernel(const uint8_t* src_base,
                                                                 uint8_t* dst_base,
                                                                 const int64_t* ids, int L,
                                                                 int NB, int64_t page_bytes,
                                                                 int64_t pieces) {
  const int64_t w = xcd_run_piece(blockIdx.x, gridDim.x);
  const int64_t pc = w / pieces;
  const int64_t piece = w - pc * pieces;
  const int c = (int)(pc & 1);
  const int64_t il = pc >> 1;
  const int64_t i = il / L;
  const int l = (int)(il - i * L);
  const int64_t id = ids[i];
  if (id < 0 || id >= NB) return;
  const int64_t pool_off = (((int64_t)l * 2 + c) * NB + id) * page_bytes;
  const int64_t pack_off = pc * page_bytes;
  const uint8_t* src = src_base + (kUnpack ? pack_off : pool_off);
  uint8_t* dst = dst_base + (kUnpack ? pool_off : pack_off);
  if constexpr (kVec16) copy_piece16(src, dst, page_bytes, piece);
  else copy_piece1(src, dst, page_bytes, piece);
}

// out[b, t] = cache[bt[b][t / BS], t % BS], one row = row_bytes.
template <bool kVec16>
__global__ __launch_bounds__(kCopyThreads) void gather_rows_kernel(
    const uint8_t* cache, uint8_t* out, const int32_t* bt, int NB, int BS, int MB, int length,
    int64_t row_bytes, int64_t pieces) {
  const int64_t w = xcd_run_piece(blockIdx.x, gridDim.x);
  const int64_t rf = w / pieces;  // b * length + t
  const int64_t piece = w - rf * pieces;
  const int b = (int)(rf / length);
  const int t = (int)(rf - (int64_t)b * length);
  const int64_t blk = safe_block(bt[(int64_t)b * MB + t / BS], NB);
  const uint8_t* src = cache + (blk * BS + t % BS) * row_bytes;
  uint8_t* dst = out + rf * row_bytes;
  if constexpr (kVec16) copy_piece16(src, dst, row_bytes, piece);
  else copy_piece1(src, dst, row_bytes, piece);
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int launch_page_copy(const void* pool, void* buf, bool unpack, int L, int NB,
                     int64_t page_bytes, const int64_t* ids, int n, hipStream_t stream) {
  const int64_t pieces = ceil_div(page_bytes, kCopyPiece);
  const int64_t grid = sat_mul(n, L, 2, pieces);
  if (grid == 0) return HS_OK;
  if (grid > 0x7fffffffLL) return fail(HS_EUNSUPPORTED, "pack grid too large");
  if (sat_mul(L, 2, NB, page_bytes) == INT64_MAX)
    return fail(HS_EUNSUPPORTED, "pool too large for 64-bit offsets");
  const bool vec = page_bytes % 16 == 0 && aligned16(pool) && aligned16(buf);
  const uint8_t* pool_b = static_cast<const uint8_t*>(pool);
  uint8_t* buf_b = static_cast<uint8_t*>(buf);
  const dim3 g((unsigned)grid), blk(kCopyThreads);
  profile_begin(stream);
  if (!unpack) {
    if (vec)
      hipLaunchKernelGGL((page_copy_kernel<false, true>), g, blk, 0, stream, pool_b, buf_b, ids,
                         L, NB, page_bytes, pieces);
    else
      hipLaunchKernelGGL((page_copy_kernel<false, false>), g, blk, 0, stream, pool_b, buf_b, ids,
                         L, NB, page_bytes, pieces);
  } else {
    // unpack: source is the pack buffer, destination the pool
    uint8_t* pool_w = const_cast<uint8_t*>(pool_b);
    if (vec)
      hipLaunchKernelGGL((page_copy_kernel<true, true>), g, blk, 0, stream, buf_b, pool_w, ids, L,
                         NB, page_bytes, pieces);
    else
      hipLaunchKernelGGL((page_copy_kernel<true, false>), g, blk, 0, stream, buf_b, pool_w, ids,
                         L, NB, page_bytes, pieces);
  }
  profile_end(stream);
  return check_launch(unpack ? "kv unpack" : "kv pack");
}

int launch_gather_rows(const void* cache, int NB, int BS, int64_t row_bytes, const int32_t* bt,
                       int MB, int B, int length, void* out, hipStream_t stream) {
  const int64_t pieces = ceil_div(row_bytes, kCopyPiece);
  const int64_t grid = sat_mul(B, length, pieces);
  if (grid == 0) return HS_OK;
  if (grid > 0x7fffffffLL) return fail(HS_EUNSUPPORTED, "gather grid too large");
  const bool vec = row_bytes % 16 == 0 && aligned16(cache) && aligned16(out);
  const uint8_t* src = static_cast<const uint8_t*>(cache);
  uint8_t* dst = static_cast<uint8_t*>(out);
  profile_begin(stream);
  if (vec)
    hipLaunchKernelGGL((gather_rows_kernel<true>), dim3((unsigned)grid), dim3(kCopyThreads), 0,
                       stream, src, dst, bt, NB, BS, MB, length, row_bytes, pieces);
  else
    hipLaunchKernelGGL((gather_rows_kernel<false>), dim3((unsigned)grid), dim3(kCopyThreads), 0,
                       stream, src, dst, bt, NB, BS, MB, length, row_bytes, pieces);
  profile_end(stream);
  return check_launch("kv gather");
}

}  // namespace hs
