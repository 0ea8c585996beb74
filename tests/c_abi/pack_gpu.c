/*
 * A C host moving KV blocks through libhsattn on the GPU, the migration
 * path (hs_kv_pack on the sender, hs_kv_unpack on the receiver): a pool of
 * L layers x {K, V} x NB pages of bytes filled with a pattern, n scattered
 * block ids packed into one buffer, checked byte for byte against
 * out[i, l, c] = pool[l, c, ids[i]] computed here, then unpacked into a
 * second, zeroed pool at other ids and checked the same way (every other
 * page still zero).  Prints each check and "OK" when all are exact.
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "hsattn.h"

enum { L = 3, NB = 40, N = 7 };
#define PAGE ((int64_t)16 * 2 * 64 * 2) /* BS 16, 2 KV heads, D 64, 2-byte elements */
#define POOL_BYTES ((size_t)L * 2 * NB * PAGE)
#define PACK_BYTES ((size_t)N * L * 2 * PAGE)

#define HIP_OK(x)                                                 \
  do {                                                            \
    hipError_t e_ = (x);                                          \
    if (e_ != hipSuccess) {                                       \
      printf("%s: %s\n", #x, hipGetErrorString(e_));              \
      return 1;                                                   \
    }                                                             \
  } while (0)

static size_t page_at(int l, int c, int64_t blk) {
  return (((size_t)l * 2 + (size_t)c) * NB + (size_t)blk) * (size_t)PAGE;
}

int main(void) {
  const int64_t src_ids[N] = {5, 0, 39, 17, 18, 2, 33};
  const int64_t dst_ids[N] = {1, 38, 7, 20, 11, 30, 4};
  uint8_t *pool = malloc(POOL_BYTES), *back = malloc(POOL_BYTES), *packed = malloc(PACK_BYTES);
  uint8_t *dpool, *dpacked, *dback;
  int64_t* dids;
  size_t j;
  int i, l, c, rc, fails = 0, bad;

  if (!pool || !back || !packed) return 1;
  for (j = 0; j < POOL_BYTES; ++j) pool[j] = (uint8_t)((j * 2654435761u) >> 13);

  HIP_OK(hipMalloc((void**)&dpool, POOL_BYTES));
  HIP_OK(hipMalloc((void**)&dback, POOL_BYTES));
  HIP_OK(hipMalloc((void**)&dpacked, PACK_BYTES));
  HIP_OK(hipMalloc((void**)&dids, sizeof src_ids));
  HIP_OK(hipMemcpy(dpool, pool, POOL_BYTES, hipMemcpyHostToDevice));
  HIP_OK(hipMemset(dback, 0, POOL_BYTES));

  /* pack */
  HIP_OK(hipMemcpy(dids, src_ids, sizeof src_ids, hipMemcpyHostToDevice));
  rc = hs_kv_pack(dpool, L, NB, PAGE, dids, N, dpacked, NULL);
  if (rc != HS_OK) {
    printf("hs_kv_pack: %d %s\n", rc, hs_last_error());
    return 1;
  }
  HIP_OK(hipDeviceSynchronize());
  HIP_OK(hipMemcpy(packed, dpacked, PACK_BYTES, hipMemcpyDeviceToHost));
  bad = 0;
  for (i = 0; i < N; ++i)
    for (l = 0; l < L; ++l)
      for (c = 0; c < 2; ++c)
        bad += memcmp(packed + (((size_t)i * L + l) * 2 + c) * PAGE, pool + page_at(l, c, src_ids[i]),
                      PAGE) != 0;
  printf("pack of %d blocks (%zu bytes): %d pages differ  %s\n", N, PACK_BYTES, bad,
         bad ? "WRONG" : "ok");
  fails += bad != 0;

  /* unpack into the zeroed pool at other ids */
  HIP_OK(hipMemcpy(dids, dst_ids, sizeof dst_ids, hipMemcpyHostToDevice));
  rc = hs_kv_unpack(dback, L, NB, PAGE, dids, N, dpacked, NULL);
  if (rc != HS_OK) {
    printf("hs_kv_unpack: %d %s\n", rc, hs_last_error());
    return 1;
  }
  HIP_OK(hipDeviceSynchronize());
  HIP_OK(hipMemcpy(back, dback, POOL_BYTES, hipMemcpyDeviceToHost));
  for (j = 0; j < POOL_BYTES; ++j) pool[j] = 0;    /* the expected receiver pool */
  for (i = 0; i < N; ++i)
    for (l = 0; l < L; ++l)
      for (c = 0; c < 2; ++c)
        memcpy(pool + page_at(l, c, dst_ids[i]), packed + (((size_t)i * L + l) * 2 + c) * PAGE,
               PAGE);
  bad = memcmp(pool, back, POOL_BYTES) != 0;
  printf("unpack into another pool: %s\n", bad ? "WRONG" : "ok (every other page still zero)");
  fails += bad;

  /* a bad argument comes back as a status code */
  rc = hs_kv_pack(dpool, L, NB, PAGE, dids, -1, dpacked, NULL);
  printf("pack of -1 blocks: rc %d \"%s\"  %s\n", rc, hs_last_error(),
         rc == HS_EINVAL ? "ok" : "WRONG");
  fails += rc != HS_EINVAL;

  HIP_OK(hipFree(dpool));
  HIP_OK(hipFree(dback));
  HIP_OK(hipFree(dpacked));
  HIP_OK(hipFree(dids));
  free(pool);
  free(back);
  free(packed);
  printf("%s\n", fails ? "FAIL" : "OK");
  return fails != 0;
}
