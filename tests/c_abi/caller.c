/*
 * A C host of libhsattn: compiled against include/hsattn.h as C99 with
 * -pedantic -Werror and linked against libhsattn.so, as a non-Python caller
 * of the paged-attention boundary would be.  It makes the calls a host makes
 * before any device work (version check, workspace-size queries) and checks
 * that bad arguments come back as status codes with messages, which the
 * library reports before touching the GPU, so this runs on a machine
 * without one.  Prints one line per check and "OK" when all pass.
 */
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "hsattn.h"

typedef void (*any_fn)(void);

/* Every declared entry point, by address: a symbol the library does not
 * export fails the link. */
static const any_fn kEntryPoints[] = {
    (any_fn)hs_abi_version,         (any_fn)hs_last_error,
    (any_fn)hs_profile_next_launch, (any_fn)hs_device_cu_count,
    (any_fn)hs_choose_num_splits,   (any_fn)hs_decode_workspace_bytes,
    (any_fn)hs_decode,              (any_fn)hs_decode_noalloc,
    (any_fn)hs_decode_shared_workspace_bytes, (any_fn)hs_decode_shared,
    (any_fn)hs_prefill_workspace_bytes, (any_fn)hs_prefill,
    (any_fn)hs_prefill_varlen,      (any_fn)hs_kv_pack,
    (any_fn)hs_kv_unpack,           (any_fn)hs_kv_gather,
    (any_fn)hs_kv_scatter,          (any_fn)hs_kv_append,
    (any_fn)hs_block_tables,
};

static int fails = 0;

static void expect(const char* what, int rc, int want, const char* needle) {
  const char* msg = hs_last_error();
  const int ok = rc == want && strstr(msg, needle) != NULL;
  printf("%-34s rc %d  \"%s\"  %s\n", what, rc, msg, ok ? "ok" : "WRONG");
  fails += !ok;
}

int main(void) {
  /* a pointer the library must never dereference: every call below fails
   * validation first */
  const void* fake = (const void*)(uintptr_t)0x1000;
  const float* fq = (const float*)fake;
  const int32_t* fi = (const int32_t*)fake;
  float* fo = (float*)(uintptr_t)0x1000;
  size_t need;
  int rc;

  printf("entry points linked: %d\n", (int)(sizeof kEntryPoints / sizeof kEntryPoints[0]));
  if (hs_abi_version() != HS_ABI_VERSION) {
    printf("abi version %d, header %d  WRONG\n", hs_abi_version(), HS_ABI_VERSION);
    fails++;
  }

  /* workspace queries: partitioned decode needs one, a single pass none */
  need = hs_decode_workspace_bytes(2, 4, 4, 64, 16, 64, 0, 0);
  printf("decode workspace (default split): %zu bytes  %s\n", need, need > 0 ? "ok" : "WRONG");
  fails += need == 0;
  need = hs_decode_workspace_bytes(2, 4, 4, 64, 16, 64, 1, 0);
  printf("decode workspace (one pass): %zu bytes  %s\n", need, need == 0 ? "ok" : "WRONG");
  fails += need != 0;

  /* argument errors: hs_decode's reference checks, as status codes */
  rc = hs_decode(NULL, NULL, NULL, HS_DTYPE_F32, 8, NULL, NULL, NULL, 1, 4, 4, 64, 16, 2,
                 0.125f, 0, 0, NULL, 0, NULL);
  expect("decode, null pointers", rc, HS_EINVAL, "null");
  rc = hs_decode(fq, fake, fake, HS_DTYPE_F32, 8, fi, fi, fo, 1, 6, 4, 64, 16, 2, 0.125f, 0, 0,
                 NULL, 0, NULL);
  expect("decode, 6 heads over 4 KV heads", rc, HS_EINVAL, "divisible");
  rc = hs_decode(fq, fake, fake, HS_DTYPE_F32, 8, fi, fi, fo, 1, 4, 4, 96, 16, 2, 0.125f, 0, 0,
                 NULL, 0, NULL);
  expect("decode, head_dim 96", rc, HS_EUNSUPPORTED, "head_dim");
  rc = hs_decode(fq, fake, fake, 7, 8, fi, fi, fo, 1, 4, 4, 64, 16, 2, 0.125f, 0, 0, NULL, 0,
                 NULL);
  expect("decode, unknown kv dtype", rc, HS_EINVAL, "dtype");
  rc = hs_decode(fq, fake, fake, HS_DTYPE_F16, 8, fi, fi, fo, 2, 4, 4, 64, 16, 64, 0.125f, 0, 0,
                 NULL, 0, NULL);
  expect("decode, partitions without workspace", rc, HS_EWORKSPACE, "workspace");

  printf("%s\n", fails ? "FAIL" : "OK");
  return fails != 0;
}
