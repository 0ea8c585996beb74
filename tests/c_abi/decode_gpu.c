/*
 * A C host running paged decode through libhsattn on the GPU: device memory
 * and copies through the HIP runtime's C API, the call through
 * include/hsattn.h, the result against a double-precision decode computed
 * here from the same data (softmax(scale * q.k) . v over the first ctx_b
 * keys of each sequence, keys found through the block table, query head h
 * reading KV head h / (H / Hkv)).  Small fp32 cache, both the default
 * decomposition (with its workspace) and the single pass.  Prints the error
 * of each and "OK" when both are within 1e-5.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include <hip/hip_runtime_api.h>

#include "hsattn.h"

enum { B = 3, H = 4, HKV = 2, D = 64, BS = 16, MB = 8, NB = 32 };

static float frand(uint32_t* s) {
  *s = *s * 1664525u + 1013904223u;
  return (float)((*s >> 8) & 0xffff) / 32768.0f - 1.0f;
}

#define HIP_OK(x)                                                 \
  do {                                                            \
    hipError_t e_ = (x);                                          \
    if (e_ != hipSuccess) {                                       \
      printf("%s: %s\n", #x, hipGetErrorString(e_));              \
      return 1;                                                   \
    }                                                             \
  } while (0)

int main(void) {
  static float q[B * H * D], kc[NB * BS * HKV * D], vc[NB * BS * HKV * D], out[B * H * D];
  static double want[B * H * D];
  int32_t bt[B * MB], ctx[B] = {1, 77, MB * BS};
  const float scale = 0.125f;
  uint32_t seed = 12345u;
  int i, b, h, t, d, pass, fails = 0;

  for (i = 0; i < B * H * D; ++i) q[i] = frand(&seed);
  for (i = 0; i < NB * BS * HKV * D; ++i) kc[i] = frand(&seed);
  for (i = 0; i < NB * BS * HKV * D; ++i) vc[i] = frand(&seed);
  for (b = 0; b < B; ++b)          /* row b's pages, scattered over the pool */
    for (i = 0; i < MB; ++i) bt[b * MB + i] = (i * 11 + b * 3 + 5) % NB;

  for (b = 0; b < B; ++b)
    for (h = 0; h < H; ++h) {
      const int kvh = h / (H / HKV);
      double s[MB * BS], m = -1e300, l = 0.0;
      for (t = 0; t < ctx[b]; ++t) {
        const float* k = kc + (((int64_t)bt[b * MB + t / BS] * BS + t % BS) * HKV + kvh) * D;
        double dot = 0.0;
        for (d = 0; d < D; ++d) dot += (double)q[(b * H + h) * D + d] * k[d];
        s[t] = scale * dot;
        if (s[t] > m) m = s[t];
      }
      for (t = 0; t < ctx[b]; ++t) l += (s[t] = exp(s[t] - m));
      for (d = 0; d < D; ++d) {
        double o = 0.0;
        for (t = 0; t < ctx[b]; ++t)
          o += s[t] * vc[(((int64_t)bt[b * MB + t / BS] * BS + t % BS) * HKV + kvh) * D + d];
        want[(b * H + h) * D + d] = o / l;
      }
    }

  {
    float *dq, *dk, *dv, *dout;
    int32_t *dbt, *dctx;
    void* ws = NULL;
    HIP_OK(hipMalloc((void**)&dq, sizeof q));
    HIP_OK(hipMalloc((void**)&dk, sizeof kc));
    HIP_OK(hipMalloc((void**)&dv, sizeof vc));
    HIP_OK(hipMalloc((void**)&dout, sizeof out));
    HIP_OK(hipMalloc((void**)&dbt, sizeof bt));
    HIP_OK(hipMalloc((void**)&dctx, sizeof ctx));
    HIP_OK(hipMemcpy(dq, q, sizeof q, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(dk, kc, sizeof kc, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(dv, vc, sizeof vc, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(dbt, bt, sizeof bt, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(dctx, ctx, sizeof ctx, hipMemcpyHostToDevice));
    for (pass = 0; pass < 2; ++pass) {
      const int splits = pass == 0 ? 0 : 1;   /* default decomposition, one pass */
      const size_t need = hs_decode_workspace_bytes(B, H, HKV, D, BS, MB, splits, 0);
      double err = 0.0;
      int rc;
      if (need > 0) HIP_OK(hipMalloc(&ws, need));
      rc = hs_decode(dq, dk, dv, HS_DTYPE_F32, NB, dbt, dctx, dout, B, H, HKV, D, BS, MB,
                     scale, splits, 0, ws, need, NULL);
      if (rc != HS_OK) {
        printf("hs_decode(num_splits=%d): %d %s\n", splits, rc, hs_last_error());
        return 1;
      }
      HIP_OK(hipDeviceSynchronize());
      HIP_OK(hipMemcpy(out, dout, sizeof out, hipMemcpyDeviceToHost));
      for (i = 0; i < B * H * D; ++i) {
        const double e = fabs(out[i] - want[i]);
        if (!(e <= err)) err = e;   /* NaN counts */
      }
      printf("num_splits=%d workspace %zu bytes: max abs err %.3e  %s\n", splits, need, err,
             err <= 1e-5 ? "ok" : "WRONG");
      fails += !(err <= 1e-5);
      if (ws) HIP_OK(hipFree(ws));
      ws = NULL;
    }
    HIP_OK(hipFree(dq));
    HIP_OK(hipFree(dk));
    HIP_OK(hipFree(dv));
    HIP_OK(hipFree(dout));
    HIP_OK(hipFree(dbt));
    HIP_OK(hipFree(dctx));
  }
  printf("%s\n", fails ? "FAIL" : "OK");
  return fails != 0;
}
