/*
 * A C host running chunked causal prefill through libhsattn on the GPU
 * (hs_prefill_varlen, two ragged chunks in one call): a bf16 KV cache built
 * here from values that bf16 holds exactly, q in fp32, device memory through
 * the HIP runtime's C API.  The result is checked against a double-precision
 * prefill computed here from the same data (query i of sequence b sits at
 * position ctx_b - S_b + i and sees keys 0..position; query head h reads KV
 * head h / (H / Hkv)): the matrix-core path (use_mfma = 1, with the
 * workspace its query asks for) within the 2e-3 bar, the fp32 row kernel
 * (use_mfma = 0) within 1e-5.  Prints each error and "OK" when both pass.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "hsattn.h"

enum { B = 2, H = 8, HKV = 2, D = 128, BS = 16, MB = 20, NB = 2 * MB, T = 40 + 300 };

#define HIP_OK(x)                                                 \
  do {                                                            \
    hipError_t e_ = (x);                                          \
    if (e_ != hipSuccess) {                                       \
      printf("%s: %s\n", #x, hipGetErrorString(e_));              \
      return 1;                                                   \
    }                                                             \
  } while (0)

static uint32_t seed = 777u;
static uint32_t next(void) { return seed = seed * 1664525u + 1013904223u; }

/* a value bf16 holds exactly: k / 128 for k in [-127, 127] */
static float bf16_value(void) { return (float)((int)((next() >> 9) % 255u) - 127) / 128.0f; }

static uint16_t bf16_bits(float x) {
  uint32_t u;
  memcpy(&u, &x, sizeof u);
  return (uint16_t)(u >> 16);   /* exact: the low 16 bits are zero */
}

int main(void) {
  static float q[T * H * D], out[T * H * D], kf[NB * BS * HKV * D], vf[NB * BS * HKV * D];
  static uint16_t kc[NB * BS * HKV * D], vc[NB * BS * HKV * D];
  static double want[T * H * D], s[MB * BS];
  const int32_t prefix[B] = {100, 0}, chunk[B] = {40, 300};
  int32_t cu[B + 1] = {0, 40, 340}, ctx[B], bt[B * MB];
  const float scale = 0.08838834764831845f;   /* 1 / sqrt(128) */
  int i, b, h, t, d, r, pass, fails = 0;

  for (i = 0; i < T * H * D; ++i) q[i] = bf16_value() * 1.7f;
  for (i = 0; i < NB * BS * HKV * D; ++i) {
    kf[i] = bf16_value();
    vf[i] = bf16_value();
    kc[i] = bf16_bits(kf[i]);
    vc[i] = bf16_bits(vf[i]);
  }
  for (b = 0; b < B; ++b) {
    ctx[b] = prefix[b] + chunk[b];
    for (i = 0; i < MB; ++i) bt[b * MB + i] = (b * MB + i * 7) % NB;   /* distinct per row */
  }

  for (b = 0; b < B; ++b)
    for (r = 0; r < chunk[b]; ++r) {
      const int pos = ctx[b] - chunk[b] + r;
      for (h = 0; h < H; ++h) {
        const int kvh = h / (H / HKV);
        const float* qr = q + ((size_t)(cu[b] + r) * H + h) * D;
        double m = -1e300, l = 0.0;
        for (t = 0; t <= pos; ++t) {
          const float* k = kf + (((size_t)bt[b * MB + t / BS] * BS + t % BS) * HKV + kvh) * D;
          double dot = 0.0;
          for (d = 0; d < D; ++d) dot += (double)qr[d] * k[d];
          s[t] = scale * dot;
          if (s[t] > m) m = s[t];
        }
        for (t = 0; t <= pos; ++t) l += (s[t] = exp(s[t] - m));
        for (d = 0; d < D; ++d) {
          double o = 0.0;
          for (t = 0; t <= pos; ++t)
            o += s[t] * vf[(((size_t)bt[b * MB + t / BS] * BS + t % BS) * HKV + kvh) * D + d];
          want[((size_t)(cu[b] + r) * H + h) * D + d] = o / l;
        }
      }
    }

  {
    float *dq, *dout;
    uint16_t *dk, *dv;
    int32_t *dcu, *dctx, *dbt;
    void* ws = NULL;
    HIP_OK(hipMalloc((void**)&dq, sizeof q));
    HIP_OK(hipMalloc((void**)&dout, sizeof out));
    HIP_OK(hipMalloc((void**)&dk, sizeof kc));
    HIP_OK(hipMalloc((void**)&dv, sizeof vc));
    HIP_OK(hipMalloc((void**)&dcu, sizeof cu));
    HIP_OK(hipMalloc((void**)&dctx, sizeof ctx));
    HIP_OK(hipMalloc((void**)&dbt, sizeof bt));
    HIP_OK(hipMemcpy(dq, q, sizeof q, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(dk, kc, sizeof kc, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(dv, vc, sizeof vc, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(dcu, cu, sizeof cu, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(dctx, ctx, sizeof ctx, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(dbt, bt, sizeof bt, hipMemcpyHostToDevice));
    for (pass = 0; pass < 2; ++pass) {
      const int mfma = pass == 0;
      const double bar = mfma ? 2e-3 : 1e-5;
      const size_t need = hs_prefill_workspace_bytes(B, 300, H, D, mfma);
      double err = 0.0;
      int rc;
      if (need > 0) HIP_OK(hipMalloc(&ws, need));
      rc = hs_prefill_varlen(dq, dcu, 300, dk, dv, HS_DTYPE_BF16, NB, dbt, dctx, dout, B, H, HKV,
                             D, BS, MB, scale, mfma, ws, need, NULL);
      if (rc != HS_OK) {
        printf("hs_prefill_varlen(use_mfma=%d): %d %s\n", mfma, rc, hs_last_error());
        return 1;
      }
      HIP_OK(hipDeviceSynchronize());
      HIP_OK(hipMemcpy(out, dout, sizeof out, hipMemcpyDeviceToHost));
      for (i = 0; i < T * H * D; ++i) {
        const double e = fabs(out[i] - want[i]);
        if (!(e <= err)) err = e;   /* NaN counts */
      }
      printf("use_mfma=%d workspace %zu bytes: max abs err %.3e (bar %.0e)  %s\n", mfma, need, err,
             bar, err <= bar ? "ok" : "WRONG");
      fails += !(err <= bar);
      if (ws) HIP_OK(hipFree(ws));
      ws = NULL;
    }
    HIP_OK(hipFree(dq));
    HIP_OK(hipFree(dout));
    HIP_OK(hipFree(dk));
    HIP_OK(hipFree(dv));
    HIP_OK(hipFree(dcu));
    HIP_OK(hipFree(dctx));
    HIP_OK(hipFree(dbt));
  }
  printf("%s\n", fails ? "FAIL" : "OK");
  return fails != 0;
}
