/* A plain C program that runs the Moebius and affine scans through the C ABI on
 * the GPU (HIP runtime C API for memory and the stream; no C++, no torch) and
 * checks them against a double-precision per-step loop written here:
 *   lam_t = (A_t lam_{t-1} + B_t) / max(C_t lam_{t-1} + 1, 1e-12), lam_{-1} = lam0
 *   h_t   = g_t h_{t-1} + u_t, h_{-1} = 0
 * at rtol 1e-5 / atol 1e-6. Built and run by tests/test_abi_c_client.py (GPU). */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include "kla_hip.h"

#define CHECK_HIP(x)                                                      \
  do {                                                                    \
    hipError_t e_ = (x);                                                  \
    if (e_ != hipSuccess) {                                               \
      fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));             \
      return 1;                                                           \
    }                                                                     \
  } while (0)

static uint64_t rng = 88172645463325252ull;

static double uniform01(void) { /* xorshift64 */
  rng ^= rng << 13;
  rng ^= rng >> 7;
  rng ^= rng << 17;
  return (double)(rng >> 11) / 9007199254740992.0;
}

static int close_enough(const float *got, const double *want, size_t n, const char *name) {
  double worst = 0.0;
  for (size_t i = 0; i < n; ++i) {
    const double r = fabs((double)got[i] - want[i]) / (1e-6 + 1e-5 * fabs(want[i]));
    if (!(r <= worst)) worst = r; /* NaN counts as worst */
  }
  printf("%s: worst |d|/(atol+rtol|ref|) = %.3f\n", name, worst);
  return worst <= 1.0;
}

int main(void) {
  const int64_t B = 2, T = 300, N = 130;
  const size_t n = (size_t)(B * T * N), ns = (size_t)(B * N);
  float *hA = malloc(n * 4), *hB = malloc(n * 4), *hC = malloc(n * 4), *hl0 = malloc(ns * 4), *hout = malloc(n * 4);
  double *want = malloc(n * 8);
  if (!hA || !hB || !hC || !hl0 || !hout || !want) return 1;
  for (size_t i = 0; i < n; ++i) {
    hA[i] = (float)(0.3 + 0.6 * uniform01());
    hB[i] = (float)uniform01();
    hC[i] = (float)uniform01();
  }
  for (size_t i = 0; i < ns; ++i) hl0[i] = (float)(0.5 + uniform01());

  float *dA, *dB, *dC, *dl0, *dout;
  void *wsm, *wsa; /* one workspace per scan kind, each zero-filled once */
  const size_t wsm_bytes = kla_scan_workspace_bytes(KLA_SCAN_MOBIUS_FWD, B, T, N);
  const size_t wsa_bytes = kla_scan_workspace_bytes(KLA_SCAN_AFFINE_FWD, B, T, N);
  CHECK_HIP(hipMalloc((void **)&dA, n * 4));
  CHECK_HIP(hipMalloc((void **)&dB, n * 4));
  CHECK_HIP(hipMalloc((void **)&dC, n * 4));
  CHECK_HIP(hipMalloc((void **)&dl0, ns * 4));
  CHECK_HIP(hipMalloc((void **)&dout, n * 4));
  CHECK_HIP(hipMalloc(&wsm, wsm_bytes));
  CHECK_HIP(hipMalloc(&wsa, wsa_bytes));
  CHECK_HIP(hipMemset(wsm, 0, wsm_bytes));
  CHECK_HIP(hipMemset(wsa, 0, wsa_bytes));
  CHECK_HIP(hipMemcpy(dA, hA, n * 4, hipMemcpyHostToDevice));
  CHECK_HIP(hipMemcpy(dB, hB, n * 4, hipMemcpyHostToDevice));
  CHECK_HIP(hipMemcpy(dC, hC, n * 4, hipMemcpyHostToDevice));
  CHECK_HIP(hipMemcpy(dl0, hl0, ns * 4, hipMemcpyHostToDevice));
  hipStream_t stream;
  CHECK_HIP(hipStreamCreate(&stream));

  int ok = 1;
  /* Moebius forward. */
  int rc = kla_mobius_scan_fwd(dA, dB, dC, NULL, dl0, dout, B, T, N, wsm, wsm_bytes, stream);
  if (rc != KLA_OK) {
    fprintf(stderr, "kla_mobius_scan_fwd: %d %s\n", rc, kla_hip_last_error());
    return 1;
  }
  CHECK_HIP(hipStreamSynchronize(stream));
  CHECK_HIP(hipMemcpy(hout, dout, n * 4, hipMemcpyDeviceToHost));
  for (int64_t b = 0; b < B; ++b)
    for (int64_t l = 0; l < N; ++l) {
      double x = hl0[b * N + l];
      for (int64_t t = 0; t < T; ++t) {
        const size_t i = (size_t)((b * T + t) * N + l);
        double den = (double)hC[i] * x + 1.0;
        if (den < 1e-12) den = 1e-12;
        x = ((double)hA[i] * x + (double)hB[i]) / den;
        want[i] = x;
      }
    }
  ok &= close_enough(hout, want, n, "mobius lam");

  /* Affine forward on g = A, u = B - 0.5. */
  for (size_t i = 0; i < n; ++i) hB[i] = hB[i] - 0.5f;
  CHECK_HIP(hipMemcpy(dB, hB, n * 4, hipMemcpyHostToDevice));
  rc = kla_affine_scan_fwd(KLA_DTYPE_F32, dA, dB, NULL, dout, B, T, N, wsa, wsa_bytes, stream);
  if (rc != KLA_OK) {
    fprintf(stderr, "kla_affine_scan_fwd: %d %s\n", rc, kla_hip_last_error());
    return 1;
  }
  CHECK_HIP(hipStreamSynchronize(stream));
  CHECK_HIP(hipMemcpy(hout, dout, n * 4, hipMemcpyDeviceToHost));
  for (int64_t b = 0; b < B; ++b)
    for (int64_t l = 0; l < N; ++l) {
      double x = 0.0;
      for (int64_t t = 0; t < T; ++t) {
        const size_t i = (size_t)((b * T + t) * N + l);
        x = (double)hA[i] * x + (double)hB[i];
        want[i] = x;
      }
    }
  ok &= close_enough(hout, want, n, "affine h");
  uint32_t gave_up = 1;
  ok &= kla_workspace_failures(wsm, stream, &gave_up) == KLA_OK && gave_up == 0;
  gave_up = 1;
  ok &= kla_workspace_failures(wsa, stream, &gave_up) == KLA_OK && gave_up == 0;

  CHECK_HIP(hipStreamDestroy(stream));
  CHECK_HIP(hipFree(dA));
  CHECK_HIP(hipFree(dB));
  CHECK_HIP(hipFree(dC));
  CHECK_HIP(hipFree(dl0));
  CHECK_HIP(hipFree(dout));
  CHECK_HIP(hipFree(wsm));
  CHECK_HIP(hipFree(wsa));
  free(hA);
  free(hB);
  free(hC);
  free(hl0);
  free(hout);
  free(want);
  if (ok) printf("gpu abi client ok\n");
  return ok ? 0 : 1;
}
