/*
 * abi_smoke.c -- the C ABI of libloopback_read.so used from C alone (no Python, no torch): device buffers from
 * hipMalloc, one read of n = 3 fp32 sources of width 64 over 37 tokens, checked on the host against what needs no
 * restatement of the read:
 *   - ldr_rstd_fwd: r = 1 / sqrt(mean(v^2) + eps) per token (the closed form), to 1e-6 relative;
 *   - ldr_read_fwd_online with a zero query and cbar == c0: out == base and tc == c0 bitwise (the softmax is then the
 *     prior's own);
 *   - with a random query: sum_i tc_i == sum_i c0_i per token (the installed coefficients keep the prior's mass),
 *     and out == base + sum_i (tc_i - cbar_i) v_i from the returned tc, to 1e-5 of the output's RMS;
 *   - argument errors come back as negative codes before any launch, with a message from ldr_strerror.
 * Prints "abi smoke: ok" and exits 0, or names the failed check and exits 1. Built by loopback_amd.build.
 */
#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "loopback_read.h"

#define T 37
#define D 64
#define N 3

static int fails = 0;

static void check(int ok, const char* what) {
  if (!ok) {
    fprintf(stderr, "abi smoke: FAILED %s\n", what);
    ++fails;
  }
}

static int hip_ok(hipError_t e, const char* what) {
  if (e != hipSuccess) {
    fprintf(stderr, "abi smoke: %s: %s\n", what, hipGetErrorString(e));
    exit(2);
  }
  return 1;
}

static void* dev_copy(const void* host, size_t bytes) {
  void* p = NULL;
  hip_ok(hipMalloc(&p, bytes), "hipMalloc");
  if (host) hip_ok(hipMemcpy(p, host, bytes, hipMemcpyHostToDevice), "hipMemcpy to device");
  return p;
}

static float frand(unsigned* s) {   /* uniform in [-1, 1): a fixed linear congruential sequence */
  *s = *s * 1664525u + 1013904223u;
  return (float)((*s >> 8) & 0xffffff) / 8388608.0f - 1.0f;
}

int main(void) {
  unsigned seed = 12345u;
  static float v[N][T * D], base[T * D], cbar[T * N], c0[N], q[D], out[T * D], tc[T * N], r[N][T];
  for (int i = 0; i < N; ++i)
    for (int k = 0; k < T * D; ++k) v[i][k] = frand(&seed) * (0.5f + 0.25f * (float)i);
  for (int k = 0; k < T * D; ++k) base[k] = frand(&seed);
  for (int i = 0; i < N; ++i) c0[i] = 0.3f + 0.2f * (float)i;
  for (int t = 0; t < T; ++t)
    for (int i = 0; i < N; ++i) cbar[t * N + i] = c0[i];   /* cbar == c0 for the identity */
  const float eps = 1e-6f, inv = 1.0f / sqrtf((float)D);

  float* dv[N];
  float* dr[N];
  uint64_t vp[N], rp[N];
  for (int i = 0; i < N; ++i) {
    dv[i] = (float*)dev_copy(v[i], sizeof(v[i]));
    dr[i] = (float*)dev_copy(NULL, sizeof(r[i]));
    vp[i] = (uint64_t)(uintptr_t)dv[i];
    rp[i] = (uint64_t)(uintptr_t)dr[i];
  }
  float* dbase = (float*)dev_copy(base, sizeof(base));
  float* dcbar = (float*)dev_copy(cbar, sizeof(cbar));
  float* dc0 = (float*)dev_copy(c0, sizeof(c0));
  float* dq = (float*)dev_copy(NULL, sizeof(q));
  float* dout = (float*)dev_copy(NULL, sizeof(out));
  float* dtc = (float*)dev_copy(NULL, sizeof(tc));
  float* ddots = (float*)dev_copy(NULL, sizeof(float) * N * T);
  hipStream_t st;
  hip_ok(hipStreamCreate(&st), "hipStreamCreate");

  check(ldr_abi_version() == LDR_ABI_VERSION, "ldr_abi_version == the header's LDR_ABI_VERSION");
  /* the scale of every source, against its closed form */
  for (int i = 0; i < N; ++i) check(ldr_rstd_fwd(dv[i], dr[i], T, D, eps, LDR_F32, st) == LDR_OK, "ldr_rstd_fwd");
  hip_ok(hipStreamSynchronize(st), "sync");
  for (int i = 0; i < N; ++i) {
    hip_ok(hipMemcpy(r[i], dr[i], sizeof(r[i]), hipMemcpyDeviceToHost), "hipMemcpy r");
    for (int t = 0; t < T; ++t) {
      double ss = 0.0;
      for (int k = 0; k < D; ++k) ss += (double)v[i][t * D + k] * v[i][t * D + k];
      const double want = 1.0 / sqrt(ss / D + eps);
      if (fabs(r[i][t] - want) > 1e-6 * want) { check(0, "rstd against its closed form"); t = T; i = N; }
    }
  }

  /* zero query, cbar == c0: out == base and tc == c0 bitwise */
  memset(q, 0, sizeof(q));
  hip_ok(hipMemcpy(dq, q, sizeof(q), hipMemcpyHostToDevice), "hipMemcpy q");
  check(ldr_read_fwd_online(vp, rp, N, dq, ddots, T, dbase, NULL, 0.f, dcbar, N, dc0, N, 1.f, inv, dout, dtc, NULL,
                            NULL, T, D, LDR_F32, st) == LDR_OK, "ldr_read_fwd_online (zero query)");
  hip_ok(hipStreamSynchronize(st), "sync");
  hip_ok(hipMemcpy(out, dout, sizeof(out), hipMemcpyDeviceToHost), "hipMemcpy out");
  hip_ok(hipMemcpy(tc, dtc, sizeof(tc), hipMemcpyDeviceToHost), "hipMemcpy tc");
  check(memcmp(out, base, sizeof(out)) == 0, "zero query: out == base bitwise");
  int tc_eq = 1;
  for (int t = 0; t < T; ++t)
    for (int i = 0; i < N; ++i) tc_eq &= memcmp(&tc[t * N + i], &c0[i], sizeof(float)) == 0;
  check(tc_eq, "zero query: tc == c0 bitwise");

  /* a random query and cbar: the prior's mass kept, and out from the returned coefficients */
  for (int k = 0; k < D; ++k) q[k] = frand(&seed) * 2.0f;
  for (int k = 0; k < T * N; ++k) cbar[k] = 0.4f + 0.3f * frand(&seed);
  hip_ok(hipMemcpy(dq, q, sizeof(q), hipMemcpyHostToDevice), "hipMemcpy q");
  hip_ok(hipMemcpy(dcbar, cbar, sizeof(cbar), hipMemcpyHostToDevice), "hipMemcpy cbar");
  check(ldr_read_fwd_online(vp, rp, N, dq, ddots, T, dbase, NULL, 0.f, dcbar, N, dc0, N, 1.f, inv, dout, dtc, NULL,
                            NULL, T, D, LDR_F32, st) == LDR_OK, "ldr_read_fwd_online");
  hip_ok(hipStreamSynchronize(st), "sync");
  hip_ok(hipMemcpy(out, dout, sizeof(out), hipMemcpyDeviceToHost), "hipMemcpy out");
  hip_ok(hipMemcpy(tc, dtc, sizeof(tc), hipMemcpyDeviceToHost), "hipMemcpy tc");
  const double mass = (double)c0[0] + c0[1] + c0[2];
  double worst_mass = 0.0, worst = 0.0, ss_out = 0.0;
  for (int t = 0; t < T; ++t) {
    double m = 0.0;
    for (int i = 0; i < N; ++i) m += tc[t * N + i];
    if (fabs(m - mass) > worst_mass) worst_mass = fabs(m - mass);
    for (int k = 0; k < D; ++k) {
      double want = base[t * D + k];
      for (int i = 0; i < N; ++i) want += ((double)tc[t * N + i] - cbar[t * N + i]) * v[i][t * D + k];
      const double e = fabs(out[t * D + k] - want);
      if (e > worst) worst = e;
      ss_out += want * want;
    }
  }
  const double rms = sqrt(ss_out / (T * D));
  check(worst_mass <= 1e-5 * mass, "sum of tc == sum of c0");
  check(worst <= 1e-5 * rms, "out == base + sum (tc - cbar) v");

  /* argument errors: negative codes before any launch */
  const int e1 = ldr_read_fwd_online(vp, rp, N, dq, ddots, T, dbase, NULL, 0.f, dcbar, N, dc0, N, 1.f, inv, dout,
                                     dtc, NULL, NULL, T, D, 7, st);
  check(e1 == LDR_E_DTYPE && ldr_strerror(e1) != NULL && strlen(ldr_strerror(e1)) > 0, "bad dtype rejected");
  check(ldr_rstd_fwd(NULL, dr[0], T, D, eps, LDR_F32, st) == LDR_E_ARG, "null pointer rejected");

  for (int i = 0; i < N; ++i) { hipFree(dv[i]); hipFree(dr[i]); }
  hipFree(dbase); hipFree(dcbar); hipFree(dc0); hipFree(dq); hipFree(dout); hipFree(dtc); hipFree(ddots);
  hipStreamDestroy(st);
  if (fails) return 1;
  printf("abi smoke: ok (max |out - ref| / rms %.2e, mass %.2e)\n", worst / rms, worst_mass);
  return 0;
}
