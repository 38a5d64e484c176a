/*
 * abi_smoke.c -- the C ABI of libloopback_read.so used from C alone (no Python, no torch): device buffers from
 * hipMalloc, reads of n = 3 sources of width 64 over 37 tokens, every result checked on the host against what needs
 * no restatement of the read -- a closed form, an identity, another entry point, or a plain dot product:
 *   - ldr_rstd_fwd: r = 1 / sqrt(mean(v^2) + eps) per token, to 1e-6 relative; ldr_rstd_bwd: gr (-r^3) / d v;
 *   - ldr_read_fwd_online with a zero query and cbar == c0: out == base and tc == c0 bitwise (the prior's softmax);
 *     with a random query: sum_i tc_i == sum_i c0_i per token (the prior's mass kept), and out == base +
 *     sum_i (tc_i - cbar_i) v_i from the returned tc, to 1e-5 of the output's RMS;
 *   - ldr_read_fwd on the scores the online read stored: tc and p bitwise the online read's, out to 1e-5 x RMS;
 *     ldr_read_fwd_any (addresses in device arrays) the same read to 1e-5 x RMS;
 *   - ldr_read_bwd1 + ldr_reduce_rows and ldr_read_bwd1_noalloc: the same bits (dq, dcbar, dr, the pass-2 pairs);
 *     dcbar == -g . v_i per token and source (a dot product);
 *   - ldr_read_bwd2_list: dv_i == w_i g + dzr_i q from the returned pairs; ldr_dv_assemble of one read, per-read
 *     rounding: the same bits, and dv_neg == -dv bitwise;
 *   - ldr_write_dots, fp32 and bf16 (matrix cores, the operand table from ldr_split_queries): the
 *     update bitwise h - x rounded as torch rounds it, its scale against the closed form, the scores against a
 *     double-precision dot product to 1e-5 x RMS;
 *   - ldr_blend_sum: the sum of beta g_j, to fp32 rounding;
 *   - argument errors come back as negative codes before any launch, with a message from ldr_strerror.
 * Prints "abi smoke: ok" and exits 0, or names every failed check and exits 1 (2 on a HIP runtime error). Built by
 * loopback_amd.build; run by tests/test_gpu_c_abi.py.
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
#define NQ 5

static int fails = 0;

static void check(int ok, const char* what) {
  if (!ok) {
    fprintf(stderr, "abi smoke: FAILED %s\n", what);
    ++fails;
  }
}

static void hip_ok(hipError_t e, const char* what) {
  if (e != hipSuccess) {
    fprintf(stderr, "abi smoke: %s: %s\n", what, hipGetErrorString(e));
    exit(2);
  }
}

static void* dev_copy(const void* host, size_t bytes) {
  void* p = NULL;
  hip_ok(hipMalloc(&p, bytes), "hipMalloc");
  if (host) hip_ok(hipMemcpy(p, host, bytes, hipMemcpyHostToDevice), "hipMemcpy to device");
  return p;
}

static void to_host(void* host, const void* dev, size_t bytes) {
  hip_ok(hipMemcpy(host, dev, bytes, hipMemcpyDeviceToHost), "hipMemcpy to host");
}

static uint64_t addr(const void* p) { return (uint64_t)(uintptr_t)p; }

static float frand(unsigned* s) {   /* uniform in [-1, 1): a fixed linear congruential sequence */
  *s = *s * 1664525u + 1013904223u;
  return (float)((*s >> 8) & 0xffffff) / 8388608.0f - 1.0f;
}

static uint16_t to_bf16(float f) {   /* round to nearest even, as torch converts */
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static float from_bf16(uint16_t b) {
  const uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* max |a - b| / RMS(b) over n values */
static double err_rms(const float* a, const double* b, int n) {
  double worst = 0.0, ss = 0.0;
  for (int k = 0; k < n; ++k) {
    const double e = fabs((double)a[k] - b[k]);
    if (e > worst) worst = e;
    ss += b[k] * b[k];
  }
  return ss > 0.0 ? worst / sqrt(ss / n) : worst;
}

static double err_rms_f(const float* a, const float* b, int n) {
  static double tmp[T * D * N];
  for (int k = 0; k < n; ++k) tmp[k] = b[k];
  return err_rms(a, tmp, n);
}

int main(void) {
  unsigned seed = 12345u;
  static float v[N][T * D], base[T * D], cbar[T * N], c0[N], q[D], out[T * D], tc[T * N], p[T * N], r[N][T];
  static double ref[T * D * N];
  const float eps = 1e-6f, inv = 1.0f / sqrtf((float)D);
  for (int i = 0; i < N; ++i)
    for (int k = 0; k < T * D; ++k) v[i][k] = frand(&seed) * (0.5f + 0.25f * (float)i);
  for (int k = 0; k < T * D; ++k) base[k] = frand(&seed);
  for (int i = 0; i < N; ++i) c0[i] = 0.3f + 0.2f * (float)i;
  for (int t = 0; t < T; ++t)
    for (int i = 0; i < N; ++i) cbar[t * N + i] = c0[i];   /* cbar == c0 for the identity */

  float *dv[N], *dr[N];
  uint64_t vp[N], rp[N];
  for (int i = 0; i < N; ++i) {
    dv[i] = (float*)dev_copy(v[i], sizeof(v[i]));
    dr[i] = (float*)dev_copy(NULL, sizeof(r[i]));
    vp[i] = addr(dv[i]);
    rp[i] = addr(dr[i]);
  }
  float* dbase = (float*)dev_copy(base, sizeof(base));
  float* dcbar = (float*)dev_copy(cbar, sizeof(cbar));
  float* dc0 = (float*)dev_copy(c0, sizeof(c0));
  float* dq = (float*)dev_copy(NULL, sizeof(q));
  float* dout = (float*)dev_copy(NULL, sizeof(out));
  float* dtc = (float*)dev_copy(NULL, sizeof(tc));
  float* dp = (float*)dev_copy(NULL, sizeof(p));
  float* ddots = (float*)dev_copy(NULL, sizeof(float) * N * T);
  hipStream_t st;
  hip_ok(hipStreamCreate(&st), "hipStreamCreate");

  check(ldr_abi_version() == LDR_ABI_VERSION, "ldr_abi_version == the header's LDR_ABI_VERSION");

  /* ---- the scale and its gradient, against their closed forms ---- */
  for (int i = 0; i < N; ++i) check(ldr_rstd_fwd(dv[i], dr[i], T, D, eps, LDR_F32, st) == LDR_OK, "ldr_rstd_fwd");
  hip_ok(hipStreamSynchronize(st), "sync");
  for (int i = 0; i < N; ++i) {
    to_host(r[i], dr[i], sizeof(r[i]));
    for (int t = 0; t < T; ++t) {
      double ss = 0.0;
      for (int k = 0; k < D; ++k) ss += (double)v[i][t * D + k] * v[i][t * D + k];
      const double want = 1.0 / sqrt(ss / D + eps);
      if (fabs(r[i][t] - want) > 1e-6 * want) { check(0, "rstd against its closed form"); t = T; i = N; }
    }
  }
  {
    static float gr[T], gx[T * D];
    for (int t = 0; t < T; ++t) gr[t] = frand(&seed);
    float* dgr = (float*)dev_copy(gr, sizeof(gr));
    float* dgx = (float*)dev_copy(NULL, sizeof(gx));
    check(ldr_rstd_bwd(dv[0], dr[0], dgr, dgx, T, D, LDR_F32, st) == LDR_OK, "ldr_rstd_bwd");
    hip_ok(hipStreamSynchronize(st), "sync");
    to_host(gx, dgx, sizeof(gx));
    for (int t = 0; t < T; ++t)
      for (int k = 0; k < D; ++k)
        ref[t * D + k] = (double)gr[t] * -((double)r[0][t] * r[0][t] * r[0][t]) / D * v[0][t * D + k];
    check(err_rms(gx, ref, T * D) <= 1e-6, "rstd gradient against its closed form");
    hipFree(dgr);
    hipFree(dgx);
  }

  /* ---- zero query, cbar == c0: out == base and tc == c0 bitwise ---- */
  memset(q, 0, sizeof(q));
  hip_ok(hipMemcpy(dq, q, sizeof(q), hipMemcpyHostToDevice), "hipMemcpy q");
  check(ldr_read_fwd_online(vp, rp, N, dq, ddots, T, dbase, NULL, 0.f, dcbar, N, dc0, N, 1.f, inv, dout, dtc, NULL,
                            NULL, T, D, LDR_F32, st) == LDR_OK, "ldr_read_fwd_online (zero query)");
  hip_ok(hipStreamSynchronize(st), "sync");
  to_host(out, dout, sizeof(out));
  to_host(tc, dtc, sizeof(tc));
  check(memcmp(out, base, sizeof(out)) == 0, "zero query: out == base bitwise");
  int tc_eq = 1;
  for (int t = 0; t < T; ++t)
    for (int i = 0; i < N; ++i) tc_eq &= memcmp(&tc[t * N + i], &c0[i], sizeof(float)) == 0;
  check(tc_eq, "zero query: tc == c0 bitwise");

  /* ---- a random query and cbar: the prior's mass kept, and out from the returned coefficients ---- */
  for (int k = 0; k < D; ++k) q[k] = frand(&seed) * 2.0f;
  for (int k = 0; k < T * N; ++k) cbar[k] = 0.4f + 0.3f * frand(&seed);
  hip_ok(hipMemcpy(dq, q, sizeof(q), hipMemcpyHostToDevice), "hipMemcpy q");
  hip_ok(hipMemcpy(dcbar, cbar, sizeof(cbar), hipMemcpyHostToDevice), "hipMemcpy cbar");
  check(ldr_read_fwd_online(vp, rp, N, dq, ddots, T, dbase, NULL, 0.f, dcbar, N, dc0, N, 1.f, inv, dout, dtc, dp,
                            NULL, T, D, LDR_F32, st) == LDR_OK, "ldr_read_fwd_online");
  hip_ok(hipStreamSynchronize(st), "sync");
  to_host(out, dout, sizeof(out));
  to_host(tc, dtc, sizeof(tc));
  to_host(p, dp, sizeof(p));
  const double mass = (double)c0[0] + c0[1] + c0[2];
  double worst_mass = 0.0;
  for (int t = 0; t < T; ++t) {
    double m = 0.0;
    for (int i = 0; i < N; ++i) m += tc[t * N + i];
    if (fabs(m - mass) > worst_mass) worst_mass = fabs(m - mass);
    for (int k = 0; k < D; ++k) {
      double want = base[t * D + k];
      for (int i = 0; i < N; ++i) want += ((double)tc[t * N + i] - cbar[t * N + i]) * v[i][t * D + k];
      ref[t * D + k] = want;
    }
  }
  const double out_err = err_rms(out, ref, T * D);
  check(worst_mass <= 1e-5 * mass, "sum of tc == sum of c0");
  check(out_err <= 1e-5, "out == base + sum (tc - cbar) v");

  /* ---- the read from the stored scores, and the any-shape read, against the online read ---- */
  {
    static float out2[T * D], tc2[T * N], p2[T * N], nxt[N];
    float* dout2 = (float*)dev_copy(NULL, sizeof(out2));
    float* dtc2 = (float*)dev_copy(NULL, sizeof(tc2));
    float* dp2 = (float*)dev_copy(NULL, sizeof(p2));
    float* dnxt = (float*)dev_copy(NULL, sizeof(nxt));
    check(ldr_read_fwd(vp, rp, N, ddots, T, dbase, NULL, 0.f, dcbar, N, dc0, N, 1.f, inv, dout2, dtc2, dp2, dnxt, T,
                       D, LDR_F32, st) == LDR_OK, "ldr_read_fwd");
    hip_ok(hipStreamSynchronize(st), "sync");
    to_host(out2, dout2, sizeof(out2));
    to_host(tc2, dtc2, sizeof(tc2));
    to_host(p2, dp2, sizeof(p2));
    to_host(nxt, dnxt, sizeof(nxt));
    check(memcmp(tc2, tc, sizeof(tc)) == 0 && memcmp(p2, p, sizeof(p)) == 0,
          "stored-score read: tc and p bitwise the online read's");
    check(err_rms_f(out2, out, T * D) <= 1e-5, "stored-score read: out == the online read's");
    check(memcmp(nxt, c0, sizeof(c0)) == 0, "stored-score read: next_prior == c0");

    uint64_t* dvp = (uint64_t*)dev_copy(vp, sizeof(vp));
    uint64_t* drp = (uint64_t*)dev_copy(rp, sizeof(rp));
    check(ldr_read_fwd_any(dvp, drp, N, NULL, ddots, T, dbase, NULL, 0.f, dcbar, N, dc0, N, 1.f, inv, dout2, dtc2,
                           dp2, NULL, T, D, LDR_F32, st) == LDR_OK, "ldr_read_fwd_any");
    hip_ok(hipStreamSynchronize(st), "sync");
    to_host(out2, dout2, sizeof(out2));
    to_host(tc2, dtc2, sizeof(tc2));
    check(err_rms_f(out2, out, T * D) <= 1e-5, "any-shape read: out == the row-layout read's");
    check(err_rms_f(tc2, tc, T * N) <= 1e-6, "any-shape read: tc == the row-layout read's");
    hipFree(dout2); hipFree(dtc2); hipFree(dp2); hipFree(dnxt); hipFree(dvp); hipFree(drp);
  }

  /* ---- backward pass 1: with a workspace and without, the same bits; dcbar == -g . v_i ---- */
  static float g[T * D], wz[2][N * T * 2], dcb[2][T * N], dra[2][N][T], dqv[2][D];
  for (int k = 0; k < T * D; ++k) g[k] = frand(&seed);
  float* dg = (float*)dev_copy(g, sizeof(g));
  float* dwz[2];
  float* ddcb[2];
  float* dqo[2];
  float* ddr[2][N];
  uint64_t drv[2][N];
  for (int c = 0; c < 2; ++c) {
    dwz[c] = (float*)dev_copy(NULL, sizeof(wz[c]));
    ddcb[c] = (float*)dev_copy(NULL, sizeof(dcb[c]));
    dqo[c] = (float*)dev_copy(NULL, sizeof(dqv[c]));
    for (int i = 0; i < N; ++i) {
      ddr[c][i] = (float*)dev_copy(NULL, sizeof(dra[c][i]));
      drv[c][i] = addr(ddr[c][i]);
    }
  }
  const int64_t parts = ldr_read_bwd1_parts(T, D);
  check(parts > 0, "ldr_read_bwd1_parts");
  float* dpart = (float*)dev_copy(NULL, sizeof(float) * (size_t)(parts > 0 ? parts : 1) * D);
  check(ldr_read_bwd1(vp, rp, N, dg, NULL, dp, ddots, T, dtc, dcbar, N, dc0, N, 1.f, inv, ddcb[0], N, drv[0], 0,
                      dwz[0], T, dpart, D, NULL, NULL, 0.f, T, D, LDR_F32, st) == LDR_OK, "ldr_read_bwd1");
  check(ldr_reduce_rows(dpart, parts, D, dqo[0], st) == LDR_OK, "ldr_reduce_rows");
  check(ldr_read_bwd1_noalloc(vp, rp, N, dg, NULL, dp, ddots, T, dtc, dcbar, N, dc0, N, 1.f, inv, ddcb[1], N, drv[1],
                              0, dwz[1], T, dqo[1], NULL, NULL, 0.f, T, D, LDR_F32, st) == LDR_OK,
        "ldr_read_bwd1_noalloc");
  hip_ok(hipStreamSynchronize(st), "sync");
  for (int c = 0; c < 2; ++c) {
    to_host(wz[c], dwz[c], sizeof(wz[c]));
    to_host(dcb[c], ddcb[c], sizeof(dcb[c]));
    to_host(dqv[c], dqo[c], sizeof(dqv[c]));
    for (int i = 0; i < N; ++i) to_host(dra[c][i], ddr[c][i], sizeof(dra[c][i]));
  }
  check(memcmp(dqv[0], dqv[1], sizeof(dqv[0])) == 0 && memcmp(dcb[0], dcb[1], sizeof(dcb[0])) == 0 &&
        memcmp(wz[0], wz[1], sizeof(wz[0])) == 0 && memcmp(dra[0], dra[1], sizeof(dra[0])) == 0,
        "backward pass 1 without a workspace: the bits of the workspace path");
  for (int t = 0; t < T; ++t)
    for (int i = 0; i < N; ++i) {
      double gd = 0.0;
      for (int k = 0; k < D; ++k) gd += (double)g[t * D + k] * v[i][t * D + k];
      ref[t * N + i] = -gd;
    }
  check(err_rms(dcb[0], ref, T * N) <= 1e-5, "dcbar == -g . v");
  int finite = 1;
  for (int k = 0; k < D; ++k) finite &= isfinite(dqv[0][k]) != 0;
  check(finite, "dq finite");

  /* ---- backward pass 2: the list layout's gradients from the pairs, and the stacked assembly of one read ---- */
  {
    static float gl[N][T * D], ga[T * D], gn[T * D];
    float* dgl[N];
    uint64_t glp[N];
    for (int i = 0; i < N; ++i) {
      dgl[i] = (float*)dev_copy(NULL, sizeof(gl[i]));
      glp[i] = addr(dgl[i]);
    }
    check(ldr_read_bwd2_list(glp, N, 0, dg, dq, dwz[0], T, T, D, LDR_F32, st) == LDR_OK, "ldr_read_bwd2_list");
    hip_ok(hipStreamSynchronize(st), "sync");
    double worst = 0.0;
    for (int i = 0; i < N; ++i) {
      to_host(gl[i], dgl[i], sizeof(gl[i]));
      for (int t = 0; t < T; ++t) {
        const double w = wz[0][(i * T + t) * 2], dzr = wz[0][(i * T + t) * 2 + 1];
        for (int k = 0; k < D; ++k) ref[t * D + k] = w * g[t * D + k] + dzr * q[k];
      }
      const double e = err_rms(gl[i], ref, T * D);
      if (e > worst) worst = e;
    }
    check(worst <= 1e-6, "list gradients == w g + dzr q from the returned pairs");
    float* dga = (float*)dev_copy(NULL, sizeof(ga));
    float* dgn = (float*)dev_copy(NULL, sizeof(gn));
    int same = 1, neg = 1;
    for (int i = 0; i < N; ++i) {
      const uint64_t gt1[1] = {addr(dg)}, wz1[1] = {addr(dwz[0] + (size_t)i * T * 2)}, q1[1] = {addr(dq)};
      check(ldr_dv_assemble(gt1, wz1, q1, 1, dv[i], dr[i], NULL, NULL, 0.f, 1, dga, dgn, T, D, LDR_F32, st) == LDR_OK,
            "ldr_dv_assemble");
      hip_ok(hipStreamSynchronize(st), "sync");
      to_host(ga, dga, sizeof(ga));
      to_host(gn, dgn, sizeof(gn));
      same &= memcmp(ga, gl[i], sizeof(ga)) == 0;
      for (int k = 0; k < T * D; ++k) neg &= gn[k] == -ga[k] && !signbit(gn[k]) != !signbit(ga[k]);
    }
    check(same, "stacked assembly of one read, per-read rounding: the list layout's bits");
    check(neg, "dv_neg == -dv bitwise");
    for (int i = 0; i < N; ++i) hipFree(dgl[i]);
    hipFree(dga);
    hipFree(dgn);
  }

  /* ---- the write: fp32 on the vector units, bf16 on the matrix cores ---- */
  {
    static float h[T * D], x[T * D], vo[T * D], ro[T], qw[NQ * D], sc[NQ * T];
    static uint16_t h16[T * D], x16[T * D], v16[T * D];
    for (int k = 0; k < T * D; ++k) { h[k] = frand(&seed); x[k] = frand(&seed); }
    for (int k = 0; k < NQ * D; ++k) qw[k] = 0.3f * frand(&seed);
    float* dh = (float*)dev_copy(h, sizeof(h));
    float* dx = (float*)dev_copy(x, sizeof(x));
    float* dvo = (float*)dev_copy(NULL, sizeof(vo));
    float* dro = (float*)dev_copy(NULL, sizeof(ro));
    float* dqw = (float*)dev_copy(qw, sizeof(qw));
    float* dsc = (float*)dev_copy(NULL, sizeof(sc));
    for (int pass = 0; pass < 2; ++pass) {   /* 0: fp32, 1: bf16 */
      const int dt = pass ? LDR_BF16 : LDR_F32;
      if (pass) {
        for (int k = 0; k < T * D; ++k) { h16[k] = to_bf16(h[k]); x16[k] = to_bf16(x[k]); }
        hip_ok(hipMemcpy(dh, h16, sizeof(h16), hipMemcpyHostToDevice), "hipMemcpy h");
        hip_ok(hipMemcpy(dx, x16, sizeof(x16), hipMemcpyHostToDevice), "hipMemcpy x");
      }
      /* the queries' bf16 parts: the matrix cores' operand for every update dtype */
      const int64_t elems = ldr_query_parts_elems(NQ, D);
      check(elems > 0, "ldr_query_parts_elems");
      void* qb = dev_copy(NULL, sizeof(uint16_t) * (size_t)(elems > 0 ? elems : 1));
      check(ldr_split_queries(dqw, NQ, D, qb, st) == LDR_OK, "ldr_split_queries");
      check(ldr_write_dots(dh, dx, dvo, dro, dqw, qb, NQ, 0, dsc, T, D, T, eps, dt, st) == LDR_OK, "ldr_write_dots");
      hip_ok(hipStreamSynchronize(st), "sync");
      to_host(ro, dro, sizeof(ro));
      to_host(sc, dsc, sizeof(sc));
      static float vf[T * D];   /* the update as fp32 values */
      int exact = 1;
      if (pass) {
        to_host(v16, dvo, sizeof(v16));
        for (int k = 0; k < T * D; ++k) {
          exact &= v16[k] == to_bf16(from_bf16(h16[k]) - from_bf16(x16[k]));
          vf[k] = from_bf16(v16[k]);
        }
      } else {
        to_host(vo, dvo, sizeof(vo));
        for (int k = 0; k < T * D; ++k) {
          const float want = h[k] - x[k];
          exact &= memcmp(&vo[k], &want, sizeof(float)) == 0;
          vf[k] = vo[k];
        }
      }
      check(exact, pass ? "bf16 write: the update == round(h - x) bitwise" : "fp32 write: the update == h - x bitwise");
      int scale_ok = 1;
      for (int t = 0; t < T; ++t) {
        double ss = 0.0;
        for (int k = 0; k < D; ++k) ss += (double)vf[t * D + k] * vf[t * D + k];
        const double want = 1.0 / sqrt(ss / D + eps);
        scale_ok &= fabs(ro[t] - want) <= 1e-6 * want;
      }
      check(scale_ok, pass ? "bf16 write: the scale of the rounded update" : "fp32 write: the scale");
      for (int j = 0; j < NQ; ++j)
        for (int t = 0; t < T; ++t) {
          double s = 0.0;
          for (int k = 0; k < D; ++k) s += (double)qw[j * D + k] * vf[t * D + k];
          ref[j * T + t] = s;
        }
      check(err_rms(sc, ref, NQ * T) <= 1e-5, pass ? "bf16 write: scores (matrix cores)" : "fp32 write: scores");
      hipFree(qb);
    }
    hipFree(dh); hipFree(dx); hipFree(dvo); hipFree(dro); hipFree(dqw); hipFree(dsc);
  }

  /* ---- the iteration-end blends' h0 gradient: sum_j beta g_j ---- */
  {
    static float bs[T * D];
    float* dbs = (float*)dev_copy(NULL, sizeof(bs));
    check(ldr_blend_sum(vp, N, 0.75f, 0, dbs, T, D, LDR_F32, st) == LDR_OK, "ldr_blend_sum");
    hip_ok(hipStreamSynchronize(st), "sync");
    to_host(bs, dbs, sizeof(bs));
    for (int k = 0; k < T * D; ++k) {
      double s = 0.0;
      for (int i = 0; i < N; ++i) s += 0.75 * v[i][k];
      ref[k] = s;
    }
    check(err_rms(bs, ref, T * D) <= 1e-6, "blend sum == sum beta g");
    hipFree(dbs);
  }

  /* ---- argument errors: negative codes before any launch ---- */
  const int e1 = ldr_read_fwd_online(vp, rp, N, dq, ddots, T, dbase, NULL, 0.f, dcbar, N, dc0, N, 1.f, inv, dout,
                                     dtc, NULL, NULL, T, D, 7, st);
  check(e1 == LDR_E_DTYPE && ldr_strerror(e1) != NULL && strlen(ldr_strerror(e1)) > 0, "bad dtype rejected");
  check(ldr_rstd_fwd(NULL, dr[0], T, D, eps, LDR_F32, st) == LDR_E_ARG, "null pointer rejected");
  check(ldr_read_fwd(vp, rp, N, ddots, T, (const char*)dbase + 4, NULL, 0.f, dcbar, N, dc0, N, 1.f, inv, dout, dtc,
                     NULL, NULL, T, D, LDR_F32, st) == LDR_E_ALIGN, "unaligned row rejected");
  int vpt = 0, tpr = 0;
  check(ldr_row_layout(7, &vpt, &tpr) == LDR_E_SHAPE, "width 7 has no row layout");
  check(ldr_row_layout(D, &vpt, &tpr) == LDR_OK && vpt * tpr * 8 >= D, "the row layout of width 64");

  for (int i = 0; i < N; ++i) { hipFree(dv[i]); hipFree(dr[i]); }
  for (int c = 0; c < 2; ++c) {
    hipFree(dwz[c]); hipFree(ddcb[c]); hipFree(dqo[c]);
    for (int i = 0; i < N; ++i) hipFree(ddr[c][i]);
  }
  hipFree(dbase); hipFree(dcbar); hipFree(dc0); hipFree(dq); hipFree(dout); hipFree(dtc); hipFree(dp);
  hipFree(ddots); hipFree(dg); hipFree(dpart);
  hipStreamDestroy(st);
  if (fails) return 1;
  printf("abi smoke: ok (read out %.2e x RMS, mass %.2e)\n", out_err, worst_mass);
  return 0;
}
