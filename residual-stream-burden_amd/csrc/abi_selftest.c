/*
 * abi_selftest.c -- a plain C caller of the SiHC C ABI (include/sihc_hip.h).
 *
 * Shows that the library needs nothing but the HIP runtime and this header: it
 * allocates device buffers, calls read / write / weight gradient / triangular /
 * fused triangular backward, the per-event fused forward and backward (with and
 * without a state index; also as a deferred call followed by a chained call that
 * finalizes it) and the cell gather / scatter on small fp32 shapes, and
 * checks every result against direct loops over the cell index map (token
 * m = b*G*G + n reads cell n, or cell index[m] with a state index; cell n = wy*G + wx,
 * slot s = uy*K + ux -> carrier pixel (b, wy*K + uy, wx*K + ux)), plus one argument
 * error.
 * Exit status 0 when every check passes. Built next to libsihc_hip.so by build.py.
 */
#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "sihc_hip.h"

enum { B = 2, G = 4, K = 2, S = K * K, C = 24, E = 3, M = B * G * G, GK = G * K };
#define NX (B * GK * GK * C)
#define NZ (M * C)

static int failures;
static unsigned long long rng_state = 12345u;
static float rnd(void) { /* uniform in [-1, 1) from a 64-bit LCG */
  rng_state = rng_state * 6364136223846793005ull + 1442695040888963407ull;
  return (float)((rng_state >> 40) & 0xffffff) / (float)(1 << 23) - 1.0f;
}

static long xoff(int m, int s, int c) {
  const int b = m / (G * G), n = m % (G * G), wy = n / G, wx = n % G;
  const int row = wy * K + s / K, col = wx * K + s % K;
  return ((long)(b * GK + row) * GK + col) * C + c;
}

/* the same with a state index: token m reads cell index[m] of its batch image */
static long xoff_idx(const int32_t *index, int m, int s, int c) {
  if (!index) return xoff(m, s, c);
  const int b = m / (G * G);
  return xoff(b * G * G + index[m], s, c);
}

static int bit_equal(const char *what, const float *got, const float *want, int n) {
  const int ok = memcmp(got, want, (size_t)n * sizeof(float)) == 0;
  printf("%-28s %s\n", what, ok ? "bit-exact ok" : "FAIL (bits differ)");
  if (!ok) ++failures;
  return ok;
}

static void check(const char *what, const float *got, const double *want, int n, double tol) {
  double worst = 0.0, scale = 0.0;
  for (int i = 0; i < n; ++i) {
    const double d = fabs((double)got[i] - want[i]);
    if (d > worst) worst = d;
    if (fabs(want[i]) > scale) scale = fabs(want[i]);
  }
  const int ok = worst <= tol * (scale > 1.0 ? scale : 1.0);
  printf("%-28s max |err| %.3e (scale %.3e) %s\n", what, worst, scale, ok ? "ok" : "FAIL");
  if (!ok) ++failures;
}

#define HIP_OK(call)                                                             \
  do {                                                                           \
    hipError_t e_ = (call);                                                      \
    if (e_ != hipSuccess) {                                                      \
      fprintf(stderr, "%s failed: %s\n", #call, hipGetErrorString(e_));          \
      return 2;                                                                  \
    }                                                                            \
  } while (0)
#define SIHC_OK_(call)                                                           \
  do {                                                                           \
    if ((call) != SIHC_OK) {                                                     \
      fprintf(stderr, "%s failed: %s\n", #call, sihc_last_error());              \
      return 3;                                                                  \
    }                                                                            \
  } while (0)

int main(void) {
  static float x[NX], alpha[E * C * S], beta[E * C * S], z[E][NZ], out[NX], gam[E * C], wg[E * C * S];
  static double want_x[NX], want_z[NZ], want_w[E * C * S];
  for (int i = 0; i < NX; ++i) x[i] = rnd();
  for (int i = 0; i < E * C * S; ++i) alpha[i] = 0.25f + 0.1f * rnd();
  for (int i = 0; i < E * C * S; ++i) beta[i] = 1.0f + 0.1f * rnd();
  for (int e = 0; e < E; ++e)
    for (int i = 0; i < NZ; ++i) z[e][i] = rnd();
  for (int i = 0; i < E * C; ++i) gam[i] = rnd();
  if (sihc_abi_version() != SIHC_ABI_VERSION) {
    fprintf(stderr, "ABI version %d, expected %d\n", sihc_abi_version(), SIHC_ABI_VERSION);
    return 4;
  }

  float *dx, *dalpha, *dbeta, *dout, *dgam, *dw, *dz[E], *dr[E];
  void *work;
  HIP_OK(hipMalloc((void **)&dx, sizeof x));
  HIP_OK(hipMalloc((void **)&dalpha, sizeof alpha));
  HIP_OK(hipMalloc((void **)&dbeta, sizeof beta));
  HIP_OK(hipMalloc((void **)&dout, sizeof out));
  HIP_OK(hipMalloc((void **)&dgam, sizeof gam));
  HIP_OK(hipMalloc((void **)&dw, sizeof wg));
  for (int e = 0; e < E; ++e) {
    HIP_OK(hipMalloc((void **)&dz[e], sizeof z[e]));
    HIP_OK(hipMalloc((void **)&dr[e], sizeof z[e]));
    HIP_OK(hipMemcpy(dz[e], z[e], sizeof z[e], hipMemcpyHostToDevice));
  }
  HIP_OK(hipMemcpy(dx, x, sizeof x, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(dalpha, alpha, sizeof alpha, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(dbeta, beta, sizeof beta, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(dgam, gam, sizeof gam, hipMemcpyHostToDevice));
  size_t wbytes = sihc_weight_grad_workspace_size(E, B, G, K, C);
  const size_t tbytes = sihc_triangular_gamma_grad_workspace_size(E, M, C);
  if (tbytes > wbytes) wbytes = tbytes;
  HIP_OK(hipMalloc(&work, wbytes));
  void *zs[E], *rs[E];
  for (int e = 0; e < E; ++e) {
    zs[e] = dz[e];
    rs[e] = dr[e];
  }

  /* read: r_e[m,c] = sum_s alpha[e,c,s] x[m,s,c] */
  SIHC_OK_(sihc_read(dx, dalpha, rs, E, B, G, K, C, NULL, SIHC_DTYPE_F32, NULL));
  HIP_OK(hipDeviceSynchronize());
  for (int e = 0; e < E; ++e) {
    float got[NZ];
    HIP_OK(hipMemcpy(got, dr[e], sizeof got, hipMemcpyDeviceToHost));
    for (int m = 0; m < M; ++m)
      for (int c = 0; c < C; ++c) {
        double a = 0.0;
        for (int s = 0; s < S; ++s) a += (double)alpha[(e * C + c) * S + s] * x[xoff(m, s, c)];
        want_z[m * C + c] = a;
      }
    check("read", got, want_z, NZ, 1e-5);
  }

  /* write: out[m,s,c] = x + sum_e beta[e,c,s] z_e[m,c] */
  SIHC_OK_(sihc_write(dx, (const void *const *)zs, dbeta, dout, E, B, G, K, C, 1, NULL, SIHC_DTYPE_F32,
                      SIHC_DTYPE_F32, NULL));
  HIP_OK(hipMemcpy(out, dout, sizeof out, hipMemcpyDeviceToHost));
  for (int m = 0; m < M; ++m)
    for (int s = 0; s < S; ++s)
      for (int c = 0; c < C; ++c) {
        double a = x[xoff(m, s, c)];
        for (int e = 0; e < E; ++e) a += (double)beta[(e * C + c) * S + s] * z[e][m * C + c];
        want_x[xoff(m, s, c)] = a;
      }
  check("write (add_x)", out, want_x, NX, 1e-5);

  /* weight gradient: w[e,c,s] = sum_m x[m,s,c] z_e[m,c] */
  SIHC_OK_(sihc_weight_grad(dx, (const void *const *)zs, dw, E, B, G, K, C, NULL, SIHC_DTYPE_F32, SIHC_DTYPE_F32,
                            work, wbytes, NULL));
  HIP_OK(hipMemcpy(wg, dw, sizeof wg, hipMemcpyDeviceToHost));
  for (int e = 0; e < E; ++e)
    for (int c = 0; c < C; ++c)
      for (int s = 0; s < S; ++s) {
        double a = 0.0;
        for (int m = 0; m < M; ++m) a += (double)x[xoff(m, s, c)] * z[e][m * C + c];
        want_w[(e * C + c) * S + s] = a;
      }
  check("weight gradient", wg, want_w, E * C * S, 1e-5);

  /* triangular: t = z_0 + sum_{j<2} gamma[j] z_{j+1} (active prefix of 2) */
  SIHC_OK_(sihc_triangular(dz[0], (const void *const *)&zs[1], dgam, dout, 2, M, C, SIHC_DTYPE_F32,
                           SIHC_DTYPE_F32, NULL));
  {
    float got[NZ];
    HIP_OK(hipMemcpy(got, dout, sizeof got, hipMemcpyDeviceToHost));
    for (int i = 0; i < NZ; ++i) {
      const int c = i % C;
      want_z[i] = (double)z[0][i] + (double)gam[c] * z[1][i] + (double)gam[C + c] * z[2][i];
    }
    check("triangular", got, want_z, NZ, 1e-5);
  }

  /* fused triangular backward with grad = z_0: d_j = z_0 * gamma[j], dgamma[j] = sum z_0 z_{j+1} */
  SIHC_OK_(sihc_triangular_backward(dz[0], (const void *const *)&zs[1], dgam, rs, dw, 2, M, C, SIHC_DTYPE_F32,
                                    SIHC_DTYPE_F32, SIHC_DTYPE_F32, work, wbytes, NULL));
  for (int j = 0; j < 2; ++j) {
    float got[NZ];
    HIP_OK(hipMemcpy(got, dr[j], sizeof got, hipMemcpyDeviceToHost));
    for (int i = 0; i < NZ; ++i) want_z[i] = (double)z[0][i] * gam[j * C + i % C];
    check("triangular backward d_j", got, want_z, NZ, 1e-6);
  }
  {
    float got[2 * C];
    double want[2 * C];
    HIP_OK(hipMemcpy(got, dw, sizeof got, hipMemcpyDeviceToHost));
    for (int j = 0; j < 2; ++j)
      for (int c = 0; c < C; ++c) {
        double a = 0.0;
        for (int m = 0; m < M; ++m) a += (double)z[0][m * C + c] * z[j + 1][m * C + c];
        want[j * C + c] = a;
      }
    check("triangular backward dgamma", got, want, 2 * C, 1e-5);
  }

  /* per-event fused forward and backward, without and with a permutation state index */
  {
    static int32_t idx[M];
    for (int m = 0; m < M; ++m) idx[m] = (m % (G * G) * 7 + 3) % (G * G); /* 7 is coprime to G*G */
    int32_t *didx;
    HIP_OK(hipMalloc((void **)&didx, sizeof idx));
    HIP_OK(hipMemcpy(didx, idx, sizeof idx, hipMemcpyHostToDevice));
    static float xo[NX], gxo[NX], gx[NX], zo[NZ], gzo[NZ], gdz[NZ], gb[C * S], ga[C * S];
    static double want_b[C * S], want_a[C * S];
    for (int i = 0; i < NX; ++i) gxo[i] = 0.1f * rnd();
    for (int i = 0; i < NZ; ++i) gzo[i] = 0.1f * rnd();
    float *dxo, *dgxo, *dgx, *dzo, *dgzo, *dgdz, *dgb, *dga;
    void *ework;
    const size_t ebytes = sihc_event_backward_workspace_size(B, G, K, C);
    HIP_OK(hipMalloc((void **)&dxo, sizeof xo));
    HIP_OK(hipMalloc((void **)&dgxo, sizeof gxo));
    HIP_OK(hipMalloc((void **)&dgx, sizeof gx));
    HIP_OK(hipMalloc((void **)&dzo, sizeof zo));
    HIP_OK(hipMalloc((void **)&dgzo, sizeof gzo));
    HIP_OK(hipMalloc((void **)&dgdz, sizeof gdz));
    HIP_OK(hipMalloc((void **)&dgb, sizeof gb));
    HIP_OK(hipMalloc((void **)&dga, sizeof ga));
    HIP_OK(hipMalloc(&ework, ebytes));
    HIP_OK(hipMemcpy(dgxo, gxo, sizeof gxo, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(dgzo, gzo, sizeof gzo, hipMemcpyHostToDevice));
    const float *be = beta, *an = alpha + C * S; /* event 0's write, event 1's read */
    for (int use_idx = 0; use_idx < 2; ++use_idx) {
      const int32_t *hidx = use_idx ? idx : NULL;
      char name[64];
      /* forward: x_out = x + beta (.) dz at the token's cell, z_out = sum_s alpha' x_out */
      SIHC_OK_(sihc_event_forward(dx, dz[0], dbeta, dalpha + C * S, dxo, dzo, B, G, K, C, use_idx ? didx : NULL,
                                  SIHC_DTYPE_F32, NULL));
      HIP_OK(hipMemcpy(xo, dxo, sizeof xo, hipMemcpyDeviceToHost));
      HIP_OK(hipMemcpy(zo, dzo, sizeof zo, hipMemcpyDeviceToHost));
      for (int m = 0; m < M; ++m)
        for (int c = 0; c < C; ++c) {
          double a = 0.0;
          for (int s2 = 0; s2 < S; ++s2) {
            const long o = xoff_idx(hidx, m, s2, c);
            const float w = (float)((double)x[o] + (double)be[c * S + s2] * z[0][m * C + c]);
            want_x[o] = w;
            a += (double)an[c * S + s2] * w;
          }
          want_z[m * C + c] = a;
        }
      snprintf(name, sizeof name, "event forward x_out%s", use_idx ? " (index)" : "");
      check(name, xo, want_x, NX, 1e-6);
      snprintf(name, sizeof name, "event forward z_out%s", use_idx ? " (index)" : "");
      check(name, zo, want_z, NZ, 1e-5);
      /* backward: t = gxo + alpha' gzo; gx = t; gdz = sum_s beta t; gbeta = sum_m dz t;
         galpha' = sum_m x_out gzo */
      SIHC_OK_(sihc_event_backward(dgxo, dgzo, dxo, dz[0], dbeta, dalpha + C * S, dgx, dgdz, dgb, dga, B, G, K, C,
                                   use_idx ? didx : NULL, SIHC_DTYPE_F32, SIHC_DTYPE_F32, ework, ebytes, NULL));
      HIP_OK(hipMemcpy(gx, dgx, sizeof gx, hipMemcpyDeviceToHost));
      HIP_OK(hipMemcpy(gdz, dgdz, sizeof gdz, hipMemcpyDeviceToHost));
      HIP_OK(hipMemcpy(gb, dgb, sizeof gb, hipMemcpyDeviceToHost));
      HIP_OK(hipMemcpy(ga, dga, sizeof ga, hipMemcpyDeviceToHost));
      for (int i = 0; i < C * S; ++i) want_b[i] = want_a[i] = 0.0;
      for (int m = 0; m < M; ++m)
        for (int c = 0; c < C; ++c) {
          double d = 0.0;
          for (int s2 = 0; s2 < S; ++s2) {
            const long o = xoff_idx(hidx, m, s2, c);
            const double t = (double)gxo[o] + (double)an[c * S + s2] * gzo[m * C + c];
            want_x[o] = t;
            d += (double)be[c * S + s2] * t;
            want_b[c * S + s2] += (double)z[0][m * C + c] * t;
            want_a[c * S + s2] += (double)xo[o] * gzo[m * C + c];
          }
          want_z[m * C + c] = d;
        }
      snprintf(name, sizeof name, "event backward dX%s", use_idx ? " (index)" : "");
      check(name, gx, want_x, NX, 1e-6);
      snprintf(name, sizeof name, "event backward ddz%s", use_idx ? " (index)" : "");
      check(name, gdz, want_z, NZ, 1e-5);
      snprintf(name, sizeof name, "event backward dbeta%s", use_idx ? " (index)" : "");
      check(name, gb, want_b, C * S, 1e-5);
      snprintf(name, sizeof name, "event backward dalpha'%s", use_idx ? " (index)" : "");
      check(name, ga, want_a, C * S, 1e-5);
      /* the same backward twice as a chain: a deferred call (sihc_event_backward_partial),
         then a chained call whose trailing blocks finalize the first call's partial rows,
         then the finalize of the second call; every weight gradient bit-equal to
         sihc_event_backward's */
      {
        static float gb1[C * S], ga1[C * S], gb2[C * S], ga2[C * S];
        float *dgb1, *dga1, *dgb2, *dga2;
        void *ework2;
        int info1[2], info2[2];
        HIP_OK(hipMalloc((void **)&dgb1, sizeof gb1));
        HIP_OK(hipMalloc((void **)&dga1, sizeof ga1));
        HIP_OK(hipMalloc((void **)&dgb2, sizeof gb2));
        HIP_OK(hipMalloc((void **)&dga2, sizeof ga2));
        HIP_OK(hipMalloc(&ework2, ebytes));
        SIHC_OK_(sihc_event_backward_partial(dgxo, dgzo, dxo, dz[0], dbeta, dalpha + C * S, dgx, dgdz, dgb1, dga1,
                                             B, G, K, C, use_idx ? didx : NULL, SIHC_DTYPE_F32, SIHC_DTYPE_F32,
                                             ework, ebytes, info1, NULL));
        SIHC_OK_(sihc_event_backward_chain(dgxo, dgzo, dxo, dz[0], dbeta, dalpha + C * S, dgx, dgdz, dgb2, dga2, B,
                                           G, K, C, use_idx ? didx : NULL, SIHC_DTYPE_F32, SIHC_DTYPE_F32, ework2,
                                           ebytes, info2, ework, ebytes, info1, dgb1, dga1, NULL));
        const void *w2[1] = {ework2};
        const size_t n2[1] = {ebytes};
        void *gb2p[1] = {dgb2}, *ga2p[1] = {dga2};
        SIHC_OK_(sihc_event_finalize(1, w2, n2, info2, gb2p, ga2p, K, C, SIHC_DTYPE_F32, NULL));
        HIP_OK(hipMemcpy(gb1, dgb1, sizeof gb1, hipMemcpyDeviceToHost));
        HIP_OK(hipMemcpy(ga1, dga1, sizeof ga1, hipMemcpyDeviceToHost));
        HIP_OK(hipMemcpy(gb2, dgb2, sizeof gb2, hipMemcpyDeviceToHost));
        HIP_OK(hipMemcpy(ga2, dga2, sizeof ga2, hipMemcpyDeviceToHost));
        snprintf(name, sizeof name, "chain: carried dbeta%s", use_idx ? " (idx)" : "");
        bit_equal(name, gb1, gb, C * S);
        snprintf(name, sizeof name, "chain: carried dalpha'%s", use_idx ? " (idx)" : "");
        bit_equal(name, ga1, ga, C * S);
        snprintf(name, sizeof name, "chain: last dbeta%s", use_idx ? " (idx)" : "");
        bit_equal(name, gb2, gb, C * S);
        snprintf(name, sizeof name, "chain: last dalpha'%s", use_idx ? " (idx)" : "");
        bit_equal(name, ga2, ga, C * S);
        (void)hipFree(dgb1);
        (void)hipFree(dga1);
        (void)hipFree(dgb2);
        (void)hipFree(dga2);
        (void)hipFree(ework2);
      }
    }

    /* gather / scatter of whole cells: bit-exact copies; scatter(gather(x)) == x */
    {
      static float cells[M * S * C], want_cells[M * S * C], back[NX];
      float *dcells, *dback;
      HIP_OK(hipMalloc((void **)&dcells, sizeof cells));
      HIP_OK(hipMalloc((void **)&dback, sizeof back));
      SIHC_OK_(sihc_gather_cells(dx, didx, dcells, B, G, K, C, SIHC_DTYPE_F32, NULL));
      HIP_OK(hipMemcpy(cells, dcells, sizeof cells, hipMemcpyDeviceToHost));
      for (int m = 0; m < M; ++m)
        for (int s2 = 0; s2 < S; ++s2)
          for (int c = 0; c < C; ++c) want_cells[((long)m * S + s2) * C + c] = x[xoff_idx(idx, m, s2, c)];
      bit_equal("gather cells (index)", cells, want_cells, M * S * C);
      SIHC_OK_(sihc_scatter_cells(dcells, didx, dback, B, G, K, C, SIHC_DTYPE_F32, NULL));
      HIP_OK(hipMemcpy(back, dback, sizeof back, hipMemcpyDeviceToHost));
      bit_equal("scatter(gather(x)) == x", back, x, NX);
      (void)hipFree(dcells);
      (void)hipFree(dback);
    }
    (void)hipFree(didx);
    (void)hipFree(dxo);
    (void)hipFree(dgxo);
    (void)hipFree(dgx);
    (void)hipFree(dzo);
    (void)hipFree(dgzo);
    (void)hipFree(dgdz);
    (void)hipFree(dgb);
    (void)hipFree(dga);
    (void)hipFree(ework);
  }

  /* argument errors are reported before any launch */
  if (sihc_read(dx, dalpha, rs, E, B, G, 3, C, NULL, SIHC_DTYPE_F32, NULL) != SIHC_ERR_INVALID ||
      strlen(sihc_last_error()) == 0) {
    printf("argument error not reported: FAIL\n");
    ++failures;
  } else {
    printf("%-28s \"%s\" ok\n", "bad cell rejected", sihc_last_error());
  }

  for (int e = 0; e < E; ++e) {
    (void)hipFree(dz[e]);
    (void)hipFree(dr[e]);
  }
  (void)hipFree(dx);
  (void)hipFree(dalpha);
  (void)hipFree(dbeta);
  (void)hipFree(dout);
  (void)hipFree(dgam);
  (void)hipFree(dw);
  (void)hipFree(work);
  printf("%s\n", failures ? "FAILED" : "all checks passed");
  return failures ? 1 : 0;
}
