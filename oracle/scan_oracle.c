/*
 * scan_oracle.c -- TEST INFRASTRUCTURE ONLY: a plain-C, float64 restatement of
 * the reference's selective scan, used as the checker for the gfx950 kernels.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it; the product path never does.
 *
 * Follows mamba_metal/scan.py of the reference:
 *   forward  -- the recurrence of scan.py:13-15 (and README.md:35-39), with
 *               checkpoints of h at the end of every chunk of K steps and at
 *               t = T-1 (scan.py:117-125);
 *   backward -- the adjoint recurrence of scan.py:22-34 (dx, ddt, dAneg, dB,
 *               dC), computed here from the fully stored h (no checkpoints),
 *               plus the gradient of the final state (dh_last), which the
 *               build's scan accepts and the reference drops (scan.py:390-393).
 *
 * Layouts are the reference's: x, dt, y, dy, dx, ddt (B,T,D); Bm, Cm, dB, dC
 * (B,T,N); aneg, daneg (D,N); ckpt (B,ceil(T/K),D,N); h_last (B,D,N).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

void oracle_scan_fwd(const double* x, const double* dt, const double* aneg,
                     const double* Bm, const double* Cm, double* y, double* ckpt,
                     double* h_last, int64_t Bt, int64_t T, int64_t D, int64_t N,
                     int64_t K) {
  const int64_t nchunk = K > 0 ? (T + K - 1) / K : 0;
  double* h = (double*)malloc(sizeof(double) * (size_t)N);
  for (int64_t b = 0; b < Bt; ++b) {
    for (int64_t d = 0; d < D; ++d) {
      for (int64_t n = 0; n < N; ++n) h[n] = 0.0;
      for (int64_t t = 0; t < T; ++t) {
        const int64_t e = (b * T + t) * D + d;
        const double dtv = dt[e];
        const double xv = x[e];
        double yv = 0.0;
        for (int64_t n = 0; n < N; ++n) {
          const double da = exp(-dtv * aneg[d * N + n]);
          const double inp = dtv * Bm[(b * T + t) * N + n] * xv;
          h[n] = da * h[n] + inp;
          yv += Cm[(b * T + t) * N + n] * h[n];
        }
        if (y) y[e] = yv;
        if (ckpt && K > 0 && ((t + 1) % K == 0 || t + 1 == T)) {
          const int64_t c = (t + 1) % K == 0 ? (t + 1) / K - 1 : nchunk - 1;
          double* dst = ckpt + ((b * nchunk + c) * D + d) * N;
          for (int64_t n = 0; n < N; ++n) dst[n] = h[n];
        }
      }
      if (h_last)
        for (int64_t n = 0; n < N; ++n) h_last[(b * D + d) * N + n] = h[n];
    }
  }
  free(h);
}

void oracle_scan_bwd(const double* x, const double* dt, const double* aneg,
                     const double* Bm, const double* Cm, const double* dy,
                     const double* dh_last, double* dx, double* ddt, double* daneg,
                     double* dB, double* dC, int64_t Bt, int64_t T, int64_t D, int64_t N) {
  /* h for one (b, d) over all t, plus the zero state in row 0: hs[(t+1)*N + n]. */
  double* hs = (double*)malloc(sizeof(double) * (size_t)((T + 1) * N));
  double* g = (double*)malloc(sizeof(double) * (size_t)N);
  memset(daneg, 0, sizeof(double) * (size_t)(D * N));
  memset(dB, 0, sizeof(double) * (size_t)(Bt * T * N));
  memset(dC, 0, sizeof(double) * (size_t)(Bt * T * N));
  for (int64_t b = 0; b < Bt; ++b) {
    for (int64_t d = 0; d < D; ++d) {
      for (int64_t n = 0; n < N; ++n) hs[n] = 0.0;
      for (int64_t t = 0; t < T; ++t) {
        const int64_t e = (b * T + t) * D + d;
        for (int64_t n = 0; n < N; ++n) {
          const double da = exp(-dt[e] * aneg[d * N + n]);
          hs[(t + 1) * N + n] = da * hs[t * N + n] + dt[e] * Bm[(b * T + t) * N + n] * x[e];
        }
      }
      for (int64_t n = 0; n < N; ++n) g[n] = dh_last ? dh_last[(b * D + d) * N + n] : 0.0;
      for (int64_t t = T - 1; t >= 0; --t) {
        const int64_t e = (b * T + t) * D + d;
        const double dtv = dt[e], xv = x[e], dyv = dy[e];
        double s_gb = 0.0, s_agh = 0.0;
        for (int64_t n = 0; n < N; ++n) {
          const int64_t s = (b * T + t) * N + n;
          /* G_t = dy_t C_t + dA_{t+1} G_{t+1}: g holds dA_{t+1} G_{t+1} (or dh_last). */
          const double gt = dyv * Cm[s] + g[n];
          const double da = exp(-dtv * aneg[d * N + n]);
          const double hm = da * hs[t * N + n];          /* dA_t h_{t-1} */
          s_gb += gt * Bm[s];
          s_agh += aneg[d * N + n] * gt * hm;
          daneg[d * N + n] -= dtv * gt * hm;
          dB[s] += gt * dtv * xv;
          dC[s] += dyv * hs[(t + 1) * N + n];
          g[n] = da * gt;                                  /* carried to t-1 */
        }
        dx[e] = dtv * s_gb;
        ddt[e] = xv * s_gb - s_agh;
      }
    }
  }
  free(hs);
  free(g);
}

/* One recurrent step in place (mamba_metal/model.py:234-241). */
void oracle_scan_step(double* h, const double* x, const double* dt, const double* aneg,
                      const double* Bm, const double* Cm, double* y, int64_t Bt, int64_t D,
                      int64_t N) {
  for (int64_t b = 0; b < Bt; ++b) {
    for (int64_t d = 0; d < D; ++d) {
      const double dtv = dt[b * D + d], xv = x[b * D + d];
      double yv = 0.0;
      for (int64_t n = 0; n < N; ++n) {
        double* hp = h + (b * D + d) * N + n;
        *hp = exp(-dtv * aneg[d * N + n]) * *hp + dtv * Bm[b * N + n] * xv;
        yv += Cm[b * N + n] * *hp;
      }
      y[b * D + d] = yv;
    }
  }
}
