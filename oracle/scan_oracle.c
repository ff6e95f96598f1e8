/*
 * scan_oracle.c -- TEST INFRASTRUCTURE ONLY: a plain-C, float64 restatement of
 * the reference's selective scan, used as the checker for the gfx950 kernels.
 * Only tests/ and __graft_entry__.smoke() load it; the product path never
 * does.
 *
 * Follows mamba_metal/scan.py of the reference:
 *   forward  -- the recurrence of scan.py:13-15 (and README.md:35-39), with
 *               checkpoints of h at the end of every chunk of K steps and at
 *               t = T-1 (scan.py:117-125);
 *   conv     -- the block's causal depthwise conv1d + SiLU (model.py:174-175,
 *               :244), forward and backward (oracle_conv_fwd / _bwd below);
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

/*
 * Causal depthwise conv1d + SiLU, the reference block's
 * F.silu(nn.Conv1d(D, D, K, padding=K-1, groups=D)(x^T)[:, :, :T])
 * (mamba_metal/model.py:174-175, :244), on contiguous (B,T,D) x:
 *   pre[b,t,d] = bias[d] + sum_k w[d,k] x[b, t-K+1+k, d]  (x = 0 before t = 0)
 *   out = pre * sigmoid(pre)
 */
static double sig(double v) { return 1.0 / (1.0 + exp(-v)); }

static double conv_pre(const double* x, const double* w, const double* bias, int64_t b,
                       int64_t t, int64_t d, int64_t T, int64_t D, int64_t K) {
  double p = bias[d];
  for (int64_t k = 0; k < K; ++k) {
    const int64_t s = t - K + 1 + k;
    if (s >= 0) p += w[d * K + k] * x[(b * T + s) * D + d];
  }
  return p;
}

void oracle_conv_fwd(const double* x, const double* w, const double* bias, double* out,
                     int64_t Bt, int64_t T, int64_t D, int64_t K) {
  for (int64_t b = 0; b < Bt; ++b)
    for (int64_t t = 0; t < T; ++t)
      for (int64_t d = 0; d < D; ++d) {
        const double p = conv_pre(x, w, bias, b, t, d, T, D, K);
        out[(b * T + t) * D + d] = p * sig(p);
      }
}

/* Gradients of sum(out * dout) with respect to x, w and bias. */
void oracle_conv_bwd(const double* x, const double* w, const double* bias, const double* dout,
                     double* dx, double* dw, double* dbias, int64_t Bt, int64_t T, int64_t D,
                     int64_t K) {
  memset(dx, 0, sizeof(double) * (size_t)(Bt * T * D));
  memset(dw, 0, sizeof(double) * (size_t)(D * K));
  memset(dbias, 0, sizeof(double) * (size_t)D);
  for (int64_t b = 0; b < Bt; ++b)
    for (int64_t t = 0; t < T; ++t)
      for (int64_t d = 0; d < D; ++d) {
        const double p = conv_pre(x, w, bias, b, t, d, T, D, K);
        const double sg = sig(p);
        const double s = dout[(b * T + t) * D + d] * (sg + p * sg * (1.0 - sg));
        dbias[d] += s;
        for (int64_t k = 0; k < K; ++k) {
          const int64_t src = t - K + 1 + k;
          if (src < 0) continue;
          dw[d * K + k] += s * x[(b * T + src) * D + d];
          dx[(b * T + src) * D + d] += s * w[d * K + k];
        }
      }
}
