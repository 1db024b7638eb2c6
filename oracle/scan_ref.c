/*
 * TEST INFRASTRUCTURE ONLY -- CPU oracle for the Naju gated state-space scan.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * this library, and only as the checker. The product path (naju_amd/) never
 * calls it.
 *
 * This is a plain-C, fp64 restatement of the reference's sequential scan and of
 * its explicit recompute backward:
 *   forward  : /root/reference/naju/scan.py:79-93 (naju_scan_reference),
 *              semantics stated at scan.py:15-19
 *   backward : /root/reference/naju/cuda/naju_cuda.cu:104-141 (adjoint carry,
 *              d_f, sumdB, du/df/di, dB/dC accumulation) and :284 (dD = sum
 *              over batch of per-(b,d) sums)
 * Extension (absent from the reference, whose state always starts at zero,
 * scan.py:84): optional initial state h0 [B,D,N]; its gradient is
 * dh0 = f_0 * xbar_0, the adjoint carry that flows past t = 0.
 *
 * All inputs are fp32 arrays (bf16/fp16 data is upcast by the caller before
 * the call, the practice of reference tests/test_affine_chunk.py:149-153);
 * all arithmetic and outputs are fp64.
 *
 * Layouts (row-major, last index fastest), matching scan.py:7-11:
 *   u, fl, il, y, dy, du, dfl, dil : [Bsz, T, D]
 *   Bm, Cm, dB, dC                 : [Bsz, T, N]
 *   Dsk, dD                        : [D]
 *   h0, hT, dh0                    : [Bsz, D, N]
 *
 * Parity pins for this file (see tests/test_oracle.py): closed forms
 * (geometric series, f==0, f==1 prefix sum, i==0), torch autograd of the
 * independent torch-loop restatement in oracle/scan_ref.py, finite
 * differences, causality and channel independence.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static double sig(double x) { return 1.0 / (1.0 + exp(-x)); }

/* Forward: scan.py:82-93.  f = sigmoid(fl), i = sigmoid(il) (scan.py:82-83);
 * x = f*x + i*B*u (scan.py:90); y = sum_n C*x + D*u (scan.py:91).
 * hT (nullable) receives the final state x_{T-1}. */
void naju_oracle_fwd(const float* u, const float* fl, const float* il,
                     const float* Bm, const float* Cm, const float* Dsk,
                     const float* h0, int64_t Bsz, int64_t T, int64_t D,
                     int64_t N, double* y, double* hT) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t b = 0; b < Bsz; ++b) {
    for (int64_t d = 0; d < D; ++d) {
      double* x = (double*)malloc(sizeof(double) * (size_t)N);
      for (int64_t n = 0; n < N; ++n)
        x[n] = h0 ? (double)h0[(b * D + d) * N + n] : 0.0;
      for (int64_t t = 0; t < T; ++t) {
        const int64_t btd = (b * T + t) * D + d;
        const double f = sig(fl[btd]), i = sig(il[btd]), ut = u[btd];
        double acc = 0.0;
        for (int64_t n = 0; n < N; ++n) {
          const int64_t btn = (b * T + t) * N + n;
          x[n] = f * x[n] + i * (double)Bm[btn] * ut;
          acc += (double)Cm[btn] * x[n];
        }
        y[btd] = acc + (double)Dsk[d] * ut;
      }
      if (hT)
        for (int64_t n = 0; n < N; ++n) hT[(b * D + d) * N + n] = x[n];
      free(x);
    }
  }
}

/* Backward (adjoint of the forward above), following naju_cuda.cu:104-141:
 *   xbar_t[n] = C_t[n]*dy_t + f_{t+1}*xbar_{t+1}[n]          (:116, :120)
 *   dfl_t     = f_t(1-f_t) * sum_n xbar_t[n] * x_{t-1}[n]      (:123-126, :136)
 *   dws_t     = sum_n xbar_t[n] * B_t[n]                       (:129-132)
 *   du_t      = i_t*dws_t + D*dy_t                             (:138)
 *   dil_t     = dws_t * u_t * i_t(1-i_t)                       (:137)
 *   dB_t[n]   = sum_d xbar_t[d,n] * i_t[d] * u_t[d]            (:140)
 *   dC_t[n]   = sum_d dy_t[d] * x_t[d,n]                       (:118)
 *   dD[d]     = sum_{b,t} dy*u                                 (:119, :284)
 *   dh0[n]    = f_0 * xbar_0[n]                 (extension; zero-init ref)
 * Every output pointer is nullable.  dB/dC are reduced over d in a fixed
 * order (deterministic) from a [D,T,N] per-channel buffer per batch row. */
void naju_oracle_bwd(const float* u, const float* fl, const float* il,
                     const float* Bm, const float* Cm, const float* Dsk,
                     const float* h0, const float* dy, int64_t Bsz, int64_t T,
                     int64_t D, int64_t N, double* du, double* dfl,
                     double* dil, double* dB, double* dC, double* dD,
                     double* dh0) {
  double* dDacc = (double*)calloc((size_t)(Bsz * D), sizeof(double));
  /* Per (b, d) channel: recompute the forward state history, then run the
   * adjoint backwards.  Parallel over d inside each b; dB/dC partials are
   * accumulated per channel into a [D][T][N] scratch only when requested. */
  const int want_bc = (dB != NULL) || (dC != NULL);
  for (int64_t b = 0; b < Bsz; ++b) {
    double* pB = want_bc ? (double*)calloc((size_t)(D * T * N), sizeof(double)) : NULL;
    double* pC = want_bc ? (double*)calloc((size_t)(D * T * N), sizeof(double)) : NULL;
#pragma omp parallel for schedule(static)
    for (int64_t d = 0; d < D; ++d) {
      double* xs = (double*)malloc(sizeof(double) * (size_t)((T + 1) * N));
      double* xb = (double*)malloc(sizeof(double) * (size_t)N);
      /* xs[(t+1)*N + n] = x_t[n]; xs[0..N) = x_{-1} = h0 or 0 */
      for (int64_t n = 0; n < N; ++n) {
        xs[n] = h0 ? (double)h0[(b * D + d) * N + n] : 0.0;
        xb[n] = 0.0;
      }
      for (int64_t t = 0; t < T; ++t) {
        const int64_t btd = (b * T + t) * D + d;
        const double f = sig(fl[btd]), i = sig(il[btd]), ut = u[btd];
        for (int64_t n = 0; n < N; ++n)
          xs[(t + 1) * N + n] = f * xs[t * N + n] + i * (double)Bm[(b * T + t) * N + n] * ut;
      }
      double dDs = 0.0;
      double fnext = 1.0; /* f_{t+1}; unused at t = T-1 because xb == 0 */
      for (int64_t t = T - 1; t >= 0; --t) {
        const int64_t btd = (b * T + t) * D + d;
        const double f = sig(fl[btd]), i = sig(il[btd]), ut = u[btd];
        const double g = dy[btd];
        double sf = 0.0, sb = 0.0;
        for (int64_t n = 0; n < N; ++n) {
          const int64_t btn = (b * T + t) * N + n;
          xb[n] = (double)Cm[btn] * g + fnext * xb[n];
          sf += xb[n] * xs[t * N + n];
          sb += xb[n] * (double)Bm[btn];
          if (want_bc) {
            pB[(d * T + t) * N + n] = xb[n] * i * ut;
            pC[(d * T + t) * N + n] = g * xs[(t + 1) * N + n];
          }
        }
        if (dfl) dfl[btd] = sf * f * (1.0 - f);
        if (dil) dil[btd] = sb * ut * i * (1.0 - i);
        if (du) du[btd] = i * sb + (double)Dsk[d] * g;
        dDs += g * ut;
        fnext = f;
      }
      if (dh0)
        for (int64_t n = 0; n < N; ++n) dh0[(b * D + d) * N + n] = fnext * xb[n];
      dDacc[b * D + d] = dDs;
      free(xs);
      free(xb);
    }
    if (want_bc) {
#pragma omp parallel for schedule(static)
      for (int64_t tn = 0; tn < T * N; ++tn) {
        double sB = 0.0, sC = 0.0;
        for (int64_t d = 0; d < D; ++d) {
          sB += pB[d * T * N + tn];
          sC += pC[d * T * N + tn];
        }
        if (dB) dB[b * T * N + tn] = sB;
        if (dC) dC[b * T * N + tn] = sC;
      }
      free(pB);
      free(pC);
    }
  }
  if (dD)
    for (int64_t d = 0; d < D; ++d) {
      double s = 0.0;
      for (int64_t b = 0; b < Bsz; ++b) s += dDacc[b * D + d];
      dD[d] = s;
    }
  free(dDacc);
}

/* Per-channel forward on a subset of channels (for size-independent sliced
 * checks at the full benchmark shapes: y, du, dfl, dil are per-(b,d) independent).
 * chans[k] = b*D + d; outputs y_s[k*T + t]. */
void naju_oracle_fwd_channels(const float* u, const float* fl, const float* il,
                              const float* Bm, const float* Cm,
                              const float* Dsk, const float* h0, int64_t Bsz,
                              int64_t T, int64_t D, int64_t N,
                              const int64_t* chans, int64_t nch, double* y_s) {
  (void)Bsz;
#pragma omp parallel for schedule(dynamic)
  for (int64_t k = 0; k < nch; ++k) {
    const int64_t b = chans[k] / D, d = chans[k] % D;
    double* x = (double*)malloc(sizeof(double) * (size_t)N);
    for (int64_t n = 0; n < N; ++n) x[n] = h0 ? (double)h0[(b * D + d) * N + n] : 0.0;
    for (int64_t t = 0; t < T; ++t) {
      const int64_t btd = (b * T + t) * D + d;
      const double f = sig(fl[btd]), i = sig(il[btd]), ut = u[btd];
      double acc = 0.0;
      for (int64_t n = 0; n < N; ++n) {
        const int64_t btn = (b * T + t) * N + n;
        x[n] = f * x[n] + i * (double)Bm[btn] * ut;
        acc += (double)Cm[btn] * x[n];
      }
      y_s[k * T + t] = acc + (double)Dsk[d] * ut;
    }
    free(x);
  }
}

/* Per-channel backward on a subset of channels: du, dfl, dil ([nch, T]) and
 * dh0 ([nch, N]); same formulas as naju_oracle_bwd (naju_cuda.cu:104-141).
 * These outputs depend only on their own (b,d) channel, so a slice of
 * channels checks a full-size run. Any output pointer may be NULL. */
void naju_oracle_bwd_channels(const float* u, const float* fl, const float* il,
                              const float* Bm, const float* Cm,
                              const float* Dsk, const float* h0,
                              const float* dy, int64_t Bsz, int64_t T,
                              int64_t D, int64_t N, const int64_t* chans,
                              int64_t nch, double* du_s, double* dfl_s,
                              double* dil_s, double* dh0_s) {
  (void)Bsz;
#pragma omp parallel for schedule(dynamic)
  for (int64_t k = 0; k < nch; ++k) {
    const int64_t b = chans[k] / D, d = chans[k] % D;
    double* xs = (double*)malloc(sizeof(double) * (size_t)((T + 1) * N));
    double* xb = (double*)malloc(sizeof(double) * (size_t)N);
    for (int64_t n = 0; n < N; ++n) {
      xs[n] = h0 ? (double)h0[(b * D + d) * N + n] : 0.0;
      xb[n] = 0.0;
    }
    for (int64_t t = 0; t < T; ++t) {
      const int64_t btd = (b * T + t) * D + d;
      const double f = sig(fl[btd]), i = sig(il[btd]), ut = u[btd];
      for (int64_t n = 0; n < N; ++n)
        xs[(t + 1) * N + n] = f * xs[t * N + n] + i * (double)Bm[(b * T + t) * N + n] * ut;
    }
    double fnext = 1.0;
    for (int64_t t = T - 1; t >= 0; --t) {
      const int64_t btd = (b * T + t) * D + d;
      const double f = sig(fl[btd]), i = sig(il[btd]), ut = u[btd];
      const double g = dy[btd];
      double sf = 0.0, sb = 0.0;
      for (int64_t n = 0; n < N; ++n) {
        const int64_t btn = (b * T + t) * N + n;
        xb[n] = (double)Cm[btn] * g + fnext * xb[n];
        sf += xb[n] * xs[t * N + n];
        sb += xb[n] * (double)Bm[btn];
      }
      if (dfl_s) dfl_s[k * T + t] = sf * f * (1.0 - f);
      if (dil_s) dil_s[k * T + t] = sb * ut * i * (1.0 - i);
      if (du_s) du_s[k * T + t] = i * sb + (double)Dsk[d] * g;
      fnext = f;
    }
    if (dh0_s)
      for (int64_t n = 0; n < N; ++n) dh0_s[k * N + n] = fnext * xb[n];
    free(xs);
    free(xb);
  }
}
