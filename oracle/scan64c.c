/* Float64 CPU oracle of the fused Mamba-1 selective scan, in C with OpenMP — TEST
 * INFRASTRUCTURE ONLY (tests, smoke and the bench's CPU-baseline leg; never the product).
 *
 * The same restatement as oracle/scan64.py (numpy), written as plain loops so that the
 * full-size configurations (up to 16 x 2560 x 8192 x 16 state-steps) are checked in
 * seconds. Math followed:
 *   - recurrence and discretisation: mamba/selective_scan_cuda.py:56-90
 *     (a_bar = exp(delta*A); Euler b_bar = delta*B; ZOH b_bar = expm1(delta*A)/A*B;
 *     h_t = a_bar_t h_{t-1} + b_bar_t u_t from h_{-1} = x0; y = sum_n C h; final = h_{L-1});
 *   - chunk residual (prod a_bar, h) at 2048-step chunk ends: native/selective_scan_cuda.cu:306-320;
 *   - caller fusions: softplus(delta + bias) with the identity above 20
 *     (mamba/mamba1.py:117-126, 165; native/upstream_mamba/selective_scan_bwd_kernel.cuh:157),
 *     y += D u (mamba/mamba1.py:195-196), out = y silu(z) (mamba/mamba1.py:308, 332);
 *   - adjoint: native/upstream_mamba/selective_scan_bwd_kernel.cuh:175-203, 244-299, 442-485.
 * Variable length: steps t >= len_b are the identity, out is 0 there and every gradient
 * contribution of those steps is 0 (the build's contract, as in scan64.py).
 *
 * Besides each reduction gradient (dA, dB, dC, dD, dbias) the backward can return the sum
 * of the absolute values of the terms it adds up: the scale that bounds the rounding error
 * of any order of summation, used as the per-element tolerance of those gradients.
 *
 * Layouts (contiguous, float64): u, delta, z, out, y, dout, du, ddelta, dz: [B][D][L];
 * Bm, Cm, dB, dC: [B][N][L]; A, dA: [D][N]; Dv, bias, dD, dbias: [D]; x0, last, dlast,
 * dx0: [B][D][N]; ref_states: [B][D][ceil(L/2048)][N][2]; lens: int32 [B] or NULL.
 * Optional pointers may be NULL. */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define REF_CHUNK 2048
#define SOFTPLUS_THRESHOLD 20.0

static double softplus64(double x) { return x > SOFTPLUS_THRESHOLD ? x : log1p(exp(x)); }
static double sigmoid64(double x) { return 0.5 * (1.0 + tanh(0.5 * x)); }

static int row_len(const int* lens, int b, int L) {
  if (!lens) return L;
  int v = lens[b];
  return v < 0 ? 0 : (v > L ? L : v);
}

/* delta after bias, softplus and the length mask; also the pre-activation x. */
static void prep_delta(const double* drow, double bias, int softplus, int len, int L, double* dl,
                       double* xpre) {
  for (int t = 0; t < L; ++t) {
    const double x = drow[t] + bias;
    xpre[t] = x;
    dl[t] = t < len ? (softplus ? softplus64(x) : x) : 0.0;
  }
}

/* Forward of one (b, d) channel. hist (nullable): [L][N] states after each step. */
static void fwd_channel(int b, int d, int Dm, int L, int N, int zoh, const double* urow, const double* dl,
                        const double* A, const double* Bm, const double* Cm, double Dd, const double* x0,
                        double* h, double* prod, double* y, double* hist, double* ref_states, int n_ref) {
  for (int n = 0; n < N; ++n) {
    h[n] = x0 ? x0[((size_t)b * Dm + d) * N + n] : 0.0;
    prod[n] = 1.0;
  }
  const double* Ad = A + (size_t)d * N;
  for (int t = 0; t < L; ++t) {
    double acc = 0.0;
    for (int n = 0; n < N; ++n) {
      const double dA = dl[t] * Ad[n];
      const double ab = exp(dA);
      const double E = zoh ? expm1(dA) / Ad[n] : dl[t];
      const double bu = E * Bm[((size_t)b * N + n) * L + t] * urow[t];
      h[n] = ab * h[n] + bu;
      prod[n] *= ab;
      acc += Cm[((size_t)b * N + n) * L + t] * h[n];
      if (hist) hist[(size_t)t * N + n] = h[n];
    }
    y[t] = acc + Dd * urow[t];
    if (ref_states && ((t + 1) % REF_CHUNK == 0 || t == L - 1)) {
      const int c = t / REF_CHUNK;
      for (int n = 0; n < N; ++n) {
        double* rs = ref_states + ((((size_t)b * Dm + d) * n_ref + c) * N + n) * 2;
        rs[0] = prod[n];
        rs[1] = h[n];
      }
    }
  }
}

int scan64c_fwd(int Bsz, int Dm, int L, int N, int zoh, int softplus, const double* u, const double* delta,
                const double* A, const double* Bm, const double* Cm, const double* Dv, const double* z,
                const double* bias, const double* x0, const int* lens, double* out, double* y_out,
                double* last, double* ref_states) {
  if (Bsz <= 0 || Dm <= 0 || L <= 0 || N <= 0) return 1;
  const int n_ref = (L + REF_CHUNK - 1) / REF_CHUNK;
  int fail = 0;
#pragma omp parallel
  {
    double* dl = (double*)malloc(sizeof(double) * (size_t)L * 3 + sizeof(double) * 2 * N);
    if (!dl) {
#pragma omp atomic write
      fail = 1;
    }
#pragma omp barrier
    if (!fail) {
      double* xpre = dl + L;
      double* y = xpre + L;
      double* h = y + L;
      double* prod = h + N;
#pragma omp for schedule(static)
      for (long long ch = 0; ch < (long long)Bsz * Dm; ++ch) {
        const int b = (int)(ch / Dm), d = (int)(ch % Dm);
        const int len = row_len(lens, b, L);
        const double* urow = u + (size_t)ch * L;
        prep_delta(delta + (size_t)ch * L, bias ? bias[d] : 0.0, softplus, len, L, dl, xpre);
        fwd_channel(b, d, Dm, L, N, zoh, urow, dl, A, Bm, Cm, Dv ? Dv[d] : 0.0, x0, h, prod, y, NULL,
                    ref_states, n_ref);
        for (int t = 0; t < L; ++t) {
          double o = y[t];
          if (z) {
            const double zz = z[(size_t)ch * L + t];
            o *= zz * sigmoid64(zz);
          }
          out[(size_t)ch * L + t] = t < len ? o : 0.0;
          if (y_out) y_out[(size_t)ch * L + t] = y[t];
        }
        if (last)
          for (int n = 0; n < N; ++n) last[(size_t)ch * N + n] = h[n];
      }
    }
    free(dl);
  }
  return fail ? 2 : 0;
}

/* Backward. Gradient outputs are overwritten. *_abs (nullable): sums of |terms|. */
int scan64c_bwd(int Bsz, int Dm, int L, int N, int zoh, int softplus, const double* u, const double* delta,
                const double* A, const double* Bm, const double* Cm, const double* Dv, const double* z,
                const double* bias, const double* x0, const int* lens, const double* dout,
                const double* dlast, double* du, double* ddelta, double* dA, double* dB, double* dC,
                double* dD, double* dz, double* dbias, double* dx0, double* dA_abs, double* dB_abs,
                double* dC_abs, double* dD_abs, double* dbias_abs) {
  if (Bsz <= 0 || Dm <= 0 || L <= 0 || N <= 0) return 1;
  const size_t NL = (size_t)N * L;
  memset(dA, 0, sizeof(double) * (size_t)Dm * N);
  memset(dB, 0, sizeof(double) * Bsz * NL);
  memset(dC, 0, sizeof(double) * Bsz * NL);
  if (dD) memset(dD, 0, sizeof(double) * Dm);
  if (dbias) memset(dbias, 0, sizeof(double) * Dm);
  const int want_abs = dA_abs && dB_abs && dC_abs;
  if (want_abs) {
    memset(dA_abs, 0, sizeof(double) * (size_t)Dm * N);
    memset(dB_abs, 0, sizeof(double) * Bsz * NL);
    memset(dC_abs, 0, sizeof(double) * Bsz * NL);
  }
  if (dD_abs) memset(dD_abs, 0, sizeof(double) * Dm);
  if (dbias_abs) memset(dbias_abs, 0, sizeof(double) * Dm);
  int nthr = 1;
#ifdef _OPENMP
  nthr = omp_get_max_threads();
#endif
  /* per-thread dB/dC partials of one batch row ([N][L] each, plus their |term| sums) */
  double* part = (double*)calloc((size_t)nthr * NL * 4, sizeof(double));
  if (!part) return 2;
  int fail = 0;
  for (int b = 0; b < Bsz; ++b) {
    const int len = row_len(lens, b, L);
    memset(part, 0, sizeof(double) * (size_t)nthr * NL * 4);
#pragma omp parallel num_threads(nthr)
    {
      int tid = 0;
#ifdef _OPENMP
      tid = omp_get_thread_num();
#endif
      double* pB = part + (size_t)tid * NL * 4;
      double* pC = pB + NL;
      double* pBa = pC + NL;
      double* pCa = pBa + NL;
      const size_t per = (size_t)L * 8 + (size_t)N * 4 + (size_t)L * N;
      double* buf = (double*)malloc(sizeof(double) * per);
      if (!buf) {
#pragma omp atomic write
        fail = 1;
      }
#pragma omp barrier
      if (!fail) {
        double* dl = buf;
        double* xpre = dl + L;
        double* y = xpre + L;
        double* g = y + L;
        double* dub = g + L;
        double* ddl = dub + L;
        double* ddl_abs = ddl + L;
        double* s1 = ddl_abs + L;
        double* h = s1 + L;
        double* prod = h + N;
        double* mu = prod + N;
        double* x0n = mu + N;
        double* hist = x0n + N;
#pragma omp for schedule(static)
        for (int d = 0; d < Dm; ++d) {
          const size_t ch = (size_t)b * Dm + d;
          const double* urow = u + ch * L;
          const double* Ad = A + (size_t)d * N;
          prep_delta(delta + ch * L, bias ? bias[d] : 0.0, softplus, len, L, dl, xpre);
          fwd_channel(b, d, Dm, L, N, zoh, urow, dl, A, Bm, Cm, Dv ? Dv[d] : 0.0, x0, h, prod, y, hist,
                      NULL, 0);
          for (int n = 0; n < N; ++n) {
            x0n[n] = x0 ? x0[ch * N + n] : 0.0;
            mu[n] = dlast ? dlast[ch * N + n] : 0.0;
          }
          for (int t = 0; t < L; ++t) {
            const double go = t < len ? dout[ch * L + t] : 0.0;
            if (z) {
              const double zz = z[ch * L + t];
              const double sz = sigmoid64(zz);
              g[t] = go * zz * sz;
              if (dz) dz[ch * L + t] = t < len ? go * y[t] * sz * (1.0 + zz * (1.0 - sz)) : 0.0;
            } else {
              g[t] = go;
            }
            dub[t] = 0.0;
            ddl[t] = 0.0;
            ddl_abs[t] = 0.0;
          }
          for (int t = L - 1; t >= 0; --t) {
            const double ut = urow[t];
            double sum_lb = 0.0, sum_lb_abs = 0.0, sum_q = 0.0, sum_q_abs = 0.0;
            double sum_du = 0.0;
            for (int n = 0; n < N; ++n) {
              const double dAv = dl[t] * Ad[n];
              const double ab = exp(dAv);
              const double hp = t > 0 ? hist[(size_t)(t - 1) * N + n] : x0n[n];
              const double ht = hist[(size_t)t * N + n];
              const double Bt = Bm[((size_t)b * N + n) * L + t];
              const double Ct = Cm[((size_t)b * N + n) * L + t];
              const double lam = Ct * g[t] + mu[n];
              const double q = lam * Ad[n] * ab * hp; /* lambda A a_bar h_{t-1} */
              if (zoh) {
                const double E = expm1(dAv) / Ad[n];
                const double dEdA = (dl[t] * Ad[n] * ab - expm1(dAv)) / (Ad[n] * Ad[n]);
                sum_du += lam * Bt * E;
                const double r = lam * Bt * ut * ab;
                sum_q += q + r;
                sum_q_abs += fabs(q) + fabs(r);
                const double ta = lam * dl[t] * ab * hp, tb = lam * Bt * ut * dEdA;
                dA[(size_t)d * N + n] += ta + tb;
                const double tB = lam * E * ut;
                pB[(size_t)n * L + t] += tB;
                if (want_abs) {
                  dA_abs[(size_t)d * N + n] += fabs(ta) + fabs(tb);
                  pBa[(size_t)n * L + t] += fabs(tB);
                }
              } else {
                sum_lb += lam * Bt;
                sum_lb_abs += fabs(lam * Bt);
                sum_q += q;
                sum_q_abs += fabs(q);
                const double ta = lam * dl[t] * ab * hp;
                dA[(size_t)d * N + n] += ta;
                const double tB = lam * dl[t] * ut;
                pB[(size_t)n * L + t] += tB;
                if (want_abs) {
                  dA_abs[(size_t)d * N + n] += fabs(ta);
                  pBa[(size_t)n * L + t] += fabs(tB);
                }
              }
              const double tC = g[t] * ht;
              pC[(size_t)n * L + t] += tC;
              if (want_abs) pCa[(size_t)n * L + t] += fabs(tC);
              mu[n] = ab * lam;
            }
            if (zoh) {
              dub[t] = sum_du;
              ddl[t] = sum_q;
              ddl_abs[t] = sum_q_abs;
            } else {
              dub[t] = dl[t] * sum_lb;
              ddl[t] = sum_q + ut * sum_lb;
              ddl_abs[t] = sum_q_abs + fabs(ut) * sum_lb_abs;
            }
          }
          for (int n = 0; n < N; ++n)
            if (dx0) dx0[ch * N + n] = mu[n];
          double dDs = 0.0, dDa = 0.0, dbs = 0.0, dba = 0.0;
          const double Dd = Dv ? Dv[d] : 0.0;
          for (int t = 0; t < L; ++t) {
            const double valid = t < len ? 1.0 : 0.0;
            double duv = dub[t] + (Dv ? Dd * g[t] : 0.0);
            dDs += g[t] * urow[t];
            dDa += fabs(g[t] * urow[t]);
            double dx = ddl[t], dxa = ddl_abs[t];
            if (softplus && xpre[t] <= SOFTPLUS_THRESHOLD) {
              const double s = sigmoid64(xpre[t]);
              dx *= s;
              dxa *= s;
            }
            dx *= valid;
            dxa *= valid;
            du[ch * L + t] = duv * valid;
            ddelta[ch * L + t] = dx;
            dbs += dx;
            dba += dxa;
          }
          if (dD) dD[d] += dDs;
          if (dD_abs) dD_abs[d] += dDa;
          if (dbias) dbias[d] += dbs;
          if (dbias_abs) dbias_abs[d] += dba;
        }
      }
      free(buf);
    }
    if (fail) break;
    /* fixed-order sum of the per-thread partials */
    for (int k = 0; k < nthr; ++k) {
      const double* pB = part + (size_t)k * NL * 4;
      double* oB = dB + (size_t)b * NL;
      double* oC = dC + (size_t)b * NL;
      for (size_t i = 0; i < NL; ++i) {
        oB[i] += pB[i];
        oC[i] += pB[NL + i];
      }
      if (want_abs) {
        double* aB = dB_abs + (size_t)b * NL;
        double* aC = dC_abs + (size_t)b * NL;
        for (size_t i = 0; i < NL; ++i) {
          aB[i] += pB[2 * NL + i];
          aC[i] += pB[3 * NL + i];
        }
      }
    }
  }
  free(part);
  return fail ? 2 : 0;
}
